"""ctypes loader for the float64 brute-force oracle (attn_f64.c) -- test infrastructure."""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB = _HERE / "_build" / "libattn_f64.so"
_lib = None


def build(force=False):
    """Compile attn_f64.c with gcc (via oracle/Makefile) into oracle/_build/."""
    if force or not _LIB.exists():
        subprocess.run(["make", "-s", "-C", str(_HERE)] + (["-B"] if force else []), check=True)
    return _LIB


def _load():
    global _lib
    if _lib is None:
        build()
        lib = ctypes.CDLL(str(_LIB))
        p, i64, f64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_double
        lib.oracle_attention_f64.argtypes = [p, p, p, p, i64, i64, i64, ctypes.c_int, f64]
        lib.oracle_attention_f64.restype = ctypes.c_int
        lib.oracle_paged_decode_f64.argtypes = [p, p, p, p, p, p] + [i64] * 7 + [f64]
        lib.oracle_paged_decode_f64.restype = ctypes.c_int
        _lib = lib
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def attention_f64(q, k, v, causal=False, scale=None):
    """softmax(scale*QK^T [+ mask]) V in float64; q, k, v: [..., N, D]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    n, d = q.shape[-2], q.shape[-1]
    scale = 1.0 / np.sqrt(d) if scale is None else float(scale)
    out = np.empty(q.shape, dtype=np.float64)
    bh = int(np.prod(q.shape[:-2], dtype=np.int64))
    rc = _load().oracle_attention_f64(_ptr(q), _ptr(k), _ptr(v), _ptr(out), bh, n, d,
                                      int(bool(causal)), float(scale))
    if rc != 0:
        raise RuntimeError("oracle_attention_f64 failed")
    return out


def paged_decode_f64(q, k_cache, v_cache, block_tables, context_lens, scale=None):
    """Paged decode in float64 through explicit page-index arithmetic; q: [B, Hq, D]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    kc = np.ascontiguousarray(k_cache, dtype=np.float32)
    vc = np.ascontiguousarray(v_cache, dtype=np.float32)
    bt = np.ascontiguousarray(block_tables, dtype=np.int32)
    cl = np.ascontiguousarray(context_lens, dtype=np.int32)
    B, hq, d = q.shape
    nb, hkv, bs = kc.shape[0], kc.shape[1], kc.shape[2]
    scale = 1.0 / np.sqrt(d) if scale is None else float(scale)
    out = np.empty((B, hq, d), dtype=np.float64)
    rc = _load().oracle_paged_decode_f64(_ptr(q), _ptr(kc), _ptr(vc), _ptr(bt), _ptr(cl),
                                         _ptr(out), B, hq, hkv, d, nb, bs, bt.shape[1],
                                         float(scale))
    if rc != 0:
        raise ValueError("oracle_paged_decode_f64: page id or context length out of range")
    return out
