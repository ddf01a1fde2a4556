"""The C-ABI library loads, exports every symbol include/attnkernels.h declares,
and rejects bad arguments before touching a GPU (runs on the CPU)."""
import ctypes
import re

import pytest

from conftest import ROOT, PKG_DIR

HEADER = ROOT / "include" / "attnkernels.h"
LIB = PKG_DIR / "attnkernels" / "libattnkernels.so"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ak_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        from attnkernels import build
        build.build_library()
    import torch  # noqa: F401  -- share torch's HIP runtime, as in real use
    L = ctypes.CDLL(str(LIB))
    L.ak_last_error.restype = ctypes.c_char_p
    vp, i64, f64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_double
    L.ak_flash_wmma.argtypes = [vp] * 4 + [i64] * 4 + [ctypes.c_int, f64, i64, vp]
    L.ak_flash_simt.argtypes = [vp] * 4 + [i64] * 4 + [ctypes.c_int, f64, vp]
    L.ak_naive_attention.argtypes = [vp] * 4 + [i64] * 4 + [ctypes.c_int, f64, vp]
    L.ak_paged_decode_workspace_size.argtypes = [i64] * 5
    L.ak_paged_decode_workspace_size.restype = ctypes.c_size_t
    L.ak_paged_decode.argtypes = [vp] * 6 + [i64] * 8 + [f64, i64, vp, ctypes.c_size_t, vp]
    L.ak_reshape_and_cache.argtypes = [vp] * 5 + [i64] * 7 + [vp]
    L.ak_paged_decode_noalloc.argtypes = [vp] * 6 + [i64] * 8 + [f64, i64, vp]
    L.ak_paged_decode_fused.argtypes = [vp] * 6 + [i64] * 8 + [f64, i64, vp, ctypes.c_size_t, vp, i64, vp]
    L.ak_prefill_gqa.argtypes = [vp] * 4 + [i64] * 5 + [ctypes.c_int, f64, vp]
    L.ak_prefill_varlen.argtypes = [vp] * 5 + [i64] * 6 + [ctypes.c_int, f64, vp]
    return L


def test_header_declares_the_reference_entry_points():
    names = declared_functions()
    for n in ("ak_naive_attention", "ak_flash_simt", "ak_flash_wmma", "ak_paged_decode",
              "ak_paged_decode_workspace_size", "ak_last_error", "ak_abi_version"):
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.ak_abi_version() == 101


FAKE = ctypes.c_void_p(4096)  # never dereferenced: validation fails first


@pytest.mark.parametrize("d,bn", [(32, 64), (64, 16), (256, 32)])
def test_flash_wmma_rejects_unsupported_config(lib, d, bn):
    rc = lib.ak_flash_wmma(FAKE, FAKE, FAKE, FAKE, 1, 1, 16, d, 0, 0.1, bn, None)
    assert rc == 2
    assert b"head_dim must be 64 or 128 and block_n 32 or 64" in lib.ak_last_error()


def test_simt_and_naive_reject_head_dim(lib):
    assert lib.ak_flash_simt(FAKE, FAKE, FAKE, FAKE, 1, 1, 16, 96, 0, 0.1, None) == 2
    assert b"flash_simt: head_dim must be 64 or 128" in lib.ak_last_error()
    assert lib.ak_naive_attention(FAKE, FAKE, FAKE, FAKE, 1, 1, 16, 96, 0, 0.1, None) == 2


def test_prefill_rejects_misaligned_and_null(lib):
    bad = ctypes.c_void_p(4098)
    assert lib.ak_flash_wmma(bad, FAKE, FAKE, FAKE, 1, 1, 16, 64, 0, 0.1, 64, None) == 1
    assert b"16-byte aligned" in lib.ak_last_error()
    assert lib.ak_flash_wmma(None, FAKE, FAKE, FAKE, 1, 1, 16, 64, 0, 0.1, 64, None) == 1
    assert lib.ak_flash_wmma(FAKE, FAKE, FAKE, FAKE, 1, -1, 16, 64, 0, 0.1, 64, None) == 1


def test_prefill_empty_is_a_no_op(lib):
    assert lib.ak_flash_wmma(None, None, None, None, 0, 4, 16, 64, 1, 0.1, 64, None) == 0
    assert lib.ak_flash_simt(None, None, None, None, 2, 4, 0, 128, 0, 0.1, None) == 0


def decode(lib, **kw):
    a = dict(q=FAKE, kc=FAKE, vc=FAKE, bt=FAKE, cl=FAKE, out=FAKE, B=2, hq=8, hkv=2, d=128, nb=10,
             bs=16, maxb=4, max_ctx=64, scale=0.1, part=256, ws=None, ws_bytes=0)
    a.update(kw)
    return lib.ak_paged_decode(a["q"], a["kc"], a["vc"], a["bt"], a["cl"], a["out"], a["B"], a["hq"],
                               a["hkv"], a["d"], a["nb"], a["bs"], a["maxb"], a["max_ctx"], a["scale"],
                               a["part"], a["ws"], a["ws_bytes"], None)


def test_paged_decode_checks_in_reference_order(lib):
    assert decode(lib, hq=6, hkv=4, part=100) == 1
    assert lib.ak_last_error() == b"num_heads must be a multiple of num_kv_heads"
    assert decode(lib, part=100) == 1
    assert lib.ak_last_error() == b"partition size must be a positive multiple of 256"
    assert decode(lib, d=96) == 2
    assert b"head_dim must be 64/128 and num_heads/num_kv_heads in {1,2,4,8}" in lib.ak_last_error()
    assert decode(lib, hq=32, hkv=2) == 2  # G = 16 is not built


def test_paged_decode_requires_workspace_for_splits(lib):
    need = lib.ak_paged_decode_workspace_size(2, 8, 128, 1000, 256)
    assert need == 2 * 8 * 4 * (128 + 2) * 4
    assert decode(lib, max_ctx=1000, ws=None, ws_bytes=0) == 3
    assert b"workspace" in lib.ak_last_error()
    assert decode(lib, max_ctx=1000, ws=FAKE, ws_bytes=need - 4) == 3
    assert lib.ak_paged_decode_workspace_size(2, 8, 128, 256, 256) == 0   # one split
    assert lib.ak_paged_decode_workspace_size(2, 8, 128, 1000, 0) == 0    # invalid


def test_paged_decode_rejects_bad_sizes(lib):
    assert decode(lib, max_ctx=0) == 1
    assert decode(lib, bs=0) == 1
    assert decode(lib, maxb=0) == 1
    assert decode(lib, B=0) == 0  # nothing to do


def test_reshape_and_cache_validation(lib):
    # key, value, k_cache, v_cache, slots, T, Hkv, D, num_blocks, bs, key_stride, value_stride
    rc = lib.ak_reshape_and_cache(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 8, 12, 10, 16, 96, 96, None)
    assert rc == 2 and b"head_dim must be a multiple of 8" in lib.ak_last_error()
    rc = lib.ak_reshape_and_cache(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 8, 128, 10, 16, 512, 1024, None)
    assert rc == 1 and b"token strides" in lib.ak_last_error()
    rc = lib.ak_reshape_and_cache(FAKE, FAKE, FAKE, FAKE, FAKE, 4, 8, 128, 10, 16, 1028, 1024, None)
    assert rc == 1 and b"token strides" in lib.ak_last_error()
    rc = lib.ak_reshape_and_cache(FAKE, FAKE, FAKE, FAKE, FAKE, -1, 8, 128, 10, 16, 1024, 1024, None)
    assert rc == 1 and b"invalid size" in lib.ak_last_error()
    rc = lib.ak_reshape_and_cache(FAKE, None, FAKE, FAKE, FAKE, 4, 8, 128, 10, 16, 1024, 1024, None)
    assert rc == 1 and b"null pointer" in lib.ak_last_error()
    rc = lib.ak_reshape_and_cache(ctypes.c_void_p(4104), FAKE, FAKE, FAKE, FAKE, 4, 8, 128, 10, 16, 1024, 1024,
                                  None)
    assert rc == 1 and b"16-byte aligned" in lib.ak_last_error()
    # nothing to write: no GPU work, no pointer use
    assert lib.ak_reshape_and_cache(None, None, None, None, None, 0, 8, 128, 10, 16, 1024, 1024, None) == 0
    assert lib.ak_reshape_and_cache(None, None, None, None, None, 4, 8, 128, 0, 16, 1024, 1024, None) == 0


def test_gqa_and_varlen_validation(lib):
    # q, k, v, o, B, H, H_kv, N, D, causal, scale
    rc = lib.ak_prefill_gqa(FAKE, FAKE, FAKE, FAKE, 1, 6, 4, 16, 64, 0, 0.1, None)
    assert rc == 1 and b"multiple of num_kv_heads" in lib.ak_last_error()
    rc = lib.ak_prefill_gqa(FAKE, FAKE, FAKE, FAKE, 1, 8, 2, 16, 96, 0, 0.1, None)
    assert rc == 2 and b"head_dim must be 64 or 128" in lib.ak_last_error()
    assert lib.ak_prefill_gqa(None, None, None, None, 0, 8, 2, 16, 64, 0, 0.1, None) == 0
    # q, k, v, o, cu, B, total, H, H_kv, max_seqlen, D, causal, scale
    rc = lib.ak_prefill_varlen(FAKE, FAKE, FAKE, FAKE, None, 2, 100, 8, 2, 64, 128, 1, 0.1, None)
    assert rc == 1 and b"cu_seqlens" in lib.ak_last_error()
    rc = lib.ak_prefill_varlen(FAKE, FAKE, FAKE, FAKE, ctypes.c_void_p(4098), 2, 100, 8, 2, 64, 128, 1, 0.1, None)
    assert rc == 1 and b"cu_seqlens" in lib.ak_last_error()
    rc = lib.ak_prefill_varlen(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 100, 8, 3, 64, 128, 1, 0.1, None)
    assert rc == 1 and b"multiple of num_kv_heads" in lib.ak_last_error()
    assert lib.ak_prefill_varlen(FAKE, FAKE, FAKE, FAKE, FAKE, 2, 0, 8, 2, 64, 128, 1, 0.1, None) == 0


def test_noalloc_decode_rejects_oversized_partials_before_any_hip_call(lib):
    # 64 x 32 heads x 4096 splits x (128 + 2) floats = 4.4 GB > the 32 MiB static array
    rc = lib.ak_paged_decode_noalloc(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 64, 32, 8, 128, 100, 16, 65536,
                                     1 << 20, 0.1, 256, None)
    assert rc == 3
    assert b"static scratch" in lib.ak_last_error()
    # the shared validation still applies first
    assert lib.ak_paged_decode_noalloc(FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1, 6, 4, 128, 100, 16, 8, 100,
                                       0.1, 256, None) == 1


def test_fused_decode_validates_counters_before_any_hip_call(lib):
    """ak_paged_decode_fused rejects a counter array shorter than batch *
    num_kv_heads, or misaligned, before touching the GPU."""
    need = lib.ak_paged_decode_workspace_size(2, 8, 128, 1000, 256)
    args = [FAKE] * 6 + [2, 8, 4, 128, 64, 16, 63, 1000, 0.1, 256, FAKE, need]
    assert lib.ak_paged_decode_fused(*args, FAKE, 7, None) == 1
    assert b"counters" in lib.ak_last_error()
    assert lib.ak_paged_decode_fused(*args, ctypes.c_void_p(4098), 8, None) == 1
    assert b"counters" in lib.ak_last_error()


def test_stream_checksum_validates_before_any_hip_call(lib):
    lib.ak_stream_checksum.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
    assert lib.ak_stream_checksum(FAKE, 24, FAKE, None) == 1  # not a multiple of 16 bytes
    assert b"multiple of 16" in lib.ak_last_error()
    assert lib.ak_stream_checksum(ctypes.c_void_p(4104), 32, FAKE, None) == 1  # src misaligned
    assert lib.ak_stream_checksum(FAKE, 32, None, None) == 1  # no output
    assert lib.ak_stream_checksum(None, 0, FAKE, None) == 0  # nothing to read
