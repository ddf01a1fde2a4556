"""CPU oracle for the attention hot path -- test infrastructure, not product.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker: no kernel entry
point of ``attnkernels`` calls it, and the product fails loudly when its HIP
library is missing instead of falling back here.

Every function restates an algorithm of sonhoang/flash-attention-from-scratch
(cited as ``file:line`` of that repository) in numpy float32, the precision of
the reference's own oracle ``attnkernels/reference.py``.  What pins each
function (closed forms, a float64 brute force written independently in C in
``attn_f64.c``, torch's CPU attention routine, the reference's recorded
``decode_partition`` values, planted-mistake checks) lives in
``tests/test_oracle.py``.  No function here is left "parity unpinned".

``reshape_and_cache`` and ``append_slots`` restate the paged-cache writer,
which has no counterpart in the reference: they follow the cache layout the
reference reads (attnkernels/reference.py:21-51, paged_decode.cu:95-96) and are
pinned by round trips through ``gather_kv`` and an element-wise loop.
"""
from __future__ import annotations

import math

import numpy as np

LOG2E = 1.4426950408889634  # log2(e): kernels use exp(x) = 2^(x*log2 e) (README.md:80-82)
CHUNK = 256                 # partitions are multiples of it (attnkernels/__init__.py:29)


def _as_f32(x):
    return np.asarray(x).astype(np.float32, copy=False)


def attention_fp32(q, k, v, causal=False, scale=None):
    """Exact attention in float32: softmax(scale*Q K^T [+ causal mask]) V.

    Follows attnkernels/reference.py:9-18: scores in fp32, key j is masked
    (-inf) for query i iff j > i (``triu(1)``), row softmax, then P V.
    q, k, v: [..., N, D] of any float dtype (fp16 inputs are upcast exactly).
    The leading dims are processed one slice at a time so memory stays
    O(N^2) for a single (batch, head).
    """
    q, k, v = _as_f32(q), _as_f32(k), _as_f32(v)
    n, d = q.shape[-2], q.shape[-1]
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    lead = q.shape[:-2]
    qf = q.reshape(-1, n, d)
    kf = k.reshape(-1, k.shape[-2], d)
    vf = v.reshape(-1, v.shape[-2], v.shape[-1])
    out = np.empty((qf.shape[0], n, vf.shape[-1]), dtype=np.float32)
    mask = np.triu(np.ones((n, kf.shape[1]), dtype=bool), 1) if causal else None
    for i in range(qf.shape[0]):
        s = (qf[i] @ kf[i].T) * np.float32(scale)
        if mask is not None:
            s[mask] = -np.inf
        s -= s.max(axis=-1, keepdims=True)
        np.exp(s, out=s)
        s /= s.sum(axis=-1, keepdims=True)
        out[i] = s @ vf[i]
    return out.reshape(*lead, n, vf.shape[-1])


def prefill_flops(batch, heads, seq, head_dim, causal):
    """Algorithmic prefill FLOP: 4*B*H*N^2*D, halved if causal (bench/bench.py:153)."""
    return 4.0 * batch * heads * seq * seq * head_dim * (0.5 if causal else 1.0)


def decode_kv_bytes(context_lens, num_kv_heads, head_dim):
    """Useful K+V bytes of one decode step: sum(ctx)*Hkv*D*2 (K and V)*2 B (bench/bench.py:199-200)."""
    return int(sum(int(c) for c in context_lens)) * num_kv_heads * head_dim * 2 * 2


def decode_partition(batch, num_kv_heads, max_context_len, sm_count, wg_per_sm=4):
    """Tokens per split, attnkernels/__init__.py:93-101.

    want = ceil(wg_per_sm*SMs / (B*Hkv)); splits = clamp(want, 1, ceil(max_ctx/256));
    partition = ceil(chunks/splits)*256.  The reference's factor is 4.
    """
    blocks = batch * num_kv_heads
    want = -(-wg_per_sm * sm_count // blocks)
    max_chunks = -(-max_context_len // CHUNK)
    splits = max(1, min(want, max_chunks))
    return -(-max_chunks // splits) * CHUNK


def round_partition(partition):
    """Round a partition up to a multiple of 256 (attnkernels/__init__.py:124)."""
    return -(-int(partition) // CHUNK) * CHUNK


def make_paged_cache(context_lens, num_kv_heads, head_dim, block_size=16, extra_blocks=0,
                     seed=0, dtype=np.float16):
    """Random K/V caches and block tables, attnkernels/reference.py:21-44.

    Each sequence needs ceil(ctx/bs) pages; the pool holds their sum plus
    ``extra_blocks``; physical pages are handed out by a seeded random
    permutation, sequence after sequence; unused table slots are page 0.
    Returns (k_cache, v_cache [pool, Hkv, bs, D], block_tables int32
    [B, max_blocks], context_lens int32 [B]).
    """
    rng = np.random.default_rng(seed)
    nblk = [-(-int(c) // block_size) for c in context_lens]
    total = sum(nblk) + int(extra_blocks)
    perm = rng.permutation(total).astype(np.int32)
    tables = np.zeros((len(context_lens), max(nblk)), dtype=np.int32)
    pos = 0
    for b, nb in enumerate(nblk):
        tables[b, :nb] = perm[pos:pos + nb]
        pos += nb
    shape = (total, num_kv_heads, block_size, head_dim)
    k_cache = rng.standard_normal(shape, dtype=np.float32).astype(dtype)
    v_cache = rng.standard_normal(shape, dtype=np.float32).astype(dtype)
    return k_cache, v_cache, tables, np.asarray(context_lens, dtype=np.int32)


def gather_kv(cache, block_tables, n_blocks):
    """[num_blocks, Hkv, bs, D] -> [B, Hkv, n_blocks*bs, D], attnkernels/reference.py:47-51.

    Token t of sequence b is cache[block_tables[b, t // bs], :, t % bs, :].
    """
    g = np.asarray(cache)[np.asarray(block_tables)[:, :n_blocks].astype(np.int64)]
    b, nb, h, bs, d = g.shape
    return g.transpose(0, 2, 1, 3, 4).reshape(b, h, nb * bs, d)


def paged_decode_fp32(q, k_cache, v_cache, block_tables, context_lens, scale=None):
    """Per-sequence float32 paged decode, attnkernels/reference.py:54-70.

    q: [B, Hq, D].  Query head h reads kv head h // G with G = Hq/Hkv
    (``repeat_interleave``, reference.py:66-67; paged_decode.cu:68,183).
    """
    q = _as_f32(q)
    B, H, D = q.shape
    hkv, bs = k_cache.shape[1], k_cache.shape[2]
    g = H // hkv
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    tables = np.asarray(block_tables)
    out = np.empty((B, H, D), dtype=np.float32)
    for b in range(B):
        c = int(context_lens[b])
        nb = -(-c // bs)
        kk = _as_f32(gather_kv(k_cache, tables[b:b + 1], nb)[0, :, :c])  # [Hkv, c, D]
        vv = _as_f32(gather_kv(v_cache, tables[b:b + 1], nb)[0, :, :c])
        kk = np.repeat(kk, g, axis=0)
        vv = np.repeat(vv, g, axis=0)
        # batched matrix products (BLAS): [H, c, D] x [H, D, 1] and [H, 1, c] x [H, c, D]
        s = np.matmul(kk, q[b][:, :, None])[..., 0] * np.float32(scale)
        s -= s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        out[b] = np.matmul(p[:, None, :], vv)[:, 0, :]
    return out


def split_partials(q, k_cache, v_cache, block_tables, context_lens, partition, num_splits,
                   scale=None):
    """Per-split softmax partials in the log2 domain, as paged_decode.cu:39-194 defines them.

    For split s of sequence b covering tokens [s*P, min(ctx, (s+1)*P)):
    x_t = (q*scale*log2e).k_t, m = max x_t, l = sum 2^(x_t - m),
    o = sum 2^(x_t - m) v_t / l.  Splits past the context are left as
    m = -inf, l = 0, o = 0 (the kernel never writes them, paged_decode.cu:61-62).
    Returns m, l [B, Hq, S] and o [B, Hq, S, D], all float32.
    """
    q = _as_f32(q)
    B, H, D = q.shape
    hkv, bs = k_cache.shape[1], k_cache.shape[2]
    g = H // hkv
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    sl2 = np.float32(scale * LOG2E)
    tables = np.asarray(block_tables)
    m = np.full((B, H, num_splits), -np.inf, dtype=np.float32)
    l = np.zeros((B, H, num_splits), dtype=np.float32)
    o = np.zeros((B, H, num_splits, D), dtype=np.float32)
    for b in range(B):
        c = int(context_lens[b])
        nb = -(-c // bs)
        kk = np.repeat(_as_f32(gather_kv(k_cache, tables[b:b + 1], nb)[0, :, :c]), g, axis=0)
        vv = np.repeat(_as_f32(gather_kv(v_cache, tables[b:b + 1], nb)[0, :, :c]), g, axis=0)
        x = np.einsum("hd,hcd->hc", q[b] * sl2, kk)
        for s in range(num_splits):
            lo, hi = s * partition, min(c, (s + 1) * partition)
            if lo >= hi:
                continue
            xs = x[:, lo:hi]
            ms = xs.max(axis=-1)
            p = np.exp2(xs - ms[:, None])
            ls = p.sum(axis=-1)
            m[b, :, s] = ms
            l[b, :, s] = ls
            o[b, :, s] = np.einsum("hc,hcd->hd", p, vv[:, lo:hi]) / ls[:, None]
    return m, l, o


def merge_partials(m, l, o, context_lens, partition):
    """LSE merge of split partials, paged_decode.cu:196-216.

    ns = ceil(ctx/P) splits are read; M = max m_s; w_s = l_s*2^(m_s - M);
    O = sum w_s o_s / sum w_s.  Returns float32 [B, Hq, D].
    """
    B, H, S = m.shape
    out = np.empty((B, H, o.shape[-1]), dtype=np.float32)
    for b in range(B):
        ns = min(S, -(-int(context_lens[b]) // partition))
        mb, lb, ob = m[b, :, :ns], l[b, :, :ns], o[b, :, :ns]
        M = mb.max(axis=-1, keepdims=True)
        w = lb * np.exp2(mb - M)
        out[b] = np.einsum("hs,hsd->hd", w, ob) / w.sum(axis=-1)[:, None]
    return out


def paged_decode_splitk(q, k_cache, v_cache, block_tables, context_lens, max_context_len,
                        partition, scale=None):
    """Split-K decode as the reference's kernel pair computes it (paged_decode.cu:256-277):
    S = ceil(max_ctx/P) splits of per-split partials, then the LSE merge.  With
    S == 1 the single split's normalised o is the output (paged_decode.cu:184-185)."""
    S = -(-int(max_context_len) // int(partition))
    m, l, o = split_partials(q, k_cache, v_cache, block_tables, context_lens, partition, S,
                             scale)
    if S == 1:
        return o[:, :, 0]
    return merge_partials(m, l, o, context_lens, partition)


def append_slots(block_tables, positions, block_size):
    """Cache slot of token ``positions[b]`` of sequence b: the page the block
    table holds for it times block_size plus the row in the page (the address
    map of paged_decode.cu:95-96 / reference.py:47-51, written as one index).
    A negative position gives slot -1 (skip)."""
    bt = np.asarray(block_tables)
    pos = np.asarray(positions, dtype=np.int64)
    slots = np.full(pos.shape, -1, dtype=np.int64)
    ok = pos >= 0
    rows = np.nonzero(ok)[0]
    slots[ok] = bt[rows, pos[ok] // block_size].astype(np.int64) * block_size + pos[ok] % block_size
    return slots


def reshape_and_cache(key, value, k_cache, v_cache, slot_mapping):
    """Write token t of key/value [T, Hkv, D] to page slot // bs, row slot % bs
    of copies of the caches [num_blocks, Hkv, bs, D]; negative slots and slots
    past the pool are skipped.  Bit copy: the dtype is kept.  Returns the new
    (k_cache, v_cache)."""
    kc, vc = np.array(k_cache, copy=True), np.array(v_cache, copy=True)
    nb, _, bs, _ = kc.shape
    slots = np.asarray(slot_mapping, dtype=np.int64)
    ok = (slots >= 0) & (slots < nb * bs)
    t = np.nonzero(ok)[0]
    kc[slots[ok] // bs, :, slots[ok] % bs, :] = np.asarray(key)[t]
    vc[slots[ok] // bs, :, slots[ok] % bs, :] = np.asarray(value)[t]
    return kc, vc


def attention_gqa(q, k, v, causal=False, scale=None):
    """Attention with grouped kv heads: q [..., H, N, D], k/v [..., H_kv, N, D];
    query head h reads kv head h // (H / H_kv) (the head map of the reference's
    decode, paged_decode.cu:68, 183 / reference.py:66-67, applied to prefill)."""
    q, k, v = np.asarray(q), np.asarray(k), np.asarray(v)
    g = q.shape[-3] // k.shape[-3]
    return attention_fp32(q, np.repeat(k, g, axis=-3), np.repeat(v, g, axis=-3), causal, scale)


def attention_varlen(q, k, v, cu_seqlens, causal=False, scale=None):
    """Packed variable-length attention: q [total, H, D], k/v [total, H_kv, D];
    sequence b is rows cu[b]..cu[b+1]-1 and attends only within itself, each
    sequence computed as an independent [H, n_b, D] problem with attention_gqa.
    Returns float32 [total, H, D]."""
    q, k, v = np.asarray(q), np.asarray(k), np.asarray(v)
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    out = np.zeros(q.shape, dtype=np.float32)
    for b in range(len(cu) - 1):
        s0, s1 = int(cu[b]), int(cu[b + 1])
        if s1 > s0:
            sl = slice(s0, s1)
            out[sl] = attention_gqa(q[sl].transpose(1, 0, 2), k[sl].transpose(1, 0, 2), v[sl].transpose(1, 0, 2),
                                    causal, scale).transpose(1, 0, 2)
    return out
