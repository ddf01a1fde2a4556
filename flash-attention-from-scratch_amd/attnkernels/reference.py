"""Plain-PyTorch baselines with the reference's names (attnkernels/reference.py).

The reference's tests and benchmark import these helpers: the fp32 attention
used as their oracle, the paged-cache generator, the page gather, and the
"gather + SDPA" decode baseline.  They are kept here so that code written
against the reference keeps working.  No kernel entry point of ``attnkernels``
calls this module; this repository's own parity checks use the CPU oracle in
``oracle/`` instead.  All functions are device-agnostic.
"""
from __future__ import annotations

import math

import torch


def attention_fp32(q, k, v, causal=False, scale=None):
    """Exact attention in fp32; q, k, v: [B, H, N, D] of any float dtype
    (reference attnkernels/reference.py:9-18)."""
    qf, kf, vf = q.float(), k.float(), v.float()
    if scale is None:
        scale = 1.0 / math.sqrt(qf.shape[-1])
    scores = torch.matmul(qf, kf.transpose(-1, -2).contiguous()) * scale
    if causal:
        n_q, n_k = scores.shape[-2], scores.shape[-1]
        future = torch.triu(torch.ones(n_q, n_k, dtype=torch.bool, device=scores.device), 1)
        scores = scores.masked_fill(future, float("-inf"))
    return torch.matmul(torch.softmax(scores, dim=-1), vf)


def make_paged_cache(context_lens, num_kv_heads, head_dim, block_size=16, dtype=torch.float16,
                     device="cuda", extra_blocks=0, generator=None):
    """Random K/V caches and block tables for the given context lengths
    (reference attnkernels/reference.py:21-44).

    Physical pages are assigned by a random permutation of the pool, one
    sequence after another; unused table slots hold page 0 and are never read.
    Returns k_cache, v_cache [num_blocks, H_kv, block_size, D], block_tables
    [B, max_blocks] int32 and context_lens int32.
    """
    pages_per_seq = [(int(c) + block_size - 1) // block_size for c in context_lens]
    pool = sum(pages_per_seq) + extra_blocks
    order = torch.randperm(pool, generator=generator).to(torch.int32)
    tables = torch.zeros(len(pages_per_seq), max(pages_per_seq), dtype=torch.int32)
    cursor = 0
    for row, count in enumerate(pages_per_seq):
        tables[row, :count] = order[cursor:cursor + count]
        cursor += count
    shape = (pool, num_kv_heads, block_size, head_dim)
    k_cache = torch.randn(shape, device=device, dtype=dtype)
    v_cache = torch.randn(shape, device=device, dtype=dtype)
    lens = torch.tensor(list(context_lens), dtype=torch.int32, device=device)
    return k_cache, v_cache, tables.to(device), lens


def gather_kv(cache, block_tables, n_blocks):
    """[num_blocks, H_kv, bs, D] -> contiguous [B, H_kv, n_blocks * bs, D]
    (reference attnkernels/reference.py:47-51)."""
    pages = cache[block_tables[:, :n_blocks].long()]  # [B, n_blocks, H_kv, bs, D]
    b, nb, h, bs, d = pages.shape
    return pages.permute(0, 2, 1, 3, 4).reshape(b, h, nb * bs, d)


def paged_decode_fp32(q, k_cache, v_cache, block_tables, context_lens, scale=None):
    """Per-sequence fp32 paged decode; q: [B, H, D]; query head h reads kv head
    h // (H / H_kv) (reference attnkernels/reference.py:54-70)."""
    B, H, D = q.shape
    hkv, bs = k_cache.shape[1], k_cache.shape[2]
    group = H // hkv
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = torch.empty(B, H, D, dtype=torch.float32, device=q.device)
    for b in range(B):
        ctx = int(context_lens[b])
        nb = (ctx + bs - 1) // bs
        keys = gather_kv(k_cache, block_tables[b:b + 1], nb)[0, :, :ctx].float()
        vals = gather_kv(v_cache, block_tables[b:b + 1], nb)[0, :, :ctx].float()
        keys = keys.repeat_interleave(group, dim=0)   # [H, ctx, D]
        vals = vals.repeat_interleave(group, dim=0)
        scores = (keys * q[b].float()[:, None, :]).sum(-1) * scale
        probs = torch.softmax(scores, dim=-1)
        out[b] = (probs[:, :, None] * vals).sum(1)
    return out


def paged_decode_torch(q, k_cache, v_cache, block_tables, n_blocks, context_lens=None):
    """Decode without a paged kernel: gather the pages into a contiguous padded
    cache, then SDPA, with the G query heads of a kv head folded into G query
    rows; with context_lens, tokens past each length are masked
    (reference attnkernels/reference.py:73-89)."""
    B, H, D = q.shape
    hkv = k_cache.shape[1]
    keys = gather_kv(k_cache, block_tables, n_blocks)
    vals = gather_kv(v_cache, block_tables, n_blocks)
    qg = q.view(B, hkv, H // hkv, D)
    mask = None
    if context_lens is not None:
        pos = torch.arange(keys.shape[2], device=q.device)
        mask = (pos[None, :] < context_lens[:, None].long())[:, None, None, :]
    o = torch.nn.functional.scaled_dot_product_attention(qg, keys, vals, attn_mask=mask)
    return o.reshape(B, H, D)
