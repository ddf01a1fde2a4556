"""Attention kernels for LLM inference, hand-written for AMD MI355X (gfx950, CDNA4).

Drop-in for the ``attnkernels`` package of sonhoang/flash-attention-from-scratch
(attnkernels/__init__.py): same functions, arguments, defaults and errors.

Prefill (many query tokens per sequence):
    naive_attention   softmax(scale Q K^T [+ causal mask]) V
    flash_attention   same maths; variant "simt" or "wmma" as in the reference
All three run one gfx950 flash kernel on the f16 MFMA matrix cores with fp32
accumulation and an online softmax; none materialises the N x N scores.  The
same kernel also serves two layouts the reference does not have:
    flash_attention_gqa     fewer kv heads than query heads (GQA / MQA)
    flash_attention_varlen  packed variable-length sequences, no padding

Decode (one query token per sequence) over a paged KV cache:
    paged_decode      split-K ("flash-decoding") kernel plus an LSE-merge reduce
    reshape_and_cache writes new tokens' K/V into that cache (fp16 or bf16)

The native code (``libattnkernels.so``, C-ABI in ``include/attnkernels.h``, and
the torch glue module ``attnkernels_ext``) is built in-tree by
``attnkernels.build`` for gfx950.  There is no fallback: without the built
extension and a GPU the entry points raise.
"""
from __future__ import annotations

import functools
import importlib.util
import math
import os

import torch

__all__ = ["naive_attention", "flash_attention", "paged_decode", "decode_partition",
           "reshape_and_cache", "flash_attention_gqa", "flash_attention_varlen", "load_extension"]

CHUNK = 256  # partitions are multiples of it (reference attnkernels/__init__.py:29)

# Default block_n of the "wmma" variant per head dim, kept from the reference
# (attnkernels/__init__.py:31-33).  On gfx950 block_n is validated (32 or 64)
# but the MFMA kernel uses its own key tile (64 keys for D=128, 128 for D=64).
WMMA_BLOCK_N = {64: 64, 128: 64}


@functools.lru_cache(maxsize=None)
def load_extension():
    """Import the in-tree ``attnkernels_ext`` module, building it first if absent."""
    from . import build as _build

    if not _build.is_built():
        _build.build(verbose=os.environ.get("ATTN_VERBOSE") == "1")
    path = _build.ext_path()
    spec = importlib.util.spec_from_file_location(_build.EXT_NAME, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _check_prefill(q, k, v):
    """Reference attnkernels/__init__.py:53-61 (same checks, same ValueErrors)."""
    for t in (q, k, v):
        if not (t.is_cuda and t.dtype == torch.float16 and t.dim() == 4):
            raise ValueError("q, k, v must be fp16 CUDA tensors of shape [B, H, N, D]")
    if not (q.shape == k.shape == v.shape):
        raise ValueError("q, k, v must have the same shape (self-attention prefill)")
    if q.shape[-1] not in (64, 128):
        raise ValueError("head_dim must be 64 or 128")
    return q.contiguous(), k.contiguous(), v.contiguous()


def naive_attention(q, k, v, causal=False, scale=None):
    """softmax(scale * Q K^T [+ causal mask]) V (reference attnkernels/__init__.py:64-68).

    The reference keeps the scores in DRAM; here the same call runs the MFMA
    flash kernel, so it needs no O(N^2) buffer.
    """
    q, k, v = _check_prefill(q, k, v)
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    return load_extension().naive_attention(q, k, v, causal, scale)


def flash_attention(q, k, v, causal=False, scale=None, variant="wmma", block_n=None):
    """Tiled attention with online softmax. q, k, v: fp16 [B, H, N, D], D in {64, 128}.

    variant: "simt" or "wmma" (both run the gfx950 MFMA kernel).
    block_n: key-tile width accepted by "wmma" (32 or 64), as in the reference.
    Reference: attnkernels/__init__.py:71-85.
    """
    q, k, v = _check_prefill(q, k, v)
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    ext = load_extension()
    if variant == "simt":
        return ext.flash_simt(q, k, v, causal, scale)
    if variant == "wmma":
        bn = WMMA_BLOCK_N[q.shape[-1]] if block_n is None else block_n
        return ext.flash_wmma(q, k, v, causal, scale, bn)
    raise ValueError(f"unknown variant {variant!r}")


@functools.lru_cache(maxsize=None)
def _sm_count(device_index):
    """Compute units of the device (multi_processor_count is the CU count on ROCm)."""
    return torch.cuda.get_device_properties(device_index).multi_processor_count


# Split-count target of decode_partition.  The reference's rule aims at 4
# blocks per SM (attnkernels/__init__.py:94-98, tuned on a T4).  The partition
# is chosen from max_context_len alone (reading the lengths would cost a host
# sync), so the rule must hold for uniform, mixed-length and skewed batches.
# The MI355X split-K ablation of ``attnkernels.benchsuite`` (every power-of-two
# partition; 19 uniform, 6 mixed-length and 5 skewed batches (one long sequence
# among short ones) over one, four and eight query heads per kv head;
# results/mi355x.md), with the splits merged in the decode kernel, sets the
# constants:
#   * about one workgroup per CU in all: uniform batches run fastest with
#     256-512 workgroups (B=1: 16-32 splits, B=4: 8, B=16: 2); every split pays
#     a workgroup's fixed costs (page ids, q, then K/V before any work; the
#     merge) for its share of the bytes;
#   * splits of at most 4 chunks (1024 tokens): a long sequence among short
#     ones (which the rule cannot see) is then cut into enough splits that it
#     does not finish long after the rest.  Uniform batches of 8-16 sequences
#     would take larger splits (3-10% faster at 2048-4096 tokens with eight
#     query heads per kv head), but 2048-token splits cost the skewed batches
#     with four and eight query heads per kv head 10-11% (21-27% with 16 and
#     32 sequences);
#   * no split once B * Hkv reaches 2 workgroups per CU and the context is at
#     most 32 chunks (8192 tokens): the batch alone fills the GPU;
#   * with that many blocks and a longer context, splits sized so that one
#     sequence of max_context_len spreads its Hkv blocks over about 2
#     workgroups per CU (2 * CUs / Hkv splits, at least 2 chunks, not capped
#     at 4): if it is one long sequence among short ones, the short ones fill
#     the GPU and the long one ends with them.  That gives 512 tokens for
#     Hkv=8 at 16384 and 32768 tokens, 1024 and 2048 for Hkv=32.  The skewed
#     batches with Hkv=8 run fastest at 256-512 tokens (1024 reads 73-87% of
#     the best), uniform and mixed ones at 1024-16384 (512 reads 79-94% over
#     three runs); a floor of 1 chunk would cost the uniform ones 14-26%;
#   * tokens per split a power-of-two number of chunks.
# Together they reach 97% of the best partition on average and 88% in the
# worst case in the committed ablation (without the long-context clause 95%
# and 74%; the previous rule, 8 per CU with 1024-token splits and no split at
# 2 per CU: 85% and 19%, on a skewed batch).
DECODE_WG_PER_CU = 1
DECODE_MIN_CHUNKS = 1
DECODE_MAX_SPLIT_CHUNKS = 4
DECODE_NO_SPLIT_BLOCKS_PER_CU = 2
DECODE_NO_SPLIT_MAX_CHUNKS = 32
DECODE_LONG_WG_PER_CU = 2
DECODE_LONG_MIN_CHUNKS = 2
REFERENCE_WG_PER_SM = 4


def decode_partition(batch, num_kv_heads, max_context_len, device=None, wg_per_cu=DECODE_WG_PER_CU,
                     min_chunks=DECODE_MIN_CHUNKS, no_split_blocks_per_cu=DECODE_NO_SPLIT_BLOCKS_PER_CU,
                     no_split_max_chunks=DECODE_NO_SPLIT_MAX_CHUNKS, max_split_chunks=DECODE_MAX_SPLIT_CHUNKS,
                     pow2_chunks=True, long_wg_per_cu=DECODE_LONG_WG_PER_CU,
                     long_min_chunks=DECODE_LONG_MIN_CHUNKS):
    """Tokens per split for paged_decode: enough splits for about ``wg_per_cu``
    workgroups per CU in total, at least ``min_chunks`` and at most
    ``max_split_chunks`` 256-token chunks per split (a power of two of them if
    ``pow2_chunks``), and one split once ``batch * num_kv_heads`` reaches
    ``no_split_blocks_per_cu`` per CU with at most ``no_split_max_chunks``
    chunks of context; with that many blocks and a longer context, enough
    splits for ``long_wg_per_cu`` workgroups per CU from one sequence's kv
    heads, of at least ``long_min_chunks`` chunks (reference attnkernels/__init__.py:93-101, whose rule is
    ``wg_per_cu=REFERENCE_WG_PER_SM, min_chunks=1, no_split_blocks_per_cu=None,
    max_split_chunks=None, pow2_chunks=False``)."""
    dev = torch.cuda.current_device() if device is None else device
    blocks = batch * num_kv_heads
    cus = _sm_count(dev)
    max_chunks = -(-max_context_len // CHUNK)
    if no_split_blocks_per_cu is not None and blocks >= no_split_blocks_per_cu * cus:
        if no_split_max_chunks is None or max_chunks <= no_split_max_chunks:
            return max(1, max_chunks) * CHUNK
        if long_wg_per_cu is not None:
            splits = -(-int(long_wg_per_cu) * cus // num_kv_heads)
            chunks = max(int(long_min_chunks), -(-max_chunks // splits))
            if pow2_chunks:
                chunks = 1 << (chunks - 1).bit_length()
            return chunks * CHUNK
    want = -(-int(wg_per_cu) * cus // blocks)
    splits = max(1, min(want, -(-max_chunks // int(min_chunks))))
    chunks = -(-max_chunks // splits)
    if max_split_chunks is not None:
        chunks = min(chunks, int(max_split_chunks))
    if pow2_chunks:
        chunks = 1 << (chunks - 1).bit_length()
    return chunks * CHUNK


def paged_decode(q, k_cache, v_cache, block_tables, context_lens, max_context_len,
                 scale=None, partition_size=None):
    """Decode attention over a paged KV cache (reference attnkernels/__init__.py:104-128).

    q:            [B, H, D] fp16, one query token per sequence
    k_cache:      [num_blocks, H_kv, block_size, D] fp16 (v_cache the same)
    block_tables: [B, max_blocks_per_seq] int32, physical block ids
    context_lens: [B] int32, tokens of context per sequence (>= 1)
    max_context_len: Python int, max(context_lens) (passed in to avoid a sync)
    partition_size: tokens per split (multiple of 256). None picks one from the
                  batch size; a value >= max_context_len disables split-K.
    """
    if not (q.dtype == k_cache.dtype == v_cache.dtype == torch.float16):
        raise ValueError("q and caches must be fp16")
    if q.shape[-1] not in (64, 128) or k_cache.shape[-1] != q.shape[-1]:
        raise ValueError("head_dim must be 64 or 128 and match the cache")
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    if partition_size is None:
        partition_size = decode_partition(q.shape[0], k_cache.shape[1], max_context_len,
                                          q.device.index)
    partition_size = -(-int(partition_size) // CHUNK) * CHUNK
    return load_extension().paged_decode(
        q.contiguous(), k_cache.contiguous(), v_cache.contiguous(),
        block_tables.to(torch.int32).contiguous(), context_lens.to(torch.int32).contiguous(),
        int(max_context_len), float(scale), partition_size)


def flash_attention_gqa(q, k, v, causal=False, scale=None):
    """Prefill with grouped-query attention: q [B, H, N, D], k and v [B, H_kv,
    N, D] fp16 with H a multiple of H_kv; query head h reads kv head
    h // (H / H_kv).  Same kernel as ``flash_attention``, which (like the
    reference, attnkernels/__init__.py:57-58) requires H_kv == H."""
    for t in (q, k, v):
        if not (t.is_cuda and t.dtype == torch.float16 and t.dim() == 4):
            raise ValueError("q, k, v must be fp16 CUDA tensors of shape [B, H, N, D]")
    if k.shape != v.shape or (k.shape[0], k.shape[2], k.shape[3]) != (q.shape[0], q.shape[2], q.shape[3]):
        raise ValueError("k and v must be [B, H_kv, N, D] with the B, N and D of q")
    if k.shape[1] == 0 or q.shape[1] % k.shape[1]:
        raise ValueError("the query heads must be a multiple of the kv heads")
    if q.shape[-1] not in (64, 128):
        raise ValueError("head_dim must be 64 or 128")
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    return load_extension().flash_gqa(q.contiguous(), k.contiguous(), v.contiguous(), causal, float(scale))


def flash_attention_varlen(q, k, v, cu_seqlens, max_seqlen, causal=False, scale=None):
    """Prefill over packed variable-length sequences (no padding).

    q: [total, H, D], k and v: [total, H_kv, D] fp16 (H a multiple of H_kv);
    sequence b is rows cu_seqlens[b] .. cu_seqlens[b+1]-1 and attends only to
    itself (causal: key j <= query i within the sequence).  cu_seqlens: int32
    [B + 1]; max_seqlen: Python int >= every length (it sizes the grid).  A
    host cu_seqlens is checked here; a device one is used as given (no sync):
    inconsistent offsets then give wrong rows, never an out-of-bounds access.
    """
    for t in (q, k, v):
        if not (t.is_cuda and t.dtype == torch.float16 and t.dim() == 3):
            raise ValueError("q, k, v must be fp16 CUDA tensors of shape [total, H, D]")
    if k.shape != v.shape or (k.shape[0], k.shape[2]) != (q.shape[0], q.shape[2]):
        raise ValueError("k and v must be [total, H_kv, D] with the total and D of q")
    if k.shape[1] == 0 or q.shape[1] % k.shape[1]:
        raise ValueError("the query heads must be a multiple of the kv heads")
    if q.shape[-1] not in (64, 128):
        raise ValueError("head_dim must be 64 or 128")
    if cu_seqlens.dim() != 1 or cu_seqlens.shape[0] < 1:
        raise ValueError("cu_seqlens must be [B + 1]")
    if not cu_seqlens.is_cuda:
        c = cu_seqlens.to(torch.int64)
        lens = c[1:] - c[:-1]
        if (lens < 0).any() or (c.numel() and (c[0] < 0 or c[-1] > q.shape[0])):
            raise ValueError("cu_seqlens must be non-decreasing offsets into the packed rows")
        if lens.numel() and int(lens.max()) > int(max_seqlen):
            raise ValueError("max_seqlen is shorter than a sequence")
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    cu = cu_seqlens.to(device=q.device, dtype=torch.int32).contiguous()
    return load_extension().flash_varlen(q.contiguous(), k.contiguous(), v.contiguous(), cu, int(max_seqlen),
                                         causal, float(scale))


def reshape_and_cache(key, value, k_cache, v_cache, slot_mapping):
    """Write new tokens' keys and values into the paged caches, in place.

    The step before ``paged_decode`` reads them (after a prefill, or after each
    decode step); not part of the reference, whose decode only reads the cache
    in the layout of attnkernels/reference.py:21-44.

    key, value:   [T, H_kv, D] fp16 or bf16 (heads contiguous; any token stride,
                  e.g. a slice of a fused QKV projection output)
    k_cache:      [num_blocks, H_kv, block_size, D], same dtype (v_cache the same)
    slot_mapping: [T] int64 (or int32): token t goes to page slot // block_size,
                  row slot % block_size.  Negative slots (padding) and slots
                  past the pool are skipped.
    """
    if key.dim() != 3 or value.shape != key.shape:
        raise ValueError("key and value must be [num_tokens, H_kv, D] of the same shape")
    if key.dtype not in (torch.float16, torch.bfloat16) or not (
            key.dtype == value.dtype == k_cache.dtype == v_cache.dtype):
        raise ValueError("key, value and the caches must all be fp16 or all bf16")
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape or \
            (k_cache.shape[1], k_cache.shape[3]) != (key.shape[1], key.shape[2]):
        raise ValueError("caches must be [num_blocks, H_kv, block_size, D] matching key")
    if key.shape[-1] % 8:
        raise ValueError("head_dim must be a multiple of 8")
    if slot_mapping.dim() != 1 or slot_mapping.shape[0] != key.shape[0]:
        raise ValueError("slot_mapping must be [num_tokens]")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("caches must be contiguous (they are written in place)")

    def rows(x):  # heads contiguous, token stride a multiple of 8 elements
        ok = x.stride(2) == 1 and x.stride(1) == x.shape[2] and (x.shape[0] <= 1 or x.stride(0) % 8 == 0)
        return x if ok and x.data_ptr() % 16 == 0 else x.contiguous()

    slots = slot_mapping.to(device=key.device, dtype=torch.int64).contiguous()  # a host tensor is copied over
    load_extension().reshape_and_cache(rows(key), rows(value), k_cache, v_cache, slots)
