"""Prefill parity on the GPU: the gfx950 MFMA kernel behind every prefill entry
point against the CPU oracle on identical seeded fp16 inputs.

Mirrors the reference's suite (tests/test_prefill.py:14-81: 4 variants x causal
x d x n, long sequence, large logits, causal row 0, SDPA, bad input) with the
north-star tolerances (max-abs 2e-3 for d=64, 4e-3 for d=128), and adds the
full-size BASELINE configs through slices and size-independent properties.
"""
import numpy as np
import pytest
import torch

import attnkernels as ak
import oracle
from conftest import TOL, max_err

pytestmark = pytest.mark.gpu

VARIANTS = {
    "naive": lambda q, k, v, c, s=None: ak.naive_attention(q, k, v, causal=c, scale=s),
    "simt": lambda q, k, v, c, s=None: ak.flash_attention(q, k, v, causal=c, scale=s, variant="simt"),
    "wmma32": lambda q, k, v, c, s=None: ak.flash_attention(q, k, v, causal=c, scale=s, variant="wmma",
                                                            block_n=32),
    "wmma64": lambda q, k, v, c, s=None: ak.flash_attention(q, k, v, causal=c, scale=s, variant="wmma",
                                                            block_n=64),
}


def rand_qkv(b, h, n, d, q_scale=1.0, seed=0):
    """fp16 N(0,1) from a seeded CPU generator; the same values go to the GPU and the oracle."""
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(b, h, n, d, generator=g) * q_scale).half()
    k = torch.randn(b, h, n, d, generator=g).half()
    v = torch.randn(b, h, n, d, generator=g).half()
    return q, k, v


def run(variant, q, k, v, causal, scale=None):
    out = VARIANTS[variant](q.cuda(), k.cuda(), v.cuda(), causal, scale)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("variant", list(VARIANTS))
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("n", [1, 17, 64, 100, 129, 256, 333])
def test_matches_fp32(variant, causal, d, n):
    q, k, v = rand_qkv(2, 3, n, d, seed=n * 7 + d)
    out = run(variant, q, k, v, causal)
    ref = oracle.attention_fp32(q.numpy(), k.numpy(), v.numpy(), causal)
    assert out.shape == q.shape and out.dtype == torch.float16
    assert torch.isfinite(out).all()
    assert max_err(out, ref) < TOL[d]


@pytest.mark.parametrize("variant", ["simt", "wmma32", "wmma64"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("d", [64, 128])
def test_long_sequence(variant, causal, d):
    q, k, v = rand_qkv(1, 2, 2048 + 7, d, seed=3)
    out = run(variant, q, k, v, causal)
    assert max_err(out, oracle.attention_fp32(q.numpy(), k.numpy(), v.numpy(), causal)) < TOL[d]


@pytest.mark.parametrize("variant", list(VARIANTS))
@pytest.mark.parametrize("d", [64, 128])
def test_large_logits(variant, d):
    """Scores with a std of about 6: exp would overflow without the running max."""
    q, k, v = rand_qkv(1, 2, 300, d, q_scale=6.0, seed=4)
    out = run(variant, q, k, v, True)
    assert torch.isfinite(out).all()
    assert max_err(out, oracle.attention_fp32(q.numpy(), k.numpy(), v.numpy(), True)) < 2 * TOL[d]


@pytest.mark.parametrize("causal,b,h,n", [(False, 2, 2, 700), (True, 2, 2, 700), (False, 1, 64, 1100),
                                          (True, 1, 64, 2100)])
@pytest.mark.parametrize("d", [64, 128])
def test_running_max_moves_late(causal, b, h, n, d):
    """Key j's scores grow with j (K row j scaled by 1 + j/40) and keys 500, 650
    and 1000 are 3-4x larger still: the subtracted maximum must move after the
    first tile, by small steps and by very large ones (exp would overflow fp16
    without them).  Keys 500 and 1000 sit in the second half of their key tile
    and key 650 in the first, for both tile widths (64 and 128 keys); two heads
    run on 4-wave workgroups and 64 heads on 8-wave ones."""
    q, k, v = rand_qkv(b, h, n, d, seed=11 + d)
    ramp = 1.0 + torch.arange(n, dtype=torch.float32) / 40.0
    k = (k.float() * ramp[None, None, :, None]).half()
    for key, f in ((500, 3), (650, 4), (1000, 3)):
        if key < n:
            k[:, :, key] *= f
    out = run("wmma64", q, k, v, causal)
    assert torch.isfinite(out).all()
    for hi in sorted({0, h - 1}):
        ref = oracle.attention_fp32(q[:, hi].numpy(), k[:, hi].numpy(), v[:, hi].numpy(), causal)
        assert max_err(out[:, hi], ref) < 2 * TOL[d], hi


@pytest.mark.parametrize("causal,h,n", [(False, 16, 3071), (False, 16, 3072), (False, 12, 4100), (True, 16, 6143),
                                        (True, 16, 6144)])
def test_mfma_shape_boundaries(causal, h, n):
    """D = 128 on 8-wave workgroups either side of the switch from 32x32x16 to
    16x16x32 MFMAs (non-causal at N = 3072, causal at N = 6144), ragged and
    whole key tiles: first and last head against the oracle."""
    print(f"mfma shape boundary causal={causal} h={h} n={n}", flush=True)
    q, k, v = rand_qkv(1, h, n, 128, seed=n)
    out = run("wmma64", q, k, v, causal)
    assert torch.isfinite(out).all()
    for hi in (0, h - 1):
        ref = oracle.attention_fp32(q[:, hi].numpy(), k[:, hi].numpy(), v[:, hi].numpy(), causal)
        assert max_err(out[:, hi], ref) < TOL[128], hi


def test_causal_first_row_is_v0():
    q, k, v = rand_qkv(1, 1, 128, 64, seed=5)
    for name in VARIANTS:
        out = run(name, q, k, v, True)
        assert max_err(out[0, 0, 0], v[0, 0, 0]) < 1e-3, name


@pytest.mark.parametrize("variant", list(VARIANTS))
def test_matches_cpu_sdpa(variant):
    """Second, independent reference: torch's CPU SDPA in fp32 (GPU SDPA is not used)."""
    q, k, v = rand_qkv(2, 4, 512, 64, seed=6)
    out = run(variant, q, k, v, True)
    sdpa = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float(),
                                                            is_causal=True)
    assert max_err(out, sdpa) < TOL[64]


@pytest.mark.parametrize("scale", [0.3, -0.05, 0.0, 1e-3, 4.0, -30.0])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("d", [64, 128])
def test_explicit_scales(scale, causal, d):
    """Explicit scales, including large ones (scores in the hundreds of powers of
    two: a nearly one-hot softmax whose running maximum keeps moving) and
    negative ones (folded into Q's sign bits)."""
    q, k, v = rand_qkv(1, 2, 150, d, seed=8)
    out = run("wmma64", q, k, v, causal, scale)
    ref = oracle.attention_fp32(q.numpy(), k.numpy(), v.numpy(), causal, scale)
    assert max_err(out, ref) < TOL[d]


def test_rejects_bad_input():
    q, k, v = rand_qkv(1, 1, 16, 32)
    with pytest.raises(ValueError):
        ak.flash_attention(q.cuda(), k.cuda(), v.cuda())
    q, k, v = rand_qkv(1, 1, 16, 64)
    with pytest.raises(ValueError):
        ak.flash_attention(q.cuda(), k.cuda(), v.cuda(), variant="tensor")
    with pytest.raises(RuntimeError, match="block_n 32 or 64"):
        ak.flash_attention(q.cuda(), k.cuda(), v.cuda(), block_n=128)
    with pytest.raises(ValueError):
        ak.flash_attention(q.cuda(), k[:, :, :8].cuda(), v.cuda())


def test_non_contiguous_inputs_are_accepted():
    q, k, v = rand_qkv(1, 4, 96, 64, seed=9)
    qt = q.transpose(1, 2).contiguous().cuda().transpose(1, 2)  # [B, H, N, D] view, not contiguous
    out = ak.flash_attention(qt, k.cuda(), v.cuda(), causal=True)
    assert max_err(out, oracle.attention_fp32(q.numpy(), k.numpy(), v.numpy(), True)) < TOL[64]


@pytest.mark.parametrize("causal,n", [(False, 1100), (True, 2100)])
@pytest.mark.parametrize("d", [64, 128])
def test_workgroup_sizes_agree(causal, n, d):
    """64 heads fill the GPU and run on 8-wave workgroups (256 query rows); two
    heads alone form a small grid and run on 4-wave workgroups (128 rows).  At
    D = 128 each query row sees the same 64-key tiles in the same order either
    way, so the two results are bit-identical.  At D = 64 the 4-wave workgroups
    take 64-key tiles instead of 128, a different summation order: the results
    then agree to rounding.  Both match the oracle."""
    q, k, v = rand_qkv(1, 64, n, d, seed=n + d)
    big = run("wmma64", q, k, v, causal)
    small = run("wmma64", q[:, :2], k[:, :2], v[:, :2], causal)
    if d == 128:
        assert torch.equal(big[:, :2], small)
    else:
        assert max_err(big[:, :2], small) < TOL[d]
    ref = oracle.attention_fp32(q[:, :2].numpy(), k[:, :2].numpy(), v[:, :2].numpy(), causal)
    assert max_err(small, ref) < TOL[d]
    assert max_err(big[:, :2], ref) < TOL[d]


# ---------------------------------------------------- BASELINE full sizes --

def _device_qkv(b, h, n, d, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return [torch.randn(b, h, n, d, generator=g, device="cuda", dtype=torch.float16) for _ in range(3)]


@pytest.mark.parametrize("cfg", [(1, 4, 256, 64, False), (4, 16, 2048, 64, False), (2, 32, 8192, 128, True),
                                 (2, 32, 8191, 128, True)],
                         ids=["cfg1_d64_n256", "cfg2_d64_n2048", "cfg3_d128_n8192_causal", "cfg3_d128_n8191_causal"])
def test_baseline_config_slices(cfg):
    """Full-size launch; (batch, head) slices at both ends checked against the
    oracle (every slice of the small configuration)."""
    b, h, n, d, causal = cfg
    print(f"baseline slices B={b} H={h} N={n} D={d} causal={causal}", flush=True)
    q, k, v = _device_qkv(b, h, n, d, seed=11)
    out = ak.flash_attention(q, k, v, causal=causal)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    pairs = [(bi, hi) for bi in range(b) for hi in range(h)] if b * h <= 8 else [(0, 0), (b - 1, h - 1)]
    for bi, hi in pairs:
        qs, ks, vs = (t[bi, hi].cpu().numpy() for t in (q, k, v))
        ref = oracle.attention_fp32(qs, ks, vs, causal)
        assert max_err(out[bi, hi], ref) < TOL[d], (bi, hi)


@pytest.mark.parametrize("cfg", [(2, 32, 8192, 128, True), (2, 32, 8191, 128, True),
                                 (4, 16, 2048, 64, False)],
                         ids=["cfg3", "cfg3_odd", "cfg2"])
def test_baseline_config_properties(cfg):
    """Size-independent checks over every row: V = 1 gives O = 1 exactly (the
    softmax weights of each row sum to one); scaling V by 2 scales O by 2."""
    b, h, n, d, causal = cfg
    q, k, v = _device_qkv(b, h, n, d, seed=12)
    ones = torch.ones_like(v)
    o1 = ak.flash_attention(q, k, ones, causal=causal)
    assert (o1.float() - 1).abs().max().item() < 2e-3
    o = ak.flash_attention(q, k, v, causal=causal)
    o2 = ak.flash_attention(q, k, v * 2, causal=causal)
    assert (o2.float() - 2 * o.float()).abs().max().item() < 2 * TOL[d]


@pytest.mark.parametrize("n", [65536, 100003])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_long_context_rows(n, d, causal):
    """Beyond the BASELINE sizes: single query rows of a 64k / 100k-token
    sequence against the oracle over exactly the keys they see (causal: keys
    0..row), and V = 1 giving O = 1 on every row.  Exercises the row/tile
    index arithmetic far past 8192 and long running sums."""
    q, k, v = _device_qkv(1, 2, n, d, seed=13 + n % 7)
    out = ak.flash_attention(q, k, v, causal=causal)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    hc = 1
    qs, ks, vs = (t[0, hc].cpu().numpy() for t in (q, k, v))
    for row in (0, 1, 8191, 8192, n // 2, n - 2, n - 1):
        lim = row + 1 if causal else n
        ref = oracle.attention_fp32(qs[row:row + 1], ks[:lim], vs[:lim], False)
        assert max_err(out[0, hc, row:row + 1], ref) < TOL[d], row
    o1 = ak.flash_attention(q, k, torch.ones_like(v), causal=causal)
    assert (o1.float() - 1).abs().max().item() < 2e-3
