"""CPU model of the lane algebra of the eight-head decode kernel on the matrix
cores (paged_decode_gqa_mfma_kernel in attnkernels/csrc/decode.hip).

The model replays the kernel's own index formulas on byte images of fp16 pages:
the K and V byte offsets inside a page (koff, voff), the Q^T fragment, the
v_perm selectors that regroup the V rows per head dim, the operand and
accumulator layouts of v_mfma_f32_16x16x32_f16 (lane l: row or column l % 16,
eight k values chosen by l / 16 and the element index, the same for A and B;
accumulator r is row 4 (l / 16) + r), the reference-max softmax with its
lane exchanges (l ^ 16, l ^ 32, and each accumulator row's factor from lane
4g + r), the l sum over the head's four lanes and the rows written for the
workgroup merge.  A wave takes page pairs of a context that rises (so the
reference max moves mid-way) and ends inside the last pair (the checked
path's masking), and the result must match attention in float64 to the
rounding of fp16 P.  Planted mistakes in the same formulas must fail.
"""
import numpy as np
import pytest

P_SHIFT, P_MAX = 7.0, 32768.0


def mfma16x16x32(a, b, c):
    """a, b: [64, 8] per-lane operands (fp16 values); c: [64, 4] accumulators.
    Element e of lane l's A and element e of lane l' s B meet in one k when
    l // 16 == l' // 16; A's row and B's column are l % 16."""
    am = a.reshape(4, 16, 8).transpose(1, 0, 2).reshape(16, 32).astype(np.float32)
    bm = b.reshape(4, 16, 8).transpose(1, 0, 2).reshape(16, 32).astype(np.float32)
    cm = am @ bm.T  # [row, col]
    out = c.copy()
    for lane in range(64):
        for r in range(4):
            out[lane, r] += cm[4 * (lane // 16) + r, lane % 16]
    return out


def perm(hi, lo, sel):
    """v_perm_b32: result byte i = byte sel_i of the 8 bytes {hi:lo} (lo = bytes 0-3)."""
    src = int(lo) | (int(hi) << 32)
    out = 0
    for i in range(4):
        bsel = (sel >> (8 * i)) & 0xFF
        out |= ((src >> (8 * bsel)) & 0xFF) << (8 * i)
    return out


def halves(words):
    """uint32 words -> fp16 values, low half first."""
    w = np.asarray(words, dtype=np.uint32)
    return np.stack([w & 0xFFFF, w >> 16], -1).reshape(-1).astype(np.uint16).view(np.float16)


def read_bytes(page_bytes, off, n):
    return page_bytes[off:off + n]


def model(q, kpages, vpages, pair_tokens, ctx_end, kvh, scale, mistake=None):
    """One wave of the kernel over the given page pairs.  kpages/vpages: per
    pair, two pages [hkv, 16, D] fp16; pair_tokens: first token of each pair;
    q: [G, D] fp16.  Returns the merged rows [G, D] (the wave's o / l) and
    whether the reference max moved after the first pair."""
    g_heads, d = q.shape
    ks, dpl = d // 32, d // 16
    sl2 = np.float32(scale * np.log2(np.e))
    lanes = np.arange(64)
    n_of, g_of = lanes % 16, lanes // 16
    # Q^T fragments: head n, dims 32 s + 8 g .. +7 (zeros for n >= G)
    qf = np.zeros((ks, 64, 8), np.float16)
    for s in range(ks):
        for lane in lanes:
            n, g = n_of[lane], g_of[lane]
            if n < g_heads:
                d0 = 32 * s + 8 * g if mistake != "kq" else 8 * s + 32 * g
                qf[s, lane] = q[n, d0:d0 + 8]
    m_own = np.full(64, -np.inf, np.float32)
    l_own = np.zeros(64, np.float32)
    acc = np.zeros((dpl, 64, 4), np.float32)
    moved_late = False
    for pi, (t0, (ka_page, kb_page), (va_page, vb_page)) in enumerate(zip(pair_tokens, kpages, vpages)):
        hkv = ka_page.shape[0]
        pages_k = [ka_page.reshape(-1).view(np.uint8), kb_page.reshape(-1).view(np.uint8)]
        pages_v = [va_page.reshape(-1).view(np.uint8), vb_page.reshape(-1).view(np.uint8)]
        kv_off = kvh * 16 * d
        # K fragments (A operand): token n of the page, dims 32 s + 8 g
        kf = np.zeros((2, ks, 64, 8), np.float16)
        for pg in range(2):
            for s in range(ks):
                for lane in lanes:
                    n, g = n_of[lane], g_of[lane]
                    tok = t0 + 16 * pg + n
                    koff = (kv_off + n * d + 32 * s + 8 * g) * 2
                    if tok < ctx_end:
                        kf[pg, s, lane] = read_bytes(pages_k[pg], koff, 16).view(np.float16)
        # V rows: token 4g + r of each page, dims dpl n .. +dpl-1, as uint32 words
        vu = np.zeros((64, 8, dpl // 2), np.uint32)
        valid = np.zeros((64, 8), bool)
        for lane in lanes:
            n, g = n_of[lane], g_of[lane]
            for i in range(8):
                pg, r = i // 4, i % 4
                tok = t0 + 16 * pg + 4 * g + r
                row = 4 * g + r if mistake != "voff" else 4 * r + g
                voff = (kv_off + row * d + dpl * n) * 2
                valid[lane, i] = tok < ctx_end
                if valid[lane, i]:
                    vu[lane, i] = read_bytes(pages_v[pg], voff, 2 * dpl).view(np.uint32)
        # scores
        sa = np.zeros((64, 4), np.float32)
        sb = np.zeros((64, 4), np.float32)
        for s in range(ks):
            sa = mfma16x16x32(kf[0, s], qf[s], sa)
            sb = mfma16x16x32(kf[1, s], qf[s], sb)
        x = np.concatenate([sa, sb], 1)
        with np.errstate(over="ignore", invalid="ignore"):
            bias = np.float32(P_SHIFT) - m_own
            p = np.where(valid, np.exp2(x * sl2 + bias[:, None]), np.float32(0))
            ok = np.all(p <= P_MAX, 1)
            if not ok.all():
                moved_late |= pi > 0
                mx = np.where(valid, x * sl2, -np.inf).max(1).astype(np.float32)
                mx = np.maximum(mx, mx[lanes ^ 16])
                mx = np.maximum(mx, mx[lanes ^ 32])
                m_new = np.maximum(m_own, mx)
                m_use = np.where(m_new == -np.inf, np.float32(0), m_new)
                alpha = np.exp2(m_own - m_use).astype(np.float32)
                l_own = l_own * alpha
                m_own = m_new
                for r in range(4):
                    src = 4 * g_of + r if mistake != "alpha" else 4 * r + g_of
                    acc[:, :, r] *= alpha[src][None, :]
                bias = np.float32(P_SHIFT) - m_use
                p = np.where(valid, np.exp2(x * sl2 + bias[:, None]), np.float32(0))
        ph = p.astype(np.float16)
        l_own = l_own + ph.astype(np.float32).sum(1)
        # V fragment j: the 8 tokens' dim dpl n + j, two tokens per register
        for j in range(dpl):
            sel = 0x07060302 if (j & 1) else 0x05040100
            if mistake == "perm":
                sel = 0x05040100 if (j & 1) else 0x07060302
            bj = np.zeros((64, 8), np.float16)
            for lane in lanes:
                words = [perm(vu[lane, 2 * k + 1, j >> 1], vu[lane, 2 * k, j >> 1], sel) for k in range(4)]
                bj[lane] = halves(words)
            acc[j] = mfma16x16x32(ph, bj, acc[j])
    # merge the wave: l over the head's four lanes; rows to the workgroup merge
    l_tot = l_own + l_own[lanes ^ 16]
    l_tot = l_tot + l_tot[lanes ^ 32]
    out = np.zeros((g_heads, d), np.float64)
    lsum = np.zeros(g_heads)
    for lane in lanes:
        n, g = n_of[lane], g_of[lane]
        if g == 0 and n < g_heads:
            lsum[n] = l_tot[lane]
        for r in range(4):
            h = 4 * g + r
            if h < g_heads:
                for j in range(dpl):
                    out[h, dpl * n + j] = acc[j, lane, r]
    return out / lsum[:, None], moved_late


def make_case(d, g_heads, hkv=2, kvh=1, pairs=3, tail=21, seed=0):
    rng = np.random.default_rng(seed)
    ntok = 32 * (pairs - 1) + tail
    k = rng.standard_normal((ntok, d)).astype(np.float32)
    v = rng.standard_normal((ntok, d)).astype(np.float32)
    k[:, 0] = np.linspace(0.0, 6.0, ntok)  # scores rise along the context: the max moves
    q = (0.3 * rng.standard_normal((g_heads, d))).astype(np.float32)
    q[:, 0] = 3.0
    q, k, v = (a.astype(np.float16) for a in (q, k, v))
    kpages, vpages, starts = [], [], []
    for p in range(pairs):
        t0 = 32 * p
        pair_k, pair_v = [], []
        for pg in range(2):
            pk = rng.standard_normal((hkv, 16, d)).astype(np.float16)  # other kv heads: noise
            pv = rng.standard_normal((hkv, 16, d)).astype(np.float16)
            for t in range(16):
                tok = t0 + 16 * pg + t
                if tok < ntok:
                    pk[kvh, t], pv[kvh, t] = k[tok], v[tok]
                else:  # past the context: garbage the kernel must not read
                    pk[kvh, t], pv[kvh, t] = np.float16(np.nan), np.float16(np.nan)
            pair_k.append(pk)
            pair_v.append(pv)
        kpages.append(pair_k)
        vpages.append(pair_v)
        starts.append(t0)
    return q, k, v, kpages, vpages, starts, ntok


def attention(q, k, v, scale):
    s = q.astype(np.float64) @ k.astype(np.float64).T * scale
    p = np.exp(s - s.max(1, keepdims=True))
    return (p / p.sum(1, keepdims=True)) @ v.astype(np.float64)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("g_heads", [8, 4, 2])
def test_mfma_decode_lane_model_matches_attention(d, g_heads):
    scale = 1.0
    q, k, v, kp, vp, starts, ntok = make_case(d, g_heads, seed=d + g_heads)
    got, moved_late = model(q, kp, vp, starts, ntok, kvh=1, scale=scale)
    assert moved_late  # the reference max moved after the first pair
    want = attention(q, k, v, scale)
    err = np.abs(got - want).max()
    assert err < 2e-3, err  # fp16 P: a relative step of 2^-11 per weight


@pytest.mark.parametrize("mistake", ["perm", "alpha", "voff", "kq"])
def test_mfma_decode_lane_model_planted_mistakes_fail(mistake):
    """Each planted mistake is one formula of the kernel changed: the V
    regrouping selectors swapped, the rescale factor taken from lane 4r + g,
    the V row offset of token 4r + g, or Q read with another head-dim order
    than K."""
    scale = 1.0
    q, k, v, kp, vp, starts, ntok = make_case(128, 8, seed=7)
    got, _ = model(q, kp, vp, starts, ntok, kvh=1, scale=scale, mistake=mistake)
    want = attention(q, k, v, scale)
    err = np.abs(got - want).max()
    assert not err < 2e-2, (mistake, err)
