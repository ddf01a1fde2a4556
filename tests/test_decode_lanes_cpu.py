"""CPU model of the lane algebra of the grouped-query decode kernel on dot
products (paged_decode_gqa_kernel in attnkernels/csrc/decode.hip; two and four
query heads per kv head, eight run on the matrix-core kernel modelled in
tests/test_decode_mfma_lanes_cpu.py).

A lane group of D/8 lanes holds, per chunk, G*U partial dot products (head h,
token slot u, 8 head dims each).  The kernel sums them across the group with a
reduce-scatter butterfly whose partners are lane ^ 8, ^ 7, ^ 2, ^ 1 (16-lane
groups; 7, 2, 1 for 8-lane groups), in a lane-dependent register order
(register r holds value r ^ f(lane), value index j = (u >> 1) * 2G + 2h + (u & 1)),
then all-gathers the fp16 P pairs back by the inverse butterfly.  This model
replays exactly those index formulas on random partial sums and checks what
the kernel relies on: every lane ends with the full scores of its own head and
its own token slots 0 and 1; after the gather, register pr * G + a holds the
pair of head a ^ fh for V registers 2 pr and 2 pr + 1; the l merge, the
slow-path max and the head-lane masks cover exactly the right lanes; and the 8
lanes of a 128-byte cache line always read the same token row.
"""
import random

import pytest

MASKS16 = [8, 7, 2, 1]


def coord(li, s, lb):
    l2 = (li >> 2) & 1
    c = [(li >> 3) & 1, l2, ((li >> 1) & 1) ^ l2, (li & 1) ^ l2]
    return c[s + 4 - lb]


def layout(d, g):
    lpt = d // 8
    tpl = 64 // lpt
    u = 16 // tpl
    lb = 4 if d == 128 else 3
    n = g * u
    logn = n.bit_length() - 1
    s = min(lb, logn - 1)
    lg = g.bit_length() - 1
    masks = MASKS16[4 - lb:]
    return lpt, u, lb, n, s, lg, masks


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("g", [2, 4])
def test_butterfly_lane_algebra(d, g):
    lpt, U, lb, n, S, lg, masks = layout(d, g)
    assert n >> S == 2 and S >= lg  # the kernel's static_asserts

    # the masks are a basis: every lane has unique coordinates
    for li in range(lpt):
        acc = 0
        for s in range(lb):
            if coord(li, s, lb):
                acc ^= masks[s]
        assert acc == li

    head_of = lambda j: (j >> 1) & (g - 1)          # noqa: E731
    slot_of = lambda j: ((j >> (1 + lg)) << 1) | (j & 1)  # noqa: E731
    f = []
    for li in range(lpt):
        v = 0
        for s in range(S):
            if coord(li, s, lb):
                v ^= n >> (s + 1)
        f.append(v)
    fh = [head_of(v) for v in f]
    fu = [slot_of(v) for v in f]
    # cache lines: lanes 0-7 and 8-15 read the two 128-byte halves of a row
    for li in range(lpt):
        assert fu[li] == fu[li & ~7]

    rng = random.Random(d * 10 + g)
    part = [[[rng.random() for _ in range(lpt)] for _ in range(U)] for _ in range(g)]
    full = [[sum(part[h][u]) for u in range(U)] for h in range(g)]
    x = [[part[head_of(r) ^ fh[li]][slot_of(r) ^ fu[li]][li] for r in range(n)] for li in range(lpt)]
    for s in range(S):                              # reduce-scatter
        half = (n >> s) // 2
        x = [[x[li][r] + x[li ^ masks[s]][r + half] for r in range(half)] for li in range(lpt)]
    for s in range(S, lb):                          # plain stages on the two left
        x = [[x[li][r] + x[li ^ masks[s]][r] for r in range(2)] for li in range(lpt)]
    for li in range(lpt):
        for r in range(2):
            assert x[li][r] == pytest.approx(full[fh[li]][fu[li] ^ r])

    P = [[(x[li][0], x[li][1])] for li in range(lpt)]  # all-gather of the pairs
    for k in range(S):
        s = S - 1 - k
        m = n >> (s + 2)
        P = [P[li] + [P[li ^ masks[s]][j] for j in range(m)] for li in range(lpt)]
    for li in range(lpt):
        assert len(P[li]) == n // 2
        for pr in range(U // 2):
            for a in range(g):
                h, s0 = a ^ fh[li], (2 * pr) ^ fu[li]
                assert P[li][pr * g + a] == (pytest.approx(full[h][s0]), pytest.approx(full[h][s0 + 1]))

    slot_stage = lambda s: (n >> (s + 1)) >= 2 * g  # noqa: E731  stage s resolves a slot bit
    lown = [x[li][0] + x[li][1] for li in range(lpt)]
    for s in range(S):
        if slot_stage(s):
            lown = [lown[li] + lown[li ^ masks[s]] for li in range(lpt)]
    mx = [max(x[li]) for li in range(lpt)]
    for s in range(lb):
        if s >= S or slot_stage(s):
            mx = [max(mx[li], mx[li ^ masks[s]]) for li in range(lpt)]
    for li in range(lpt):
        assert lown[li] == pytest.approx(sum(full[fh[li]]))
        assert mx[li] == pytest.approx(max(full[fh[li]]))

    for a in range(g):                              # head_lane_mask
        hm = 0
        for s in range(lb):
            bit = n >> (s + 1)
            if bit < 2:
                break
            if bit < 2 * g and a & (bit >> 1):
                hm ^= masks[s]
        for li in range(lpt):
            assert fh[li ^ hm] == fh[li] ^ a


@pytest.mark.parametrize("g", [2, 4])
def test_head_major_value_order_splits_cache_lines(g):
    """The value order the kernel avoids: j = h * U + u (slot bits last) resolves
    a slot bit on a mask whose coordinate varies inside a cache line, so lanes
    of one 128-byte line would read different token rows (measured 6-19%
    slower at G = 4 on MI355X)."""
    lpt, U, lb, n, S, lg, masks = layout(128, g)
    fu = []
    for li in range(lpt):
        v = 0
        for s in range(S):
            if coord(li, s, lb):
                v ^= n >> (s + 1)
        fu.append(v % U)
    assert any(fu[li] != fu[li & ~7] for li in range(lpt))
