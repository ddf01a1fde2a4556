"""GPU timing shared by bench.py (the driver's one-line benchmark) and
attnkernels.benchsuite (the comparison tables).

Two protocols:
  * steady_steps: back-to-back calls, as a serving loop issues them, after a
    settle phase that takes the GPU's clock out of its idle state; a start and
    an end event around the timed calls (plus marked calls for a per-step
    median);
  * flushed: every call after FLUSH_BYTES of device memory have been
    overwritten, so its inputs come from HBM and not from the 256 MB Infinity
    Cache or the L2s; a start and an end event bracket the call alone.  The
    reference times every rep that way (bench/bench.py:37-60, with a 32 MiB
    flush sized for a T4's L2).

Events are recorded on the current stream, the one the attnkernels entry
points launch on.
"""
from __future__ import annotations

import statistics
import time

import torch

# Twice MI355X's 256 MB Infinity Cache, and far more than its 8 x 4 MB of L2.
FLUSH_BYTES = 512 << 20
_flush_buf = None


def flush_caches():
    """Overwrite FLUSH_BYTES of device memory (one fill kernel on the current stream)."""
    global _flush_buf
    if _flush_buf is None:
        _flush_buf = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device="cuda")
    _flush_buf.fill_(1)


def one_flushed_call_ms(fn):
    """Flush, then time one call of fn with a start and an end event."""
    flush_caches()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    fn()
    b.record()
    b.synchronize()
    return a.elapsed_time(b)


def flushed_samples(fn, min_calls=5, max_calls=40, budget_s=0.25):
    """Flushed timings of fn (ms): at least min_calls, then more until the
    wall-clock budget is spent or max_calls is reached.  One untimed call first."""
    fn()
    torch.cuda.synchronize()
    out, t_end = [], time.perf_counter() + budget_s
    while len(out) < min_calls or (len(out) < max_calls and time.perf_counter() < t_end):
        out.append(one_flushed_call_ms(fn))
    return out


def steady_steps(fn, steps, warmup, settle_s=0.25, flushed_steps=None):
    """Untimed calls for settle_s seconds, then W untimed calls, then exactly K
    calls bracketed by synchronize: the timed steps, with only a start and an
    end HIP event around all K (an event recorded after every step adds 3-4 us
    to each step on MI355X, 4-5% of an 80 us kernel).  Then K more calls with
    one event at each step boundary, for the per-step median, and
    ``flushed_steps`` (default K) flushed calls.

    Returns dict(total_ms: wall clock of the timed K, mean_ms: their event span
    / K, median_ms: median of the marked steps, flushed_mean_ms,
    flushed_median_ms, calls_before_timed): the last counts the calls made
    before the first timed one, including one the caller made before this
    function, so that a profiler trace can pick out the timed dispatches."""
    calls = 1
    settle_end = time.perf_counter() + settle_s
    while time.perf_counter() < settle_end:
        for _ in range(8):
            fn()
        calls += 8
        torch.cuda.synchronize()
    for _ in range(warmup):
        fn()
    calls += warmup
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    total_ms = (time.perf_counter() - t0) * 1e3
    mean_ms = start.elapsed_time(end) / max(steps, 1)
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    marks[0].record()
    for i in range(steps):
        fn()
        marks[i + 1].record()
    torch.cuda.synchronize()
    ev = [a.elapsed_time(b) for a, b in zip(marks[:-1], marks[1:])]
    fl = [one_flushed_call_ms(fn) for _ in range(steps if flushed_steps is None else flushed_steps)]
    return dict(total_ms=total_ms, mean_ms=mean_ms, median_ms=statistics.median(ev) if ev else None,
                flushed_mean_ms=statistics.fmean(fl) if fl else None,
                flushed_median_ms=statistics.median(fl) if fl else None, calls_before_timed=calls)


def extra_peak_bytes(fn):
    """Device memory one call of fn allocates above what is already live, at its
    peak (its output included)."""
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    live = torch.cuda.memory_allocated()
    out = fn()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - live
    del out
    return peak
