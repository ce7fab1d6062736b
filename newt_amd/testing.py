"""Benchmark helpers: event timing with a cache flush between reps.

Same API as the reference (newt/testing.py:6-34), two MI355X differences:
  * the flush buffer is 512 MiB: MI355X's 256 MiB Infinity Cache (MALL) would
    hold the reference's 256 MiB flush entirely, so rep after rep would run
    from cache;
  * the flush READS the buffer instead of zeroing it. L2 and MALL are
    write-back: a 512 MiB zero fill leaves them full of dirty lines, and
    writing those back to HBM competes with the kernel being timed (a plain
    256 MiB device copy measured 25 % slower after a zero fill than after a
    read). A read evicts the kernel's inputs just as well and leaves clean
    lines, so the timed kernel sees cold, HBM-resident inputs only.
"""

import torch

FLUSH_BYTES = 512 * 1024 * 1024
_flush = {}


def _flush_buffer():
    dev = torch.cuda.current_device()
    buf = _flush.get(dev)
    if buf is None:
        buf = torch.zeros(FLUSH_BYTES // 4, dtype=torch.float32, device="cuda")
        _flush[dev] = buf
    return buf


def do_bench(fn, warmup=10, rep=50, quantile=0.5, flush=True):
    """Median wall time of fn() in milliseconds, caches flushed between reps."""
    fn()  # trigger compilation
    torch.cuda.synchronize()
    cache = _flush_buffer() if flush else None
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = [torch.cuda.Event(enable_timing=True) for _ in range(rep)]
    end = [torch.cuda.Event(enable_timing=True) for _ in range(rep)]
    for i in range(rep):
        if cache is not None:
            cache.sum()
        start[i].record()
        fn()
        end[i].record()
    torch.cuda.synchronize()
    times = sorted(s.elapsed_time(e) for s, e in zip(start, end))
    return times[min(int(len(times) * quantile), len(times) - 1)]


def assert_close(actual, expected, rtol=1e-3, atol=1e-3, msg=""):
    if not torch.allclose(actual, expected, rtol=rtol, atol=atol):
        diff = (actual - expected).abs()
        rel = diff / expected.abs().clamp_min(1e-6)
        raise AssertionError(f"{msg} mismatch: max abs err {diff.max().item():.3e}, "
                             f"max rel err {rel.max().item():.3e}")
