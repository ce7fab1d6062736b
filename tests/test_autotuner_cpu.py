"""CPU tests of the autotuner's protocol (no GPU: the kernel and the timer are
stand-ins). The observable behaviour follows the reference decorators
(newt/runtime/autotuner.py:5-128): every Config is tried, failing ones are
dropped, reset_to_zero tensors are cleared before each run and after tuning,
the fastest Config is kept per key. The order of work is this backend's own:
every Config is compiled and run once before any is timed, then all are timed
back to back in two rounds and the faster round counts."""

import pytest
import torch

import newt_amd as newt
from newt_amd import testing
from newt_amd.runtime.autotuner import Autotuner


class _Kernel:
    """Stands in for a JIT function: records launches, fails for BLOCK=3."""
    param_names = ["x", "n"]
    defaults = {}

    def __init__(self):
        self.events = []

    def __getitem__(self, grid):
        def launch(*args, **kw):
            if kw["BLOCK"] == 3:
                raise RuntimeError("too much LDS")
            self.events.append(("launch", kw["BLOCK"]))
        return launch


def _configs():
    return [newt.Config({"BLOCK": b}, num_warps=4) for b in (1, 2, 3, 4)]


def test_compiles_all_then_times_two_rounds(monkeypatch):
    k = _Kernel()
    rounds = {1: [5.0, 3.0], 2: [2.0, 4.0], 4: [6.0, 2.5]}
    seen = []

    def fake_bench(fn, warmup, rep):
        fn()
        blk = k.events[-1][1]
        seen.append(blk)
        return rounds[blk][sum(1 for b in seen if b == blk) - 1]
    monkeypatch.setattr(testing, "do_bench", fake_bench)
    tuner = Autotuner(k, _configs(), key=["n"])
    x = torch.zeros(4)
    tuner[(1,)](x, 7)
    # first the compile-and-run pass over every Config (BLOCK=3 fails there),
    # then two timing rounds over the three that ran, in the same order
    first_pass = [e[1] for e in k.events[:3]]
    assert first_pass == [1, 2, 4]
    assert seen == [1, 2, 4, 1, 2, 4]
    # fastest round per Config: 1 -> 3.0, 2 -> 2.0, 4 -> 2.5
    key = next(iter(tuner.timings))
    assert [(ms, c.kwargs["BLOCK"]) for ms, c in tuner.timings[key]] == [(2.0, 2), (2.5, 4), (3.0, 1)]
    assert tuner.best_config.kwargs["BLOCK"] == 2
    assert [c.kwargs["BLOCK"] for c, _ in tuner.failures[key]] == [3]
    assert k.events[-1] == ("launch", 2)           # the real launch uses the winner
    # a second call with the same key does not tune again
    n = len(seen)
    tuner[(1,)](x, 7)
    assert len(seen) == n and k.events[-1] == ("launch", 2)


def test_reset_to_zero_before_every_run_and_after_tuning(monkeypatch):
    k = _Kernel()
    buf = torch.ones(3)
    log = []

    class Zeroing(_Kernel):
        def __getitem__(self, grid):
            inner = _Kernel.__getitem__(self, grid)

            def launch(*args, **kw):
                log.append(float(buf.sum()))        # must be zero before each run
                inner(*args, **kw)
                buf.add_(1.0)                       # a read-modify-write kernel
            return launch
    k = Zeroing()
    monkeypatch.setattr(testing, "do_bench", lambda fn, warmup, rep: (fn(), 1.0)[1])
    tuner = Autotuner(k, [newt.Config({"BLOCK": 1}), newt.Config({"BLOCK": 2})], key=["n"],
                      reset_to_zero=["x"])
    tuner[(1,)](buf, 5)
    assert log and all(v == 0.0 for v in log)
    assert float(buf.sum()) == 3.0                  # only the real launch's writes remain


def test_no_valid_config_raises_chained(monkeypatch):
    k = _Kernel()
    monkeypatch.setattr(testing, "do_bench", lambda fn, warmup, rep: 1.0)
    tuner = Autotuner(k, [newt.Config({"BLOCK": 3})], key=["n"])
    with pytest.raises(RuntimeError, match="no valid config") as e:
        tuner[(1,)](torch.zeros(1), 1)
    assert "too much LDS" in str(e.value.__cause__)
