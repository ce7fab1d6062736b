"""CPU tests of bench.py's host-side helpers that need no GPU: the power
sampler's summary (over a stand-in for amdsmi) and the argument checks."""

import sys
import types

import pytest

import bench


class _FakeSmi(types.SimpleNamespace):
    """amdsmi stand-in: a scripted metrics table and violation counters."""

    def __init__(self, metrics, violations):
        super().__init__()
        self.metrics = list(metrics)
        self.violations = list(violations)

    def amdsmi_get_gpu_metrics_info(self, h):
        return self.metrics.pop(0) if len(self.metrics) > 1 else self.metrics[0]

    def amdsmi_get_violation_status(self, h):
        return self.violations.pop(0)

    def amdsmi_get_power_cap_info(self, h):
        return {"power_cap": 1400 * 10 ** 6}


def _violation(counter, ppt):
    return {"acc_counter": counter, "acc_ppt_pwr": ppt, "acc_socket_thrm": 0,
            "acc_vr_thrm": 0, "acc_hbm_thrm": 0}


def _sampler(smi):
    ps = bench.PowerSampler.__new__(bench.PowerSampler)
    ps.sm, ps.h, ps.period, ps.samples = smi, None, 0.0, []
    return ps


def test_power_summary_percentiles_and_ppt_fraction():
    smi = _FakeSmi([], [_violation(100, 40), _violation(1100, 640)])
    ps = _sampler(smi)
    ps.first = dict(bench.PowerSampler._state(ps), t=0.0)
    # the first 0.5 s is skipped as the ramp; the steady samples are 1000-1400 W
    ps.samples = [(0.1, 300, [2400] * 8)] + [(1.0 + i, 1000 + 100 * i, [1800 + i] * 8)
                                            for i in range(5)]
    ps.last = dict(bench.PowerSampler._state(ps), t=6.0)
    s = ps.summary()
    assert s["steady_samples"] == 5
    assert s["socket_power_w_p10_p50_p90"] == [1000, 1200, 1400]
    assert s["gfxclk_mhz_p10_p50_p90"] == [1800, 1802, 1804]
    assert s["power_cap_w"] == 1400.0
    assert s["violation_intervals"] == 1000
    assert s["ppt_limited_frac"] == 0.6
    assert s["thermal_limited_frac"] == 0.0


def test_power_summary_ignores_unavailable_fields():
    smi = _FakeSmi([], [_violation(5, 0), _violation(5, 0)])
    ps = _sampler(smi)
    ps.first = dict(bench.PowerSampler._state(ps), t=0.0)
    ps.samples = [(1.0, "N/A", "N/A"), (2.0, 900, [0, 2100])]
    ps.last = dict(bench.PowerSampler._state(ps), t=3.0)
    s = ps.summary()
    assert s["socket_power_w_p10_p50_p90"] == [900, 900, 900]
    assert s["gfxclk_mhz_p10_p50_p90"] == [2100, 2100, 2100]
    # no interval elapsed in the firmware's accounting: no fraction
    assert s["violation_intervals"] == 0 and s["ppt_limited_frac"] is None


@pytest.mark.parametrize("argv", [["--power", "2"], ["--only", "matmul", "--torch-mm"],
                                  ["--timeline"], ["--dtype", "bf16"]])
def test_option_combinations_rejected(monkeypatch, argv):
    monkeypatch.setattr(sys, "argv", ["bench.py"] + argv)
    with pytest.raises(SystemExit):
        bench.parse()
