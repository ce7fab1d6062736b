"""newt on MI355X - headline benchmark.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-secondary] [--no-cpu]

One "step" is one launch of the newt matmul kernel (the examples/04 body,
compiled by newt_amd to HIP for gfx950, autotuned over its gfx950 config space)
on fp16 A[4096,4096] @ B[4096,4096] -> C fp16 with fp32 accumulation. Inputs are
resident in HBM before the timed region; `value` is TFLOP/s over the K timed
steps (2*M*N*K flop per step). The one JSON line also carries:

  roofline      the matmul kernel vs MI355X's dense fp16 MFMA peak (2.5 PFLOP/s):
                2*M*N*K flop per launch / the kernel's average launch duration
                over the timed region (one HIP event pair, without system-scope
                fences, on the launch stream around K gap-free launches)
  cpu_baseline  the reference's oracle (torch CPU eager, A.float() @ B.float())
                timed on this host's cores on the same 4096^3 problem; cpu_info
                names the CPU model and its physical cores
  secondary     the copy ceiling (a newt copy kernel at 128 MiB, 256 MiB and
                1 GiB), vector add / softmax / layernorm (GB/s vs 8 TB/s HBM),
                flash attention, the other matmul sizes and dtypes and the
                deuteron matmul (TFLOP/s); each line's timed launches are
                checked against the oracle afterwards (sampled so that every
                program of the launch is touched) and carry their own torch
                CPU eager baseline

Everything runs on one GPU; --gpus above 1 exits with a message.
`--only NAME` runs a single workload (for rocprofv3 runs); `--only copy` runs a
256 MiB device copy used to calibrate the FETCH_SIZE / WRITE_SIZE counters.
"""

import argparse
import json
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_TFLOPS = 2500.0   # MI355X dense fp16/bf16 MFMA, published
PEAK_GBS = 8000.0      # MI355X HBM3E, published
PEAK_FP32_TFLOPS = 157.3  # MI355X dense fp32 MFMA, published
METRIC = "fp16 4096^3 matmul TFLOP/s (% MFMA peak); softmax/layernorm GB/s (% HBM)"
# HBM bytes per matmul launch from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE on
# this command, scaled by the copy-kernel calibration (see profiles/)
MATMUL_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "matmul_fp16_4096_traffic.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--size", type=int, default=4096)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--config", default=None, help="BM,BN,BK,warps,stages (skip autotune)")
    ap.add_argument("--only", default=None,
                    help="run one workload for profiler runs: 'matmul', 'copy' (torch's "
                         "device copy, counter calibration), 'newt copy' (the copy ceiling's "
                         "kernel at 128 MiB moved), or the start of a secondary workload's "
                         "name (e.g. 'softmax fp32 4096x4096')")
    ap.add_argument("--operands", default="random", choices=("random", "constant", "bf16-values"),
                    help="with --only matmul: the configuration's N(0,1)/sqrt(K) operands "
                         "(random), every element 1/64 (constant), or the random values "
                         "rounded to bf16 first; the power the matrix cores draw, and so the "
                         "clock the chip holds, depends on the operands' bits")
    ap.add_argument("--dtype", default="fp16", choices=("fp16", "bf16"),
                    help="with --only matmul: the operands' dtype (the headline is fp16)")
    ap.add_argument("--timeline", action="store_true",
                    help="with --only matmul: per-workgroup start, end-of-k-loop and end "
                         "timestamps of the headline kernel (s_memrealtime, 100 MHz), "
                         "summarised per XCD")
    ap.add_argument("--torch-mm", action="store_true",
                    help="with --only matmul --power: run torch.mm (hipBLASLt) on the same "
                         "operands instead of the newt kernel, for the power comparison")
    ap.add_argument("--power", type=float, default=0.0, metavar="SECONDS",
                    help="with --only: afterwards run the workload back to back for SECONDS "
                         "of GPU time while a thread reads the GPU's socket power, energy "
                         "counter, graphics clocks and power-limit accounting through "
                         "amdsmi; prints one JSON line of the summary")
    args = ap.parse_args()
    if args.power and not args.only:
        ap.error("--power applies to --only runs")
    if args.torch_mm and not (args.power and args.only == "matmul"):
        ap.error("--torch-mm applies to --only matmul --power runs")
    if args.timeline and args.only != "matmul":
        ap.error("--timeline applies to --only matmul runs")
    if args.dtype != "fp16" and args.only != "matmul":
        ap.error("--dtype applies to --only matmul runs (the headline is fp16)")
    if args.operands != "random" and args.only != "matmul":
        ap.error("--operands applies to --only matmul runs (the headline uses the "
                 "configuration's random operands)")
    return args


def seeded(shape, seed, scale=1.0, mean=0.0, dtype=None):
    import torch
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(shape, generator=g) * scale + mean
    return t.to(dtype or torch.float32).to("cuda")


class _HipEvents:
    """HIP events on the launch stream, created with hipEventDisableSystemFence:
    an event record then adds no system-scope cache release between launches
    (torch's events do, which puts a few microseconds between back-to-back
    kernels)."""

    DISABLE_SYSTEM_FENCE = 0x20000000

    def __init__(self):
        import ctypes
        self.ct = ctypes
        self.lib = ctypes.CDLL("libamdhip64.so")

    def make(self, n):
        out = []
        for _ in range(n):
            e = self.ct.c_void_p()
            rc = self.lib.hipEventCreateWithFlags(self.ct.byref(e), self.ct.c_uint(self.DISABLE_SYSTEM_FENCE))
            if rc != 0:
                raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")
            out.append(e)
        return out

    def record(self, e, stream):
        rc = self.lib.hipEventRecord(e, self.ct.c_void_p(stream))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def ms(self, e0, e1):
        v = self.ct.c_float()
        rc = self.lib.hipEventElapsedTime(self.ct.byref(v), e0, e1)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return v.value

    def destroy(self, evs):
        for e in evs:
            self.lib.hipEventDestroy(e)


def timed_launches(fn, steps, embedded=True, before=None, with_list=False):
    """Run fn() `steps` times back to back on the current stream (where newt
    launches) and time each launch with a HIP event pair. Returns (total ms
    between the first start and last end event, average ms of the per-launch
    event pairs).

    embedded: fn makes exactly one newt launch, whose dispatch records the
    pair itself at the kernel's start and end (hipExtModuleLaunchKernel), so
    no event packets sit between the launches. Otherwise (a library call such
    as torch.mm) the pair is recorded around each call.

    before: called ahead of every fn() (a cache flush); with embedded timing
    its own launches fall outside the pairs, which then hold the kernel's
    execution on cold caches without the host's dispatch gap."""
    import torch
    from newt_amd.runtime import jit as J
    hev = _HipEvents()
    stream = torch.cuda.current_stream().cuda_stream
    st, en = hev.make(steps), hev.make(steps)
    torch.cuda.synchronize()
    if embedded:
        pairs = list(zip(st, en))
        pos = [0]

        def next_pair():
            i = pos[0]
            if i >= steps:
                raise RuntimeError("timed_launches: more than one newt launch per step")
            pos[0] = i + 1
            return pairs[i][0].value, pairs[i][1].value
        try:
            for i in range(steps):
                if before is not None:
                    before()
                J.launch_events = next_pair
                fn()
                J.launch_events = None
        finally:
            J.launch_events = None
        if pos[0] != steps:
            raise RuntimeError("timed_launches: expected one newt launch per step")
    else:
        for i in range(steps):
            if before is not None:
                before()
            hev.record(st[i], stream)
            fn()
            hev.record(en[i], stream)
    torch.cuda.synchronize()
    per = [hev.ms(s, e) for s, e in zip(st, en)]
    total = hev.ms(st[0], en[-1])
    hev.destroy(st + en)
    if with_list:
        return total, sum(per) / len(per), per
    return total, sum(per) / len(per)


LEAD_CYCLES = 2_000_000


def bracketed_launches(fn, steps, lead=True):
    """Run fn() `steps` times back to back with one HIP event pair around all
    of them and nothing between launches. Returns the total ms.

    lead: a GPU-side spin (torch.cuda._sleep) is queued before the start
    event, so the host has queued the launches by the time the start event
    fires. Without it the span also holds the host's latency to its first
    launch after the synchronize (~90 us measured: 4% of 20 steps at 4096^3)."""
    import torch
    hev = _HipEvents()
    stream = torch.cuda.current_stream().cuda_stream
    st, en = hev.make(1), hev.make(1)
    torch.cuda.synchronize()
    if lead:
        torch.cuda._sleep(LEAD_CYCLES)
    hev.record(st[0], stream)
    for _ in range(steps):
        fn()
    hev.record(en[0], stream)
    torch.cuda.synchronize()
    total = hev.ms(st[0], en[0])
    hev.destroy(st + en)
    return total


SETTLE_S = 0.4
MM_WINDOWS = 5   # timed windows per sized-matmul secondary line (median reported)


def settle_clocks(fn, seconds):
    """Launch fn back to back, in batches timed on the GPU, until `seconds` of
    GPU time have passed; returns what ran (launches, seconds) for the
    report. Untimed with respect to the measurement that follows."""
    done, spent, batch = 0, 0.0, 50
    while spent < seconds:
        spent += bracketed_launches(lambda: [fn() for _ in range(batch)], 1, lead=False) * 1e-3
        done += batch
    return {"launches": done, "gpu_s": round(spent, 3)}


class PowerSampler:
    """The GPU's power state while kernels run, read through amdsmi (ROCm's
    SMI library: it reads the power-management firmware's metrics table from
    the driver and makes no HIP call). A thread reads the metrics table (socket
    power, per-XCD graphics clocks) every `period` seconds; the violation
    accounting (the firmware's count of the ~1 ms intervals in which the
    package power limit, PPT, or a temperature limit held the clock below the
    host's limit) is read at the start and end of the window. The firmware's
    energy counter is not read: over windows of a few seconds its averages
    disagreed with the power samples and exceeded the cap."""

    _sm = None

    def __init__(self, period=0.005):
        import threading
        if PowerSampler._sm is None:
            import amdsmi
            amdsmi.amdsmi_init()
            PowerSampler._sm = amdsmi
        self.sm = PowerSampler._sm
        self.h = self._handle()
        self.period = period
        self.samples = []
        self.stop = threading.Event()
        self.thread = threading.Thread(target=self._run, daemon=True)

    def _handle(self):
        import torch
        hs = self.sm.amdsmi_get_processor_handles()
        if len(hs) == 1:
            return hs[0]
        bus = getattr(torch.cuda.get_device_properties(0), "pci_bus_id", None)
        for h in hs:
            if bus is not None and int(self.sm.amdsmi_get_gpu_device_bdf(h).split(":")[1], 16) == bus:
                return h
        raise RuntimeError(f"PowerSampler: {len(hs)} GPUs visible to amdsmi and none matches "
                           f"cuda:0's PCI bus {bus}")

    def _state(self):
        v = self.sm.amdsmi_get_violation_status(self.h)
        st = {"t": time.perf_counter()}
        for k in ("acc_counter", "acc_ppt_pwr", "acc_socket_thrm", "acc_vr_thrm",
                  "acc_hbm_thrm"):
            st[k] = v[k]
        return st

    def _run(self):
        while not self.stop.is_set():
            m = self.sm.amdsmi_get_gpu_metrics_info(self.h)
            self.samples.append((time.perf_counter(), m["current_socket_power"],
                                 m["current_gfxclks"]))
            self.stop.wait(self.period)

    def __enter__(self):
        self.first = self._state()
        self.thread.start()
        return self

    def __exit__(self, *exc):
        self.stop.set()
        self.thread.join()
        self.last = self._state()

    def summary(self, skip_s=0.5):
        """Power and clocks over the window after its first `skip_s` seconds
        (the steady state); the violation accounting over the whole window."""
        a, b = self.first, self.last
        steady = [s for s in self.samples if s[0] >= a["t"] + skip_s] or self.samples
        watts = sorted(s[1] for s in steady if isinstance(s[1], (int, float)))
        clocks = sorted(c for s in steady if isinstance(s[2], list)
                        for c in s[2] if isinstance(c, (int, float)) and c > 0)
        n = b["acc_counter"] - a["acc_counter"]
        frac = lambda k: (round((b[k] - a[k]) / n, 4)
                          if n and b.get(k) is not None and a.get(k) is not None else None)
        pct = lambda xs, q: xs[min(len(xs) - 1, int(len(xs) * q))] if xs else None
        return {
            "window_s": round(b["t"] - a["t"], 3), "steady_samples": len(steady),
            "socket_power_w_p10_p50_p90": [pct(watts, 0.1), pct(watts, 0.5), pct(watts, 0.9)],
            "power_cap_w": self.sm.amdsmi_get_power_cap_info(self.h)["power_cap"] / 1e6,
            "gfxclk_mhz_p10_p50_p90": [pct(clocks, 0.1), pct(clocks, 0.5), pct(clocks, 0.9)],
            "violation_intervals": n,
            "ppt_limited_frac": frac("acc_ppt_pwr"),
            "thermal_limited_frac": frac("acc_socket_thrm"),
            "vr_thermal_limited_frac": frac("acc_vr_thrm"),
            "hbm_thermal_limited_frac": frac("acc_hbm_thrm"),
        }


def power_window(name, fn, seconds, flop=None, nbytes=None):
    """Run fn back to back for `seconds` of GPU time under a PowerSampler,
    with an idle window of the same sampler before it; print one JSON line."""
    import torch
    torch.cuda.synchronize()
    time.sleep(0.5)
    with PowerSampler() as idle:
        time.sleep(1.0)
    with PowerSampler() as ps:
        ran = settle_clocks(fn, seconds)
    out = {"power": name, "launches": ran["launches"], "gpu_s": ran["gpu_s"],
           "idle": idle.summary(), "busy": ps.summary()}
    per = ran["gpu_s"] / ran["launches"]
    if flop:
        out["tflops"] = round(flop / per / 1e12, 1)
    if nbytes:
        out["gbs"] = round(nbytes / per / 1e9, 1)
    print(json.dumps(out), flush=True)


def cpu_info():
    """This host's CPU model and physical core count (from /proc/cpuinfo),
    logical CPUs, the CPUs this process may run on and torch's threads."""
    import torch
    model, cores = platform.processor() or platform.machine(), set()
    phys = core = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name":
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                elif not k and phys is not None:
                    cores.add((phys, core))
                    phys = core = None
    except OSError:
        pass
    if phys is not None:
        cores.add((phys, core))
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    return {"model": model, "physical_cores": len(cores) or None,
            "logical_cpus": os.cpu_count(), "usable_cpus": usable,
            "torch_threads": torch.get_num_threads()}


_CPU = {}


def cpu_time(fn, budget_s, min_reps=5, max_reps=50):
    """time.perf_counter median of fn() over >= min_reps reps (2 warm-ups
    first), stopping after about budget_s seconds or max_reps reps."""
    for _ in range(2):
        fn()
    reps, t0 = [], time.perf_counter()
    while len(reps) < min_reps or (time.perf_counter() - t0 < budget_s and len(reps) < max_reps):
        t1 = time.perf_counter()
        fn()
        reps.append(time.perf_counter() - t1)
    return statistics.median(reps), len(reps), sum(reps)


def cpu_line(work, unit, fn, budget_s, what, max_reps=50):
    """A cpu_baseline object: `work` (bytes or flop of the sample `fn`
    processes) per median second, in GB/s or TFLOP/s."""
    import torch
    info = _CPU.get("info") or _CPU.setdefault("info", cpu_info())
    med, n, tot = cpu_time(fn, budget_s, max_reps=max_reps)
    div = 1e9 if unit == "GB/s" else 1e12
    return {"value": round(work / med / div, 4), "unit": unit, "cores": info["torch_threads"],
            "kind": "port", "sample": f"{what}; median of {n} reps ({tot:.1f} s)"}


def cpu_matmul(S, dtype, budget_s, rows=None, max_reps=50):
    """torch CPU A.float() @ B.float() on the problem (or its first `rows`
    rows of A when the whole problem would take too long)."""
    import torch
    from oracle import torch_eager
    g = torch.Generator().manual_seed(4)
    r = rows or S
    a = (torch.randn(r, S, generator=g) * S ** -0.5).to(dtype)
    b = (torch.randn(S, S, generator=g) * S ** -0.5).to(dtype)
    what = (f"A.float() @ B.float(), full {S}^3" if r == S else
            f"A[:{r}].float() @ B.float() ({r} rows of {S}^3)")
    return cpu_line(2.0 * r * S * S, "TFLOP/s", lambda: torch_eager.matmul(a, b), budget_s, what,
                    max_reps=max_reps)


def pick_matmul_config(a, b, c, args):
    import newt_amd as newt
    from newt_amd import workloads as W
    if args.config:
        BM, BN, BK, nw, ns = (int(x) for x in args.config.split(","))
        return newt.Config({"BLOCK_M": BM, "BLOCK_N": BN, "BLOCK_K": BK}, num_warps=nw,
                           num_stages=ns)
    W.matmul(a, b, c)  # autotune over MATMUL_CONFIGS (untimed)
    return W.matmul_tuned.best_config


def matmul_traffic(cfg):
    """HBM bytes per launch measured for this exact tile configuration (null
    when the autotuner picked a configuration that was not measured)."""
    try:
        with open(MATMUL_TRAFFIC_FILE) as f:
            d = json.load(f)
    except (OSError, ValueError):
        return None
    want = dict(cfg.kwargs, num_warps=cfg.num_warps, num_stages=cfg.num_stages)
    return d.get("bytes_per_launch") if d.get("config") == want else None


def check_matmul(a, b, c, dtype_name):
    """Parity of a square matmul's output against the oracle on rows that
    touch every 64-row panel (plus the last row), all columns: (relative
    Frobenius error, elements beyond one ulp of the rounded exact product)."""
    import torch
    from oracle import newt_oracle as orc
    rows = orc.panel_rows(c.shape[0], 64)
    got = c[torch.from_numpy(rows).to(c.device)].float().cpu().numpy()
    ref = orc.matmul(a[torch.from_numpy(rows).to(a.device)].float().cpu().numpy(),
                     b.float().cpu().numpy(), dtype_name)
    return orc.rel_frobenius(got, ref), orc.ulp_violations(got, ref, dtype_name)


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one MI355X (every box here has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    torch.cuda.set_device(0)
    if args.only and args.only != "matmul":
        return run_only(args.only, args.power)
    from newt_amd import workloads as W
    from newt_amd.testing import _flush_buffer

    S = args.size
    dt = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    a = seeded((S, S), 4, scale=S ** -0.5, dtype=dt)
    b = seeded((S, S), 5, scale=S ** -0.5, dtype=dt)
    if args.operands == "constant":
        a.fill_(1 / 64)
        b.fill_(1 / 64)
    elif args.operands == "bf16-values":
        a.copy_(a.bfloat16())
        b.copy_(b.bfloat16())
    c = torch.empty(S, S, device="cuda", dtype=dt)
    cfg = pick_matmul_config(a, b, c, args)
    step = lambda: W.matmul(a, b, c, config=cfg)
    if args.timeline:
        return matmul_timeline(a, b, c, cfg, step)
    # warm-up straight after the autotuner's runs: the chip's clocks drop
    # while it idles (a CPU-side check here cost ~20% on the first timed
    # launches), so the oracle check of the measured configuration's output
    # follows the timed region instead of preceding it
    for _ in range(args.warmup):
        step()
    # and then until the clocks have settled: whatever W is, launches run back
    # to back for SETTLE_S seconds of GPU time (measured: right after the
    # host-side autotuning the first ~50 launches at 4096^3 run ~20% slow)
    settle = settle_clocks(step, SETTLE_S)
    # the timed region: K back-to-back launches between one event pair (any
    # per-launch event adds ~3.5-4.5 us per step); each launch's own duration
    # then comes from a second pass of K launches whose dispatches record events
    t0 = time.perf_counter()
    total_ms = bracketed_launches(step, args.steps)
    wall = time.perf_counter() - t0
    _, kern_ms, kern_list = timed_launches(step, args.steps, with_list=True)
    # parity of the measured configuration: the last timed launch's output
    err, bad = check_matmul(a, b, c, "bfloat16" if dt == torch.bfloat16 else "float16")
    if not (err <= 1e-2 and bad == 0):
        raise SystemExit(f"bench.py: matmul result differs from the oracle (rel. Frobenius "
                         f"{err}, {bad} elements beyond one ulp)")
    # the measurement protocol of the reference's do_bench: the median of
    # launches on cold caches (512 MiB read between them), each launch timed
    # by events its own dispatch records
    flush = _flush_buffer()
    for _ in range(10):
        step()
    _, _, cold = timed_launches(step, 50, before=lambda: flush.sum(), with_list=True)
    flop = 2.0 * S ** 3
    value = flop * args.steps / (total_ms * 1e-3) / 1e12
    # the kernel's average launch duration over the timed region: its launches
    # run back to back with no gap (the rocprofv3 trace of this command shows
    # 0.0 us between them), so the region's span / K is that average. The
    # second pass, whose dispatches record an event pair each, is reported
    # beside it: the events put ~8 us between launches and change the clocks
    achieved = flop / (total_ms / args.steps * 1e-3) / 1e12
    if args.only:
        log(f"matmul only ({args.dtype} {S}^3, {cfg}, {args.operands} operands): "
            f"{value:.1f} TFLOP/s, "
            f"{statistics.median(kern_list) * 1e3:.2f} us per launch with dispatch events")
        if args.power:
            if args.torch_mm:
                step = lambda: torch.mm(a, b, out=c)
                name = f"torch.mm (hipBLASLt) {args.dtype} {S}^3 {args.operands} operands"
            else:
                name = f"matmul {args.dtype} {S}^3 {args.operands} operands {cfg}"
            power_window(name, step, args.power, flop=flop)
        return
    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(total_ms / args.steps, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (seeded N(0,1)/sqrt(K) fp16 inputs)",
        "config": {"workload": f"matmul fp16 {S}x{S}x{S}, examples/04 kernel body via @newt.jit "
                               f"-> HIP for gfx950 (autotuned)",
                   "M": S, "N": S, "K": S, "tile": dict(cfg.kwargs), "num_warps": cfg.num_warps,
                   "num_stages": cfg.num_stages, "rel_frobenius_vs_oracle": err,
                   "checked_rows": "one per 64-row panel + last row, all columns; "
                                   "every element within one fp16 ulp"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_TFLOPS, 4),
                     "traffic": matmul_traffic(cfg)},
        "settle": settle,
        "kernel_ms_dispatch_events_median": round(statistics.median(kern_list), 5),
        "kernel_ms_flushed_median": round(statistics.median(cold), 5),
        "tflops_flushed_median": round(flop / (statistics.median(cold) * 1e-3) / 1e12, 2),
        "wall_s": round(wall, 3),
    }
    if not args.no_cpu:
        # the headline's sample runs for the whole --cpu-seconds budget
        out["cpu_baseline"] = cpu_matmul(S, torch.float16, args.cpu_seconds, max_reps=10 ** 6)
        out["cpu_info"] = _CPU["info"]
    if not args.no_secondary:
        out["secondary"] = secondary(cpu=not args.no_cpu)
        # last, so that the end of the line (what a driver keeps of a long
        # line) holds every configuration's figure
        out["baseline_configs"] = summarize(out, out["secondary"])
    print(json.dumps(out), flush=True)


def _short_name(workload):
    """A compact key for a workload line of the summary."""
    w = workload
    for long, short in (("copy ceiling: newt copy kernel, ", "copy "), (" moved (read + write)", ""),
                        (" (extra: larger than the configuration)", ""), (" (+mean/rstd)", ""),
                        ("attention bf16 [4,32,4096,128] ", "attention "),
                        (" (examples/05 plain form)", " plain"),
                        (" (fp32 MFMA, full precision; the reference runs tf32)", ""),
                        (" (autotuned tile DSL)", ""), ("fp32 ", ""), ("fp16 ", ""),
                        ("host launch cost: add n=1e6 via @newt.jit (value) and torch.add(out=)",
                         "host launch (newt add)")):
        w = w.replace(long, short)
    if workload.startswith("matmul"):
        w = workload.split(" (")[0]
    return w


def summarize(head, lines):
    """Every measured configuration in one small object: per workload the
    value, its unit, the fraction of the peak that bounds it (HBM 8 TB/s or
    the dense MFMA peak; for memory-bound lines do_bench-timed), the
    kernel-only fraction on flushed caches (dispatch events; the headline's
    flushed median) where measured, and the torch CPU eager baseline's value
    in the same unit."""
    rows = {"matmul fp16 4096^3 (headline)": [
        head["value"], "TFLOP/s", head["roofline"]["frac"],
        round(head["tflops_flushed_median"] / PEAK_TFLOPS, 4),
        head.get("cpu_baseline", {}).get("value")]}
    for line in lines:
        if "workload" not in line:
            rows["error"] = line.get("error")
            continue
        frac = line.get("frac_hbm", line.get("frac_mfma"))
        if "frac_hbm" not in line and "frac_hbm_kernel_flushed" in line:
            frac = line["frac_hbm_kernel_flushed"]
        kern = line.get("frac_hbm_kernel_flushed", line.get("frac_mfma_kernel_flushed"))
        rows[_short_name(line["workload"])] = [
            line["value"], line["unit"], frac, kern, line.get("cpu_baseline", {}).get("value")]
    return {"fields": ["value", "unit", "frac_peak", "frac_peak_kernel_flushed", "cpu_baseline"],
            "rows": rows}


def timeline_source(src):
    """A generated matmul kernel's source with per-workgroup timestamps: one
    more parameter, `unsigned long long* _ts` (4 values per workgroup: start,
    end of the k-loop, end, XCC_ID), written by the workgroup's first thread."""
    import re
    head = re.search(r'extern "C" __global__ void [^{]*?\) \{', src)
    src = (src[:head.end() - 3] + ", unsigned long long* __restrict__ _ts) {\n"
           "  const unsigned long long _tsw_start = __builtin_amdgcn_s_memrealtime();" + src[head.end():])
    lines = src.split("\n")
    last_mfma = max(i for i, ln in enumerate(lines) if "newt::mfma" in ln)
    first = next(i for i in range(last_mfma, len(lines)) if "c_ptr" in lines[i])
    while not (lines[first].startswith("  ") and not lines[first].startswith("   ")):
        first -= 1   # the top-level statement holding the first C store
    lines.insert(first, "  const unsigned long long _tsw_loop = __builtin_amdgcn_s_memrealtime();")
    src = "\n".join(lines)
    end = src.rstrip().rfind("}")
    src = src[:end] + (
        "  {\n"
        "    const unsigned long long _tsw_end = __builtin_amdgcn_s_memrealtime();\n"
        "    const unsigned int _tsw_xcc = __builtin_amdgcn_s_getreg((15 << 11) | 20);\n"
        "    if (threadIdx.x == 0) {\n"
        "      const int _tsw_wg = blockIdx.x + gridDim.x * blockIdx.y;\n"
        "      _ts[_tsw_wg * 4 + 0] = _tsw_start; _ts[_tsw_wg * 4 + 1] = _tsw_loop; _ts[_tsw_wg * 4 + 2] = _tsw_end;\n"
        "      _ts[_tsw_wg * 4 + 3] = _tsw_xcc;\n"
        "    }\n"
        "  }\n") + src[end:]
    return src


def matmul_timeline(a, b, c, cfg, step, launches=40, keep=30):
    """Per-workgroup timestamps of the headline matmul: a copy of the kernel's
    generated source that reads the 100 MHz real-time counter at the start, at
    the end of the k-loop (before the C tile's first store) and at the end,
    and writes them with the workgroup's XCC_ID from its first thread. The
    copy runs `launches` times back to back behind a GPU spin; the last `keep`
    are summarised per XCD. Diagnostic only: the timed headline never runs it."""
    import re
    import torch
    from newt_amd import workloads as W
    from newt_amd.runtime import hip
    S = a.shape[0]
    args = (a, b, c, S, S, S, a.stride(0), a.stride(1), b.stride(0), b.stride(1),
            c.stride(0), c.stride(1))
    ck = W.matmul_kernel.specialize(*args, **cfg.kwargs, num_warps=cfg.num_warps,
                                    num_stages=cfg.num_stages)
    src = timeline_source(ck.source)
    kern = hip.Kernel(hip.compile_hip(src, ck.name), ck.name, ck.lds_bytes)
    packer = hip.pack_format(ck.kinds + ["ptr"])
    named = dict(zip(W.matmul_kernel.param_names, args))
    vals = [named[n].data_ptr() if torch.is_tensor(named[n]) else named[n] for n in ck.param_names]
    gx, gy = S // cfg.kwargs["BLOCK_M"], S // cfg.kwargs["BLOCK_N"]
    bufs = [torch.zeros(gx * gy * 4, dtype=torch.int64, device="cuda") for _ in range(launches)]
    stream = torch.cuda.current_stream().cuda_stream
    for _ in range(50):
        step()
    settle_clocks(step, SETTLE_S)
    torch.cuda._sleep(LEAD_CYCLES)
    for buf in bufs:
        kern.launch_packed(gx, gy, 1, 64 * cfg.num_warps, stream, packer.pack(*(vals + [buf.data_ptr()])))
    torch.cuda.synchronize()
    err, bad = check_matmul(a, b, c, "float16")
    runs = [buf.view(-1, 4).cpu().tolist() for buf in bufs[-keep:]]
    per = {}
    for run in runs:
        for t0, t1, t2, x in run:
            d = per.setdefault(x & 0xF, {"loop": [], "store": []})
            d["loop"].append((t1 - t0) / 100)
            d["store"].append((t2 - t1) / 100)
    spans = [(max(r[2] for r in run) - min(r[0] for r in run)) / 100 for run in runs]
    starts = [(max(r[0] for r in run) - min(r[0] for r in run)) / 100 for run in runs]
    log(f"matmul timeline: {keep} launches of {ck.name}, {gx * gy} workgroups each; "
        f"rel. Frobenius {err:.2e}, {bad} elements beyond one ulp")
    log(f"  launch span median {statistics.median(spans):.2f} us (workgroup start to last end); "
        f"start spread median {statistics.median(starts):.2f} us")
    for x in sorted(per):
        lp, stv = per[x]["loop"], per[x]["store"]
        log(f"  XCD {x}: {len(lp) // keep} workgroups, k-loop median {statistics.median(lp):.2f} us "
            f"(min {min(lp):.2f}, max {max(lp):.2f}), C store median {statistics.median(stv):.2f} us")


def run_only(name, power=0.0):
    """One workload for profiler runs (counters / kernel traces); with
    `power`, then that many seconds of it under the PowerSampler."""
    import torch
    if name == "copy":
        src = torch.ones(64 << 20, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy: 5 x 256 MiB device-to-device copies")
        return
    if name.startswith("newt copy"):
        # the copy ceiling's kernel at 128 MiB moved (the layernorm's bytes)
        from newt_amd import workloads as W
        src = torch.ones(128 << 20 >> 3, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(10):
            W.copy(src, dst)
        torch.cuda.synchronize()
        assert torch.equal(dst, src)
        log("newt copy: 10 x 128 MiB moved (64 MiB read, 64 MiB written)")
        return
    for wl in _secondary_workloads():
        if wl["name"].startswith(name):
            for _ in range(10):
                wl["fn"]()
            torch.cuda.synchronize()
            wl["check"]()
            log(f"{name}: ran {wl['name']}")
            if power:
                flops = wl["name"].startswith("attention")
                power_window(wl["name"], wl["fn"], power, flop=wl["work"] if flops else None,
                             nbytes=None if flops else wl["work"])
            return
    raise SystemExit(f"bench.py: no workload named {name!r}")


def _secondary_workloads():
    """One dict per memory-bound or attention workload: name, algorithmic
    bytes or flop per launch, the launch, the oracle check of the launch's
    output buffer (run after the timing, so it reads what the timed launches
    wrote), and the torch CPU eager baseline of the same workload."""
    import numpy as np
    import torch
    from newt_amd import workloads as W
    from oracle import newt_oracle as orc
    from oracle import torch_eager as te
    npf = lambda t: t.detach().float().cpu().numpy()
    out = []

    def add_line(n, name, extra=False):
        x1, y1 = seeded(n, 0), seeded(n, 1)
        o1 = torch.empty_like(x1)
        xc, yc = x1.cpu(), y1.cpu()

        def chk():
            idx = torch.from_numpy(orc.spread(n, min(n, 1 << 20))).cuda()
            assert np.array_equal(npf(o1[idx]), orc.vector_add(npf(x1[idx]), npf(y1[idx])))
        out.append({"name": name, "work": 12 * n, "fn": lambda: W.add(x1, y1, o1), "check": chk,
                    "cpu": (12 * n, lambda: te.vector_add(xc, yc), "x + y (fp32, same n)", 1.0),
                    "extra": extra})
    add_line(1_000_000, "add fp32 n=1e6")

    for C in (1000, 4096, 8192):
        xs = seeded((4096, C), 0, scale=4.0)
        os_ = torch.empty_like(xs)
        xsc = xs.cpu()

        def chk_sm(xs=xs, os_=os_, C=C):
            # every row, rtol 1e-5 on every element (relative)
            bad = orc.rel_violations(npf(os_), orc.softmax_rows(npf(xs)), 1e-5)
            assert bad == 0, f"softmax 4096x{C}: {bad} elements beyond rtol 1e-5"
        out.append({"name": f"softmax fp32 4096x{C}", "work": 2 * 4 * 4096 * C,
                    "fn": (lambda xs=xs, os_=os_: W.softmax(xs, os_)), "check": chk_sm,
                    "cpu": (2 * 4 * 4096 * C, (lambda xsc=xsc: te.softmax(xsc)),
                            f"torch.softmax (fp32 [4096, {C}])", 1.0)})

    xl = seeded((4096, 8192), 0, dtype=torch.float16)
    wl = seeded(8192, 2, scale=0.1, mean=1.0, dtype=torch.float16)
    bl = seeded(8192, 3, scale=0.1, dtype=torch.float16)
    ol = torch.empty_like(xl)
    ln_out = {}
    xlc, wlc, blc = xl.cpu(), wl.cpu(), bl.cpu()

    def run_ln():
        ln_out["r"] = W.layernorm(xl, wl, bl, 1e-5, ol)

    def chk_ln():
        # every row: y within one fp16 ulp, mean and rstd rtol 1e-5
        # (oracle.layernorm_violations states the floors)
        y, mean, rstd = ln_out["r"]
        bad = orc.layernorm_violations(npf(y), npf(mean), npf(rstd), npf(xl), npf(wl), npf(bl),
                                       1e-5, "float16")
        assert bad == {"y": 0, "mean": 0, "rstd": 0}, f"layernorm: {bad}"
    out.append({"name": "layernorm fp16 4096x8192 (+mean/rstd)", "work": 134_283_264,
                "fn": run_ln, "check": chk_ln,
                "cpu": (134_283_264, lambda: te.layernorm(xlc, wlc, blc, 1e-5),
                        "torch.native_layer_norm on fp32 upcasts of x, w, b (fp16 [4096, 8192])",
                        1.0)})

    q, k, v = (seeded((4, 32, 4096, 128), s, dtype=torch.bfloat16) for s in (6, 7, 8))
    oa = torch.empty_like(q)
    # CPU sample: 2 of the 128 (batch, head) pairs in fp32
    qc, kc, vc = (t[:1, :2].float().cpu() for t in (q, k, v))
    for causal, plain in ((False, False), (True, False), (False, True), (True, True)):
        flop = 4 * 4 * 32 * 128 * (4096 ** 2 if not causal else 4096 * 4097 // 2)

        def chk_at(causal=causal):
            # every program: one row of every 128-row query block of every
            # (batch, head), plus three whole blocks of eight pairs
            res = orc.attention_sampled_errors(npf(q), npf(k), npf(v), npf(oa), 128 ** -0.5,
                                               causal, block=128)
            assert res["worst_row"] <= 1e-2 and res["worst_pair"] <= 1e-2, f"attention: {res}"
        form = " (examples/05 plain form)" if plain else ""
        out.append({"name": f"attention bf16 [4,32,4096,128] {'causal' if causal else 'non-causal'}"
                            f"{form}", "work": flop,
                    "fn": (lambda causal=causal, plain=plain:
                           W.attention(q, k, v, causal, out=oa, plain=plain)),
                    "check": chk_at,
                    "cpu": (flop / 64, (lambda causal=causal: te.attention(qc, kc, vc, causal)),
                            "F.scaled_dot_product_attention in fp32 on 2 of the 128 "
                            "(batch, head) pairs", 64.0)})

    # larger vector adds (the reference benches 2^20..2^27 elements): the add
    # lowering's HBM efficiency once launch overhead no longer dominates
    add_line(1 << 27, "add fp32 n=2^27 (extra: larger than the configuration)", extra=True)
    return out


def warm_up(fn, seconds=0.2):
    """Run fn back to back for about `seconds` of GPU time, so the timing that
    follows does not start on clocks that dropped while the host was busy."""
    import torch
    fn()
    torch.cuda.synchronize()
    settle_clocks(fn, seconds)


def host_launch_cost(launches=1000):
    """Host time per launch of the vector add (n = 10^6) through @newt.jit,
    and of torch.add(x, y, out=o) for comparison: `launches` calls queued
    behind a GPU spin long enough that the GPU never waits for the host, so
    the loop's wall time divided by `launches` is the host's own cost."""
    import torch
    from newt_amd import workloads as W
    x, y = seeded(1_000_000, 0), seeded(1_000_000, 1)
    o = torch.empty_like(x)
    out = {}
    for name, fn in (("newt", lambda: W.add(x, y, o)), ("torch", lambda: torch.add(x, y, out=o))):
        for _ in range(50):
            fn()
        reps = []
        for _ in range(3):
            torch.cuda.synchronize()
            torch.cuda._sleep(LEAD_CYCLES * 20)
            t0 = time.perf_counter()
            for _ in range(launches):
                fn()
            reps.append((time.perf_counter() - t0) / launches * 1e6)
            torch.cuda.synchronize()
        out[name] = round(min(reps), 2)
    return {"workload": "host launch cost: add n=1e6 via @newt.jit (value) and torch.add(out=)",
            "value": out["newt"], "unit": "us/launch", "torch_add_us": out["torch"],
            "launches": launches}


def secondary(cpu=True, cpu_budget=2.0):
    import torch
    from newt_amd import workloads as W
    from newt_amd.testing import _flush_buffer, do_bench
    res = []
    try:
        flush = _flush_buffer()
        # the copy ceiling: a newt copy kernel at the memory-bound lines' sizes,
        # on cold caches, timed by events its own dispatch records
        for nbytes in (134_217_728, 268_435_456, 1 << 30):
            n = nbytes // 2 // 4
            src = torch.ones(n, device="cuda")
            dst = torch.empty_like(src)
            fn = lambda: W.copy(src, dst)
            warm_up(fn)
            _, _, cold = timed_launches(fn, 20, before=lambda: flush.sum(), with_list=True)
            ms = statistics.median(cold)
            assert torch.equal(dst, src)
            res.append({"workload": f"copy ceiling: newt copy kernel, {nbytes >> 20} MiB moved "
                                    f"(read + write)", "value": round(nbytes / (ms * 1e-3) / 1e9, 1),
                        "unit": "GB/s", "ms_kernel_flushed": round(ms, 5),
                        "frac_hbm_kernel_flushed": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_GBS, 4),
                        "bytes": nbytes})
            del src, dst
        for wl in _secondary_workloads():
            name, work, fn = wl["name"], wl["work"], wl["fn"]
            warm_up(fn)
            ms = do_bench(fn, warmup=5, rep=20)        # caches flushed before each rep
            _, kern = timed_launches(fn, 20)            # back to back, per-launch events
            # flushed like do_bench, timed by the dispatch's own events
            _, _, cold = timed_launches(fn, 20, before=lambda: flush.sum(), with_list=True)
            kern_cold = statistics.median(cold)
            wl["check"]()                               # the timed launches' output
            if name.startswith("attention"):
                line = {"workload": name, "value": round(work / (ms * 1e-3) / 1e12, 2),
                        "unit": "TFLOP/s", "ms": round(ms, 5),
                        "frac_mfma": round(work / (ms * 1e-3) / 1e12 / PEAK_TFLOPS, 4),
                        "ms_kernel_flushed": round(kern_cold, 5),
                        "frac_mfma_kernel_flushed": round(work / (kern_cold * 1e-3) / 1e12
                                                          / PEAK_TFLOPS, 4),
                        "flop": work}
                unit = "TFLOP/s"
            else:
                v = work / (ms * 1e-3) / 1e9
                line = {"workload": name, "value": round(v, 1), "unit": "GB/s",
                        "ms_flushed": round(ms, 5), "frac_hbm": round(v / PEAK_GBS, 4),
                        "ms_kernel_flushed": round(kern_cold, 5),
                        "frac_hbm_kernel_flushed": round(work / (kern_cold * 1e-3) / 1e9
                                                         / PEAK_GBS, 4),
                        "ms_back_to_back": round(kern, 5), "bytes": work}
                unit = "GB/s"
            if cpu:
                cwork, cfn, what, _ = wl["cpu"]
                line["cpu_baseline"] = cpu_line(cwork, unit, cfn, cpu_budget, what)
            res.append(line)
        # the other square sizes and dtypes of the matmul configuration, each
        # autotuned and checked like the headline; torch.mm (hipBLASLt) is timed
        # beside the fp16/bf16 ones for context
        for dt, S, tuned, peak, name in (
                (torch.float16, 1024, W.matmul_tuned, PEAK_TFLOPS, "matmul fp16 1024^3"),
                (torch.float16, 2048, W.matmul_tuned, PEAK_TFLOPS, "matmul fp16 2048^3"),
                (torch.float16, 8192, W.matmul_tuned, PEAK_TFLOPS, "matmul fp16 8192^3"),
                (torch.bfloat16, 1024, W.matmul_tuned, PEAK_TFLOPS, "matmul bf16 1024^3"),
                (torch.bfloat16, 2048, W.matmul_tuned, PEAK_TFLOPS, "matmul bf16 2048^3"),
                (torch.bfloat16, 4096, W.matmul_tuned, PEAK_TFLOPS, "matmul bf16 4096^3"),
                (torch.bfloat16, 8192, W.matmul_tuned, PEAK_TFLOPS, "matmul bf16 8192^3"),
                (torch.float32, 4096, W.matmul_tuned_fp32, PEAK_FP32_TFLOPS,
                 "matmul fp32 4096^3 (fp32 MFMA, full precision; the reference runs tf32)")):
            a = seeded((S, S), 4, scale=S ** -0.5, dtype=dt)
            b = seeded((S, S), 5, scale=S ** -0.5, dtype=dt)
            c = torch.empty(S, S, device="cuda", dtype=dt)
            W.matmul(a, b, c)                           # autotune
            cfg = tuned.best_config
            run = lambda: W.matmul(a, b, c, config=cfg)
            warm_up(run)
            # like the headline: K launches queued behind a GPU spin, one event
            # pair around them (at 1024^3 the host's ~30 us per launch would
            # otherwise leave the GPU idle, and clocking down, between kernels).
            # The median of five such windows: one window of a short kernel
            # (~0.4 ms at 2048^3) samples a single point of the clock the power
            # limit moves up and down
            kern = statistics.median(bracketed_launches(run, 20) / 20 for _ in range(MM_WINDOWS))
            _, kern_ev = timed_launches(run, 20)
            v = 2.0 * S ** 3 / (kern * 1e-3) / 1e12
            dname = {torch.float16: "float16", torch.bfloat16: "bfloat16",
                     torch.float32: "float32"}[dt]
            err, bad = check_matmul(a, b, c, dname)     # the timed launches' output
            assert err <= (1e-2 if dt != torch.float32 else 1e-5), f"{name}: rel. Frobenius {err}"
            assert dt == torch.float32 or bad == 0, f"{name}: {bad} elements beyond one ulp"
            line = {"workload": name, "value": round(v, 2), "unit": "TFLOP/s",
                    "ms": round(kern, 5), "frac_mfma": round(v / peak, 4),
                    "ms_dispatch_events": round(kern_ev, 5),
                    "rel_frobenius_vs_oracle": err,
                    "tile": dict(cfg.kwargs), "num_warps": cfg.num_warps,
                    "num_stages": cfg.num_stages}
            if dt != torch.float32:
                for _ in range(3):
                    torch.mm(a, b, out=c)
                tk = statistics.median(bracketed_launches(lambda: torch.mm(a, b, out=c), 20) / 20
                                       for _ in range(MM_WINDOWS))
                line["torch_mm_tflops"] = round(2.0 * S ** 3 / (tk * 1e-3) / 1e12, 2)
            if cpu:
                line["cpu_baseline"] = cpu_matmul(S, dt, cpu_budget,
                                                  rows=None if S <= 2048 else 512)
            res.append(line)
            del a, b, c
        res.append(host_launch_cost())
        S = 4096
        # deuteron: the same matmul written as tiles, traced to newt and
        # autotuned against its eager oracle (examples/deuteron/01_matmul.py)
        import tempfile
        os.environ["DEUTERON_CACHE_DIR"] = tempfile.mkdtemp(prefix="deuteron-bench-")  # tune here
        k = W.dt_matmul
        a = seeded((S, S), 4, scale=S ** -0.5, dtype=torch.float16)
        b = seeded((S, S), 5, scale=S ** -0.5, dtype=torch.float16)
        c = torch.empty(S, S, device="cuda", dtype=torch.float16)
        k(a, b, c)                                      # trace + autotune
        warm_up(lambda: k(a, b, c))
        kern = bracketed_launches(lambda: k(a, b, c), 20) / 20
        v = 2.0 * S ** 3 / (kern * 1e-3) / 1e12
        err, bad = check_matmul(a, b, c, "float16")
        assert err <= 1e-2 and bad == 0, f"deuteron matmul: rel. Frobenius {err}, {bad} bad"
        line = {"workload": "deuteron matmul fp16 4096^3 (autotuned tile DSL)",
                "value": round(v, 2), "unit": "TFLOP/s", "ms": round(kern, 5),
                "frac_mfma": round(v / PEAK_TFLOPS, 4), "rel_frobenius_vs_oracle": err,
                "config": dict(k.best_config)}
        if cpu:
            line["cpu_baseline"] = cpu_matmul(S, torch.float16, cpu_budget, rows=512)
        res.append(line)
    except Exception as e:  # report what was measured, and why the rest was not
        res.append({"error": f"{type(e).__name__}: {str(e)[:300]}"})
    return res


if __name__ == "__main__":
    main()
