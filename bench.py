"""newt on MI355X - headline benchmark.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-secondary] [--no-cpu]

One "step" is one launch of the newt matmul kernel (the examples/04 body,
compiled by newt_amd to HIP for gfx950, autotuned over its gfx950 config space)
on fp16 A[4096,4096] @ B[4096,4096] -> C fp16 with fp32 accumulation. Inputs are
resident in HBM before the timed region; `value` is TFLOP/s over the K timed
steps (2*M*N*K flop per step). The one JSON line also carries:

  roofline      the matmul kernel vs MI355X's dense fp16 MFMA peak (2.5 PFLOP/s):
                2*M*N*K flop per launch / the average launch duration from HIP
                events (without system-scope fences) recorded around each
                launch on the launch stream
  cpu_baseline  the reference's oracle (torch CPU eager, A.float() @ B.float())
                timed on this host's cores on the same 4096^3 problem
  secondary     vector add / softmax / layernorm (GB/s vs 8 TB/s HBM), bf16
                matmul and flash attention (TFLOP/s), each checked against the
                oracle before it is timed

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
                    help="run one workload for profiler runs: 'matmul', 'copy', or the "
                         "start of a secondary workload's name (e.g. 'softmax fp32 4096x4096')")
    return ap.parse_args()


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


def timed_launches(fn, steps, embedded=True, before=None):
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
    return total, sum(per) / len(per)


def bracketed_launches(fn, steps):
    """Run fn() `steps` times back to back with one HIP event pair around all
    of them and nothing between launches. Returns the total ms."""
    import torch
    hev = _HipEvents()
    stream = torch.cuda.current_stream().cuda_stream
    st, en = hev.make(1), hev.make(1)
    torch.cuda.synchronize()
    hev.record(st[0], stream)
    for _ in range(steps):
        fn()
    hev.record(en[0], stream)
    torch.cuda.synchronize()
    total = hev.ms(st[0], en[0])
    hev.destroy(st + en)
    return total


def cpu_baseline(S, budget_s):
    """torch CPU eager A.float() @ B.float() (the reference's oracle) on the full
    problem, median of >= 5 reps after 2 warm-ups."""
    import torch
    from oracle import torch_eager
    threads = torch.get_num_threads()
    g = torch.Generator().manual_seed(4)
    a = (torch.randn(S, S, generator=g) * S ** -0.5).half()
    b = (torch.randn(S, S, generator=g) * S ** -0.5).half()
    for _ in range(2):
        torch_eager.matmul(a, b)
    reps, t0 = [], time.perf_counter()
    while len(reps) < 5 or (time.perf_counter() - t0 < budget_s and len(reps) < 50):
        t1 = time.perf_counter()
        torch_eager.matmul(a, b)
        reps.append(time.perf_counter() - t1)
    med = statistics.median(reps)
    return {"value": round(2.0 * S ** 3 / med / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"torch {torch.__version__} CPU eager A.float() @ B.float() (oracle/"
                      f"torch_eager.py) on the full fp16 {S}^3 problem, median of {len(reps)} reps "
                      f"({sum(reps):.1f} s), {threads} threads, {os.cpu_count()} logical CPUs, "
                      f"{platform.processor() or platform.machine()}"}


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


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one MI355X (every box here has one GPU); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    torch.cuda.set_device(0)
    if args.only and args.only != "matmul":
        return run_only(args.only)
    from newt_amd import workloads as W
    from oracle import newt_oracle as orc

    S = args.size
    a = seeded((S, S), 4, scale=S ** -0.5, dtype=torch.float16)
    b = seeded((S, S), 5, scale=S ** -0.5, dtype=torch.float16)
    c = torch.empty(S, S, device="cuda", dtype=torch.float16)
    cfg = pick_matmul_config(a, b, c, args)
    step = lambda: W.matmul(a, b, c, config=cfg)
    # warm-up straight after the autotuner's runs: the chip's clocks drop
    # while it idles (a CPU-side check here cost ~20% on the first timed
    # launches), so the oracle check of the measured configuration's output
    # follows the timed region instead of preceding it
    for _ in range(args.warmup):
        step()
    # the timed region: K back-to-back launches between one event pair (any
    # per-launch event adds ~3.5-4.5 us per step); each launch's own duration
    # then comes from a second pass of K launches whose dispatches record events
    t0 = time.perf_counter()
    total_ms = bracketed_launches(step, args.steps)
    wall = time.perf_counter() - t0
    _, kern_ms = timed_launches(step, args.steps)
    # parity of the measured configuration against the oracle (sampled rows of
    # the last timed step's output)
    rows = slice(0, 256)
    ref = orc.matmul(a[rows].float().cpu().numpy(), b.float().cpu().numpy(), "float16")
    err = orc.rel_frobenius(c[rows].float().cpu().numpy(), ref)
    if not err <= 1e-2:
        raise SystemExit(f"bench.py: matmul result differs from the oracle (rel. Frobenius {err})")
    flop = 2.0 * S ** 3
    value = flop * args.steps / (total_ms * 1e-3) / 1e12
    achieved = flop / (kern_ms * 1e-3) / 1e12
    if args.only:
        log(f"matmul only: {value:.1f} TFLOP/s")
        return
    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(total_ms / args.steps, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic (seeded N(0,1)/sqrt(K) fp16 inputs)",
        "config": {"workload": f"matmul fp16 {S}x{S}x{S}, examples/04 kernel body via @newt.jit "
                               f"-> HIP for gfx950 (autotuned)",
                   "M": S, "N": S, "K": S, "tile": dict(cfg.kwargs), "num_warps": cfg.num_warps,
                   "num_stages": cfg.num_stages, "rel_frobenius_vs_oracle": err},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_TFLOPS, 4),
                     "traffic": matmul_traffic(cfg)},
        "wall_s": round(wall, 3),
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(S, args.cpu_seconds)
    if not args.no_secondary:
        out["secondary"] = secondary()
    print(json.dumps(out), flush=True)


def run_only(name):
    """One workload for profiler runs (counters / kernel traces)."""
    import torch
    from newt_amd import workloads as W
    if name == "copy":
        src = torch.ones(64 << 20, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy: 5 x 256 MiB device-to-device copies")
        return
    for wl in _secondary_workloads():
        if wl[0].startswith(name):
            _, nbytes_or_flop, fn, check = wl
            check()
            for _ in range(10):
                fn()
            torch.cuda.synchronize()
            log(f"{name}: ran {wl[0]}")
            return


def _secondary_workloads():
    """(name, algorithmic bytes or flop, launch fn, oracle check) per workload."""
    import numpy as np
    import torch
    from newt_amd import workloads as W
    from oracle import newt_oracle as orc
    npf = lambda t: t.detach().float().cpu().numpy()
    out = []

    x1, y1 = seeded(1_000_000, 0), seeded(1_000_000, 1)
    o1 = torch.empty_like(x1)

    def chk_add():
        W.add(x1, y1, o1)
        assert np.array_equal(npf(o1), orc.vector_add(npf(x1), npf(y1)))
    out.append(("add fp32 n=1e6", 12_000_000, lambda: W.add(x1, y1, o1), chk_add))

    for C in (1000, 4096, 8192):
        xs = seeded((4096, C), 0, scale=4.0)
        os_ = torch.empty_like(xs)

        def chk_sm(xs=xs, os_=os_):
            W.softmax(xs, os_)
            np.testing.assert_allclose(npf(os_[:64]), orc.softmax_rows(npf(xs[:64])),
                                       rtol=1e-5, atol=1e-6)
        out.append((f"softmax fp32 4096x{C}", 2 * 4 * 4096 * C,
                    (lambda xs=xs, os_=os_: W.softmax(xs, os_)), chk_sm))

    xl = seeded((4096, 8192), 0, dtype=torch.float16)
    wl = seeded(8192, 2, scale=0.1, mean=1.0, dtype=torch.float16)
    bl = seeded(8192, 3, scale=0.1, dtype=torch.float16)
    ol = torch.empty_like(xl)

    def chk_ln():
        y, mean, rstd = W.layernorm(xl, wl, bl, 1e-5, ol)
        ry, rm, rr = orc.layernorm_rows(npf(xl[:64]), npf(wl), npf(bl), 1e-5, "float16")
        np.testing.assert_allclose(npf(y[:64]), ry, rtol=2e-3, atol=2e-3)
        np.testing.assert_allclose(npf(rstd[:64]), rr, rtol=1e-5, atol=1e-6)
    out.append(("layernorm fp16 4096x8192 (+mean/rstd)", 134_283_264,
                lambda: W.layernorm(xl, wl, bl, 1e-5, ol), chk_ln))

    q, k, v = (seeded((4, 32, 4096, 128), s, dtype=torch.bfloat16) for s in (6, 7, 8))
    oa = torch.empty_like(q)
    for causal in (False, True):
        flop = 4 * 4 * 32 * 128 * (4096 ** 2 if not causal else 4096 * 4097 // 2)

        def chk_at(causal=causal):
            o = W.attention(q[:1, :2], k[:1, :2], v[:1, :2], causal)
            ref = orc.attention(npf(q[:1, :2]), npf(k[:1, :2]), npf(v[:1, :2]), 128 ** -0.5,
                                causal, p_dtype="bfloat16", out_dtype="bfloat16")
            assert orc.rel_frobenius(npf(o), ref) <= 1e-2
        out.append((f"attention bf16 [4,32,4096,128] {'causal' if causal else 'non-causal'}",
                    flop, (lambda causal=causal: W.attention(q, k, v, causal, out=oa)), chk_at))
    return out


def warm_up(fn, seconds=0.03):
    """Run fn back to back for about `seconds` of GPU time, so the timing that
    follows does not start on clocks that dropped while the host was busy."""
    import torch
    fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    fn()
    torch.cuda.synchronize()
    one = max(time.perf_counter() - t0, 1e-6)
    for _ in range(min(2000, int(seconds / one))):
        fn()
    torch.cuda.synchronize()


def secondary():
    import torch
    from newt_amd import workloads as W
    from newt_amd.testing import _flush_buffer, do_bench
    res = []
    try:
        for name, work, fn, check in _secondary_workloads():
            check()
            warm_up(fn)
            ms = do_bench(fn, warmup=5, rep=20)        # caches flushed before each rep
            _, kern = timed_launches(fn, 20)            # back to back, per-launch events
            flush = _flush_buffer()
            # flushed like do_bench, timed by the dispatch's own events
            _, kern_cold = timed_launches(fn, 20, before=lambda: flush.sum())
            if name.startswith("attention"):
                res.append({"workload": name, "value": round(work / (ms * 1e-3) / 1e12, 2),
                            "unit": "TFLOP/s", "ms": round(ms, 5),
                            "frac_mfma": round(work / (ms * 1e-3) / 1e12 / PEAK_TFLOPS, 4),
                            "flop": work})
            else:
                v = work / (ms * 1e-3) / 1e9
                res.append({"workload": name, "value": round(v, 1), "unit": "GB/s",
                            "ms_flushed": round(ms, 5), "frac_hbm": round(v / PEAK_GBS, 4),
                            "ms_kernel_flushed": round(kern_cold, 5),
                            "frac_hbm_kernel_flushed": round(work / (kern_cold * 1e-3) / 1e9
                                                             / PEAK_GBS, 4),
                            "ms_back_to_back": round(kern, 5), "bytes": work})
        from oracle import newt_oracle as orc
        # the other square sizes and dtypes of the matmul configuration, each
        # autotuned and checked like the headline; torch.mm (hipBLASLt) is timed
        # beside the fp16/bf16 ones for context
        for dt, S, tuned, peak, name in (
                (torch.float16, 1024, W.matmul_tuned, PEAK_TFLOPS, "matmul fp16 1024^3"),
                (torch.float16, 2048, W.matmul_tuned, PEAK_TFLOPS, "matmul fp16 2048^3"),
                (torch.float16, 8192, W.matmul_tuned, PEAK_TFLOPS, "matmul fp16 8192^3"),
                (torch.bfloat16, 4096, W.matmul_tuned, PEAK_TFLOPS, "matmul bf16 4096^3"),
                (torch.float32, 4096, W.matmul_tuned_fp32, PEAK_FP32_TFLOPS,
                 "matmul fp32 4096^3 (fp32 MFMA, full precision; the reference runs tf32)")):
            a = seeded((S, S), 4, scale=S ** -0.5, dtype=dt)
            b = seeded((S, S), 5, scale=S ** -0.5, dtype=dt)
            c = torch.empty(S, S, device="cuda", dtype=dt)
            W.matmul(a, b, c)                           # autotune
            cfg = tuned.best_config
            run = lambda: W.matmul(a, b, c, config=cfg)
            for _ in range(min(500, max(10, int(0.02 / (2.0 * S ** 3 / 1e15))))):
                run()                                   # ~20 ms warm-up (clocks)
            _, kern = timed_launches(run, 20)
            v = 2.0 * S ** 3 / (kern * 1e-3) / 1e12
            rows = slice(0, 128)                        # then the check (CPU)
            ref = orc.matmul(a[rows].float().cpu().numpy(), b.float().cpu().numpy(),
                             "bfloat16" if dt == torch.bfloat16 else "float32")
            err = orc.rel_frobenius(c[rows].float().cpu().numpy(), ref)
            assert err <= 1e-2, f"{name}: rel. Frobenius {err}"
            line = {"workload": name, "value": round(v, 2), "unit": "TFLOP/s",
                    "ms": round(kern, 5), "frac_mfma": round(v / peak, 4),
                    "rel_frobenius_vs_oracle": err,
                    "tile": dict(cfg.kwargs), "num_warps": cfg.num_warps,
                    "num_stages": cfg.num_stages}
            if dt != torch.float32:
                for _ in range(3):
                    torch.mm(a, b, out=c)
                _, tk = timed_launches(lambda: torch.mm(a, b, out=c), 20, embedded=False)
                line["torch_mm_tflops"] = round(2.0 * S ** 3 / (tk * 1e-3) / 1e12, 2)
            res.append(line)
            del a, b, c
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
        for _ in range(150):
            k(a, b, c)                                  # warm-up (clocks)
        _, kern = timed_launches(lambda: k(a, b, c), 20)
        v = 2.0 * S ** 3 / (kern * 1e-3) / 1e12
        ref = orc.matmul(a[:128].float().cpu().numpy(), b.float().cpu().numpy(), "float16")
        err = orc.rel_frobenius(c[:128].float().cpu().numpy(), ref)
        assert err <= 1e-2, f"deuteron matmul: rel. Frobenius {err}"
        res.append({"workload": "deuteron matmul fp16 4096^3 (autotuned tile DSL)",
                    "value": round(v, 2), "unit": "TFLOP/s", "ms": round(kern, 5),
                    "frac_mfma": round(v / PEAK_TFLOPS, 4), "rel_frobenius_vs_oracle": err,
                    "config": dict(k.best_config)})
    except Exception as e:  # report what was measured, and why the rest was not
        res.append({"error": f"{type(e).__name__}: {str(e)[:300]}"})
    return res


if __name__ == "__main__":
    main()
