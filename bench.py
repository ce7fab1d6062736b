"""newt on MI355X - headline benchmark.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-secondary]

One "step" = one launch of the newt matmul kernel (examples/04 body, compiled by
newt_amd to HIP for gfx950) on fp16 A[4096,4096] @ B[4096,4096] -> C fp16 with
fp32 accumulation, inputs resident in HBM. `value` is TFLOP/s over the K timed
steps (2*M*N*K flop per step). The same JSON line carries:
  roofline      the matmul kernel vs the dense fp16 MFMA peak, kernel time from
                HIP events on the launch stream
  cpu_baseline  the numpy oracle (fp32 GEMM) timed on this host's cores on a
                bounded slice of the same problem
  secondary     softmax / layernorm / vector add (GB/s vs 8 TB/s HBM), bf16
                matmul, and flash attention causal / non-causal (TFLOP/s)
Everything runs on one GPU; --gpus above 1 exits with a message.
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_TFLOPS = 2500.0   # MI355X dense fp16/bf16 MFMA
PEAK_GBS = 8000.0      # MI355X HBM3E
METRIC = "fp16 4096^3 matmul TFLOP/s (% MFMA peak); softmax/layernorm GB/s (% HBM)"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--size", type=int, default=4096)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--config", default=None, help="BM,BN,BK,warps,stages (skip autotune)")
    return ap.parse_args()


def seeded(shape, seed, scale=1.0, mean=0.0, dtype=None):
    import torch
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(shape, generator=g) * scale + mean
    return t.to(dtype or torch.float32).to("cuda")


def event_time_ms(fn, reps):
    """Average device time per call of fn over `reps` back-to-back calls,
    HIP events recorded on the current (launch) stream."""
    import torch
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps


def cpu_baseline(size):
    """numpy fp32 GEMM (the oracle's matmul) on a bounded slice: rows of A
    chosen so the timed work is ~10 s or less."""
    import numpy as np
    try:
        from threadpoolctl import threadpool_info
        cores = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        cores = os.cpu_count() or 1
    rng = np.random.default_rng(0)
    b = rng.standard_normal((size, size), dtype=np.float32)
    rows = 256
    a = rng.standard_normal((rows, size), dtype=np.float32)
    a @ b  # warm
    t0 = time.perf_counter()
    reps = 0
    while True:
        a @ b
        reps += 1
        el = time.perf_counter() - t0
        if el > 3.0 or reps >= 50:
            break
    tflops = 2.0 * rows * size * size * reps / el / 1e12
    return {"value": round(tflops, 4), "unit": "TFLOP/s", "cores": int(cores), "kind": "port",
            "sample": f"oracle matmul (numpy fp32 BLAS) on A[{rows},{size}] @ B[{size},{size}], "
                      f"{reps} reps, {el:.1f} s; scaled to TFLOP/s"}


def pick_matmul_config(a, b, c, args):
    import newt_amd as newt
    from newt_amd import workloads as W
    if args.config:
        BM, BN, BK, nw, ns = (int(x) for x in args.config.split(","))
        return newt.Config({"BLOCK_M": BM, "BLOCK_N": BN, "BLOCK_K": BK}, num_warps=nw,
                           num_stages=ns)
    W.matmul(a, b, c)  # autotune over MATMUL_CONFIGS (untimed)
    return W.matmul_tuned.best_config


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one MI355X only (one GPU per box); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    from newt_amd import workloads as W
    from newt_amd.testing import do_bench

    S = args.size
    a = seeded((S, S), 4, scale=S ** -0.5, dtype=torch.float16)
    b = seeded((S, S), 5, scale=S ** -0.5, dtype=torch.float16)
    c = torch.empty(S, S, device="cuda", dtype=torch.float16)
    cfg = pick_matmul_config(a, b, c, args)
    step = lambda: W.matmul(a, b, c, config=cfg)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ms = event_time_ms(step, args.steps)
    wall = time.perf_counter() - t0
    flop = 2.0 * S ** 3
    tflops = flop / (ms * 1e-3) / 1e12
    # parity of the measured configuration against the oracle (sampled rows)
    from oracle import newt_oracle as orc
    rows = slice(0, 256)
    ref = orc.matmul(a[rows].float().cpu().numpy(), b.float().cpu().numpy(), "float16")
    err = orc.rel_frobenius(c[rows].float().cpu().numpy(), ref)

    out = {
        "metric": METRIC, "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": f"matmul fp16 {S}^3 (examples/04 body via @newt.jit -> HIP gfx950)",
                   "M": S, "N": S, "K": S, "tile": dict(cfg.kwargs), "num_warps": cfg.num_warps,
                   "num_stages": cfg.num_stages, "rel_frobenius_vs_oracle": err},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_TFLOPS, 4), "traffic": None},
        "wall_s": round(wall, 3),
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(S)
    if not args.no_secondary:
        out["secondary"] = secondary(do_bench)
    print(json.dumps(out))


def secondary(do_bench):
    import torch
    from newt_amd import workloads as W
    res = []

    def gbs(name, nbytes, fn):
        ms = do_bench(fn, warmup=5, rep=20)
        v = nbytes / (ms * 1e-3) / 1e9
        res.append({"workload": name, "value": round(v, 1), "unit": "GB/s", "ms": round(ms, 5),
                    "frac_hbm": round(v / PEAK_GBS, 4), "bytes": nbytes})

    def tfl(name, flop, fn):
        ms = do_bench(fn, warmup=3, rep=10)
        v = flop / (ms * 1e-3) / 1e12
        res.append({"workload": name, "value": round(v, 2), "unit": "TFLOP/s", "ms": round(ms, 5),
                    "frac_mfma": round(v / PEAK_TFLOPS, 4), "flop": flop})

    try:
        x = seeded(1_000_000, 0)
        y = seeded(1_000_000, 1)
        o = torch.empty_like(x)
        gbs("vector add fp32 n=1e6", 12_000_000, lambda: W.add(x, y, o))
        x = seeded(1 << 26, 0)
        y = seeded(1 << 26, 1)
        o = torch.empty_like(x)
        gbs("vector add fp32 n=2^26 (extra, large)", 3 * 4 << 26, lambda: W.add(x, y, o, BLOCK=4096))
        del x, y, o
        for C in (1000, 4096, 8192):
            x = seeded((4096, C), 0, scale=4.0)
            o = torch.empty_like(x)
            gbs(f"softmax fp32 4096x{C}", 2 * 4 * 4096 * C, lambda: W.softmax(x, o))
        x = seeded((4096, 8192), 0, dtype=torch.float16)
        w = seeded(8192, 2, scale=0.1, mean=1.0, dtype=torch.float16)
        bb = seeded(8192, 3, scale=0.1, dtype=torch.float16)
        o = torch.empty_like(x)
        gbs("layernorm fp16 4096x8192 (+mean/rstd)", 134_283_264,
            lambda: W.layernorm(x, w, bb, 1e-5, o))
        S = 4096
        a = seeded((S, S), 4, scale=S ** -0.5, dtype=torch.bfloat16)
        b = seeded((S, S), 5, scale=S ** -0.5, dtype=torch.bfloat16)
        c = torch.empty(S, S, device="cuda", dtype=torch.bfloat16)
        W.matmul(a, b, c)
        cfg = W.matmul_tuned.best_config
        tfl("matmul bf16 4096^3", 2.0 * S ** 3, lambda: W.matmul(a, b, c, config=cfg))
        q, k, v = (seeded((4, 32, 4096, 128), s, dtype=torch.bfloat16) for s in (6, 7, 8))
        o = torch.empty_like(q)
        tfl("attention bf16 [4,32,4096,128] non-causal", 4 * 4 * 32 * 4096 ** 2 * 128,
            lambda: W.attention(q, k, v, False, out=o))
        tfl("attention bf16 [4,32,4096,128] causal", 4 * 4 * 32 * 128 * 4096 * 4097 // 2,
            lambda: W.attention(q, k, v, True, out=o))
    except Exception as e:  # report what was measured, and why the rest was not
        res.append({"error": f"{type(e).__name__}: {str(e)[:300]}"})
    return res


if __name__ == "__main__":
    main()
