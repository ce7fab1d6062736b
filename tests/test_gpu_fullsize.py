"""Parity at the benchmark configurations' full sizes.

The matmul configuration is fp16 and bf16 A[S,S] @ B[S,S] for S in
{1024, 2048, 4096, 8192}, autotuned (reference: tests/test_matmul.py:52-71,
benchmarks/bench.py:258-290); the attention configuration is bf16 Q, K, V
[4, 32, 4096, 128], causal and not (examples/05_fused_attention.py:14-48
generalised to batch and heads). Both run here exactly as bench.py launches
them. The oracle cannot afford the whole output at these sizes, so each check
samples it so that every program of the launch is touched:

  matmul     one row from every 64-row panel (the smallest BLOCK_M in the
             autotune space) at an offset that cycles through the panel, plus
             the last row, against all N columns: relative Frobenius error
             <= 1e-2 (north_star) and every sampled element within one ulp of
             the fp64 product rounded to the output dtype.
  softmax    fp32 [4096, C] for C in {1000, 4096, 8192} and layernorm fp16
             [4096, 8192] (examples/02 and 03 at the benchmark shapes, both
             paths of their in-bounds test: 1000 < BLOCK_N takes the masked
             body, 4096 and 8192 the straight-line one): every row against the
             oracle, at the tolerances of the small-shape tests: softmax
             rtol 1e-5 on every element (relative, no absolute floor
             beyond 1e-30); layernorm y within one fp16 ulp of the exact
             result rounded to fp16, mean rtol 1e-5 with a floor of one
             fp32 unit of mean(|x|) for rows whose sum cancels, rstd rtol
             1e-5 (oracle.layernorm_violations).
  attention  (the default kernel and the examples/05 plain form) every
             (batch, head) pair, one query row of every 128-row block (each
             256-row program of the default launch owns two such blocks, a
             128-row one exactly one) at an offset that cycles through the block and moves
             with the pair, plus every row of the first, a middle and the
             last block of eight pairs spread over all 128: relative
             Frobenius error <= 1e-2 per row and per pair
             (oracle.attention_sampled_errors).
"""

import numpy as np
import pytest
import torch

from oracle import newt_oracle as orc

pytestmark = pytest.mark.gpu


def seeded(shape, seed, scale=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype).to("cuda")


def npf(t):
    return t.detach().float().cpu().numpy()


@pytest.fixture(scope="module")
def W():
    from newt_amd import workloads
    return workloads


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["fp16", "bf16"])
@pytest.mark.parametrize("S", [1024, 2048, 4096, 8192])
def test_matmul_square_autotuned(W, S, dtype):
    name = "float16" if dtype == torch.float16 else "bfloat16"
    print(f"matmul {name} {S}^3 autotuned", flush=True)
    a = seeded((S, S), 4, scale=S ** -0.5, dtype=dtype)
    b = seeded((S, S), 5, scale=S ** -0.5, dtype=dtype)
    c = W.matmul(a, b)                       # autotune, then the chosen config's launch
    c = W.matmul(a, b, c)                    # a second launch of the cached choice
    torch.cuda.synchronize()
    rows = orc.panel_rows(S, 64)
    got = npf(c[torch.from_numpy(rows).cuda()])
    ref = orc.matmul(npf(a)[rows], npf(b), name)
    err = orc.rel_frobenius(got, ref)
    bad = orc.ulp_violations(got, ref, name)
    cfg = W.matmul_tuned.best_config
    print(f"  config {cfg} rows {len(rows)} rel_frobenius {err:.3e} ulp_violations {bad}",
          flush=True)
    assert err <= 1e-2
    assert bad == 0, f"{bad} of {got.size} sampled elements beyond one ulp"


QUERY_BLOCK = 128   # at most the query rows of one program (the default launches 256)


@pytest.mark.parametrize("plain", [False, True], ids=["default", "plain_form"])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_attention_benchmark_shape(W, causal, plain):
    B, H, S, D = 4, 32, 4096, 128
    print(f"attention bf16 [{B},{H},{S},{D}] causal={causal} plain={plain}", flush=True)
    q, k, v = (seeded((B, H, S, D), s, dtype=torch.bfloat16) for s in (6, 7, 8))
    o = W.attention(q, k, v, causal=causal, plain=plain)
    torch.cuda.synchronize()
    # every program: one row of every 128-row query block of every (batch,
    # head) pair, plus every row of three blocks of eight pairs
    res = orc.attention_sampled_errors(npf(q), npf(k), npf(v), npf(o), D ** -0.5, causal,
                                       block=QUERY_BLOCK)
    print(f"  {res}", flush=True)
    assert res["rows"] >= B * H * (S // QUERY_BLOCK)
    assert res["worst_row"] <= 1e-2, res
    assert res["worst_pair"] <= 1e-2, res


@pytest.mark.parametrize("C", [1000, 4096, 8192])
def test_softmax_benchmark_shapes(W, C):
    print(f"softmax fp32 [4096, {C}]", flush=True)
    x = seeded((4096, C), 0, scale=4.0)
    out = W.softmax(x)
    got, ref = npf(out), orc.softmax_rows(npf(x))
    bad = orc.rel_violations(got, ref, 1e-5)
    rel = float(np.max(np.abs(got.astype(np.float64) - ref) / np.maximum(ref, 1e-30)))
    print(f"  max relative error {rel:.3e}, smallest probability {ref.min():.3e}", flush=True)
    assert bad == 0, f"{bad} of {got.size} elements beyond rtol 1e-5 (max {rel:.3e})"


def test_layernorm_benchmark_shape(W):
    print("layernorm fp16 [4096, 8192]", flush=True)
    M, N = 4096, 8192
    x = seeded((M, N), 0, dtype=torch.float16)
    w = (seeded((N,), 2, scale=0.1) + 1.0).half()
    b = seeded((N,), 3, scale=0.1, dtype=torch.float16)
    y, mean, rstd = W.layernorm(x, w, b, 1e-5)
    bad = orc.layernorm_violations(npf(y), npf(mean), npf(rstd), npf(x), npf(w), npf(b), 1e-5,
                                   "float16")
    print(f"  violations {bad}", flush=True)
    assert bad == {"y": 0, "mean": 0, "rstd": 0}
