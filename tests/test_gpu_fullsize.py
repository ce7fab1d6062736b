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
             oracle, at the tolerances of the small-shape tests.
  attention  (the default kernel and the examples/05 plain form)
             eight (batch, head) pairs spread over all 128, with the query
             rows of the first, a middle and the last 128-row query block:
             relative Frobenius error <= 1e-2 per (batch, head) and per row.
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


QUERY_BLOCK = 128


@pytest.mark.parametrize("plain", [False, True], ids=["default", "plain_form"])
@pytest.mark.parametrize("causal", [False, True], ids=["full", "causal"])
def test_attention_benchmark_shape(W, causal, plain):
    B, H, S, D = 4, 32, 4096, 128
    print(f"attention bf16 [{B},{H},{S},{D}] causal={causal} plain={plain}", flush=True)
    q, k, v = (seeded((B, H, S, D), s, dtype=torch.bfloat16) for s in (6, 7, 8))
    o = W.attention(q, k, v, causal=causal, plain=plain)
    torch.cuda.synchronize()
    blocks = S // QUERY_BLOCK
    rows = np.concatenate([np.arange(i * QUERY_BLOCK, (i + 1) * QUERY_BLOCK)
                           for i in (0, blocks // 2, blocks - 1)])
    rows_t = torch.from_numpy(rows).cuda()
    worst = 0.0
    for bh in orc.spread(B * H, 8):
        bi, hi = divmod(int(bh), H)
        ref = orc.attention(npf(q[bi, hi, rows_t]), npf(k[bi, hi]), npf(v[bi, hi]), D ** -0.5,
                            causal, p_dtype="bfloat16", out_dtype="bfloat16", q_pos=rows)
        got = npf(o[bi, hi, rows_t])
        err = orc.rel_frobenius(got, ref)
        row_err = max(orc.rel_frobenius(got[r], ref[r]) for r in range(len(rows)))
        worst = max(worst, row_err)
        assert err <= 1e-2, f"(b={bi}, h={hi}) rel_frobenius {err}"
        assert row_err <= 1e-2, f"(b={bi}, h={hi}) worst row rel_frobenius {row_err}"
    print(f"  worst per-row rel_frobenius {worst:.3e}", flush=True)


@pytest.mark.parametrize("C", [1000, 4096, 8192])
def test_softmax_benchmark_shapes(W, C):
    print(f"softmax fp32 [4096, {C}]", flush=True)
    x = seeded((4096, C), 0, scale=4.0)
    out = W.softmax(x)
    np.testing.assert_allclose(npf(out), orc.softmax_rows(npf(x)), rtol=1e-5, atol=1e-6)


def test_layernorm_benchmark_shape(W):
    print("layernorm fp16 [4096, 8192]", flush=True)
    M, N = 4096, 8192
    x = seeded((M, N), 0, dtype=torch.float16)
    w = (seeded((N,), 2, scale=0.1) + 1.0).half()
    b = seeded((N,), 3, scale=0.1, dtype=torch.float16)
    y, mean, rstd = W.layernorm(x, w, b, 1e-5)
    ry, rmean, rrstd = orc.layernorm_rows(npf(x), npf(w), npf(b), 1e-5, "float16")
    np.testing.assert_allclose(npf(y), ry, rtol=2e-3, atol=2e-3)
    np.testing.assert_allclose(npf(mean), rmean, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(npf(rstd), rrstd, rtol=1e-5, atol=1e-6)
