"""Parity of the five hot-path kernels on the GPU against the CPU oracle.

Each test runs the newt kernel through the HIP backend (hipRTC code object
launched through libnewt_hip.so) on seeded inputs and compares with
oracle/newt_oracle.py at the tolerance north_star states:
  vector add (elementwise): bit-exact
  softmax fp32: rtol 1e-5 on every element (relative; no absolute floor
    beyond 1e-30, so small probabilities are held as tightly as large ones)
  layernorm: fp16 output within one fp16 ulp of the exact result rounded to
    fp16 (2^-24 slack for subnormals); fp32 output rtol 1e-5 of the terms'
    magnitude; mean rtol 1e-5 with a floor of one fp32 unit of mean(|x|)
    for rows whose sum cancels; rstd rtol 1e-5 (oracle.layernorm_violations)
  matmul, attention (fp16/bf16): relative Frobenius error <= 1e-2
"""

import math
import numpy as np
import pytest
import torch

from oracle import newt_oracle as orc

pytestmark = pytest.mark.gpu


def seeded(shape, seed, scale=1.0, mean=0.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale + mean).to(dtype).to("cuda")


def npf(t):
    return t.detach().float().cpu().numpy()


@pytest.fixture(scope="module")
def W():
    from newt_amd import workloads
    return workloads


@pytest.mark.parametrize("n", [1024, 1 << 20, 12345, 1_000_000, 1])
def test_vector_add_bit_exact(W, n):
    x, y = seeded(n, 0), seeded(n, 1)
    out = W.add(x, y)
    torch.cuda.synchronize()
    ref = orc.vector_add(npf(x), npf(y))
    assert np.array_equal(npf(out), ref), f"n={n}"


def test_vector_add_golden(W):
    g = np.load("tests/golden/vector_add_12345.npz")
    x = torch.from_numpy(g["x"]).cuda()
    y = torch.from_numpy(g["y"]).cuda()
    out = W.add(x, y)
    assert np.array_equal(npf(out), g["out"])


def assert_softmax_close(got, ref, what=""):
    """rtol 1e-5 on every element, relative (oracle.rel_violations)."""
    bad = orc.rel_violations(got, ref, 1e-5)
    rel = float(np.max(np.abs(got.astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-30)))
    print(f"  softmax{what}: max relative error {rel:.3e}", flush=True)
    assert bad == 0, f"softmax{what}: {bad} of {got.size} elements beyond rtol 1e-5 (max {rel:.3e})"


def assert_layernorm_close(y, mean, rstd, x, w, b, dtype, what=""):
    bad = orc.layernorm_violations(npf(y), npf(mean), npf(rstd), npf(x), npf(w), npf(b), 1e-5,
                                   dtype)
    print(f"  layernorm{what}: violations {bad}", flush=True)
    assert bad == {"y": 0, "mean": 0, "rstd": 0}, f"layernorm{what}: {bad}"


@pytest.mark.parametrize("M,N", [(8, 128), (128, 1024), (32, 781), (64, 1000), (16, 4096),
                                 (4, 8192), (3, 5)])
def test_softmax(W, M, N):
    x = seeded((M, N), 0, scale=4.0)
    out = W.softmax(x)
    assert_softmax_close(npf(out), orc.softmax_rows(npf(x)), f" [{M}, {N}]")


def test_softmax_golden(W):
    for name in ("softmax_8x128", "softmax_32x781"):
        g = np.load(f"tests/golden/{name}.npz")
        out = W.softmax(torch.from_numpy(g["x"]).cuda())
        assert_softmax_close(npf(out), g["out"], f" {name}")


@pytest.mark.parametrize("M,N", [(8, 128), (16, 300), (64, 2048), (4, 8192), (2, 1000)])
def test_layernorm_fp16(W, M, N):
    x = seeded((M, N), 0, dtype=torch.float16)
    w = seeded(N, 2, scale=0.1, mean=1.0, dtype=torch.float16)
    b = seeded(N, 3, scale=0.1, dtype=torch.float16)
    y, mean, rstd = W.layernorm(x, w, b, 1e-5)
    assert_layernorm_close(y, mean, rstd, x, w, b, "float16", f" [{M}, {N}]")


def test_layernorm_fp32(W):
    M, N = 16, 3000
    x = seeded((M, N), 0)
    w = seeded(N, 2)
    b = seeded(N, 3)
    y, mean, rstd = W.layernorm(x, w, b, 1e-5)
    assert_layernorm_close(y, mean, rstd, x, w, b, "float32", f" fp32 [{M}, {N}]")


def test_layernorm_golden(W):
    for name in ("layernorm_16x300", "layernorm_8x128"):
        g = np.load(f"tests/golden/{name}.npz")
        t = lambda k: torch.from_numpy(g[k]).half().cuda()
        y, mean, rstd = W.layernorm(t("x"), t("w"), t("b"), 1e-5)
        # the golden y is torch's float64 result: one fp16 ulp of it rounded
        want = orc.round_to(g["out"], "float16")
        assert orc.ulp_violations(npf(y), want, "float16", atol=orc.U_FP16_SUB) == 0, name
        assert orc.mean_violations(npf(mean), g["mean"], g["x"]) == 0, name
        assert orc.rel_violations(npf(rstd), g["rstd"], 1e-5) == 0, name


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,N,K,cfg", [
    (64, 64, 32, (64, 64, 32, 4, 2)),
    (256, 256, 128, (64, 64, 32, 4, 2)),
    (300, 200, 100, (64, 64, 32, 4, 2)),
    (512, 512, 256, (128, 128, 64, 4, 2)),
    (512, 384, 512, (256, 128, 64, 8, 2)),
])
def test_matmul(W, dtype, M, N, K, cfg):
    import newt_amd as newt
    a = seeded((M, K), 4, scale=K ** -0.5, dtype=dtype)
    b = seeded((K, N), 5, scale=K ** -0.5, dtype=dtype)
    BM, BN, BK, nw, ns = cfg
    c = W.matmul(a, b, config=newt.Config({"BLOCK_M": BM, "BLOCK_N": BN, "BLOCK_K": BK},
                                         num_warps=nw, num_stages=ns))
    ref = orc.matmul(npf(a), npf(b), "float16" if dtype == torch.float16 else "bfloat16")
    assert orc.rel_frobenius(npf(c), ref) <= 1e-2


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", [(512, 512, 512), (300, 200, 100), (256, 256, 64),
                                   (1024, 768, 1056), (64, 96, 32), (520, 264, 136)])
@pytest.mark.parametrize("cfg", [(256, 256, 32, 8, 4), (256, 256, 32, 4, 4), (128, 128, 32, 4, 3), (64, 64, 32, 4, 4),
                                 (128, 256, 64, 8, 2)])
def test_matmul_pipelined(W, dtype, M, N, K, cfg):
    """The software-pipelined k-loop (direct-to-LDS stages, ragged fallbacks,
    trip counts shorter than the pipeline) against the oracle."""
    import newt_amd as newt
    a = seeded((M, K), 4, scale=K ** -0.5, dtype=dtype)
    b = seeded((K, N), 5, scale=K ** -0.5, dtype=dtype)
    BM, BN, BK, nw, ns = cfg
    print(f"matmul_pipelined M={M} N={N} K={K} cfg={cfg} {dtype}", flush=True)
    c = W.matmul(a, b, config=newt.Config({"BLOCK_M": BM, "BLOCK_N": BN, "BLOCK_K": BK},
                                         num_warps=nw, num_stages=ns))
    ref = orc.matmul(npf(a), npf(b), "float16" if dtype == torch.float16 else "bfloat16")
    assert orc.rel_frobenius(npf(c), ref) <= 1e-2


@pytest.mark.parametrize("ta,tb", [(False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K", [(512, 384, 256), (300, 200, 136), (1024, 1024, 512)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_matmul_transposed_operands(W, dtype, M, N, K, ta, tb):
    """Column-major A and/or B (transposed views: unit stride along the other
    dim) take other LDS tile formats and copy paths than row-major inputs."""
    a = seeded((K, M) if ta else (M, K), 30, scale=K ** -0.5, dtype=dtype)
    b = seeded((N, K) if tb else (K, N), 31, scale=K ** -0.5, dtype=dtype)
    a = a.t() if ta else a
    b = b.t() if tb else b
    c = W.matmul(a, b)
    ref = orc.matmul(npf(a), npf(b), "float16" if dtype == torch.float16 else "bfloat16")
    assert orc.rel_frobenius(npf(c), ref) <= 1e-2


@pytest.mark.parametrize("cfg", [(256, 256, 16, 8, 3), (256, 128, 16, 8, 4), (128, 128, 32, 4, 3),
                                 (128, 128, 16, 4, 4)])
@pytest.mark.parametrize("M,N,K", [(512, 384, 256), (300, 200, 136), (1024, 1024, 512)])
def test_matmul_fp32_pipelined(W, M, N, K, cfg):
    """fp32 operands through the pipelined k-loop (direct-to-LDS stages, four
    k per fragment read in the permuted order, ragged tails): full precision,
    relative Frobenius error <= 1e-5 against the float64 oracle."""
    import newt_amd as newt
    a = seeded((M, K), 34, scale=K ** -0.5)
    b = seeded((K, N), 35, scale=K ** -0.5)
    BM, BN, BK, nw, ns = cfg
    print(f"matmul_fp32_pipelined M={M} N={N} K={K} cfg={cfg}", flush=True)
    c = W.matmul(a, b, config=newt.Config({"BLOCK_M": BM, "BLOCK_N": BN, "BLOCK_K": BK},
                                         num_warps=nw, num_stages=ns))
    ref = orc.matmul(npf(a), npf(b), "float32")
    assert orc.rel_frobenius(npf(c), ref) <= 1e-5


@pytest.mark.parametrize("ta,tb", [(False, True), (True, False), (True, True)])
def test_matmul_fp32_transposed_operands(W, ta, tb):
    """Column-major fp32 A (an R-major tile read four floats at a time) and
    K-contiguous B (a K-major tile read with 16-byte loads)."""
    import newt_amd as newt
    M, N, K = 384, 256, 200
    a = seeded((K, M) if ta else (M, K), 36, scale=K ** -0.5)
    b = seeded((N, K) if tb else (K, N), 37, scale=K ** -0.5)
    a = a.t() if ta else a
    b = b.t() if tb else b
    c = W.matmul(a, b, config=newt.Config({"BLOCK_M": 128, "BLOCK_N": 128, "BLOCK_K": 16},
                                         num_warps=4, num_stages=3))
    ref = orc.matmul(npf(a), npf(b), "float32")
    assert orc.rel_frobenius(npf(c), ref) <= 1e-5


@pytest.mark.parametrize("cfg", [(256, 256, 32, 4, 4), (256, 256, 32, 8, 4), (128, 128, 64, 4, 3)])
def test_matmul_strided_rows(W, cfg):
    """Row strides larger than the row (views into a wider buffer) and an
    output written into a strided view."""
    import newt_amd as newt
    BM, BN, BK, nw, ns = cfg
    big_a = seeded((512, 768), 32, scale=0.05, dtype=torch.float16)
    big_b = seeded((512, 640), 33, scale=0.05, dtype=torch.float16)
    a, b = big_a[:, 64:576], big_b[:, 32:544]        # [512, 512] each, strides 768 / 640
    out = torch.zeros(512, 1024, device="cuda", dtype=torch.float16)
    c = out[:, 256:768]
    W.matmul(a, b, c, config=newt.Config({"BLOCK_M": BM, "BLOCK_N": BN, "BLOCK_K": BK},
                                         num_warps=nw, num_stages=ns))
    ref = orc.matmul(npf(a), npf(b), "float16")
    assert orc.rel_frobenius(npf(c), ref) <= 1e-2
    assert not out[:, :256].any() and not out[:, 768:].any()


def test_matmul_golden(W):
    import newt_amd as newt
    cfg = newt.Config({"BLOCK_M": 64, "BLOCK_N": 64, "BLOCK_K": 32}, num_warps=4, num_stages=2)
    for name in ("matmul_64x64x32", "matmul_300x200x100"):
        g = np.load(f"tests/golden/{name}.npz")
        a = torch.from_numpy(g["a"]).half().cuda()
        b = torch.from_numpy(g["b"]).half().cuda()
        c = W.matmul(a, b, config=cfg)
        assert orc.rel_frobenius(npf(c), g["out"]) <= 1e-2


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,H,S,D", [(1, 2, 64, 32), (1, 2, 256, 64), (2, 2, 200, 128)])
def test_attention(W, causal, B, H, S, D):
    q, k, v = (seeded((B, H, S, D), s, dtype=torch.bfloat16) for s in (6, 7, 8))
    o = W.attention(q, k, v, causal=causal, BLOCK_M=64, BLOCK_N=64, num_warps=4)
    ref = orc.attention(npf(q), npf(k), npf(v), D ** -0.5, causal, p_dtype="bfloat16",
                        out_dtype="bfloat16")
    assert orc.rel_frobenius(npf(o), ref) <= 1e-2


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,H,S,D", [(1, 2, 256, 128), (2, 2, 300, 128), (1, 1, 1000, 128),
                                     (1, 2, 64, 128)])
def test_attention_default_config(W, causal, B, H, S, D):
    """The configuration bench.py and users get (BLOCK_M=256, BLOCK_N=64, 8
    waves, 2 stages, waves_per_eu=2), including ragged sequence lengths."""
    q, k, v = (seeded((B, H, S, D), s, dtype=torch.bfloat16) for s in (16, 17, 18))
    o = W.attention(q, k, v, causal=causal)
    ref = orc.attention(npf(q), npf(k), npf(v), D ** -0.5, causal, p_dtype="bfloat16",
                        out_dtype="bfloat16")
    assert orc.rel_frobenius(npf(o), ref) <= 1e-2


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("BM,BN,warps", [(256, 32, 8), (128, 32, 4), (128, 128, 4), (64, 32, 2),
                                         (128, 16, 4)])
def test_attention_key_block_sizes(W, causal, D, BM, BN, warps):
    """Key blocks of 32 and 128 (one and four 16x16x32 P @ V steps per block,
    the score accumulator fed in place) and 16 to 32 query rows per wave, on a
    ragged sequence, both kernels. 16-key blocks fit no 16x16x32 step: P @ V
    runs on 32x32x16 with P converted through LDS (this configuration failed
    to compile while the in-place check built a 32-wide accumulator layout
    for the 16-wide P)."""
    q, k, v = (seeded((1, 2, 333, D), s, dtype=torch.bfloat16) for s in (36, 37, 38))
    ref = orc.attention(npf(q), npf(k), npf(v), D ** -0.5, causal, p_dtype="bfloat16",
                        out_dtype="bfloat16")
    for plain in (False, True):
        print(f"attention D={D} BM={BM} BN={BN} warps={warps} causal={causal} plain={plain}",
              flush=True)
        o = W.attention(q, k, v, causal=causal, plain=plain, BLOCK_M=BM, BLOCK_N=BN,
                        num_warps=warps)
        assert orc.rel_frobenius(npf(o), ref) <= 1e-2, plain


@pytest.mark.parametrize("B,H,S", [(1, 8, 1000), (2, 8, 300), (3, 8, 777), (1, 24, 513),
                                   (1, 32, 300), (2, 32, 300), (1, 96, 200)])
def test_attention_causal_heads_split_over_xcds(W, B, H, S):
    """Causal launches whose B*H heads split evenly over the 8 XCDs take the
    heaviest-first renumbering of programs (every head's last query block
    first, over groups of 4 of an XCD's heads when 4 divides their count: one,
    two and three groups in the last three cases); each (batch, head, query
    block) must still be computed exactly once: the output starts as NaN and
    every row is held to the oracle."""
    D = 128
    q, k, v = (seeded((B, H, S, D), s, dtype=torch.bfloat16) for s in (40, 41, 42))
    o = torch.full_like(q, float("nan"))
    W.attention(q, k, v, causal=True, out=o)
    got = npf(o)
    assert np.isfinite(got).all()
    ref = orc.attention(npf(q), npf(k), npf(v), D ** -0.5, True, p_dtype="bfloat16",
                        out_dtype="bfloat16")
    worst = max(orc.rel_frobenius(got[b, h, r], ref[b, h, r])
                for b in range(B) for h in range(H) for r in range(S))
    assert worst <= 1e-2, worst


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("growth,S", [(20.0, 1000), (4.0, 777), (200.0, 513)])
def test_attention_scores_outgrowing_the_first_block(W, causal, growth, S):
    """The default kernel refers every exponent to a row's first-block
    maximum; keys whose norms grow along the sequence (by 1 + j / growth)
    push later scores far past it, so rows' sums pass 2^80 and the programs
    take the online-softmax pass (a growth of 200 stays below it: both
    paths are checked). Every row matches the oracle."""
    B, H, D = 1, 2, 128
    g = torch.Generator().manual_seed(9)
    q = torch.randn(B, H, S, D, generator=g)
    k = torch.randn(B, H, S, D, generator=g) * (1 + torch.arange(S) / growth)[None, None, :, None]
    v = torch.randn(B, H, S, D, generator=g)
    q, k, v = (t.bfloat16().cuda() for t in (q, k, v))
    o = W.attention(q, k, v, causal=causal)
    assert torch.isfinite(o).all()
    ref = orc.attention(npf(q), npf(k), npf(v), D ** -0.5, causal, p_dtype="bfloat16",
                        out_dtype="bfloat16")
    got = npf(o)
    worst = max(orc.rel_frobenius(got[0, h, r], ref[0, h, r]) for h in range(H) for r in range(S))
    assert worst <= 1e-2, worst


@pytest.mark.parametrize("causal", [False, True])
def test_attention_large_values_with_rising_scores(W, causal):
    """Scores that rise linearly along the keys, to 2^40 (head 0) and 2^70
    (head 1) above the first key block's maximum in log2 units, over values
    in [2^110, 2^111): every row's sum l stays below 2^80, but with the
    exponents referred to the first block's maximum p * v passes fp32's
    range, where a per-block rescale keeps p <= 1 and the sums finite (at
    most S * 2^111). The kernel finds the overflow in its accumulator and
    takes the online-softmax pass; every row matches the oracle."""
    B, H, S, D = 1, 2, 1000, 128
    rise = torch.tensor([40.0, 70.0], dtype=torch.float64)       # log2 units over the keys
    slope = rise * math.log(2.0) / S                              # natural-log units per key
    score = slope[:, None] * torch.arange(S, dtype=torch.float64)[None, :]   # [H, S]
    # q = 1 everywhere; k_j = (score_j / sqrt(D)) everywhere gives q.k * D^-0.5 = score_j
    q = torch.ones(B, H, S, D)
    k = (score / math.sqrt(D))[None, :, :, None].expand(B, H, S, D).float()
    g = torch.Generator().manual_seed(12)
    v = (1.0 + torch.rand(B, H, S, D, generator=g)) * 2.0 ** 110
    q, k, v = (t.bfloat16().cuda() for t in (q, k, v))
    o = W.attention(q, k, v, causal=causal)
    assert torch.isfinite(o).all()
    ref = orc.attention(npf(q), npf(k), npf(v), D ** -0.5, causal, p_dtype="bfloat16",
                        out_dtype="bfloat16")
    got = npf(o)
    worst = max(orc.rel_frobenius(got[0, h, r], ref[0, h, r]) for h in range(H) for r in range(S))
    assert worst <= 1e-2, worst


def test_attention_golden(W):
    for causal in (False, True):
        g = np.load(f"tests/golden/attention_1x2x64x32_{'causal' if causal else 'full'}.npz")
        t = lambda k: torch.from_numpy(g[k]).bfloat16().cuda()
        o = W.attention(t("q"), t("k"), t("v"), causal=causal, BLOCK_M=64, BLOCK_N=64)
        assert orc.rel_frobenius(npf(o), g["out"]) <= 1e-2


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,H,S,D,BM,BN", [(1, 2, 256, 128, 128, 64), (2, 2, 300, 128, 128, 64),
                                           (1, 2, 200, 64, 64, 64), (1, 1, 1000, 128, 128, 64)])
def test_attention_plain_form(W, causal, B, H, S, D, BM, BN):
    """The examples/05 form (nl.exp, qk * scale, a where mask in one loop)
    compiled as written, ragged sequence lengths included."""
    q, k, v = (seeded((B, H, S, D), s, dtype=torch.bfloat16) for s in (26, 27, 28))
    o = W.attention(q, k, v, causal=causal, plain=True, BLOCK_M=BM, BLOCK_N=BN)
    ref = orc.attention(npf(q), npf(k), npf(v), D ** -0.5, causal, p_dtype="bfloat16",
                        out_dtype="bfloat16")
    assert orc.rel_frobenius(npf(o), ref) <= 1e-2


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("scale", [-0.1, 0.0, -1.0])
def test_attention_non_positive_scale(W, causal, scale):
    """Any softmax scale is valid, as in the reference (qk * scale, then the
    -inf mask): a scale <= 0 must not turn masked scores into +inf or NaN."""
    B, H, S, D = 1, 2, 300, 128
    q, k, v = (seeded((B, H, S, D), s, dtype=torch.bfloat16) for s in (36, 37, 38))
    o = W.attention(q, k, v, causal=causal, scale=scale)
    assert torch.isfinite(o).all()
    ref = orc.attention(npf(q), npf(k), npf(v), scale, causal, p_dtype="bfloat16",
                        out_dtype="bfloat16")
    assert orc.rel_frobenius(npf(o), ref) <= 1e-2


@pytest.mark.parametrize("n", [1, 4095, 4096 * 3 + 17, 1 << 22])
def test_copy_exact(W, n):
    """The streaming copy bench.py times as the HBM ceiling moves every bit."""
    src = seeded(n, 40)
    dst = torch.full_like(src, float("nan"))
    W.copy(src, dst)
    assert torch.equal(dst, src)
