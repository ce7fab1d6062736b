"""deuteron on the HIP backend: the reference's deuteron tests
(tests/test_deuteron.py) and example kernels (examples/deuteron/01-04), each
checked against torch on the GPU; autotuned kernels also against deuteron's own
eager oracle."""

import os
import tempfile

import pytest
import torch

import deuteron as dt

pytestmark = pytest.mark.gpu

os.environ.setdefault("DEUTERON_CACHE_DIR", tempfile.mkdtemp(prefix="deuteron-test-"))


@dt.kernel(config={"BLOCK_TILE_M": 64, "BLOCK_TILE_N": 64, "BLOCK_TILE_K": 32, "num_warps": 4})
def matmul_fixed(x, y, out):
    for tile_m, tile_n in dt.tile([x.shape[0], y.shape[1]]):
        acc = dt.zeros([tile_m, tile_n], dtype=dt.float32)
        for tile_k in dt.tile(x.shape[1]):
            acc += x[tile_m, tile_k] @ y[tile_k, tile_n]
        out[tile_m, tile_n] = acc


@dt.kernel(samples=6)
def matmul(x, y, out):
    for tile_m, tile_n in dt.tile([x.shape[0], y.shape[1]]):
        acc = dt.zeros([tile_m, tile_n], dtype=dt.float32)
        for tile_k in dt.tile(x.shape[1]):
            acc += x[tile_m, tile_k] @ y[tile_k, tile_n]
        out[tile_m, tile_n] = acc


@dt.kernel(samples=6)
def softmax(x, out):
    for tile_m in dt.tile(x.shape[0]):
        row = x[tile_m, :]
        m = row.amax(1)
        e = dt.exp(row - m[:, None])
        s = e.sum(1)
        out[tile_m, :] = e / s[:, None]


@dt.kernel(samples=6)
def add_relu(x, y, out):
    for tile_n in dt.tile(x.shape[0]):
        out[tile_n] = dt.relu(x[tile_n] + y[tile_n])


@dt.kernel(samples=6)
def layernorm(x, w, b, out, eps):
    for tile_m in dt.tile(x.shape[0]):
        row = x[tile_m, :]
        mean = row.sum(1) / x.shape[1]
        diff = row - mean[:, None]
        var = (diff * diff).sum(1) / x.shape[1]
        rstd = dt.rsqrt(var + eps)
        out[tile_m, :] = diff * rstd[:, None] * w[:] + b[:]


@dt.kernel(samples=6)
def fused_gelu_residual(x, y, out):
    for t in dt.tile(x.shape[0]):
        v = x[t]
        inner = 0.7978845608028654 * (v + 0.044715 * v * v * v)
        g = 0.5 * v * (1.0 + dt.tanh(inner))
        out[t] = g + y[t]


def _g(seed):
    return torch.Generator(device="cuda").manual_seed(seed)


def test_matmul_fixed_config():
    x = torch.randn(512, 256, device="cuda", dtype=torch.float16, generator=_g(0))
    y = torch.randn(256, 384, device="cuda", dtype=torch.float16, generator=_g(1))
    out = torch.empty(512, 384, device="cuda", dtype=torch.float16)
    matmul_fixed(x, y, out)
    torch.cuda.synchronize()
    ref = (x.float() @ y.float()).half()
    assert torch.allclose(out.float(), ref.float(), rtol=2e-2, atol=2e-2)


def test_matmul_autotuned():
    x = torch.randn(1024, 512, device="cuda", dtype=torch.float16, generator=_g(2))
    y = torch.randn(512, 768, device="cuda", dtype=torch.float16, generator=_g(3))
    out = torch.empty(1024, 768, device="cuda", dtype=torch.float16)
    matmul(x, y, out)
    torch.cuda.synchronize()
    ref = (x.float() @ y.float()).half()
    assert torch.allclose(out.float(), ref.float(), rtol=2e-2, atol=2e-2)
    cfg = matmul.best_config
    assert set(cfg) >= {"BLOCK_TILE_M", "BLOCK_TILE_N", "BLOCK_TILE_K", "num_warps", "num_stages"}


def test_matmul_ragged_bf16():
    x = torch.randn(300, 200, device="cuda", dtype=torch.bfloat16, generator=_g(4))
    y = torch.randn(200, 100, device="cuda", dtype=torch.bfloat16, generator=_g(5))
    out = torch.empty(300, 100, device="cuda", dtype=torch.bfloat16)
    matmul_fixed(x, y, out)
    ref = (x.float() @ y.float())
    rel = ((out.float() - ref).norm() / ref.norm()).item()
    assert rel <= 1e-2


def test_softmax():
    x = torch.randn(1000, 777, device="cuda", generator=_g(6))
    out = torch.empty_like(x)
    softmax(x, out)
    torch.cuda.synchronize()
    assert torch.allclose(out, torch.softmax(x, -1), rtol=1e-3, atol=1e-4)


def test_add_relu_exact():
    x = torch.randn(1 << 20, device="cuda", generator=_g(7))
    y = torch.randn(1 << 20, device="cuda", generator=_g(8))
    out = torch.empty_like(x)
    add_relu(x, y, out)
    torch.cuda.synchronize()
    assert torch.equal(out, torch.relu(x + y))


def test_layernorm_ragged():
    M, N = 512, 1500
    x = torch.randn(M, N, device="cuda", generator=_g(9))
    w = torch.randn(N, device="cuda", generator=_g(10))
    b = torch.randn(N, device="cuda", generator=_g(11))
    out = torch.empty_like(x)
    layernorm(x, w, b, out, 1e-5)
    ref = torch.nn.functional.layer_norm(x, (N,), w, b, 1e-5)
    assert (out - ref).abs().max().item() < 1e-3


def test_fused_gelu_residual():
    n = 1 << 20
    x = torch.randn(n, device="cuda", generator=_g(12))
    y = torch.randn(n, device="cuda", generator=_g(13))
    out = torch.empty_like(x)
    fused_gelu_residual(x, y, out)
    ref = torch.nn.functional.gelu(x, approximate="tanh") + y
    assert (out - ref).abs().max().item() < 1e-5


def test_eager_reference():
    x = torch.randn(128, 64, device="cuda", dtype=torch.float16, generator=_g(14))
    y = torch.randn(64, 32, device="cuda", dtype=torch.float16, generator=_g(15))
    out = torch.empty(128, 32, device="cuda", dtype=torch.float16)
    matmul.ref(x, y, out)
    assert torch.allclose(out.float(), (x @ y).float(), rtol=2e-2, atol=2e-2)


def test_config_cache_persists(tmp_path, monkeypatch):
    monkeypatch.setenv("DEUTERON_CACHE_DIR", str(tmp_path))
    k = dt.kernel(add_relu.fn)
    k.samples = 3
    x = torch.randn(4096, device="cuda", generator=_g(16))
    out = torch.empty_like(x)
    k(x, x, out)
    import json
    data = json.load(open(tmp_path / "configs.json"))
    assert len(data) == 1 and next(iter(data)).startswith("add_relu:")
    k2 = dt.kernel(add_relu.fn)
    k2(x, x, out)          # served from the disk cache, no autotuning
    assert dict(k2.best_config) == next(iter(data.values()))


@dt.kernel(samples=4)
def row_mean(x, out):
    for t in dt.tile(x.shape[0]):
        out[t] = x[t, :].mean(1)


def test_mean_over_a_ragged_whole_dimension():
    """mean() folds a whole dimension: padded lanes are excluded and the sum
    is divided by the true extent (777, not the 1024-wide span)."""
    x = torch.randn(300, 777, device="cuda", generator=_g(17))
    out = torch.empty(300, device="cuda")
    row_mean(x, out)
    torch.testing.assert_close(out, x.mean(1), rtol=1e-5, atol=1e-6)


@dt.kernel(config={"BLOCK_TM": 64, "BLOCK_TN": 64, "BLOCK_TK": 32, "num_warps": 4,
                   "num_stages": 2})
def exp_dot(x, y, out):
    for tm, tn in dt.tile([x.shape[0], y.shape[1]]):
        acc = dt.zeros([tm, tn], dtype=dt.float32)
        for tk in dt.tile(x.shape[1]):
            acc += dt.exp(x[tm, tk]) @ dt.exp(y[tk, tn])
        out[tm, tn] = acc


def test_dot_of_computed_tiles_over_a_ragged_k():
    """exp(0) = 1 in both operands' padded k lanes: the tracer zeroes each
    computed operand there, so K = 100 (not a multiple of 32) matches torch."""
    x = torch.randn(128, 100, device="cuda", generator=_g(18)) * 0.1
    y = torch.randn(100, 96, device="cuda", generator=_g(19)) * 0.1
    out = torch.empty(128, 96, device="cuda")
    exp_dot(x, y, out)
    ref = x.exp().double() @ y.exp().double()
    assert ((out.double() - ref).norm() / ref.norm()).item() < 1e-5


@dt.kernel(config={"BLOCK_TM": 64, "BLOCK_TN": 64, "BLOCK_TK": 32, "num_warps": 4,
                   "num_stages": 2})
def log_dot(x, y, out):
    for tm, tn in dt.tile([x.shape[0], y.shape[1]]):
        acc = dt.zeros([tm, tn], dtype=dt.float32)
        for tk in dt.tile(x.shape[1]):
            acc += dt.log(x[tm, tk]) @ y[tk, tn]
        out[tm, tn] = acc


def test_dot_of_a_non_finite_padding_and_a_load_over_a_ragged_k():
    """log(0) = -inf in the computed operand's padded k lanes and 0 in the
    loaded operand's: -inf * 0 is NaN, so the tracer zeroes the computed
    operand even though the other one is a zero-padded load (K = 100)."""
    x = torch.rand(128, 100, device="cuda", generator=_g(20)) + 0.5
    y = torch.randn(100, 96, device="cuda", generator=_g(21)) * 0.1
    out = torch.empty(128, 96, device="cuda")
    log_dot(x, y, out)
    ref = x.log().double() @ y.double()
    assert not out.isnan().any()
    assert ((out.double() - ref).norm() / ref.norm()).item() < 1e-5
