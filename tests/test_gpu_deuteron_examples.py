"""The reference's deuteron examples (examples/deuteron/01-04) at their own
shapes and tolerances, written the way the examples write them: each kernel
traces, autotunes against its eager oracle and must then match torch."""

import os
import tempfile

import pytest
import torch

import deuteron as dt

pytestmark = pytest.mark.gpu

os.environ.setdefault("DEUTERON_CACHE_DIR", tempfile.mkdtemp(prefix="deuteron-examples-"))


@dt.kernel
def matmul(x, y, out):
    for tile_m, tile_n in dt.tile([x.shape[0], y.shape[1]]):
        acc = dt.zeros([tile_m, tile_n], dtype=dt.float32)
        for tile_k in dt.tile(x.shape[1]):
            acc += x[tile_m, tile_k] @ y[tile_k, tile_n]
        out[tile_m, tile_n] = acc


@dt.kernel
def softmax(x, out):
    for tile_m in dt.tile(x.shape[0]):
        row = x[tile_m, :]
        m = row.amax(1)
        e = dt.exp(row - m[:, None])
        s = e.sum(1)
        out[tile_m, :] = e / s[:, None]


@dt.kernel
def layernorm(x, w, b, out, eps):
    for tile_m in dt.tile(x.shape[0]):
        row = x[tile_m, :]
        mean = row.sum(1) / x.shape[1]
        diff = row - mean[:, None]
        var = (diff * diff).sum(1) / x.shape[1]
        rstd = dt.rsqrt(var + eps)
        out[tile_m, :] = diff * rstd[:, None] * w[:] + b[:]


@dt.kernel
def fused_gelu_residual(x, y, out):
    for t in dt.tile(x.shape[0]):
        v = x[t]
        inner = 0.7978845608028654 * (v + 0.044715 * v * v * v)
        g = 0.5 * v * (1.0 + dt.tanh(inner))
        out[t] = g + y[t]


def test_example_01_matmul_2048x1024x2048():
    M, K, N = 2048, 1024, 2048
    x = torch.randn(M, K, device="cuda", dtype=torch.float16)
    y = torch.randn(K, N, device="cuda", dtype=torch.float16)
    out = torch.empty(M, N, device="cuda", dtype=torch.float16)
    matmul(x, y, out)
    ref = (x.float() @ y.float()).half()
    rel = ((out.float() - ref.float()).norm() / ref.float().norm()).item()
    assert rel <= 1e-2
    assert "nl.dot(" in matmul.to_newt_source(x, y, out)


def test_example_02_softmax_8192x3000():
    x = torch.randn(8192, 3000, device="cuda")
    out = torch.empty_like(x)
    softmax(x, out)
    torch.testing.assert_close(out, torch.softmax(x, -1), rtol=1e-3, atol=1e-4)


def test_example_03_layernorm_4096x1500():
    M, N = 4096, 1500
    x = torch.randn(M, N, device="cuda")
    w = torch.randn(N, device="cuda")
    b = torch.randn(N, device="cuda")
    out = torch.empty_like(x)
    layernorm(x, w, b, out, 1e-5)
    ref = torch.nn.functional.layer_norm(x, (N,), w, b, 1e-5)
    assert (out - ref).abs().max().item() < 1e-3


def test_example_04_fused_gelu_residual_4m():
    n = 1 << 22
    x = torch.randn(n, device="cuda")
    y = torch.randn(n, device="cuda")
    out = torch.empty_like(x)
    fused_gelu_residual(x, y, out)
    ref = torch.nn.functional.gelu(x, approximate="tanh") + y
    assert (out - ref).abs().max().item() < 1e-5
