"""deuteron's tracer without a GPU: the newt source it generates for the
reference's example kernels (examples/deuteron/01-04), its rejections
(TraceError messages of deuteron/codegen.py), and that the generated kernels
compile to gfx950 code objects through newt's compiler and hipRTC."""

import ast

import pytest
import torch

import deuteron as dt
from newt_amd.compiler import Param, compile_fn
from newt_amd.compiler import types as tp


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
def add_relu(x, y, out):
    for tile_n in dt.tile(x.shape[0]):
        out[tile_n] = dt.relu(x[tile_n] + y[tile_n])


def test_matmul_source_is_a_pipelineable_dot_loop():
    x, y, o = torch.empty(64, 32).half(), torch.empty(32, 48).half(), torch.empty(64, 48).half()
    src = matmul.to_newt_source(x, y, o)
    assert "@newt.jit" in src and "def matmul_newt(" in src
    assert "BLOCK_TILE_M: nl.constexpr" in src and "BLOCK_TILE_K: nl.constexpr" in src
    assert "nl.program_id(0)" in src and "nl.program_id(1)" in src
    assert "for _i_tile_k in range(0, nl.cdiv(x_d1, BLOCK_TILE_K)):" in src
    assert "acc = nl.dot(_ld1, _ld2, acc)" in src
    assert src.count("nl.load(") == 2 and "nl.store(" in src
    ks = matmul._source_for((x, y, o))
    assert ks.tunable == ["BLOCK_TILE_M", "BLOCK_TILE_N", "BLOCK_TILE_K"]
    assert ks.store_params == {"out"}


def test_dot_kernels_try_gfx950_priors_first():
    x, y, o = torch.empty(64, 32).half(), torch.empty(32, 48).half(), torch.empty(64, 48).half()
    ks = matmul._source_for((x, y, o))
    pri = matmul._priors(ks, matmul._space(ks))
    assert dict(pri[0]) == {"num_warps": 4, "num_stages": 4, "BLOCK_TILE_M": 256,
                            "BLOCK_TILE_N": 256, "BLOCK_TILE_K": 32}
    xs, os_ = torch.empty(8, 100), torch.empty(8, 100)
    ks2 = softmax._source_for((xs, os_))
    assert softmax._priors(ks2, softmax._space(ks2)) == []


def test_masks_reach_reductions():
    x = torch.empty(10, 30)
    src = softmax.to_newt_source(x, x)
    # padded lanes of the masked row load get -inf for max and 0 for sum
    assert "float('-inf')), axis=1)" in src and "0.0), axis=1)" in src
    assert "BLOCK_FULL0: nl.constexpr" in src


def test_scalars_and_1d_tensors():
    x = torch.empty(10, 30)
    src = layernorm.to_newt_source(x, x[0], x[0], x, 1e-5)
    assert "eps" in src.split("def layernorm_newt(")[1].split(")")[0]
    assert "w_ptr + offs_full1 * w_s0" in src


def _compile(ks, types, constexprs, num_warps=4, num_stages=2):
    tree = ast.parse(ks.source)
    fndef = next(n for n in tree.body if isinstance(n, ast.FunctionDef))
    import newt
    import newt.language as nl
    glb = {"newt": newt, "nl": nl}
    params = []
    for a in fndef.args.args:
        if a.arg in constexprs:
            continue
        params.append((a.arg, Param(types(a.arg), a.arg, eq1=a.arg.endswith("_s1"),
                                    aligned16=True, div=16)))
    return compile_fn(fndef, glb, params, constexprs, num_warps, "k", num_stages=num_stages)


def test_generated_matmul_compiles_pipelined_for_gfx950():
    from newt_amd.runtime import hip
    x, y, o = torch.empty(64, 32).half(), torch.empty(32, 48).half(), torch.empty(64, 48).half()
    ks = matmul._source_for((x, y, o))
    f16p = tp.pointer_type(tp.float16)
    src, lds = _compile(ks, lambda n: f16p if n.endswith("_ptr") else tp.int32,
                        {"BLOCK_TILE_M": 128, "BLOCK_TILE_N": 128, "BLOCK_TILE_K": 32},
                        num_warps=4, num_stages=3)
    assert "newt::lds_dma16" in src and "_ldsP2" in src     # 3 direct-to-LDS stages
    assert len(hip.compile_hip(src, "k")) > 0


def test_generated_softmax_compiles_for_gfx950():
    from newt_amd.runtime import hip
    x = torch.empty(10, 30)
    ks = softmax._source_for((x, x))
    f32p = tp.pointer_type(tp.float32)
    src, _ = _compile(ks, lambda n: f32p if n.endswith("_ptr") else tp.int32,
                      {"BLOCK_TILE_M": 2, "BLOCK_FULL0": 32, "BLOCK_FULL1": 32})
    assert len(hip.compile_hip(src, "k")) > 0


@pytest.mark.parametrize("body,msg", [
    ("x[0] = 1.0", "top level"),
    ("for t in range(4):\n        pass", "expected dt.tile"),
    ("for t in dt.tile(x.shape[0]):\n        out[t] = x[t].to(dt.float16)", ".to()"),
    ("for t in dt.tile(x.shape[0]):\n        out[t] = x[t].mean()", "mean"),
    ("for t in dt.tile(x.shape[0]):\n        out[t] = q[t]", "unknown name"),
    ("for t in dt.tile(x.shape[0]):\n        out[t, t] = x[t]", "dims"),
])
def test_trace_errors(tmp_path, body, msg):
    import importlib.util
    path = tmp_path / "k.py"
    path.write_text("import deuteron as dt\n\n\ndef k(x, out):\n    " + body + "\n")
    spec = importlib.util.spec_from_file_location("dtk", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    kern = dt.kernel(mod.k)
    with pytest.raises(dt.TraceError, match=msg):
        kern.to_newt_source(torch.empty(8), torch.empty(8))
