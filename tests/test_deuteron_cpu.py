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
    assert "@newt.jit" in src and "def matmul__tiles(" in src
    assert "BLOCK_TILE_M: nl.constexpr" in src and "BLOCK_TILE_K: nl.constexpr" in src
    assert "nl.program_id(0)" in src and "nl.program_id(1)" in src
    assert "for tile_k_step in range(nl.cdiv(x_d1, BLOCK_TILE_K)):" in src
    # each tensor read is its own statement; the dot consumes them directly
    assert "v_acc = nl.dot(_t1, _t2, v_acc)" in src
    assert src.count("nl.load(") == 2 and "nl.store(" in src
    assert "tile_m_in[:, None] & tile_k_in[None, :]" in src
    tr = matmul._specialize((x, y, o)).traced
    assert tr.tunable == ["BLOCK_TILE_M", "BLOCK_TILE_N", "BLOCK_TILE_K"]
    assert tr.writes == {"out"} and tr.has_dot and tr.spans == []


def test_dot_kernels_try_gfx950_seeds_first():
    from newt_amd.deuteron.runtime import SearchSpace
    x, y, o = torch.empty(64, 32).half(), torch.empty(32, 48).half(), torch.empty(64, 48).half()
    space = SearchSpace(matmul._specialize((x, y, o)).traced)
    assert dict(space.seeds()[0]) == {"num_warps": 4, "num_stages": 4, "BLOCK_TILE_M": 256,
                                      "BLOCK_TILE_N": 256, "BLOCK_TILE_K": 32}
    assert all(space.admits(c) for c in space.moves(space.seeds()[0]))
    xs = torch.empty(8, 100)
    sm = SearchSpace(softmax._specialize((xs, xs)).traced, span_elements=128)
    assert sm.seeds() == []
    # footprints beyond one workgroup's registers are not tried
    assert all(c["BLOCK_TILE_M"] * 128 <= 1 << 15 for c in sm.every())
    assert sm.admits(sm.default())


def test_a_span_wider_than_the_footprint_cap_keeps_its_smallest_tiles():
    """A whole-dimension span above the cap (a 65536-wide row) still has
    candidates: one row per program with each num_warps, and moves among
    them; the search does not start from an empty space."""
    from newt_amd.deuteron.runtime import SearchSpace
    xs = torch.empty(8, 65536)
    sm = SearchSpace(softmax._specialize((xs, xs)).traced, span_elements=65536)
    every = sm.every()
    assert every and all(c["BLOCK_TILE_M"] == 1 for c in every)
    assert sorted(c.num_warps for c in every) == [1, 2, 4, 8]
    assert sm.admits(sm.default()) and sm.default()["BLOCK_TILE_M"] == 1
    assert sm.moves(every[0])


def test_an_empty_search_space_is_its_own_error():
    from newt_amd.deuteron.runtime import Tuner

    class Empty:
        def every(self):
            return []

        def seeds(self):
            return []
    t = object.__new__(Tuner)
    t.kernel = softmax
    with pytest.raises(RuntimeError, match="no candidate configuration"):
        t.search(Empty(), 8)


def test_masks_reach_reductions():
    x = torch.empty(10, 30)
    src = softmax.to_newt_source(x, x)
    # padded lanes of the whole-row load become -inf for max and 0 for sum:
    # only the folded axis is masked
    assert "nl.max(nl.where(x_all1_in[None, :], v_row, float('-inf')), axis=1)" in src
    assert "nl.sum(nl.where(x_all1_in[None, :], v_e, 0.0), axis=1)" in src
    assert "SPAN_X_1: nl.constexpr" in src


def test_whole_dims_meeting_share_one_span():
    x = torch.empty(10, 30)
    tr = layernorm._specialize((x, x[0], x[0], x, 1e-5)).traced
    assert "eps" in tr.source.split("def layernorm__tiles(")[1].split(")")[0]
    assert "w_ptr + x_all1_idx * w_s0" in tr.source
    assert tr.spans == [("SPAN_X_1", ["x_d1", "w_d0", "b_d0", "out_d1"])]


def test_span_sizes_must_agree():
    x, w = torch.empty(10, 30), torch.empty(31)
    spec = layernorm._specialize((x, w, w, x, 1e-5))
    with pytest.raises(ValueError, match="meet in one expression"):
        spec.span_sizes(spec.extents((x, w, w, x, 1e-5)))
    ok = spec.span_sizes(spec.extents((x, x[0], x[0], x, 1e-5)))
    assert ok == {"SPAN_X_1": 32}


@dt.kernel
def row_mean(x, out):
    for t in dt.tile(x.shape[0]):
        out[t] = x[t, :].mean(1)


def test_mean_divides_by_the_true_extent():
    x, o = torch.empty(10, 30), torch.empty(10)
    src = row_mean.to_newt_source(x, o)
    assert "(nl.sum(nl.where(x_all1_in[None, :], _t1, 0.0), axis=1) / (x_d1))" in src


def test_dot_masks_every_computed_operand_over_a_padded_k():
    @dt.kernel
    def expdot(x, y, out):
        for tm, tn in dt.tile([x.shape[0], y.shape[1]]):
            acc = dt.zeros([tm, tn], dtype=dt.float32)
            for tk in dt.tile(x.shape[1]):
                acc += dt.exp(x[tm, tk]) @ dt.exp(y[tk, tn])
            out[tm, tn] = acc

    @dt.kernel
    def halfexp(x, y, out):
        for tm, tn in dt.tile([x.shape[0], y.shape[1]]):
            acc = dt.zeros([tm, tn], dtype=dt.float32)
            for tk in dt.tile(x.shape[1]):
                acc += dt.exp(x[tm, tk]) @ y[tk, tn]
            out[tm, tn] = acc
    @dt.kernel
    def loaddot(x, y, out):
        for tm, tn in dt.tile([x.shape[0], y.shape[1]]):
            acc = dt.zeros([tm, tn], dtype=dt.float32)
            for tk in dt.tile(x.shape[1]):
                acc += x[tm, tk] @ dt.log(y[tk, tn])
            out[tm, tn] = acc
    x, y, o = torch.empty(64, 32), torch.empty(32, 48), torch.empty(64, 48)
    src = expdot.to_newt_source(x, y, o)
    assert "nl.where(tk_in[None, :], nl.exp(_t1), 0.0)" in src
    assert "nl.where(tk_in[:, None], nl.exp(_t2), 0.0)" in src
    # a raw load on the other side is not enough: 0 * inf is NaN, so the
    # computed operand is zeroed in its padded k lanes all the same
    src = halfexp.to_newt_source(x, y, o)
    assert "nl.where(tk_in[None, :], nl.exp(_t1), 0.0)" in src and src.count("nl.where(") == 1
    src = loaddot.to_newt_source(x, y, o)
    assert "nl.where(tk_in[:, None], nl.log(_t2), 0.0)" in src and src.count("nl.where(") == 1
    # two raw loads (the matmul) need no mask
    assert "nl.where(" not in matmul.to_newt_source(x.half(), y.half(), o.half())


def _compile(tr, types, constexprs, num_warps=4, num_stages=2):
    tree = ast.parse(tr.source)
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
    tr = matmul._specialize((x, y, o)).traced
    f16p = tp.pointer_type(tp.float16)
    src, lds = _compile(tr, lambda n: f16p if n.endswith("_ptr") else tp.int32,
                        {"BLOCK_TILE_M": 128, "BLOCK_TILE_N": 128, "BLOCK_TILE_K": 32},
                        num_warps=4, num_stages=3)
    assert "newt::lds_dma16" in src and "_ldsP2" in src     # 3 direct-to-LDS stages
    assert len(hip.compile_hip(src, "k")) > 0


def test_generated_softmax_compiles_for_gfx950():
    from newt_amd.runtime import hip
    x = torch.empty(10, 30)
    tr = softmax._specialize((x, x)).traced
    f32p = tp.pointer_type(tp.float32)
    src, _ = _compile(tr, lambda n: f32p if n.endswith("_ptr") else tp.int32,
                      {"BLOCK_TILE_M": 2, "SPAN_X_1": 32})
    assert len(hip.compile_hip(src, "k")) > 0


@pytest.mark.parametrize("body,msg", [
    ("x[0] = 1.0", "top level"),
    ("for t in range(4):\n        pass", "dt.tile"),
    ("for t in dt.tile(x.shape[0]):\n        out[t] = x[t].to(dt.float16)", ".to()"),
    ("for t in dt.tile(x.shape[0]):\n        out[t] = x[t].mean()", "whole dimensions"),
    ("for t in dt.tile(x.shape[0]):\n        out[t] = q[t]", "not defined"),
    ("for t in dt.tile(x.shape[0]):\n        out[t, t] = x[t]", "dims"),
    ("for t in dt.tile(x.shape[0]):\n        out[t] = x[t]\n    for u in dt.tile(4):\n"
     "        out[u] = x[u]", "exactly one"),
    ("for t in dt.tile(x.shape[0]):\n        for u in dt.tile(x.shape[0]):\n"
     "            out[t] = x[u] + x[t]", "cannot be combined"),
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


def test_config_store_merges_and_replaces_atomically(tmp_path, monkeypatch):
    """configs.json: entries from several writers survive, a corrupt or
    truncated file is read as empty (and then rewritten whole), and no
    temporary file is left behind."""
    import json
    from newt_amd.deuteron.runtime import Config, ConfigStore
    monkeypatch.setenv("DEUTERON_CACHE_DIR", str(tmp_path))
    a, b = ConfigStore(), ConfigStore()
    a.put("k1", Config(BLOCK_T=64, num_warps=4))
    b.put("k2", Config(BLOCK_T=128, num_warps=8))
    data = json.loads((tmp_path / "configs.json").read_text())
    assert data == {"k1": {"BLOCK_T": 64, "num_warps": 4},
                    "k2": {"BLOCK_T": 128, "num_warps": 8}}
    assert a.get("k2") == {"BLOCK_T": 128, "num_warps": 8} and a.get("k3") is None
    (tmp_path / "configs.json").write_text('{"k1": {"BLOCK_T": 6')     # truncated
    assert a.get("k1") is None
    a.put("k3", Config(BLOCK_T=32))
    assert json.loads((tmp_path / "configs.json").read_text()) == {"k3": {"BLOCK_T": 32}}
    assert sorted(p.name for p in tmp_path.iterdir()) == ["configs.json", "configs.json.lock"]


def test_untuned_kernel_uses_a_default_and_persists_nothing(tmp_path, monkeypatch):
    from newt_amd.deuteron.runtime import SearchSpace
    monkeypatch.setenv("DEUTERON_CACHE_DIR", str(tmp_path))
    k = dt.kernel(autotune=False)(matmul.fn)
    x, y, o = torch.empty(64, 32).half(), torch.empty(32, 48).half(), torch.empty(64, 48).half()
    spec = k._specialize((x, y, o))
    cfg = SearchSpace(spec.traced).default()
    assert cfg["BLOCK_TILE_M"] == 256 and cfg.num_stages == 4
    assert not (tmp_path / "configs.json").exists()


def test_tuner_confirms_its_fastest_candidates(monkeypatch):
    """After its search, deuteron's tuner times its three fastest distinct
    candidates again, back to back and twice over, and keeps the fastest of
    those runs: a candidate timed on cold clocks during the search can still
    win."""
    from newt_amd import testing
    from newt_amd.deuteron.runtime import Config, Tuner

    cfgs = {n: Config({"BLOCK_TILE_M": n}) for n in (16, 32, 64, 128, 256)}
    t = object.__new__(Tuner)
    t.trials = [(cfgs[16], 3.0, ""), (cfgs[32], 1.0, ""), (cfgs[64], 2.0, ""),
                (cfgs[128], None, "wrong result"), (cfgs[256], 4.0, ""), (cfgs[32], 1.5, "")]
    launched = []

    class Spec:
        def launch(self, work, cfg):
            launched.append(cfg["BLOCK_TILE_M"])
    t.spec, t.work = Spec(), []
    again = {16: [0.9, 0.7], 32: [1.1, 1.0], 64: [2.0, 1.9]}

    def fake_bench(fn, warmup, rep):
        fn()
        n = launched[-1]
        return again[n][sum(1 for x in launched if x == n) - 1]
    monkeypatch.setattr(testing, "do_bench", fake_bench)
    best, ms = t.confirm(cfgs[32], 1.0)
    assert launched == [32, 64, 16, 32, 64, 16]    # the 3 fastest, two rounds
    assert best["BLOCK_TILE_M"] == 16 and ms == 0.7
