"""CPU-only compiler tests: newt kernel AST -> HIP C++ -> gfx950 code object,
with no GPU involved (the counterpart of the reference's
tests/test_codegen_cpu.py, re-targeted: instead of CUDA substrings these check
the emitted HIP and the AMD assembly of our own hipRTC builds - 16-byte global
vector accesses, wave64 DPP/ds_swizzle reductions, v_mfma matrix-core
instructions - plus LDS accounting and the compile errors the reference raises).
"""

import ast
import inspect
import re
import subprocess
import textwrap

import pytest

import newt_amd.language as nl
from newt_amd import workloads as W
from newt_amd.compiler import CompileError, Param, compile_fn
from newt_amd.compiler import types as tp

F32P = tp.pointer_type(tp.float32)
F16P = tp.pointer_type(tp.float16)
BF16P = tp.pointer_type(tp.bfloat16)
OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"


def fndef_of(fn):
    fn = getattr(fn, "fn", fn)
    return ast.parse(textwrap.dedent(inspect.getsource(fn))).body[0], fn.__globals__


def compile_source(fn, arg_types, constexprs, num_warps=4, num_stages=3, waves_per_eu=0):
    """Run the code generator directly: (HIP source, LDS bytes)."""
    fndef, glb = fndef_of(fn)
    params = []
    for n, t in arg_types.items():
        if isinstance(t, tuple):
            t, facts = t
        else:
            facts = {}
        params.append((n, Param(t, n, **facts)))
    return compile_fn(fndef, glb, params, constexprs, num_warps, "k", num_stages=num_stages,
                      waves_per_eu=waves_per_eu)


def isa(src):
    """gfx950 assembly of a generated kernel, built here with hipRTC."""
    from newt_amd.runtime import hip
    code = hip.compile_hip(src, "k")
    import os
    import tempfile
    with tempfile.NamedTemporaryFile(suffix=".co", delete=False) as f:
        f.write(code)
        path = f.name
    try:
        return subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", path], capture_output=True,
                              text=True, check=True).stdout
    finally:
        os.unlink(path)


A16 = {"aligned16": True}
D16 = {"div": 16}

ADD_ARGS = {"x_ptr": (F32P, A16), "y_ptr": (F32P, A16), "out_ptr": (F32P, A16), "n": tp.int32}


def test_vector_add_layout_and_vector_path():
    src, lds = compile_source(W.add_kernel, ADD_ARGS, {"BLOCK": 1024})
    assert "__launch_bounds__(256)" in src        # num_warps=4 wave64s
    assert "newt::load_vec<float, 4>" in src      # 16-byte fast path
    assert "newt::store_vec<float, 4>" in src
    assert "blockIdx.x" in src and "__restrict__" in src
    # no program shares data with others: hardware workgroup order
    assert "_pb" not in src
    assert lds == 0                               # pure elementwise: no LDS
    asm = isa(src)
    assert "global_load_dwordx4" in asm and "global_store_dwordx4" in asm
    assert "v_fma" not in asm                     # x + y is not contracted


def test_no_fp_contraction():
    def k(x_ptr, y_ptr, o_ptr, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        x = nl.load(x_ptr + offs)
        y = nl.load(y_ptr + offs)
        nl.store(o_ptr + offs, x * y + x)
    src, _ = compile_source(k, {"x_ptr": (F32P, A16), "y_ptr": (F32P, A16), "o_ptr": (F32P, A16)},
                            {"BLOCK": 256})
    asm = isa(src)
    assert "v_mul_f32" in asm and "v_add_f32" in asm
    assert not re.search(r"v_(fma|fmac|mac|mad)_f32", asm)


def test_softmax_wave64_reductions():
    args = {"x_ptr": (F32P, A16), "out_ptr": (F32P, A16), "N": tp.int32, "stride": tp.int32}
    src, lds = compile_source(W.softmax_kernel, args, {"BLOCK_N": 4096}, num_warps=8)
    assert "__launch_bounds__(512)" in src
    assert "newt::lane_reduce<newt::Max" in src and "newt::lane_reduce<newt::Sum" in src
    assert lds > 0                                # cross-wave partials go through LDS
    asm = isa(src)
    assert "quad_perm" in asm                     # DPP steps
    # a whole-wave butterfly stays on the VALU: DPP mirrors for lane bits 2-3,
    # permlane swaps for bits 4-5, nothing through the LDS pipe
    assert "row_half_mirror" in asm and "row_mirror" in asm
    assert "v_permlane16_swap_b32" in asm and "v_permlane32_swap_b32" in asm
    assert "ds_swizzle_b32" not in asm and "ds_bpermute_b32" not in asm


def test_layernorm_fp16_io_fp32_math():
    args = {"x_ptr": (F16P, A16), "w_ptr": (F16P, A16), "b_ptr": (F16P, A16),
            "out_ptr": (F16P, A16), "mean_ptr": (F32P, A16), "rstd_ptr": (F32P, A16),
            "N": tp.int32, "stride": tp.int32, "eps": tp.float32}
    src, _ = compile_source(W.layernorm_kernel, args, {"BLOCK_N": 8192}, num_warps=8)
    assert "newt::load_vec<_Float16, 8>" in src   # VEC = 8 halves = 16 bytes
    assert "rsqrtf" in src
    asm = isa(src)
    assert "global_load_dwordx4" in asm


@pytest.mark.parametrize("dt,ptr", [("f16", F16P), ("bf16", BF16P)])
def test_matmul_uses_mfma(dt, ptr):
    args = {"a_ptr": (ptr, A16), "b_ptr": (ptr, A16), "c_ptr": (ptr, A16)}
    for n in ("M", "N", "K", "sam", "sbk", "scm"):
        args[n] = (tp.int32, D16)
    for n in ("sak", "sbn", "scn"):
        args[n] = (tp.int32, {"eq1": True})
    # 8 waves of 64x64: the 32x32x16 MFMA
    src, lds = compile_source(W.matmul_kernel, args,
                              {"BLOCK_M": 256, "BLOCK_N": 128, "BLOCK_K": 32}, num_warps=8,
                              num_stages=4)
    assert "newt::mfma_32x32x16" in src and "newt::mfma_16x16x32" not in src
    assert 0 < lds <= 160 * 1024
    asm = isa(src)
    assert f"v_mfma_f32_32x32x16_{dt}" in asm
    assert "ds_read_b128" in asm
    # one wave per SIMD (4-wave workgroups): the 16x16x32 MFMA, whatever the
    # wave tile and k-step
    for cex, ns in (({"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": 32}, 4),
                    ({"BLOCK_M": 128, "BLOCK_N": 128, "BLOCK_K": 64}, 4),
                    ({"BLOCK_M": 64, "BLOCK_N": 64, "BLOCK_K": 64}, 4)):
        src, lds = compile_source(W.matmul_kernel, args, cex, num_warps=4, num_stages=ns)
        assert "newt::mfma_16x16x32" in src and "newt::mfma_32x32x16" not in src, cex
    assert lds == 64 * 64 * 2 * 2 * 4
    assert f"v_mfma_f32_16x16x32_{dt}" in isa(src)
    # except 128x128 wave tiles over a 64-deep k-step (their 16x16x32
    # fragments spill): 32x32x16
    src, _ = compile_source(W.matmul_kernel, args, {"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": 64},
                            num_warps=4, num_stages=2)
    assert "newt::mfma_32x32x16" in src and "newt::mfma_16x16x32" not in src


def test_attention_compiles_with_mfma():
    args = {n: (BF16P, A16) for n in ("q_ptr", "k_ptr", "v_ptr", "o_ptr")}
    args.update({"S": (tp.int32, D16), "H": (tp.int32, D16), "scale": tp.float32})
    for n in ("sqb", "sqh", "sqm", "skb", "skh", "skn", "svb", "svh", "svn", "sob", "soh", "som"):
        args[n] = (tp.int32, D16)
    for causal in (False, True):
        src, lds = compile_source(W.attention_kernel, args,
                                  {"BLOCK_M": 128, "BLOCK_N": 64, "D": 128, "CAUSAL": causal},
                                  num_warps=4, num_stages=2)
        assert lds <= 160 * 1024
        asm = isa(src)
        assert "v_mfma_f32_32x32x16_bf16" in asm or "v_mfma_f32_16x16x32_bf16" in asm


def _vgprs(src):
    """Arch + accumulation VGPRs of the gfx950 code object built here."""
    import os
    import tempfile
    from newt_amd.runtime import hip
    with tempfile.NamedTemporaryFile(suffix=".co", delete=False) as f:
        f.write(hip.compile_hip(src, "k"))
        path = f.name
    try:
        notes = subprocess.run(["/opt/rocm/llvm/bin/llvm-readelf", "--notes", path],
                               capture_output=True, text=True, check=True).stdout
    finally:
        os.unlink(path)
    return int(re.search(r"\.vgpr_count:\s+(\d+)", notes).group(1))


def test_waves_per_eu_caps_registers():
    """waves_per_eu=2 emits the occupancy attribute and keeps flash attention
    within 256 registers (two waves per SIMD); without it the kernel uses more."""
    args = {n: (BF16P, A16) for n in ("q_ptr", "k_ptr", "v_ptr", "o_ptr")}
    args.update({"S": (tp.int32, D16), "H": (tp.int32, D16), "scale": tp.float32})
    for n in ("sqb", "sqh", "sqm", "skb", "skh", "skn", "svb", "svh", "svn", "sob", "soh", "som"):
        args[n] = (tp.int32, D16)
    cx = {"BLOCK_M": 128, "BLOCK_N": 64, "D": 128, "CAUSAL": False}
    src2, _ = compile_source(W.attention_kernel, args, cx, num_warps=4, num_stages=2,
                             waves_per_eu=2)
    src0, _ = compile_source(W.attention_kernel, args, cx, num_warps=4, num_stages=2)
    assert "amdgpu_waves_per_eu(2)" in src2 and "amdgpu_waves_per_eu" not in src0
    assert _vgprs(src2) <= 256 < _vgprs(src0)


def test_exp2_is_the_hardware_instruction():
    def k(x_ptr, o_ptr, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        nl.store(o_ptr + offs, nl.exp2(nl.load(x_ptr + offs)))

    src, _ = compile_source(k, {"x_ptr": F32P, "o_ptr": F32P}, {"BLOCK": 1024})
    asm = isa(src)
    assert "v_exp_f32" in asm and "v_ldexp" not in asm


def test_constexpr_branch_pruning():
    def k(x_ptr, FLAG: nl.constexpr, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        if FLAG:
            nl.store(x_ptr + offs, nl.full((BLOCK,), 1.0, dtype=nl.float32))
        else:
            nl.store(x_ptr + offs, nl.full((BLOCK,), 2.0, dtype=nl.float32))
    s1, _ = compile_source(k, {"x_ptr": (F32P, A16)}, {"FLAG": True, "BLOCK": 256})
    s2, _ = compile_source(k, {"x_ptr": (F32P, A16)}, {"FLAG": False, "BLOCK": 256})
    assert "1.0f" in s1 and "2.0f" not in s1
    assert "2.0f" in s2 and "1.0f" not in s2


def _expect_error(fn, args, ce, pattern):
    with pytest.raises(CompileError, match=pattern):
        compile_source(fn, args, ce)


def test_errors_block_if_condition():
    def k(x_ptr, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        x = nl.load(x_ptr + offs)
        if x > 0:
            nl.store(x_ptr + offs, x)
    _expect_error(k, {"x_ptr": F32P}, {"BLOCK": 64}, "scalar")


def test_errors_return_value():
    def k(x_ptr):
        return 1
    _expect_error(k, {"x_ptr": F32P}, {}, "return")


def test_errors_non_pow2_arange():
    def k(x_ptr, BLOCK: nl.constexpr):
        nl.store(x_ptr + nl.arange(0, BLOCK), 0.0)
    _expect_error(k, {"x_ptr": F32P}, {"BLOCK": 100}, "power of two")


def test_errors_unknown_function():
    def k(x_ptr):
        print(x_ptr)
    _expect_error(k, {"x_ptr": F32P}, {}, "unknown")


def test_errors_scalar_pointer_block_mask():
    def k(x_ptr, BLOCK: nl.constexpr):
        m = nl.arange(0, BLOCK) < 3
        v = nl.load(x_ptr, mask=m)
    _expect_error(k, {"x_ptr": F32P}, {"BLOCK": 64}, "scalar")


def test_errors_dot_shapes():
    def k(a_ptr, b_ptr, c_ptr):
        r = nl.arange(0, 32)
        a = nl.load(a_ptr + r[:, None] * 16 + nl.arange(0, 16)[None, :])
        b = nl.load(b_ptr + r[:, None] * 32 + r[None, :])
        c = nl.dot(a, b)
    _expect_error(k, {"a_ptr": F16P, "b_ptr": F16P, "c_ptr": F32P}, {}, "mismatch")


def test_errors_int_pow():
    def k(x_ptr, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        nl.store(x_ptr + offs, offs ** 3)
    _expect_error(k, {"x_ptr": tp.pointer_type(tp.int32)}, {"BLOCK": 64}, r"\*\*")


def test_lds_budget_check():
    # a dot whose staged operands exceed 160 KB of LDS is rejected at compile time
    def k(a_ptr, b_ptr, c_ptr, BM: nl.constexpr, BN: nl.constexpr, BK: nl.constexpr):
        rm = nl.arange(0, BM)
        rn = nl.arange(0, BN)
        rk = nl.arange(0, BK)
        a = nl.load(a_ptr + rm[:, None] * BK + rk[None, :])
        b = nl.load(b_ptr + rk[:, None] * BN + rn[None, :])
        c = nl.dot(a, b)
        nl.store(c_ptr + rm[:, None] * BN + rn[None, :], c)
    with pytest.raises(CompileError, match="LDS"):
        compile_source(k, {"a_ptr": (F32P, A16), "b_ptr": (F32P, A16), "c_ptr": (F32P, A16)},
                       {"BM": 256, "BN": 256, "BK": 128}, num_warps=8)


def test_independent_loads_issue_before_reductions(monkeypatch):
    """With NEWT_HOIST_LOADS=1, layernorm's weight and bias loads (which do not
    depend on the row statistics) are issued before the first cross-wave
    reduction, after the row load."""
    monkeypatch.setenv("NEWT_HOIST_LOADS", "1")
    src, _ = compile_source(W.layernorm_kernel, {
        "x_ptr": (F16P, {"aligned16": True}), "w_ptr": (F16P, {"aligned16": True}),
        "b_ptr": (F16P, {"aligned16": True}), "out_ptr": (F16P, {"aligned16": True}),
        "mean_ptr": tp.pointer_type(tp.float32), "rstd_ptr": tp.pointer_type(tp.float32),
        "N": tp.int32, "stride": tp.int32, "eps": tp.float32}, {"BLOCK_N": 8192})
    first_reduce = src.index("lane_reduce")
    xs, ws, bs = (src.index(f"({p} + ") if p != "x" else src.index("load_vec<_Float16, 8>((_p")
                  for p in ("x", "w_ptr", "b_ptr"))
    assert xs < ws < bs < first_reduce


def test_loads_do_not_move_across_stores():
    from newt_amd.compiler import hoist_loads

    def k(x_ptr, y_ptr, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        a = nl.load(x_ptr + offs)
        nl.store(x_ptr + offs, a * 2.0)
        s = nl.sum(a, axis=0)
        b = nl.load(x_ptr + offs)
        nl.store(y_ptr + offs, b + s)

    fndef, _ = fndef_of(k)
    order = [ast.unparse(st).split(" =")[0].split("(")[0] for st in hoist_loads(fndef).body]
    # b may pass the reduction but not the store before it
    assert order == ["offs", "a", "nl.store", "b", "s", "nl.store"]


def _matmul_args(ptr=F16P):
    args = {"a_ptr": (ptr, A16), "b_ptr": (ptr, A16), "c_ptr": (ptr, A16)}
    for n in ("M", "N", "K", "sam", "sbk", "scm"):
        args[n] = (tp.int32, D16)
    for n in ("sak", "sbn", "scn"):
        args[n] = (tp.int32, {"eq1": True})
    return args


def test_split_dot_axes_detection():
    """Grouped program ids are chosen for kernels whose dot operands follow
    different program axes (a tiled matmul, either operand order), not where
    an operand follows both (attention's q) or the ids are one axis."""
    from newt_amd.compiler import _split_dot_axes

    def mm_swapped(a_ptr, b_ptr, c_ptr, B: nl.constexpr):
        r = nl.arange(0, B)
        pn = nl.program_id(1)
        pm = nl.program_id(axis=0)
        x = nl.load(b_ptr + (pn * B + r)[:, None] * B + r[None, :])
        y = nl.load(a_ptr + r[:, None] * B + (pm * B + r)[None, :])
        nl.store(c_ptr + r[:, None] * B + r[None, :], nl.dot(x, y))

    def one_axis(a_ptr, b_ptr, c_ptr, B: nl.constexpr, NPN: nl.constexpr):
        pid = nl.program_id(0)
        pm, pn = pid // NPN, pid % NPN
        r = nl.arange(0, B)
        x = nl.load(a_ptr + (pm * B + r)[:, None] * B + r[None, :])
        y = nl.load(b_ptr + r[:, None] * B + (pn * B + r)[None, :])
        nl.store(c_ptr + r[:, None] * B + r[None, :], nl.dot(x, y))

    assert _split_dot_axes(fndef_of(W.matmul_kernel)[0])
    assert _split_dot_axes(fndef_of(mm_swapped)[0])
    assert not _split_dot_axes(fndef_of(one_axis)[0])
    assert not _split_dot_axes(fndef_of(W.attention_kernel)[0])
    assert not _split_dot_axes(fndef_of(W.softmax_kernel)[0])


_PID_HARNESS = r"""
#include <stdio.h>
#include <stdlib.h>
struct dim { unsigned x, y, z; };
int main(int argc, char **argv) {
  const struct dim gridDim = {atoi(argv[1]), atoi(argv[2]), atoi(argv[3])};
  const unsigned n = gridDim.x * gridDim.y * gridDim.z;
  unsigned *hits = calloc(n, sizeof(unsigned));
  for (unsigned z = 0; z < gridDim.z; z++)
    for (unsigned y = 0; y < gridDim.y; y++)
      for (unsigned x = 0; x < gridDim.x; x++) {
        const struct dim blockIdx = {x, y, z};
%s
        if (_pid0 < 0 || _pid1 < 0 || _pid2 < 0 || (unsigned)_pid0 >= gridDim.x ||
            (unsigned)_pid1 >= gridDim.y || (unsigned)_pid2 >= gridDim.z) return 2;
        hits[((unsigned)_pid2 * gridDim.y + (unsigned)_pid1) * gridDim.x + (unsigned)_pid0]++;
      }
  for (unsigned i = 0; i < n; i++) if (hits[i] != 1) return 3;
  return 0;
}
"""


@pytest.mark.parametrize("group", ["4", "8", "3", "0"])
def test_program_id_mapping_is_a_bijection(monkeypatch, tmp_path, group):
    """The program-id prologue the matmul kernel is compiled with, built with
    gcc on the host and run over every workgroup id of ragged and even grids:
    each program id is produced exactly once and in range (grouped for
    NEWT_PID_GROUP=3/4/8, XCD remap only for 0)."""
    monkeypatch.setenv("NEWT_PID_GROUP", group)
    src, _ = compile_source(W.matmul_kernel, _matmul_args(),
                            {"BLOCK_M": 64, "BLOCK_N": 64, "BLOCK_K": 32}, num_warps=4)
    lines = src.splitlines()
    i0 = next(i for i, l in enumerate(lines) if "const unsigned _nbx" in l)
    i1 = next(i for i, l in enumerate(lines) if "const int _pid2" in l)
    prologue = "\n".join(lines[i0:i1 + 1])
    assert ("_gw" in prologue) == (group != "0")
    c = tmp_path / "pid.c"
    c.write_text(_PID_HARNESS % prologue)
    exe = tmp_path / "pid"
    subprocess.run(["gcc", "-O1", "-o", str(exe), str(c)], check=True)
    for g in ((32, 32, 1), (16, 16, 1), (13, 7, 2), (5, 4, 1), (1, 1, 1), (3, 100, 1),
              (100, 3, 1), (9, 9, 3), (1, 17, 1), (17, 1, 1), (64, 48, 1)):
        r = subprocess.run([str(exe)] + [str(v) for v in g])
        assert r.returncode == 0, (g, r.returncode)


_PID_ORDER_HARNESS = r"""
#include <stdio.h>
#include <stdlib.h>
struct dim { unsigned x, y, z; };
int main(int argc, char **argv) {
  const struct dim gridDim = {atoi(argv[1]), atoi(argv[2]), atoi(argv[3])};
  const unsigned n = gridDim.x * gridDim.y * gridDim.z;
  for (unsigned b = 0; b < n; b++) {
    const struct dim blockIdx = {b %% gridDim.x, b / gridDim.x %% gridDim.y, b / (gridDim.x * gridDim.y)};
%s
    printf("%%u %%d %%d %%d\n", b, _pid0, _pid1, _pid2);
  }
  return 0;
}
"""


def _plain_attention_prologue(causal):
    src, _ = compile_source(W.attention_plain_kernel, _attention_args(),
                            {"BLOCK_M": 256, "BLOCK_N": 64, "D": 128, "CAUSAL": causal},
                            num_warps=8, num_stages=2, waves_per_eu=2)
    lines = src.splitlines()
    i0 = next(i for i, l in enumerate(lines) if "const unsigned _nbx" in l)
    i1 = next(i for i, l in enumerate(lines) if "const int _pid2" in l)
    return "\n".join(lines[i0:i1 + 1])


def test_work_growing_along_axis0_detected():
    """The causal examples/05 form's key loop ends at its query block's
    diagonal, so its work grows with program_id(0); the hand-written kernel
    numbers its programs itself, and loops independent of axis 0, shrinking
    with it, of unknown sign, or in kernels with atomics are not matched."""
    from newt_amd.compiler import _work_grows_along_axis0 as grows
    f = lambda k: fndef_of(k)[0]
    assert grows(f(W.attention_plain_kernel), {"CAUSAL": True, "BLOCK_M": 256, "BLOCK_N": 64})
    assert not grows(f(W.attention_plain_kernel), {"CAUSAL": False, "BLOCK_M": 256, "BLOCK_N": 64})
    for causal in (True, False):
        assert not grows(f(W.attention_kernel), {"CAUSAL": causal, "BLOCK_M": 256, "BLOCK_N": 64})
    for k, cex in ((W.matmul_kernel, {"BLOCK_M": 64, "BLOCK_N": 64, "BLOCK_K": 32}),
                   (W.softmax_kernel, {"BLOCK_N": 1024}), (W.layernorm_kernel, {"BLOCK_N": 1024}),
                   (W.add_kernel, {"BLOCK": 1024})):
        assert not grows(f(k), cex)

    def tri(o_ptr, n, stride, B: nl.constexpr):
        pid = nl.program_id(0)
        acc = 0.0
        for i in range(0, (pid + 1) * B):
            acc += 1.0
        nl.store(o_ptr + pid, acc)

    def shrinking(o_ptr, n, B: nl.constexpr):
        pid = nl.program_id(0)
        for i in range(pid * B, n):
            pass

    def unknown_sign(o_ptr, n, stride, B: nl.constexpr):
        pid = nl.program_id(0)
        for i in range(0, pid * stride):
            pass

    def with_atomics(o_ptr, n, B: nl.constexpr):
        pid = nl.program_id(0)
        for i in range(0, nl.minimum(n, pid + 1)):
            nl.atomic_add(o_ptr, 1.0)

    def runtime_join(o_ptr, n, B: nl.constexpr):
        pid = nl.program_id(0)
        end = n
        if n > 4:
            end = pid
        for i in range(0, end):
            pass

    def other_axis(o_ptr, n, B: nl.constexpr):
        for i in range(0, nl.program_id(1) * B):
            pass

    assert grows(f(tri), {"B": 4})
    assert not grows(f(tri), {"B": 0})
    for k in (shrinking, unknown_sign, with_atomics, runtime_join, other_axis):
        assert not grows(f(k), {"B": 4}), k.__name__


def test_heaviest_first_program_ids(tmp_path):
    """The causal examples/05 form is compiled with the heaviest-first
    prologue (the non-causal form without it). Built with gcc and run over
    every workgroup id: a bijection on even and ragged grids; on a grid whose
    heads split evenly over the 8 XCDs, the workgroups each XCD receives
    (linear ids b = x, x + 8, ...) take its whole heads in groups of 4 (all
    of them when 4 does not divide their count), and within a group every
    head's heaviest query block (pid0 = nbx - 1) first, then every head's next."""
    pro = _plain_attention_prologue(True)
    assert "_nbx - 1u - _rr / _G" in pro
    assert "_nbx - 1u" not in _plain_attention_prologue(False)
    c = tmp_path / "pid.c"
    c.write_text(_PID_HARNESS % pro)
    exe = tmp_path / "pid"
    subprocess.run(["gcc", "-O1", "-o", str(exe), str(c)], check=True)
    for g in ((16, 128, 1), (16, 16, 1), (13, 7, 2), (5, 4, 1), (1, 1, 1), (3, 100, 1),
              (100, 3, 1), (9, 9, 3), (1, 17, 1), (17, 1, 1), (16, 24, 1), (7, 8, 2)):
        r = subprocess.run([str(exe)] + [str(v) for v in g])
        assert r.returncode == 0, (g, r.returncode)
    c2 = tmp_path / "order.c"
    c2.write_text(_PID_ORDER_HARNESS % pro)
    exe2 = tmp_path / "order"
    subprocess.run(["gcc", "-O1", "-o", str(exe2), str(c2)], check=True)
    for nbx, nby in ((16, 128), (8, 16), (5, 24), (4, 64)):
        out = subprocess.run([str(exe2), str(nbx), str(nby), "1"], capture_output=True,
                             text=True, check=True).stdout.split("\n")
        rows = [tuple(map(int, l.split())) for l in out if l]
        gh = nby // 8
        G = 4 if gh % 4 == 0 else gh
        for x in range(8):
            seq = [(p0, p1) for b, p0, p1, _ in rows if b % 8 == x]
            assert len(seq) == gh * nbx
            h0 = min(p1 for _, p1 in seq)
            assert {p1 for _, p1 in seq} == set(range(h0, h0 + gh))
            for i, (p0, p1) in enumerate(seq):
                g, rr = divmod(i, G * nbx)
                assert (p0, p1) == (nbx - 1 - rr // G, h0 + g * G + rr % G), (nbx, nby, x, i)


def test_loaded_block_keeps_its_layout_against_a_broadcast_statistic():
    """A [1, N] row block that an earlier reduction already loaded, combined
    with the broadcast row statistic (the traced softmax's
    `row - row.amax(1)[:, None]`), keeps the load's 16-byte layout: the
    block is not converted through LDS, and the store is vectorised."""
    def k(x_ptr, o_ptr, N, BLOCK: nl.constexpr):
        rows = nl.program_id(0) + nl.arange(0, 1)
        cols = nl.arange(0, BLOCK)
        x = nl.load(x_ptr + rows[:, None] * N + cols[None, :])
        m = nl.max(x, axis=1)
        nl.store(o_ptr + rows[:, None] * N + cols[None, :], x - m[:, None])

    src, _ = compile_source(k, {"x_ptr": (F32P, A16), "o_ptr": (F32P, A16), "N": (tp.int32, D16)},
                            {"BLOCK": 4096})
    assert "_cv" not in src
    assert "store_vec<float, 4>" in src


def test_chained_dots_detected():
    """Kernels that feed one dot's result into another (attention's P @ V)
    are found on the AST; a matmul's accumulator chain and dot-free kernels
    are not."""
    from newt_amd.compiler import _chained_dots as chained
    f = lambda k: fndef_of(k)[0]
    assert chained(f(W.attention_kernel)) and chained(f(W.attention_plain_kernel))
    for k in (W.matmul_kernel, W.softmax_kernel, W.layernorm_kernel, W.add_kernel):
        assert not chained(f(k))

    def two_step(a_ptr, b_ptr, c_ptr, o_ptr, B: nl.constexpr):
        r = nl.arange(0, B)
        a = nl.load(a_ptr + r[:, None] * B + r[None, :])
        b = nl.load(b_ptr + r[:, None] * B + r[None, :])
        c = nl.load(c_ptr + r[:, None] * B + r[None, :])
        t = nl.dot(a, b)
        u = t.to(nl.float16)
        nl.store(o_ptr + r[:, None] * B + r[None, :], nl.dot(u, c))

    assert chained(f(two_step))


@pytest.mark.parametrize("mode,instr,fn", [("", "16x16x32", "lds_frag_r_perm16"),
                                            ("32", "32x32x16", "lds_frag_r_perm32")])
def test_attention_p_feeds_pv_from_registers(monkeypatch, mode, instr, fn):
    """Both attention forms run both dots on 16x16x32 MFMAs by default (on
    32x32x16 with NEWT_MFMA=32): the bf16 cast of the score accumulator is the
    P @ V dot's A operand in place, with V read from LDS in the permuted k
    order, so no block goes through an LDS layout conversion. The V tile takes
    the swizzle its 16-row reader needs."""
    monkeypatch.setenv("NEWT_MFMA", mode)
    args = _attention_args()
    for kern in (W.attention_kernel, W.attention_plain_kernel):
        for D in (64, 128):
            for causal in (False, True):
                src, _ = compile_source(kern, args, {"BLOCK_M": 256, "BLOCK_N": 64, "D": D,
                                                     "CAUSAL": causal},
                                        num_warps=8, num_stages=2, waves_per_eu=2)
                assert f"newt::mfma_{instr}" in src
                assert f"newt::{fn}<__bf16, {D}, {2 if mode == '' else 3}>" in src
                assert "_cv" not in src
                assert f"LdsTileR<__bf16, {D}, {2 if mode == '' else 3}>" in src


def _chained_dots_kernel(a_ptr, k_ptr, v_ptr, o_ptr, s_ptr, N, svn, svd,
                         BLOCK_M: nl.constexpr, BLOCK_N: nl.constexpr, D: nl.constexpr):
    pid = nl.program_id(0)
    offs_m = pid * BLOCK_M + nl.arange(0, BLOCK_M)
    offs_d = nl.arange(0, D)
    a = nl.load(a_ptr + offs_m[:, None] * D + offs_d[None, :])
    acc = nl.zeros((BLOCK_M, D), dtype=nl.float32)
    rs = nl.zeros((BLOCK_M,), dtype=nl.float32)
    for start_n in range(0, N, BLOCK_N):
        offs_n = start_n + nl.arange(0, BLOCK_N)
        k = nl.load(k_ptr + offs_n[:, None] * D + offs_d[None, :])
        s = nl.dot(a, nl.trans(k))
        rs = rs + nl.sum(s, axis=1)
        v = nl.load(v_ptr + offs_n[:, None] * svn + offs_d[None, :] * svd)
        acc = nl.dot(s.to(nl.float16), v, acc)
    nl.store(o_ptr + offs_m[:, None] * D + offs_d[None, :], acc)
    nl.store(s_ptr + offs_m, rs)


@pytest.mark.parametrize("mode,instr", [("", "16x16x32"), ("32", "32x32x16")])
@pytest.mark.parametrize("v_keys_contiguous", [False, True])
def test_chained_dot_reads_v_in_accumulator_order(monkeypatch, mode, instr, v_keys_contiguous):
    """The kernel of tests/test_gpu_pipeline_dot.py::test_dot_result_feeds_next_dot
    takes the permuted reader of its V tile's format and instruction: R-major
    (rows contiguous; swizzle bit 2 at 16x16x32) or K-major (keys
    contiguous), and converts nothing through LDS."""
    monkeypatch.setenv("NEWT_MFMA", mode)
    args = {"a_ptr": (F16P, A16), "k_ptr": (F16P, A16), "v_ptr": (F16P, A16),
            "o_ptr": (F32P, A16), "s_ptr": (F32P, A16), "N": (tp.int32, D16)}
    one = (tp.int32, {"eq1": True})
    args["svn"], args["svd"] = (one, (tp.int32, D16)) if v_keys_contiguous else ((tp.int32, D16), one)
    src, _ = compile_source(_chained_dots_kernel, args, {"BLOCK_M": 128, "BLOCK_N": 64, "D": 64},
                            num_warps=4, num_stages=2)
    mi = instr.split("x")[0]
    want = (f"lds_frag_k_perm{mi}<_Float16, 64>" if v_keys_contiguous else
            f"lds_frag_r_perm{mi}<_Float16, 64, {2 if mi == '16' else 3}>")
    assert f"newt::{want}" in src
    assert f"newt::mfma_{instr}" in src
    assert "_cv" not in src


def test_chained_dot_with_a_16_wide_p_compiles():
    """16-key blocks: the score tile is 16 wide, so P @ V (K = 16) takes
    32x32x16 and P goes through an LDS conversion; the in-place check must not
    build a 32x32 accumulator layout for a 16-wide P (it asserted here)."""
    args = {"a_ptr": (F16P, A16), "k_ptr": (F16P, A16), "v_ptr": (F16P, A16),
            "o_ptr": (F32P, A16), "s_ptr": (F32P, A16), "N": (tp.int32, D16),
            "svn": (tp.int32, D16), "svd": (tp.int32, {"eq1": True})}
    for BM, D, w in ((128, 64, 4), (64, 32, 2)):
        src, _ = compile_source(_chained_dots_kernel, args, {"BLOCK_M": BM, "BLOCK_N": 16, "D": D},
                                num_warps=w, num_stages=2)
        assert "newt::mfma_32x32x16" in src and "_perm" not in src
    for kern in (W.attention_kernel, W.attention_plain_kernel):
        src, _ = compile_source(kern, _attention_args(), {"BLOCK_M": 128, "BLOCK_N": 16, "D": 64,
                                                          "CAUSAL": True},
                                num_warps=4, num_stages=2)
        assert "_perm" not in src


def test_attention_program_ids_not_grouped():
    args = {n: (BF16P, A16) for n in ("q_ptr", "k_ptr", "v_ptr", "o_ptr")}
    args.update({"S": (tp.int32, D16), "H": (tp.int32, D16), "scale": tp.float32})
    for n in ("sqb", "sqh", "sqm", "skb", "skh", "skn", "svb", "svh", "svn", "sob", "soh", "som"):
        args[n] = (tp.int32, D16)
    src, _ = compile_source(W.attention_kernel, args,
                            {"BLOCK_M": 128, "BLOCK_N": 64, "D": 128, "CAUSAL": True},
                            num_warps=4, num_stages=2)
    assert "_pid0 = (int)(_pb % _nbx)" in src and "_gw" not in src


def test_loops_reusing_a_target_name_compile():
    """Two loops with the same target name: the second loop's target is not
    loop-carried state initialised from the first loop's (out-of-scope)
    counter, and the name is unbound after each loop."""
    def k(x_ptr, o_ptr, n, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        acc = nl.zeros((BLOCK,), dtype=nl.float32)
        for i in range(0, n, 2):
            acc = acc + nl.load(x_ptr + i * BLOCK + offs)
        for i in range(1, n, 2):
            acc = acc - nl.load(x_ptr + i * BLOCK + offs)
        nl.store(o_ptr + offs, acc)

    src, _ = compile_source(k, {"x_ptr": F32P, "o_ptr": F32P, "n": tp.int32}, {"BLOCK": 64})
    isa(src)   # compiles with hipRTC

    def reads_target_after_loop(o_ptr, n, BLOCK: nl.constexpr):
        for i in range(n):
            pass
        nl.store(o_ptr + nl.arange(0, BLOCK), nl.zeros((BLOCK,), dtype=nl.float32) + i)

    with pytest.raises(CompileError):
        compile_source(reads_target_after_loop, {"o_ptr": F32P, "n": tp.int32}, {"BLOCK": 64})


def test_sequential_pipelined_loops_share_lds_stages():
    """Attention's unmasked key loop, its masked tail loop and the
    online-softmax pass it takes for rows whose scores outgrow the first
    block's maximum are all pipelined (direct-to-LDS copies, branch-free fast
    copy), and each reuses the previous one's stage arrays after a barrier:
    the kernel needs the LDS of one loop (2 stages x (K + V) = 64 KiB), not
    of three."""
    args = {n: (BF16P, A16) for n in ("q_ptr", "k_ptr", "v_ptr", "o_ptr")}
    args.update({"S": (tp.int32, D16), "H": (tp.int32, D16), "scale": tp.float32})
    for n in ("sqb", "sqh", "sqm", "skb", "skh", "skn", "svb", "svh", "svn", "sob", "soh", "som"):
        args[n] = (tp.int32, D16)
    for causal in (False, True):
        src, lds = compile_source(W.attention_kernel, args,
                                  {"BLOCK_M": 128, "BLOCK_N": 64, "D": 128, "CAUSAL": causal},
                                  num_warps=4, num_stages=2, waves_per_eu=2)
        # + the cross-wave partials of the reductions: two programs still fit
        # one CU's 160 KiB
        assert 64 * 1024 <= lds <= 64 * 1024 + 1024
        assert len(re.findall(r"for \(; _it\d+ \+ 2 <", src)) == 3   # three fast copies
        assert src.count("newt::lds_dma16(") >= 16


@pytest.mark.parametrize("cfg", [(256, 256, 16, 8, 3), (128, 128, 32, 4, 3)])
def test_fp32_matmul_is_pipelined(cfg):
    """fp32 operands take the pipelined k-loop: direct-to-LDS copies, the
    branch-free fast copy, 16-byte fragment reads of the K-major A tile and
    the full-precision fp32 MFMA."""
    BM, BN, BK, nw, ns = cfg
    src, lds = compile_source(W.matmul_kernel, _matmul_args(F32P),
                              {"BLOCK_M": BM, "BLOCK_N": BN, "BLOCK_K": BK},
                              num_warps=nw, num_stages=ns)
    assert src.count("newt::lds_dma16(") > 0
    assert re.search(r"for \(; _it\d+ \+ \d+ <", src)
    assert "newt::lds_frag_k32f<" in src and "newt::LdsTileR32<" in src
    assert lds == ns * (BM * BK + BK * BN) * 4
    asm = isa(src)
    assert "v_mfma_f32_32x32x2_f32" in asm and "ds_read_b128" in asm


def test_fast_loop_copies_take_the_buffer_form(monkeypatch):
    """In the branch-free fast loop each direct-to-LDS copy goes through a raw
    buffer descriptor on the tile's uniform start plus a 32-bit lane offset
    (buffer_load_dwordx4 ... offen lds): one loop-invariant VGPR per copy
    instead of a VGPR pair and a 64-bit add. The loop is entered only when
    every tile's lane offsets are non-negative and below 2^31 bytes; the
    prologue and the general loop keep the 64-bit form, and
    NEWT_BUFFER_DMA=0 turns the buffer form off."""
    cex = {"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": 32}
    src, _ = compile_source(W.matmul_kernel, _matmul_args(), cex, num_warps=4, num_stages=4)
    loops = [m.start() for m in re.finditer(r"for \(; _it\d+ ", src)]
    assert len(loops) == 2
    before, fast, general = src[:loops[0]], src[loops[0]:loops[1]], src[loops[1]:]
    # the fast loop and the one clamped trip after it, 8 copies per sub-iteration each
    assert fast.count("newt::lds_dma16_buf(") == 64 and "newt::lds_dma16(" not in fast
    assert "lds_dma16_buf" not in before and "lds_dma16_buf" not in general
    # the entry test reads the tiles' offsets without emitting their loads
    assert "? a_ptr[" not in fast and "? b_ptr[" not in fast
    entry = before.rsplit("const int", 1)[1]
    # fp16 lane offsets below 2^31 bytes: sam * 255 + 31 (A rows) and
    # 255 + sbk * 31 (B rows) below 2^30 elements, strides non-negative
    assert "(sam) >= 0" in entry and "(long long)(sam) * 255 + 31LL) < 1073741824LL" in entry
    assert "(sbk) >= 0" in entry and "(255LL + (long long)(sbk) * 31) < 1073741824LL" in entry
    assert re.search(r"buffer_load_dwordx4 v\d+, s\[\d+:\d+\], \S+ offen lds", isa(src))
    monkeypatch.setenv("NEWT_BUFFER_DMA", "0")
    src0, _ = compile_source(W.matmul_kernel, _matmul_args(), cex, num_warps=4, num_stages=4)
    assert "lds_dma16_buf" not in src0 and "1073741824LL" not in src0


def test_fast_loop_fills_are_spaced_evenly_over_the_mfmas():
    """Interleave hints of the 4-wave 256x256x32 matmul's branch-free loop:
    each stage's 64 MFMAs (one 32-deep k-step of a 128x128 wave tile) carry
    its 8 copies and 24 next-stage fragment reads one after every second
    MFMA, copies and reads alternating while both remain."""
    src, _ = compile_source(W.matmul_kernel, _matmul_args(),
                            {"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": 32},
                            num_warps=4, num_stages=4)
    loops = [m.start() for m in re.finditer(r"for \(; _it\d+ ", src)]
    fast = src[loops[0]:loops[1]]
    seq = re.findall(r"sched_group_barrier\((0x\w+), 1, 0\)", fast)
    # 4 stages x (64 MFMAs + 32 fills), in the loop and in the clamped trip after it
    assert len(seq) == 2 * 4 * 96
    first = seq[:96]
    after = []
    for mask in first:
        if mask == "0x008":
            after.append([])
        else:
            after[-1].append(mask)
    assert len(after) == 64
    assert [len(a) for a in after] == [1, 0] * 32
    fills = [a[0] for a in after if a]
    assert fills[:16] == ["0x020", "0x100"] * 8 and fills[16:] == ["0x100"] * 16


def _attention_args():
    args = {n: (BF16P, A16) for n in ("q_ptr", "k_ptr", "v_ptr", "o_ptr")}
    args.update({"S": (tp.int32, D16), "H": (tp.int32, D16), "scale": tp.float32})
    for n in ("sqb", "sqh", "sqm", "skb", "skh", "skn", "svb", "svh", "svn", "sob", "soh", "som"):
        args[n] = (tp.int32, D16)
    return args


def test_matmul_tiles_are_stored_non_temporal(monkeypatch):
    """A matmul's C tile (column-oriented dot accumulator) is stored with the
    non-temporal hint (`global_store_short ... nt` on gfx950); attention's O
    (row-oriented accumulator) and a streaming row kernel (softmax) keep
    plain stores; NEWT_NT_STORE=0 turns the hint off."""
    mm = lambda: compile_source(W.matmul_kernel, _matmul_args(),
                                {"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": 32},
                                num_warps=4, num_stages=4)[0]
    src = mm()
    # 256 values per thread, in both the in-bounds and the masked branch
    assert src.count("__builtin_nontemporal_store(") == 2 * 256 * 256 // 256
    assert re.search(r"global_store_short v\[\d+:\d+\], v\d+, off nt", isa(src))
    asrc, _ = compile_source(W.attention_kernel, _attention_args(),
                             {"BLOCK_M": 128, "BLOCK_N": 64, "D": 128, "CAUSAL": False},
                             num_warps=4, num_stages=2)
    assert "newt::store_vec<__bf16, 4>(" in asrc and "nontemporal_store" not in asrc
    assert "store_vec_nt" not in asrc
    sm, _ = compile_source(W.softmax_kernel, {"x_ptr": (F32P, A16), "out_ptr": (F32P, A16),
                                              "N": (tp.int32, D16), "stride": (tp.int32, D16)},
                           {"BLOCK_N": 4096}, num_warps=4)
    assert "nontemporal_store" not in sm and "store_vec_nt" not in sm
    monkeypatch.setenv("NEWT_NT_STORE", "0")
    assert "nontemporal_store" not in mm()


def test_program_data_sharing_decides_order_and_hints(monkeypatch):
    """Streaming kernels (every load private to its program or common to all)
    keep the hardware's workgroup order; kernels whose programs share data
    with a subset of the others (a matmul's panels, an attention head's keys)
    are renumbered per XCD. NEWT_NT_LOAD=1 marks exactly the program-private
    top-level loads non-temporal (a layernorm's x, not its weights)."""
    import ast as _ast
    from newt_amd.compiler import _shares_across_programs, _streamed
    def parse(k):
        return fndef_of(k)[0]
    for k in (W.add_kernel, W.copy_kernel, W.softmax_kernel, W.layernorm_kernel):
        assert not _shares_across_programs(parse(k)), k
    for k in (W.matmul_kernel, W.attention_kernel, W.attention_plain_kernel):
        assert _shares_across_programs(parse(k)), k
        assert not _streamed(parse(k), ("load",)), k
    ln = parse(W.layernorm_kernel)
    streamed = _streamed(ln, ("load",))
    loads = [n for n in _ast.walk(ln) if isinstance(n, _ast.Call)
             and getattr(n.func, "attr", None) == "load"]
    names = {_ast.unparse(n.args[0]).split(" ")[0]: id(n) in streamed for n in loads}
    assert names == {"x_ptr": True, "w_ptr": False, "b_ptr": False}
    monkeypatch.setenv("NEWT_NT_LOAD", "1")
    src, _ = compile_source(W.layernorm_kernel, {
        "x_ptr": (F16P, A16), "w_ptr": (F16P, A16), "b_ptr": (F16P, A16), "out_ptr": (F16P, A16),
        "mean_ptr": (F32P, A16), "rstd_ptr": (F32P, A16), "N": tp.int32, "stride": tp.int32,
        "eps": tp.float32}, {"BLOCK_N": 8192})
    assert "newt::load_vec_nt<_Float16, 8>((_p" in src
    assert "newt::load_vec<_Float16, 8>((w_ptr" in src and "newt::load_vec<_Float16, 8>((b_ptr" in src
    assert re.search(r"global_load_dwordx4 .* nt", isa(src))
    monkeypatch.delenv("NEWT_NT_LOAD")

    def loop_reread(x_ptr, o_ptr, BLOCK: nl.constexpr):
        row = nl.program_id(0)
        acc = nl.zeros((BLOCK,), dtype=nl.float32)
        for i in range(4):
            acc += nl.load(x_ptr + row * BLOCK + nl.arange(0, BLOCK))
        nl.store(o_ptr + row * BLOCK + nl.arange(0, BLOCK), acc)
    fd = _ast.parse(textwrap.dedent(inspect.getsource(loop_reread))).body[0]
    assert not _streamed(fd, ("load",))          # re-read in a loop: keep cached
    assert _shares_across_programs(fd)           # a load in a loop: keep the XCD order


LN_ARGS = {"x_ptr": (F16P, A16), "w_ptr": (F16P, A16), "b_ptr": (F16P, A16),
           "out_ptr": (F16P, A16), "mean_ptr": (F32P, A16), "rstd_ptr": (F32P, A16),
           "N": (tp.int32, D16), "stride": (tp.int32, D16), "eps": tp.float32}


def test_repeated_binop_is_computed_once(monkeypatch):
    """layernorm writes `x - mean` for the variance and again for the output:
    the second use takes the first block's registers (x - mean is evaluated
    once per element), and NEWT_CSE=0 restores the recomputation (counted
    in the body as generated, without the whole-body versioning copy)."""
    monkeypatch.setenv("NEWT_VERSION_BODY", "0")
    sub = re.compile(r"= \(\(\(float\)\(_r\d+\[0\]\)\) - _t\d+\);")
    src, _ = compile_source(W.layernorm_kernel, LN_ARGS, {"BLOCK_N": 8192})
    assert len(sub.findall(src)) == 1
    isa(src)
    monkeypatch.setenv("NEWT_CSE", "0")
    src0, _ = compile_source(W.layernorm_kernel, LN_ARGS, {"BLOCK_N": 8192})
    assert len(sub.findall(src0)) == 2


def test_reuse_respects_c_scopes():
    """A block computed inside a runtime `if` (or a loop body) is not visible
    after it: the same expression there is computed again, and the source
    builds. Values read from loop-carried storage are never reused across a
    write of that storage."""
    def k(x_ptr, o_ptr, flag, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        x = nl.load(x_ptr + offs)
        y = x * 0.0
        if flag > 0:
            y = x * 3.0
        z = x * 3.0
        acc = x * 1.0
        for i in range(3):
            acc = acc * 2.0
            t = acc * 2.0
            acc = t + 1.0
        nl.store(o_ptr + offs, y + z + acc)
    src, _ = compile_source(k, {"x_ptr": (F32P, A16), "o_ptr": (F32P, A16), "flag": tp.int32},
                            {"BLOCK": 256})
    mul3 = re.findall(r"\* 3\.0f\)", src)
    assert len(mul3) >= 2            # once in the branch, once after it
    assert len(re.findall(r"\* 2\.0f\)", src)) >= 2   # both products of the loop body
    isa(src)


def test_fast_loop_runs_the_last_trips_with_repeated_copies(monkeypatch):
    """When every iteration is fast, one more branch-free trip follows the
    fast loop: its copies past the end repeat the last tile (clamped loop
    variable), the carried pointers stop on it, and the copies are drained
    after the loops. The fast loop itself is unchanged; NEWT_PIPE_CLAMP=0
    drops the extra trip."""
    cex = {"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": 32}
    src, _ = compile_source(W.matmul_kernel, _matmul_args(), cex, num_warps=4, num_stages=4)
    loops = [m.start() for m in re.finditer(r"for \(; _it\d+ ", src)]
    assert len(loops) == 2
    m = re.search(r"if \(\(\((_t\d+)\) == \((_t\d+)\)\) && (_it\d+) \+ 3 < \2\) \{", src)
    assert m and loops[0] < m.start() < loops[1], "one clamped trip between the loops"
    trip = src[m.start():loops[1]]
    assert trip.count("newt::lds_dma16_buf(") == 32
    assert re.search(r"if \(\(\(_it\d+ \+ 0\) \+ 3\) < _t\d+ - 1\) \{", trip)
    assert f"{m.group(3)} += 4;" in trip
    fast = src[loops[0]:m.start()]
    assert "- 1) ?" not in fast and " - 1) {" not in fast    # no clamping in the loop
    assert "newt::wait_vmcnt<0>();" in src[loops[1]:]
    monkeypatch.setenv("NEWT_PIPE_CLAMP", "0")
    src0, _ = compile_source(W.matmul_kernel, _matmul_args(), cex, num_warps=4, num_stages=4)
    assert not re.search(r"\) && _it\d+ \+ 3 < ", src0)


def test_layout_hints_before_pipeline_fallback():
    """A first pass whose layout conversions push the LDS past 160 KB (flash
    attention with 64 query rows per wave: its accumulator starts in a blocked
    layout) is retried with the layouts it learned before the dot pipeline gives
    up a stage or falls back to synchronous staging: the kernel keeps its two
    direct-to-LDS stages and needs no conversion arena."""
    args = {n: (BF16P, A16) for n in ("q_ptr", "k_ptr", "v_ptr", "o_ptr")}
    args.update({"S": (tp.int32, D16), "H": (tp.int32, D16), "scale": tp.float32})
    for n in ("sqb", "sqh", "sqm", "skb", "skh", "skn", "svb", "svh", "svn", "sob", "soh", "som"):
        args[n] = (tp.int32, D16)
    src, lds = compile_source(W.attention_kernel, args,
                              {"BLOCK_M": 256, "BLOCK_N": 32, "D": 128, "CAUSAL": False},
                              num_warps=4, num_stages=2, waves_per_eu=1)
    assert lds < 2 * 16384 + 1024 and "lds_dma16_buf" in src


def test_bench_timeline_source_compiles():
    """bench.py --timeline instruments the headline matmul's generated source
    (real-time counter reads at the start, before the first C store and at the
    end, written with the XCC id through one more pointer parameter): the
    instrumented copy must still build for gfx950."""
    import bench
    src, _ = compile_source(W.matmul_kernel, _matmul_args(F16P),
                            {"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": 32}, num_warps=4,
                            num_stages=4)
    inst = bench.timeline_source(src)
    assert inst.count("s_memrealtime") == 3 and "_ts[_tsw_wg * 4 + 3]" in inst
    assert "s_memrealtime" in isa(inst)


def test_whole_body_versioning(monkeypatch):
    """A small loop-free kernel whose masked accesses share one uniform
    in-bounds test over scalar arguments is emitted twice: `if (test) { body,
    test folded to true } else { body }`. The fallback is the body as
    generated; the fast copy keeps the masked branches only as dead code.
    Tests over per-program values (vector add), bodies with loops, bodies over
    the size limit and NEWT_VERSION_BODY=0 keep the single body."""
    src, _ = compile_source(W.layernorm_kernel, LN_ARGS, {"BLOCK_N": 8192}, num_warps=8)
    lines = src.split("\n")
    # the first statement after the LDS declarations is the version test; the
    # lane index arithmetic is inside both copies
    i = next(i for i, ln in enumerate(lines) if re.match(r"^  if \(.*\) \{$", ln))
    assert "__shared__" in lines[i - 1] and "_tid" in lines[i + 1]
    cond = re.match(r"^  if \((.*)\) \{$", lines[i]).group(1)
    j = lines.index("  } else {", i)
    fast, slow = "\n".join(lines[i + 1:j]), "\n".join(lines[j + 1:])
    assert set(re.findall(r"[A-Za-z_]\w*", cond)) == {"N"}
    assert cond not in fast and fast.count("if ((true)) {") == slow.count(f"if ({cond})") >= 2
    asm = isa(src)
    assert "global_load_dwordx4" in asm and "global_store_dwordx4" in asm

    monkeypatch.setenv("NEWT_VERSION_BODY", "0")
    src0, _ = compile_source(W.layernorm_kernel, LN_ARGS, {"BLOCK_N": 8192}, num_warps=8)
    assert "if ((true))" not in src0 and src0.count(f"if ({cond})") == slow.count(f"if ({cond})")
    monkeypatch.delenv("NEWT_VERSION_BODY")

    # the add kernel's test is over the program's first element: one body
    assert "if ((true))" not in compile_source(W.add_kernel, ADD_ARGS, {"BLOCK": 1024})[0]

    # a loop in the body: one body
    def k(x_ptr, o_ptr, n, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        acc = nl.zeros((BLOCK,), dtype=nl.float32)
        for i in range(0, 4):
            acc += nl.load(x_ptr + i * n + offs, mask=offs < n, other=0.0)
        nl.store(o_ptr + offs, acc, mask=offs < n)
    args = {"x_ptr": (F32P, A16), "o_ptr": (F32P, A16), "n": tp.int32}
    assert "if ((true))" not in compile_source(k, args, {"BLOCK": 256})[0]

    # a body over the size limit: one body
    def big(x_ptr, o_ptr, n, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        x = nl.load(x_ptr + offs, mask=offs < n, other=0.0)
        nl.store(o_ptr + offs, x * 2.0, mask=offs < n)
    small_src = compile_source(big, args, {"BLOCK": 1024})[0]
    assert "if ((true))" in small_src
    assert "if ((true))" not in compile_source(big, args, {"BLOCK": 1 << 16}, num_warps=1)[0]


def test_whole_body_versioning_leaves_runtime_ifs_alone():
    """A runtime `if` on a scalar argument evaluates its test into a per-program
    temporary first, so repeated user tests are not taken for the in-bounds test
    and the body stays single; the masked accesses' own test still versions it,
    and the user's tests keep their text in both copies."""
    def k(x_ptr, o_ptr, m, n, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        x = nl.load(x_ptr + offs)
        if n > 0:
            x = x + 1.0
        if n > 0:
            x = x * 2.0
        nl.store(o_ptr + offs, x + (m + n > 0))
    args = {"x_ptr": (F32P, A16), "o_ptr": (F32P, A16), "m": tp.int32, "n": tp.int32}
    src = compile_source(k, args, {"BLOCK": 256})[0]
    assert "if ((true))" not in src and src.count("(n > 0)") == 2
    isa(src)

    def km(x_ptr, o_ptr, n, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        x = nl.load(x_ptr + offs, mask=offs < n, other=0.0)
        if n > 8:
            x = x + 1.0
        nl.store(o_ptr + offs, x, mask=offs < n)
    args = {"x_ptr": (F32P, A16), "o_ptr": (F32P, A16), "n": tp.int32}
    src = compile_source(km, args, {"BLOCK": 256})[0]
    assert src.count("if ((true)) {") == 2 and src.count("(n > 8)") == 2
    isa(src)
