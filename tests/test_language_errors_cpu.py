"""Compile-time rejections and host-side argument checks, on the CPU.

The same programs the reference rejects, with the same error class and the
message fragment its tests match (tests/test_review_fixes.py,
tests/test_control_flow.py):
  nl.static_assert failing with its message               test_control_flow.py:156-165
  a block-valued `if` condition ("scalar")                test_control_flow.py:168-180
  dot operands reused after a store ("consumed")          test_review_fixes.py:61-82
  a scalar pointer with a block mask ("scalar pointer")   test_review_fixes.py:172-183
  a loop-carried pointer rebased to another tensor ("base") :186-201
  int loop-carried storage updated with a float ("float")  :204-212
  unknown keyword / too many positional arguments          :266-273
  constexpr host arithmetic                                :288-292
No GPU is needed: compile_fn is a pure function of the kernel AST, the
argument types and the constexprs.
"""

import ast
import inspect
import textwrap

import pytest
import torch

import newt
import newt_amd.language as nl
from newt_amd.compiler import CompileError, Param, compile_fn
from newt_amd.compiler import types as tp

F32P = tp.pointer_type(tp.float32)
F16P = tp.pointer_type(tp.float16)


def compile_k(fn, args, constexprs, num_warps=4):
    fndef = ast.parse(textwrap.dedent(inspect.getsource(fn))).body[0]
    params = [(n, Param(t, n)) for n, t in args.items()]
    return compile_fn(fndef, fn.__globals__, params, constexprs, num_warps, "k")


def test_static_assert_message():
    def k(o_ptr, BLOCK: nl.constexpr):
        nl.static_assert(BLOCK >= 128, "BLOCK too small")
        nl.store(o_ptr + nl.arange(0, BLOCK), 1.0)

    with pytest.raises(CompileError, match="BLOCK too small"):
        compile_k(k, {"o_ptr": F32P}, {"BLOCK": 64})
    compile_k(k, {"o_ptr": F32P}, {"BLOCK": 128})


def test_block_condition_rejected():
    def k(x_ptr, o_ptr, BLOCK: nl.constexpr):
        x = nl.load(x_ptr + nl.arange(0, BLOCK))
        if x > 0:
            nl.store(o_ptr, 1.0)

    with pytest.raises(CompileError, match="scalar"):
        compile_k(k, {"x_ptr": F32P, "o_ptr": F32P}, {"BLOCK": 64})


def test_dot_operand_reused_after_store_rejected():
    def k(x_ptr, y_ptr, c1_ptr, c2_ptr, N: nl.constexpr):
        r = nl.arange(0, N)
        idx = r[:, None] * N + r[None, :]
        x = nl.load(x_ptr + idx)
        y = nl.load(y_ptr + idx)
        nl.store(c1_ptr + idx, nl.dot(x, y))
        nl.store(x_ptr + idx, nl.zeros((N, N), dtype=nl.float16))
        nl.store(c2_ptr + idx, nl.dot(x, y))

    with pytest.raises(CompileError, match="consumed"):
        compile_k(k, {"x_ptr": F16P, "y_ptr": F16P, "c1_ptr": F32P, "c2_ptr": F32P}, {"N": 32})


def test_dot_operand_reused_without_store_is_fine():
    def k(x_ptr, y_ptr, c1_ptr, c2_ptr, N: nl.constexpr):
        r = nl.arange(0, N)
        idx = r[:, None] * N + r[None, :]
        x = nl.load(x_ptr + idx)
        y = nl.load(y_ptr + idx)
        c1 = nl.dot(x, y)
        c2 = nl.dot(x, y) * 2.0
        nl.store(c1_ptr + idx, c1)
        nl.store(c2_ptr + idx, c2)

    compile_k(k, {"x_ptr": F16P, "y_ptr": F16P, "c1_ptr": F32P, "c2_ptr": F32P}, {"N": 32})


def test_scalar_pointer_with_block_mask_rejected():
    def k(x_ptr, y_ptr, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        v = nl.load(x_ptr, mask=offs < 4, other=7.0)
        nl.store(y_ptr + offs, nl.zeros((BLOCK,), dtype=nl.float32) + v)

    with pytest.raises(CompileError, match="scalar pointer"):
        compile_k(k, {"x_ptr": F32P, "y_ptr": F32P}, {"BLOCK": 64})


def test_pointer_rebased_in_loop_rejected():
    def k(a_ptr, b_ptr, out_ptr, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        p = a_ptr + offs
        for i in range(2):
            nl.store(out_ptr + i * BLOCK + offs, nl.load(p))
            p = b_ptr + offs

    with pytest.raises(CompileError, match="base"):
        compile_k(k, {"a_ptr": F32P, "b_ptr": F32P, "out_ptr": F32P}, {"BLOCK": 64})


def test_int_storage_updated_with_float_rejected():
    def k(y_ptr, ITERS: nl.constexpr):
        s = 0
        for i in range(ITERS):
            s = s + 0.5
        nl.store(y_ptr, s)

    with pytest.raises(CompileError, match="float"):
        compile_k(k, {"y_ptr": F32P}, {"ITERS": 3})


def test_return_value_and_unsupported_syntax_rejected():
    def k(x_ptr):
        return 1

    with pytest.raises(CompileError, match="return"):
        compile_k(k, {"x_ptr": F32P}, {})


def test_unknown_and_surplus_arguments():
    @newt.jit
    def k(x_ptr, BLOCK: nl.constexpr):
        nl.store(x_ptr + nl.arange(0, BLOCK), 1.0)

    x = torch.zeros(64)
    with pytest.raises(TypeError, match="unknown"):
        k[(1,)](x, BLOCK=64, BLOK=128)
    with pytest.raises(TypeError, match="arguments"):
        k[(1,)](x, 64, 999)


def test_launch_requires_a_grid():
    @newt.jit
    def k(x_ptr, BLOCK: nl.constexpr):
        nl.store(x_ptr + nl.arange(0, BLOCK), 1.0)

    with pytest.raises(RuntimeError, match="grid"):
        k(torch.zeros(64), BLOCK=64)


@pytest.mark.parametrize("warps,stages", [(3, 3), (32, 3), (4, 0), (4, 9)])
def test_launch_options_validated(warps, stages):
    @newt.jit
    def k(x_ptr, BLOCK: nl.constexpr):
        nl.store(x_ptr + nl.arange(0, BLOCK), 1.0)

    with pytest.raises(ValueError):
        k[(1,)](torch.zeros(64), BLOCK=64, num_warps=warps, num_stages=stages)


def test_constexpr_host_arithmetic():
    c = nl.constexpr(64)
    assert (c * 2).value == 128
    assert int(c) == 64
    assert c == 64
    assert c + 1 == 65 and c // 2 == 32 and 100 - c == 36


def test_launch_fast_path_tracks_specialization(monkeypatch):
    """The launch fast path is keyed on everything the slow path specializes
    on: a call differing in an int's ==1 / divisibility, a constexpr value, a
    launch option or a codegen switch must not reuse another call's kernel."""

    @newt.jit
    def k(x_ptr, n, BLOCK: nl.constexpr):
        nl.store(x_ptr + nl.arange(0, BLOCK), 1.0, mask=nl.arange(0, BLOCK) < n)

    x = torch.zeros(64)
    sig = lambda *a, **kw: k._call_signature(a, kw, (4, 3, 0))
    base = sig(x, 64, BLOCK=64)
    assert sig(x, 64, BLOCK=64) == base
    assert sig(x, 1, BLOCK=64) != base           # n == 1 specializes
    assert sig(x, 48, BLOCK=64) == base          # both divisible by 16: same kernel
    assert sig(x, 24, BLOCK=64) != base          # divisible by 8 only
    assert sig(x, 64, BLOCK=128) != base         # constexpr value
    assert sig(x, 1 << 40, BLOCK=64) != base     # int64 argument
    assert k._call_signature((x, 64), {"BLOCK": 64}, (8, 3, 0)) != base
    monkeypatch.setenv("NEWT_PID_REMAP", "0")
    assert sig(x, 64, BLOCK=64) != base
