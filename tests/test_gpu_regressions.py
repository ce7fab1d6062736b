"""Regression cases of the reference's review-fix suite (tests/test_review_fixes.py)
that need a launch, with the same known answers:
  values defined inside a loop / both branches of an if, read after it    :12-40
  `prev = x` inside a loop is a copy, not an alias                        :43-58
  two loops reusing one target name (here: the second is not loop-carried)
  bool max / sum give "any" and a count (1 and 3; 0 and 0)               :85-100
  an atomic through a scalar pointer fires once per program (10.0)        :103-111
  float atomic_max over 4 programs == x.max()                             :114-124
  autotune with reset_to_zero does not double-accumulate while tuning     :127-143
  a grid callable sees the runtime arguments in META                      :146-157
  an empty grid is a no-op                                                :160-169
  constants adopt the block dtype: uint8 200+200 = 144,
  fp16 3*0.1 = 0.299804688                                                :215-235
  broadcast_to of a uniform scalar                                        :238-247
  `other` may itself be a loaded block                                    :250-263
  uint32 tensors                                                          :276-285
  a name carried by a loop inside a runtime if and assigned again after it
The compile-time rejections of the same suite run on the CPU
(test_language_errors_cpu.py).
"""

import pytest
import torch

import newt
import newt.language as nl

pytestmark = pytest.mark.gpu


def test_value_defined_in_loop_is_read_after_it():
    @newt.jit
    def k(x_ptr, y_ptr, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        for i in range(2):
            t = nl.load(x_ptr + offs) + i
        nl.store(y_ptr + offs, t)

    x = torch.randn(64, device="cuda")
    y = torch.empty_like(x)
    k[(1,)](x, y, BLOCK=64)
    assert torch.equal(y, x + 1)


def test_value_defined_in_both_branches():
    @newt.jit
    def k(x_ptr, y_ptr, flag, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        if flag == 1:
            t = nl.load(x_ptr + offs) * 2
        else:
            t = nl.load(x_ptr + offs) * 3
        nl.store(y_ptr + offs, t)

    x = torch.randn(64, device="cuda")
    y = torch.empty_like(x)
    k[(1,)](x, y, 1, BLOCK=64)
    assert torch.equal(y, x * 2)
    k[(1,)](x, y, 0, BLOCK=64)
    assert torch.equal(y, x * 3)


def test_two_loops_share_a_target_name():
    @newt.jit
    def k(x_ptr, o_ptr, n, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        acc = nl.zeros((BLOCK,), dtype=nl.float32)
        for i in range(0, n, 2):
            acc = acc + nl.load(x_ptr + i * BLOCK + offs)
        for i in range(1, n, 2):
            acc = acc - nl.load(x_ptr + i * BLOCK + offs)
        nl.store(o_ptr + offs, acc)

    x = torch.randn(7, 64, device="cuda")
    o = torch.empty(64, device="cuda")
    k[(1,)](x, o, 7, BLOCK=64)
    torch.testing.assert_close(o, x[0::2].sum(0) - x[1::2].sum(0), rtol=1e-5, atol=1e-5)


def test_copy_in_loop_does_not_alias():
    @newt.jit
    def k(x_ptr, out_ptr, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        x = nl.load(x_ptr + offs)
        for i in range(2):
            prev = x
            x = x + 1.0
            nl.store(out_ptr + i * BLOCK + offs, prev)

    x = torch.zeros(64, device="cuda")
    out = torch.empty(128, device="cuda")
    k[(1,)](x, out, BLOCK=64)
    assert bool((out[:64] == 0.0).all()) and bool((out[64:] == 1.0).all())


def test_bool_reductions():
    @newt.jit
    def k(x_ptr, y_ptr, BLOCK: nl.constexpr):
        hit = nl.load(x_ptr + nl.arange(0, BLOCK)) > 100.0
        nl.store(y_ptr, nl.max(hit).to(nl.int32))
        nl.store(y_ptr + 1, nl.sum(hit).to(nl.int32))

    x = torch.zeros(64, device="cuda")
    x[[3, 10, 40]] = 200.0
    y = torch.empty(2, device="cuda", dtype=torch.int32)
    k[(1,)](x, y, BLOCK=64)
    assert y.tolist() == [1, 3]
    x.zero_()
    k[(1,)](x, y, BLOCK=64)
    assert y.tolist() == [0, 0]


@pytest.mark.parametrize("waves", [1, 4, 16])
def test_scalar_atomic_once_per_program(waves):
    @newt.jit
    def k(out_ptr):
        nl.atomic_add(out_ptr, 1.0)

    o = torch.zeros(1, device="cuda")
    k[(10,)](o, num_warps=waves)
    torch.cuda.synchronize()
    assert o.item() == 10.0


def test_float_atomic_max():
    @newt.jit
    def k(x_ptr, out_ptr, BLOCK: nl.constexpr):
        offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
        nl.atomic_max(out_ptr, nl.max(nl.load(x_ptr + offs)))

    x = torch.randn(4096, device="cuda")
    o = torch.full((1,), float("-inf"), device="cuda")
    k[(4,)](x, o, BLOCK=1024)
    torch.cuda.synchronize()
    assert o.item() == x.max().item()


def test_float_atomic_max_all_negative():
    @newt.jit
    def k(x_ptr, out_ptr, BLOCK: nl.constexpr):
        offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
        nl.atomic_max(out_ptr, nl.max(nl.load(x_ptr + offs)))

    x = -torch.rand(2048, device="cuda") - 1.0
    o = torch.full((1,), float("-inf"), device="cuda")
    k[(8,)](x, o, BLOCK=256)
    torch.cuda.synchronize()
    assert o.item() == x.max().item()


def test_autotune_reset_to_zero_on_first_call():
    @newt.autotune(configs=[newt.Config({"BLOCK": 64}), newt.Config({"BLOCK": 64}, num_warps=2)],
                   key=["n"], reset_to_zero=["out_ptr"])
    @newt.jit
    def rmw(x_ptr, out_ptr, n, BLOCK: nl.constexpr):
        offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
        live = offs < n
        cur = nl.load(out_ptr + offs, mask=live)
        nl.store(out_ptr + offs, cur + nl.load(x_ptr + offs, mask=live), mask=live)

    x = torch.ones(256, device="cuda")
    out = torch.zeros(256, device="cuda")
    rmw[lambda meta: (newt.cdiv(256, meta["BLOCK"]),)](x, out, 256)
    torch.cuda.synchronize()
    assert bool((out == 1.0).all())


def test_grid_callable_sees_runtime_arguments():
    @newt.jit
    def k(x_ptr, y_ptr, n, BLOCK: nl.constexpr):
        offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
        live = offs < n
        nl.store(y_ptr + offs, nl.load(x_ptr + offs, mask=live) + 1, mask=live)

    seen = {}

    def grid(meta):
        seen.update(meta)
        return (newt.cdiv(meta["n"], meta["BLOCK"]),)

    x = torch.randn(1000, device="cuda")
    y = torch.empty_like(x)
    k[grid](x, y, 1000, BLOCK=256)
    assert torch.equal(y, x + 1)
    assert seen["n"] == 1000 and seen["BLOCK"] == 256 and seen["num_warps"] == 4


@pytest.mark.parametrize("grid", [(0,), (0, 4), (3, 0, 1), 0])
def test_empty_grid_is_noop(grid):
    @newt.jit
    def k(x_ptr, BLOCK: nl.constexpr):
        nl.store(x_ptr + nl.arange(0, BLOCK), 1.0)

    x = torch.zeros(64, device="cuda")
    k[grid](x, BLOCK=64)
    torch.cuda.synchronize()
    assert bool((x == 0).all())


def test_int_constant_adopts_uint8():
    @newt.jit
    def k(a_ptr, o_ptr, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        nl.store(o_ptr + offs, nl.load(a_ptr + offs) + 200)

    a = torch.full((64,), 200, device="cuda", dtype=torch.uint8)
    o = torch.empty_like(a)
    k[(1,)](a, o, BLOCK=64)
    assert bool((o == 144).all())


def test_float_constant_rounds_to_fp16():
    @newt.jit
    def k(a_ptr, o_ptr, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        nl.store(o_ptr + offs, nl.load(a_ptr + offs) * 0.1)

    a = torch.full((64,), 3.0, device="cuda", dtype=torch.float16)
    o = torch.empty(64, device="cuda")
    k[(1,)](a, o, BLOCK=64)
    # fp16(0.1) * 3 rounded to fp16 = 0.299804688, not fp32's 0.300000012
    assert abs(o[0].item() - 0.299804688) < 1e-6


def test_broadcast_to_of_uniform_scalar():
    @newt.jit
    def k(x_ptr, y_ptr, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        s = nl.sum(nl.load(x_ptr + offs))
        nl.store(y_ptr + offs, nl.broadcast_to(s, (BLOCK,)))

    x = torch.ones(64, device="cuda")
    y = torch.empty(64, device="cuda")
    k[(1,)](x, y, BLOCK=64)
    assert bool((y == 64.0).all())


def test_other_from_a_loaded_block():
    @newt.jit
    def k(p_ptr, q_ptr, y_ptr, n, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        fallback = nl.load(q_ptr + offs)
        v = nl.load(p_ptr + offs, mask=offs < n, other=fallback)
        nl.store(y_ptr + offs, v)

    p = torch.ones(64, device="cuda")
    q = torch.full((64,), 5.0, device="cuda")
    y = torch.empty(64, device="cuda")
    k[(1,)](p, q, y, 4, BLOCK=64)
    assert bool((y[:4] == 1.0).all()) and bool((y[4:] == 5.0).all())


def test_uint32_tensors():
    @newt.jit
    def k(x_ptr, y_ptr, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        nl.store(y_ptr + offs, nl.load(x_ptr + offs) + 1)

    x = torch.zeros(64, device="cuda", dtype=torch.uint32)
    y = torch.empty_like(x)
    k[(1,)](x, y, BLOCK=64)
    assert int(y[0]) == 1 and int(y[63]) == 1


def test_cpu_tensor_rejected():
    @newt.jit
    def k(x_ptr, BLOCK: nl.constexpr):
        nl.store(x_ptr + nl.arange(0, BLOCK), 1.0)

    with pytest.raises(TypeError, match="GPU tensor"):
        k[(1,)](torch.zeros(64), BLOCK=64)


def test_name_carried_by_a_loop_inside_a_runtime_if_then_reassigned():
    """A name first defined inside a runtime `if`, carried by a loop nested in
    it, and assigned again after the `if`: the loop's storage is scoped to the
    `if` block, and the later assignment starts a fresh value (the generated
    source used to write the out-of-scope storage and failed to compile)."""
    @newt.jit
    def k(x_ptr, o_ptr, n, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        acc = nl.zeros((BLOCK,), dtype=nl.float32)
        if n > 0:
            t = nl.load(x_ptr + offs)
            for i in range(1, n):
                t = t + nl.load(x_ptr + offs + i)
            acc = acc + t
        t = nl.load(x_ptr + offs) * 2.0
        nl.store(o_ptr + offs, acc + t)

    x = torch.randn(300, device="cuda")
    for n in (0, 1, 4):
        o = torch.empty(256, device="cuda")
        k[(1,)](x, o, n, BLOCK=256)
        want = x[:256] * 2.0
        if n > 0:
            want = want + sum(x[i:i + 256] for i in range(n))
        torch.testing.assert_close(o, want, rtol=1e-5, atol=1e-5)
