"""Control flow, constexpr specialization, grids, autotuning and edge shapes on
the GPU, with the known answers of the reference's suite
(tests/test_control_flow.py):
  runtime loop accumulation; constexpr range sum 0+2+4+6+8 = 20          :16-43
  scalar loop-carried sum of squares = 285; pointer walk                  :46-74
  nested loops with break/continue; while doubling to 128                 :77-113
  runtime if/else; constexpr branch pruning                               :120-153
  3D grid -> arange; num_programs == 7                                    :187-210
  autotune picks a config; heuristics; 4 cache entries for 2x2            :217-268
  int64 argument 2**40 / 2**32 == 256                                     :271-279
  blocks smaller than the workgroup; n == 1; tuple unpacking              :286-319
"""

import pytest
import torch

import newt
import newt.language as nl

pytestmark = pytest.mark.gpu


def test_loop_accumulates_tiles():
    @newt.jit
    def k(x_ptr, o_ptr, n_iter, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        acc = nl.zeros((BLOCK,), dtype=nl.float32)
        for i in range(n_iter):
            acc = acc + nl.load(x_ptr + i * BLOCK + offs)
        nl.store(o_ptr + offs, acc)

    x = torch.randn(7 * 256, device="cuda")
    o = torch.empty(256, device="cuda")
    k[(1,)](x, o, 7, BLOCK=256)
    torch.testing.assert_close(o, x.view(7, 256).sum(0), rtol=1e-5, atol=1e-5)


def test_constexpr_range_with_step():
    @newt.jit
    def k(o_ptr, N: nl.constexpr, BLOCK: nl.constexpr):
        acc = nl.zeros((BLOCK,), dtype=nl.int32)
        for i in range(0, N, 2):
            acc = acc + i
        nl.store(o_ptr + nl.arange(0, BLOCK), acc)

    o = torch.empty(64, device="cuda", dtype=torch.int32)
    k[(1,)](o, N=10, BLOCK=64)
    assert bool((o == 20).all())


def test_scalar_carried_through_runtime_loop():
    @newt.jit
    def k(o_ptr, n, BLOCK: nl.constexpr):
        s = 0
        for i in range(n):
            s = s + i * i
        nl.store(o_ptr + nl.arange(0, BLOCK), nl.zeros((BLOCK,), dtype=nl.int32) + s)

    o = torch.empty(32, device="cuda", dtype=torch.int32)
    k[(1,)](o, 10, BLOCK=32)
    assert bool((o == 285).all())


def test_pointer_advanced_in_loop():
    @newt.jit
    def k(x_ptr, o_ptr, n_tiles, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        p = x_ptr + offs
        acc = nl.zeros((BLOCK,), dtype=nl.float32)
        for i in range(n_tiles):
            acc = acc + nl.load(p)
            p += BLOCK
        nl.store(o_ptr + offs, acc)

    x = torch.randn(5 * 512, device="cuda")
    o = torch.empty(512, device="cuda")
    k[(1,)](x, o, 5, BLOCK=512)
    torch.testing.assert_close(o, x.view(5, 512).sum(0), rtol=1e-5, atol=1e-5)


def test_break_and_continue_in_nested_loops():
    @newt.jit
    def k(o_ptr, BLOCK: nl.constexpr):
        s = 0
        for i in range(10):
            if i == 7:
                break
            if i % 2 == 1:
                continue
            for j in range(3):
                s = s + i + j
        nl.store(o_ptr + nl.arange(0, BLOCK), nl.zeros((BLOCK,), dtype=nl.int32) + s)

    want = sum(i + j for i in range(7) if i % 2 == 0 for j in range(3))
    o = torch.empty(32, device="cuda", dtype=torch.int32)
    k[(1,)](o, BLOCK=32)
    assert bool((o == want).all())


def test_while_doubles_past_bound():
    @newt.jit
    def k(o_ptr, n, BLOCK: nl.constexpr):
        v = 1
        while v < n:
            v = v * 2
        nl.store(o_ptr + nl.arange(0, BLOCK), nl.zeros((BLOCK,), dtype=nl.int32) + v)

    o = torch.empty(32, device="cuda", dtype=torch.int32)
    for n, want in ((100, 128), (1, 1), (128, 128), (129, 256)):
        k[(1,)](o, n, BLOCK=32)
        assert bool((o == want).all()), n


def test_runtime_if_else():
    @newt.jit
    def k(x_ptr, o_ptr, flag, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        x = nl.load(x_ptr + offs)
        y = nl.zeros((BLOCK,), dtype=nl.float32)
        if flag == 1:
            y = x * 2
        else:
            y = x * 3
        nl.store(o_ptr + offs, y)

    x = torch.randn(128, device="cuda")
    o = torch.empty_like(x)
    k[(1,)](x, o, 1, BLOCK=128)
    assert torch.equal(o, x * 2)
    k[(1,)](x, o, 0, BLOCK=128)
    assert torch.equal(o, x * 3)


def test_constexpr_if_prunes_the_other_branch():
    @newt.jit
    def k(x_ptr, o_ptr, MODE: nl.constexpr, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        x = nl.load(x_ptr + offs)
        if MODE == "double":
            r = x * 2
        else:
            r = nl.exp(x)
        nl.store(o_ptr + offs, r)

    x = torch.randn(64, device="cuda")
    o = torch.empty_like(x)
    k[(1,)](x, o, MODE="double", BLOCK=64)
    assert torch.equal(o, x * 2)
    assert "exp" not in next(iter(k.cache.values())).source.split("{", 1)[1]
    k[(1,)](x, o, MODE="exp", BLOCK=64)
    torch.testing.assert_close(o, torch.exp(x), rtol=1e-6, atol=1e-6)


def test_3d_grid_program_ids():
    @newt.jit
    def k(o_ptr, GX: nl.constexpr, GY: nl.constexpr):
        idx = (nl.program_id(2) * GY + nl.program_id(1)) * GX + nl.program_id(0)
        nl.store(o_ptr + idx, idx.to(nl.float32))

    o = torch.empty(4 * 3 * 2, device="cuda")
    k[(4, 3, 2)](o, GX=4, GY=3)
    assert torch.equal(o, torch.arange(24, device="cuda").float())


def test_num_programs_per_axis():
    @newt.jit
    def k(o_ptr):
        flat = (nl.program_id(1) * nl.num_programs(0) + nl.program_id(0)) * 2
        nl.store(o_ptr + flat, nl.num_programs(0).to(nl.float32))
        nl.store(o_ptr + flat + 1, nl.num_programs(1).to(nl.float32))

    o = torch.empty(7 * 3 * 2, device="cuda")
    k[(7, 3)](o)
    assert bool((o[0::2] == 7).all()) and bool((o[1::2] == 3).all())


def test_autotune_chooses_and_caches():
    @newt.autotune(configs=[newt.Config({"BLOCK": 256}, num_warps=2),
                            newt.Config({"BLOCK": 1024}, num_warps=4),
                            newt.Config({"BLOCK": 4096}, num_warps=8)],
                   key=["n"])
    @newt.jit
    def k(x_ptr, o_ptr, n, BLOCK: nl.constexpr):
        offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
        live = offs < n
        nl.store(o_ptr + offs, nl.load(x_ptr + offs, mask=live) + 1, mask=live)

    n = 1 << 20
    x = torch.randn(n, device="cuda")
    o = torch.empty_like(x)
    k[lambda meta: (newt.cdiv(n, meta["BLOCK"]),)](x, o, n)
    assert torch.equal(o, x + 1)
    assert k.best_config is not None
    o.zero_()
    k[lambda meta: (newt.cdiv(n, meta["BLOCK"]),)](x, o, n)    # cached choice
    assert torch.equal(o, x + 1)


def test_heuristics_derive_constexprs():
    @newt.heuristics({"BLOCK": lambda args: newt.next_power_of_2(min(args["n"], 1024))})
    @newt.jit
    def k(x_ptr, o_ptr, n, BLOCK: nl.constexpr):
        offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
        live = offs < n
        nl.store(o_ptr + offs, nl.load(x_ptr + offs, mask=live) * 5, mask=live)

    for n in (100, 5000):
        x = torch.randn(n, device="cuda")
        o = torch.empty_like(x)
        k[lambda meta: (newt.cdiv(n, meta["BLOCK"]),)](x, o, n)
        assert torch.equal(o, x * 5)


def test_one_specialization_per_dtype_and_block():
    @newt.jit
    def k(x_ptr, o_ptr, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        nl.store(o_ptr + offs, nl.load(x_ptr + offs) + 1)

    for dtype in (torch.float32, torch.float16):
        for block in (64, 128):
            for _ in range(2):
                x = torch.randn(block, device="cuda").to(dtype)
                o = torch.empty_like(x)
                k[(1,)](x, o, BLOCK=block)
                torch.testing.assert_close(o.float(), x.float() + 1, rtol=1e-3, atol=1e-3)
    assert len(k.cache) == 4


def test_int64_argument():
    @newt.jit
    def k(o_ptr, big, BLOCK: nl.constexpr):
        nl.store(o_ptr + nl.arange(0, BLOCK),
                 nl.zeros((BLOCK,), dtype=nl.float32) + (big / 4294967296))

    o = torch.empty(32, device="cuda")
    k[(1,)](o, 1 << 40, BLOCK=32)
    assert bool((o == 256.0).all())


@pytest.mark.parametrize("block,waves", [(16, 4), (1, 1), (64, 16), (2, 8)])
def test_block_smaller_than_workgroup(block, waves):
    @newt.jit
    def k(x_ptr, o_ptr, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        nl.store(o_ptr + offs, nl.load(x_ptr + offs) + 1)

    x = torch.randn(block, device="cuda")
    o = torch.empty_like(x)
    k[(1,)](x, o, BLOCK=block, num_warps=waves)
    assert torch.equal(o, x + 1)


def test_single_element():
    @newt.jit
    def k(x_ptr, o_ptr, n, BLOCK: nl.constexpr):
        offs = nl.arange(0, BLOCK)
        live = offs < n
        nl.store(o_ptr + offs, nl.load(x_ptr + offs, mask=live) * 3, mask=live)

    x = torch.randn(1, device="cuda")
    o = torch.empty_like(x)
    k[(1,)](x, o, 1, BLOCK=64)
    assert torch.equal(o, x * 3)


def test_tuple_unpacking():
    @newt.jit
    def k(o_ptr, BLOCK: nl.constexpr):
        a, b = nl.arange(0, BLOCK), nl.arange(0, BLOCK)
        nl.store(o_ptr + a, (a + b).to(nl.float32))

    o = torch.empty(64, device="cuda")
    k[(1,)](o, BLOCK=64)
    assert torch.equal(o, torch.arange(64, device="cuda").float() * 2)
