"""Every nl.* operation on the GPU against torch, at the reference's tolerances.

Semantics pinned here follow the reference's op suite (tests/test_ops.py):
  elementwise binary ops in fp32, fp16 and bf16: bit-exact, with
  signed zeros, infinities, NaN and subnormals (ref: rtol 1e-5 / 2e-3) :21-68
  int32 bit ops, shifts, C-truncating % and // (exact)             :71-117
  unary math (rtol/atol 1e-5)                                      :120-178
  casts: bit-exact, with specials (ref: float within 1e-3)         :181-210
  axis and full reductions, fp16 sums accumulating in fp32         :213-289
  broadcast / broadcast_to / reshape / trans (exact)               :292-337
  strided, gathered and scalar loads (exact)                       :340-391
  atomics: histogram == bincount, int atomic_max                   :394-426
  nl.dot shapes / dtypes / waves, dot epilogue                     :429-481
The kernels are launched through the HIP backend (hipRTC code objects,
libnewt_hip.so); torch on the same device is the oracle.
"""

import numpy as np
import pytest
import torch

import newt
import newt.language as nl

pytestmark = pytest.mark.gpu


def rnd(shape, dtype=torch.float32, seed=0, positive=False):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(shape, device="cuda", generator=g)
    if positive:
        x = x.abs() + 0.5
    return x.to(dtype)


# --------------------------------------------------------------- elementwise

@newt.jit
def binary_k(x_ptr, y_ptr, o_ptr, n, OP: nl.constexpr, BLOCK: nl.constexpr):
    offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
    live = offs < n
    a = nl.load(x_ptr + offs, mask=live)
    b = nl.load(y_ptr + offs, mask=live, other=1.0)
    if OP == "add":
        r = a + b
    elif OP == "sub":
        r = a - b
    elif OP == "mul":
        r = a * b
    elif OP == "div":
        r = a / b
    elif OP == "pow2":
        r = a ** 2
    elif OP == "maximum":
        r = nl.maximum(a, b)
    elif OP == "minimum":
        r = nl.minimum(a, b)
    elif OP == "fma":
        r = nl.fma(a, b, a)
    else:
        r = nl.where(a > 0, a, b)
    nl.store(o_ptr + offs, r, mask=live)


TORCH_BINARY = {
    "add": torch.add,
    "sub": torch.sub,
    "mul": torch.mul,
    "div": torch.div,
    "pow2": lambda a, b: a * a,
    "maximum": torch.maximum,
    "minimum": torch.minimum,
    "fma": lambda a, b: a * b + a,
    "where": lambda a, b: torch.where(a > 0, a, b),
}


def with_specials(x, dtype, seed):
    """x with a prefix of IEEE special values: signed zeros, infinities, NaN,
    subnormals of `dtype`, its largest finite values and values one rounding
    step apart, in every pairing the two operand seeds produce."""
    tiny = torch.finfo(dtype).tiny
    big = torch.finfo(dtype).max
    sp = torch.tensor([0.0, -0.0, float("inf"), float("-inf"), float("nan"), tiny / 4,
                       -tiny / 2, tiny, big, -big, 1.0, -1.0, 3.0, 1e-3])
    g = torch.Generator().manual_seed(seed)
    pre = sp[torch.randint(0, len(sp), (512,), generator=g)].to(dtype).to("cuda")
    return torch.cat([pre, x[512:]])


def bits(t):
    return t.view(torch.int16 if t.element_size() == 2 else torch.int32)


def assert_same_bits(got, want, op=""):
    """Bit-identical results, with NaN equal to any NaN (payloads are not
    part of the semantics) and, for max/min, +0 equal to -0 (IEEE
    maxNum/minNum leave the sign of a zero result unspecified)."""
    g, w = got.cpu(), want.cpu()
    same = bits(g) == bits(w)
    same |= g.isnan() & w.isnan()
    if op in ("maximum", "minimum"):
        same |= (g == 0) & (w == 0)
    bad = (~same).nonzero().flatten()
    assert bad.numel() == 0, (f"{op}: {bad.numel()} elements differ, first at {bad[:5].tolist()}: "
                              f"got {g[bad[:5]].tolist()} want {w[bad[:5]].tolist()}")


def binary_oracle(op, a, b):
    """The reference's elementwise semantics (codegen.py:1196-1284, :2114-2118)
    on the CPU: fp16 operands computed in fp32 and rounded once, maximum /
    minimum as C fmaxf / fminf (a NaN operand yields the other operand)."""
    af, bf = a.cpu().float(), b.cpu().float()
    if op == "maximum":
        r = torch.from_numpy(np.fmax(af.numpy(), bf.numpy()))
    elif op == "minimum":
        r = torch.from_numpy(np.fmin(af.numpy(), bf.numpy()))
    else:
        r = TORCH_BINARY[op](af, bf)
    return r.to(a.dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("op", sorted(TORCH_BINARY))
def test_binary(op, dtype):
    """Elementwise binary ops are bit-exact (north_star): no contraction, IEEE
    division, one rounding of the fp32 result for fp16/bf16, including signed
    zeros, infinities, NaN and subnormal operands. nl.fma is fused (one
    rounding of a*b+a) where torch's a*b+a rounds twice, so it is held to a
    tolerance instead."""
    n = 4321
    a = with_specials(rnd(n, dtype, 0), dtype, 10)
    b = with_specials(rnd(n, dtype, 1, positive=True), dtype, 11)
    o = torch.empty_like(a)
    binary_k[(newt.cdiv(n, 1024),)](a, b, o, n, OP=op, BLOCK=1024)
    want = binary_oracle(op, a, b)
    if op == "fma":
        tol = 1e-5 if dtype == torch.float32 else 2e-3
        torch.testing.assert_close(o[512:].float().cpu(), want[512:].float(), rtol=tol, atol=tol)
    else:
        assert_same_bits(o, want, op)


@newt.jit
def int_k(x_ptr, y_ptr, o_ptr, n, OP: nl.constexpr, BLOCK: nl.constexpr):
    offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
    live = offs < n
    a = nl.load(x_ptr + offs, mask=live)
    b = nl.load(y_ptr + offs, mask=live, other=1)
    if OP == "and":
        r = a & b
    elif OP == "or":
        r = a | b
    elif OP == "xor":
        r = a ^ b
    elif OP == "shl":
        r = a << 1
    elif OP == "shr":
        r = a >> 2
    elif OP == "mod":
        r = a % b
    else:
        r = a // b
    nl.store(o_ptr + offs, r, mask=live)


def _c_div(a, b):
    return torch.div(a, b, rounding_mode="trunc")


TORCH_INT = {
    "and": torch.bitwise_and,
    "or": torch.bitwise_or,
    "xor": torch.bitwise_xor,
    "shl": lambda a, b: a << 1,
    "shr": lambda a, b: a >> 2,
    "mod": lambda a, b: a - _c_div(a, b) * b,   # C remainder (sign of the dividend)
    "floordiv": _c_div,                         # C truncation
}


@pytest.mark.parametrize("signed", [False, True])
@pytest.mark.parametrize("op", sorted(TORCH_INT))
def test_int32(op, signed):
    n = 2048
    g = torch.Generator(device="cuda").manual_seed(3)
    a = torch.randint(-1000 if signed else 0, 1000, (n,), device="cuda", generator=g,
                      dtype=torch.int32)
    b = torch.randint(1, 50, (n,), device="cuda", generator=g, dtype=torch.int32)
    if signed:
        b = torch.where(torch.arange(n, device="cuda") % 3 == 0, -b, b)
    o = torch.empty_like(a)
    int_k[(newt.cdiv(n, 1024),)](a, b, o, n, OP=op, BLOCK=1024)
    assert torch.equal(o, TORCH_INT[op](a, b))


@newt.jit
def unary_k(x_ptr, o_ptr, n, OP: nl.constexpr, BLOCK: nl.constexpr):
    offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
    live = offs < n
    v = nl.load(x_ptr + offs, mask=live, other=1.0)
    if OP == "exp":
        r = nl.exp(v)
    elif OP == "exp2":
        r = nl.exp2(v)
    elif OP == "log":
        r = nl.log(v)
    elif OP == "log2":
        r = nl.log2(v)
    elif OP == "sqrt":
        r = nl.sqrt(v)
    elif OP == "rsqrt":
        r = nl.rsqrt(v)
    elif OP == "sin":
        r = nl.sin(v)
    elif OP == "cos":
        r = nl.cos(v)
    elif OP == "tanh":
        r = nl.tanh(v)
    elif OP == "erf":
        r = nl.erf(v)
    elif OP == "sigmoid":
        r = nl.sigmoid(v)
    elif OP == "abs":
        r = nl.abs(v)
    elif OP == "floor":
        r = nl.floor(v)
    elif OP == "ceil":
        r = nl.ceil(v)
    else:
        r = -v
    nl.store(o_ptr + offs, r, mask=live)


TORCH_UNARY = {
    "exp": torch.exp, "exp2": torch.exp2, "log": torch.log, "log2": torch.log2,
    "sqrt": torch.sqrt, "rsqrt": torch.rsqrt, "sin": torch.sin, "cos": torch.cos,
    "tanh": torch.tanh, "erf": torch.erf, "sigmoid": torch.sigmoid, "abs": torch.abs,
    "floor": torch.floor, "ceil": torch.ceil, "neg": torch.neg,
}


@pytest.mark.parametrize("op", sorted(TORCH_UNARY))
def test_unary(op):
    n = 3000
    x = rnd(n, positive=op in ("log", "log2", "sqrt", "rsqrt"))
    o = torch.empty_like(x)
    unary_k[(newt.cdiv(n, 1024),)](x, o, n, OP=op, BLOCK=1024)
    torch.testing.assert_close(o, TORCH_UNARY[op](x), rtol=1e-5, atol=1e-5)


def test_exp_over_its_whole_range():
    """nl.exp runs on the hardware exp2 unit; over every input whose result is
    a normal float it stays within the reference's rtol 1e-5 of the exact
    value (float64 on the CPU). +-0, +-inf and NaN give what expf gives. Two
    documented deviations from expf, both inside the reference's atol: a
    result below 2^-126 (x < -87.34) flushes to 0 where expf returns a
    subnormal (exp(-100) ~ 3.7e-44; from x < -103.28 on, expf gives 0 too), and an x within an ulp below ln(FLT_MAX)
    (88.7228) whose product with log2(e) rounds to 128 gives inf where expf
    gives ~3.4e38."""
    n = 1 << 16
    x = torch.linspace(-87.0, 88.5, n, device="cuda")
    o = torch.empty_like(x)
    for i in range(0, n, 4096):
        unary_k[(4,)](x[i:], o[i:], 4096, OP="exp", BLOCK=1024)
    want = torch.exp(x.cpu().double())
    rel = ((o.cpu().double() - want).abs() / want).max().item()
    assert rel < 1e-5, rel
    sp = torch.tensor([0.0, -0.0, float("inf"), float("-inf"), float("nan"), 89.0, -104.0],
                      device="cuda")
    so = torch.empty_like(sp)
    unary_k[(1,)](sp, so, sp.numel(), OP="exp", BLOCK=1024)
    got = so.cpu().tolist()
    assert got[:2] == [1.0, 1.0] and got[2] == float("inf") and got[3] == 0.0
    assert got[4] != got[4] and got[5] == float("inf") and got[6] == 0.0


@newt.jit
def cast_k(x_ptr, o_ptr, n, DT: nl.constexpr, BLOCK: nl.constexpr):
    offs = nl.arange(0, BLOCK)
    live = offs < n
    nl.store(o_ptr + offs, nl.load(x_ptr + offs, mask=live).to(DT), mask=live)


@pytest.mark.parametrize("src,dst,ndt", [
    (torch.float32, torch.float16, nl.float16),
    (torch.float16, torch.float32, nl.float32),
    (torch.float32, torch.bfloat16, nl.bfloat16),
    (torch.bfloat16, torch.float32, nl.float32),
    (torch.float16, torch.bfloat16, nl.bfloat16),
    (torch.bfloat16, torch.float16, nl.float16),
    (torch.float32, torch.int32, nl.int32),
    (torch.int32, torch.float32, nl.float32),
    (torch.int64, torch.int32, nl.int32),
    (torch.int32, torch.int64, nl.int64),
])
def test_cast(src, dst, ndt):
    """Casts are bit-exact against torch: float narrowing rounds to nearest
    even (overflow to inf, NaN kept, subnormal results), widening is exact,
    float -> int truncates toward zero (in-range values: C leaves the rest
    undefined), int -> float rounds to nearest even."""
    n = 1000
    x = (rnd(n, seed=4) * 10).to(src)
    if src.is_floating_point:
        x = with_specials(x, src, 12)
        if dst.is_floating_point:
            # values near the destination's overflow and subnormal ranges
            x[512:520] = torch.tensor([65504.0, 65520.0, 7e4, -7e4, 6e-8, 3e-8, 1e-40, -1e-39]
                                      ).to(src)
        else:
            x = torch.where(x.isfinite() & (x.abs() < 2.0 ** 31), x, torch.zeros_like(x))
    elif src == torch.int32 and dst.is_floating_point:
        x[:8] = torch.tensor([16777217, -16777219, 2 ** 31 - 1, -2 ** 31, 0, 1, 33554435,
                              -100000001], dtype=src)
    o = torch.empty(n, device="cuda", dtype=dst)
    cast_k[(1,)](x, o, n, DT=ndt, BLOCK=1024)
    want = x.cpu().to(dst)
    if dst.is_floating_point:
        assert_same_bits(o, want, "cast")
    else:
        assert torch.equal(o.cpu(), want)


def test_cast_rounds_to_nearest_even():
    """fp32 -> fp16/bf16 conversions round to nearest even, as torch does."""
    x = torch.randn(1 << 14, device="cuda") * 3
    for dt, ndt in ((torch.float16, nl.float16), (torch.bfloat16, nl.bfloat16)):
        o = torch.empty(x.numel(), device="cuda", dtype=dt)
        for i in range(0, x.numel(), 1024):
            cast_k[(1,)](x[i:], o[i:], 1024, DT=ndt, BLOCK=1024)
        assert torch.equal(o, x.to(dt))


# ---------------------------------------------------------------- reductions

@newt.jit
def reduce2d_k(x_ptr, o_ptr, M, N, sx, OP: nl.constexpr, AXIS: nl.constexpr,
               BM: nl.constexpr, BN: nl.constexpr):
    rm = nl.arange(0, BM)
    rn = nl.arange(0, BN)
    inb = (rm[:, None] < M) & (rn[None, :] < N)
    ptrs = x_ptr + rm[:, None] * sx + rn[None, :]
    if OP == "sum":
        r = nl.sum(nl.load(ptrs, mask=inb, other=0.0), axis=AXIS)
    elif OP == "max":
        r = nl.max(nl.load(ptrs, mask=inb, other=float("-inf")), axis=AXIS)
    else:
        r = nl.min(nl.load(ptrs, mask=inb, other=float("inf")), axis=AXIS)
    if AXIS == 0:
        nl.store(o_ptr + rn, r, mask=rn < N)
    else:
        nl.store(o_ptr + rm, r, mask=rm < M)


@pytest.mark.parametrize("mn", [(32, 64), (17, 100), (128, 128), (3, 1000), (300, 5)])
@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("op", ["sum", "max", "min"])
def test_reduce_axis(op, axis, mn):
    M, N = mn
    x = rnd((M, N), seed=5)
    o = torch.empty(N if axis == 0 else M, device="cuda")
    reduce2d_k[(1,)](x, o, M, N, x.stride(0), OP=op, AXIS=axis,
                     BM=newt.next_power_of_2(M), BN=newt.next_power_of_2(N))
    want = {"sum": x.sum(axis), "max": x.amax(axis), "min": x.amin(axis)}[op]
    torch.testing.assert_close(o, want, rtol=1e-4, atol=1e-4)


@newt.jit
def reduce2d_whole_k(x_ptr, o_ptr, OP: nl.constexpr, AXIS: nl.constexpr,
                     BM: nl.constexpr, BN: nl.constexpr):
    rm = nl.arange(0, BM)
    rn = nl.arange(0, BN)
    v = nl.load(x_ptr + rm[:, None] * BN + rn[None, :])
    if OP == "sum":
        r = nl.sum(v, axis=AXIS)
    elif OP == "max":
        r = nl.max(v, axis=AXIS)
    else:
        r = nl.min(v, axis=AXIS)
    if AXIS == 0:
        nl.store(o_ptr + rn, r)
    else:
        nl.store(o_ptr + rm, r)


@pytest.mark.parametrize("waves", [1, 2, 4])
@pytest.mark.parametrize("mn", [(2, 32), (4, 16), (8, 8), (16, 4), (32, 2), (64, 1), (1, 64),
                                (2, 128), (128, 2), (16, 64), (64, 16), (256, 8), (8, 256)])
@pytest.mark.parametrize("dt", [torch.int32, torch.int64])
def test_reduce_axis_exact_int(dt, mn, waves):
    # every split of a block's axes over lane bits (so each partial lane mask of
    # the wave64 butterfly, 4- and 8-byte values): integer results are exact
    M, N = mn
    g = torch.Generator().manual_seed(M * 1000 + N)
    x = torch.randint(-10**6, 10**6, (M, N), generator=g, dtype=dt).cuda()
    if dt == torch.int64:
        x = x * (1 << 20)                         # uses the upper word
    for axis in (0, 1):
        for op in ("sum", "max", "min"):
            o = torch.empty(N if axis == 0 else M, device="cuda", dtype=dt)
            reduce2d_whole_k[(1,)](x, o, OP=op, AXIS=axis, BM=M, BN=N, num_warps=waves)
            want = {"sum": x.sum(axis), "max": x.amax(axis), "min": x.amin(axis)}[op]
            assert torch.equal(o, want.to(dt)), (op, axis)


@newt.jit
def reduce_in_loop_k(x_ptr, part_ptr, col_ptr, o_ptr, ITERS: nl.constexpr,
                     BM: nl.constexpr, BN: nl.constexpr):
    rm = nl.arange(0, BM)
    rn = nl.arange(0, BN)
    total = 0
    cols = nl.zeros((BN,), dtype=nl.int32)
    for i in range(0, ITERS):
        v = nl.load(x_ptr + i * BM * BN + rm[:, None] * BN + rn[None, :])
        s = nl.sum(v)                       # across every wave, each iteration
        nl.store(part_ptr + i, s)
        if nl.max(v) > 0:                   # a branch on a cross-wave reduction
            total = total + s
        cols = cols + nl.max(v, axis=0)     # across the waves holding rows
    nl.store(o_ptr, total)
    nl.store(col_ptr + rn, cols)


@pytest.mark.parametrize("waves", [2, 4, 8])
@pytest.mark.parametrize("bm_bn", [(64, 64), (256, 16), (16, 256)])
def test_cross_wave_reductions_in_a_loop(bm_bn, waves):
    # every iteration reduces across the waves through LDS; consecutive
    # iterations alternate between two partial buffers with no barrier ahead
    # of the write: exact integer results over many iterations pin that no
    # wave reads partials a faster wave has already overwritten
    BM, BN = bm_bn
    iters = 37
    g = torch.Generator().manual_seed(BM + BN + waves)
    x = torch.randint(-1000, 1000, (iters, BM, BN), generator=g, dtype=torch.int32)
    x[5] = -x[5].abs() - 1                 # an iteration whose branch is not taken
    x = x.cuda()
    part = torch.empty(iters, device="cuda", dtype=torch.int32)
    col = torch.empty(BN, device="cuda", dtype=torch.int32)
    o = torch.empty(1, device="cuda", dtype=torch.int32)
    reduce_in_loop_k[(1,)](x, part, col, o, ITERS=iters, BM=BM, BN=BN, num_warps=waves)
    xs = x.cpu().long()
    sums = xs.sum((1, 2))
    assert part.cpu().long().tolist() == sums.tolist()
    keep = xs.amax((1, 2)) > 0
    assert int(o.item()) == int(sums[keep].sum())
    assert col.cpu().long().tolist() == xs.amax(1).sum(0).tolist()


@newt.jit
def reduce_full_k(x_ptr, o_ptr, n, OP: nl.constexpr, BLOCK: nl.constexpr):
    offs = nl.arange(0, BLOCK)
    live = offs < n
    if OP == "sum":
        r = nl.sum(nl.load(x_ptr + offs, mask=live, other=0.0))
    elif OP == "max":
        r = nl.max(nl.load(x_ptr + offs, mask=live, other=float("-inf")))
    else:
        r = nl.min(nl.load(x_ptr + offs, mask=live, other=float("inf")))
    nl.store(o_ptr, r)


@pytest.mark.parametrize("waves", [1, 4, 8, 16])
@pytest.mark.parametrize("n", [32, 100, 1024, 5000])
@pytest.mark.parametrize("op", ["sum", "max", "min"])
def test_reduce_full(op, n, waves):
    x = rnd(n, seed=6)
    o = torch.empty(1, device="cuda")
    reduce_full_k[(1,)](x, o, n, OP=op, BLOCK=newt.next_power_of_2(n), num_warps=waves)
    want = {"sum": x.sum(), "max": x.max(), "min": x.min()}[op]
    torch.testing.assert_close(o[0], want, rtol=1e-4, atol=1e-4)


@newt.jit
def sum_all_k(x_ptr, o_ptr, BLOCK: nl.constexpr):
    nl.store(o_ptr, nl.sum(nl.load(x_ptr + nl.arange(0, BLOCK))))


def test_fp16_sum_accumulates_in_fp32():
    # 4096 fp16 ones: an fp16 accumulator would stall at 2048
    x = torch.ones(4096, device="cuda", dtype=torch.float16)
    o = torch.empty(1, device="cuda")
    sum_all_k[(1,)](x, o, BLOCK=4096)
    assert o.item() == 4096.0


@newt.jit
def int_reduce_k(x_ptr, o_ptr, BLOCK: nl.constexpr):
    v = nl.load(x_ptr + nl.arange(0, BLOCK))
    nl.store(o_ptr, nl.sum(v))
    nl.store(o_ptr + 1, nl.max(v))
    nl.store(o_ptr + 2, nl.min(v))


def test_int_reductions_exact():
    x = torch.randint(-10**6, 10**6, (2048,), device="cuda", dtype=torch.int32)
    o = torch.empty(3, device="cuda", dtype=torch.int32)
    int_reduce_k[(1,)](x, o, BLOCK=2048)
    assert o.tolist() == [int(x.sum()), int(x.max()), int(x.min())]


# ------------------------------------------------------------- shape ops

@newt.jit
def outer_k(a_ptr, b_ptr, o_ptr, BM: nl.constexpr, BN: nl.constexpr):
    a = nl.load(a_ptr + nl.arange(0, BM))
    b = nl.load(b_ptr + nl.arange(0, BN))
    grid = nl.arange(0, BM)[:, None] * BN + nl.arange(0, BN)[None, :]
    nl.store(o_ptr + grid, a[:, None] * 100 + b[None, :])


def test_broadcast_outer():
    a, b = rnd(32), rnd(64, seed=1)
    o = torch.empty(32, 64, device="cuda")
    outer_k[(1,)](a, b, o, BM=32, BN=64)
    torch.testing.assert_close(o, a[:, None] * 100 + b[None, :], rtol=1e-5, atol=1e-5)


@newt.jit
def bcast_reshape_k(a_ptr, o_ptr, BM: nl.constexpr, BN: nl.constexpr):
    a = nl.load(a_ptr + nl.arange(0, BM))
    full = nl.broadcast_to(a[:, None], (BM, BN))
    nl.store(o_ptr + nl.arange(0, BM * BN), nl.reshape(full, (BM * BN,)))


def test_broadcast_to_then_reshape():
    a = rnd(16)
    o = torch.empty(16 * 32, device="cuda")
    bcast_reshape_k[(1,)](a, o, BM=16, BN=32)
    assert torch.equal(o.view(16, 32), a[:, None].expand(16, 32))


@newt.jit
def trans_k(x_ptr, o_ptr, BM: nl.constexpr, BN: nl.constexpr):
    x = nl.load(x_ptr + nl.arange(0, BM)[:, None] * BN + nl.arange(0, BN)[None, :])
    nl.store(o_ptr + nl.arange(0, BN)[:, None] * BM + nl.arange(0, BM)[None, :], nl.trans(x))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("mn", [(32, 64), (64, 32), (128, 8), (16, 16)])
def test_trans(mn, dtype):
    M, N = mn
    x = rnd((M, N), dtype)
    o = torch.empty(N, M, device="cuda", dtype=dtype)
    trans_k[(1,)](x, o, BM=M, BN=N)
    assert torch.equal(o, x.t().contiguous())


# ---------------------------------------------------------- loads and stores

@newt.jit
def strided_k(x_ptr, o_ptr, n, sx, BLOCK: nl.constexpr):
    offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
    live = offs < n
    nl.store(o_ptr + offs, nl.load(x_ptr + offs * sx, mask=live) * 2, mask=live)


def test_strided_load():
    base = rnd(2000)
    view = base[::2]
    o = torch.empty(view.numel(), device="cuda")
    strided_k[(newt.cdiv(view.numel(), 256),)](base, o, view.numel(), 2, BLOCK=256)
    assert torch.equal(o, view * 2)


@newt.jit
def gather_k(x_ptr, idx_ptr, o_ptr, n, BLOCK: nl.constexpr):
    offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
    live = offs < n
    i = nl.load(idx_ptr + offs, mask=live)
    nl.store(o_ptr + offs, nl.load(x_ptr + i, mask=live), mask=live)


def test_gather():
    n = 4096
    x = rnd(n)
    idx = torch.randperm(n, device="cuda").to(torch.int32)
    o = torch.empty(n, device="cuda")
    gather_k[(newt.cdiv(n, 1024),)](x, idx, o, n, BLOCK=1024)
    assert torch.equal(o, x[idx.long()])


@newt.jit
def scatter_k(x_ptr, idx_ptr, o_ptr, n, BLOCK: nl.constexpr):
    offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
    live = offs < n
    i = nl.load(idx_ptr + offs, mask=live)
    nl.store(o_ptr + i, nl.load(x_ptr + offs, mask=live), mask=live)


def test_scatter():
    n = 3000
    x = rnd(n)
    idx = torch.randperm(n, device="cuda").to(torch.int32)
    o = torch.zeros(n, device="cuda")
    scatter_k[(newt.cdiv(n, 512),)](x, idx, o, n, BLOCK=512)
    want = torch.zeros_like(o)
    want[idx.long()] = x
    assert torch.equal(o, want)


@newt.jit
def scalar_load_k(x_ptr, o_ptr, BLOCK: nl.constexpr):
    s = nl.load(x_ptr)
    nl.store(o_ptr + nl.arange(0, BLOCK), nl.zeros((BLOCK,), dtype=nl.float32) + s)


def test_scalar_load():
    x = torch.tensor([42.0], device="cuda")
    o = torch.empty(128, device="cuda")
    scalar_load_k[(1,)](x, o, BLOCK=128)
    assert bool((o == 42.0).all())


@newt.jit
def misaligned_k(x_ptr, o_ptr, n, BLOCK: nl.constexpr):
    offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
    live = offs < n
    nl.store(o_ptr + offs, nl.load(x_ptr + offs, mask=live) + 1.0, mask=live)


@pytest.mark.parametrize("shift", [1, 2, 3])
def test_unaligned_pointers_take_the_scalar_path(shift):
    # views starting 4/8/12 bytes into an allocation defeat 16-byte vector access
    base = rnd(5000)
    x = base[shift:]
    o = torch.zeros(5000, device="cuda")[shift:]
    misaligned_k[(newt.cdiv(x.numel(), 1024),)](x, o, x.numel(), BLOCK=1024)
    assert torch.equal(o, x + 1.0)


# ------------------------------------------------------------------ atomics

@newt.jit
def histogram_k(idx_ptr, hist_ptr, n, BLOCK: nl.constexpr):
    offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
    live = offs < n
    nl.atomic_add(hist_ptr + nl.load(idx_ptr + offs, mask=live), 1.0, mask=live)


def test_atomic_add_histogram():
    n, bins = 100_000, 64
    idx = torch.randint(0, bins, (n,), device="cuda", dtype=torch.int32)
    hist = torch.zeros(bins, device="cuda")
    histogram_k[(newt.cdiv(n, 1024),)](idx, hist, n, BLOCK=1024)
    assert torch.equal(hist, torch.bincount(idx.long(), minlength=bins).float())


@newt.jit
def block_max_k(x_ptr, o_ptr, n, BLOCK: nl.constexpr):
    offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
    v = nl.load(x_ptr + offs, mask=offs < n, other=0)
    nl.atomic_max(o_ptr, nl.max(v))


def test_atomic_max_int():
    n = 10_000
    x = torch.randint(0, 1_000_000, (n,), device="cuda", dtype=torch.int32)
    o = torch.zeros(1, device="cuda", dtype=torch.int32)
    block_max_k[(newt.cdiv(n, 1024),)](x, o, n, BLOCK=1024)
    assert o.item() == x.max().item()


# ---------------------------------------------------------------------- dot

@newt.jit
def dot_k(a_ptr, b_ptr, c_ptr, BM: nl.constexpr, BN: nl.constexpr, BK: nl.constexpr):
    rm, rk, rn = nl.arange(0, BM), nl.arange(0, BK), nl.arange(0, BN)
    a = nl.load(a_ptr + rm[:, None] * BK + rk[None, :])
    b = nl.load(b_ptr + rk[:, None] * BN + rn[None, :])
    nl.store(c_ptr + rm[:, None] * BN + rn[None, :], nl.dot(a, b))


@pytest.mark.parametrize("waves", [1, 2, 4])
@pytest.mark.parametrize("shape", [(16, 16, 16), (32, 64, 128), (64, 32, 16), (128, 128, 64)])
@pytest.mark.parametrize("dtype,tol", [(torch.float16, 2e-2), (torch.bfloat16, 3e-2),
                                       (torch.float32, 2e-2)])
def test_dot(dtype, tol, shape, waves):
    BM, BN, BK = shape
    a = rnd((BM, BK), dtype) * 0.3
    b = rnd((BK, BN), dtype, seed=1) * 0.3
    c = torch.empty(BM, BN, device="cuda")
    dot_k[(1,)](a, b, c, BM=BM, BN=BN, BK=BK, num_warps=waves)
    torch.testing.assert_close(c, a.float() @ b.float(), rtol=tol, atol=tol)


@newt.jit
def dot_epilogue_k(a_ptr, b_ptr, o_ptr, BM: nl.constexpr, BN: nl.constexpr, BK: nl.constexpr):
    rm, rk, rn = nl.arange(0, BM), nl.arange(0, BK), nl.arange(0, BN)
    a = nl.load(a_ptr + rm[:, None] * BK + rk[None, :])
    b = nl.load(b_ptr + rk[:, None] * BN + rn[None, :])
    c = nl.dot(a, b) * 2.0 + 1.0
    nl.store(o_ptr + rm, nl.sum(c, axis=1))
    nl.store(o_ptr + BM + rn, nl.max(c, axis=0))


def test_dot_epilogue_reductions():
    a = rnd((32, 32), torch.float16) * 0.3
    b = rnd((32, 32), torch.float16, seed=1) * 0.3
    o = torch.empty(64, device="cuda")
    dot_epilogue_k[(1,)](a, b, o, BM=32, BN=32, BK=32)
    c = a.float() @ b.float() * 2 + 1
    torch.testing.assert_close(o[:32], c.sum(1), rtol=2e-2, atol=2e-1)
    torch.testing.assert_close(o[32:], c.amax(0), rtol=2e-2, atol=2e-2)


@newt.jit
def dot_trans_k(a_ptr, b_ptr, c_ptr, BM: nl.constexpr, BN: nl.constexpr, BK: nl.constexpr):
    rm, rk, rn = nl.arange(0, BM), nl.arange(0, BK), nl.arange(0, BN)
    a = nl.load(a_ptr + rm[:, None] * BK + rk[None, :])
    bt = nl.load(b_ptr + rn[:, None] * BK + rk[None, :])   # B stored [N, K]
    nl.store(c_ptr + rm[:, None] * BN + rn[None, :], nl.dot(a, nl.trans(bt)))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_dot_with_transposed_operand(dtype):
    a = rnd((64, 64), dtype) * 0.3
    bt = rnd((128, 64), dtype, seed=1) * 0.3
    c = torch.empty(64, 128, device="cuda")
    dot_trans_k[(1,)](a, bt, c, BM=64, BN=128, BK=64)
    torch.testing.assert_close(c, a.float() @ bt.float().t(), rtol=2e-2, atol=2e-2)
