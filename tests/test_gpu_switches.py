"""Every codegen switch the integration notes document keeps results within the
same tolerances (reference counterpart: its env fallbacks, tests/test_codegen_cpu.py:126-137).

Each switch changes the emitted kernels (it is part of the specialization and
code-object cache keys), so each parameter compiles fresh variants of: a
ragged pipelined matmul (520x264x136, 128x128x32 tiles, 3 stages), the
4-wave 256x256x32 matmul on a shape with ragged edges (1040x768x1056), the
default attention kernel causal and not on a ragged sequence, and, for the
layout switches, softmax and layernorm rows.
"""

import pytest
import torch

import newt_amd as newt
import newt_amd.language as nl
from oracle import newt_oracle as orc

pytestmark = pytest.mark.gpu

SWITCHES = [
    ("NEWT_PIPELINE_DOT", "0"), ("NEWT_PIPE_VERSION", "0"), ("NEWT_PLR", "0"),
    ("NEWT_SCHED", "0"), ("NEWT_IGLP", "0"), ("NEWT_LDS_DMA", "0"), ("NEWT_BUFFER_DMA", "0"),
    ("NEWT_NT_STORE", "0"), ("NEWT_MFMA", "16"), ("NEWT_MFMA", "32"), ("NEWT_VEC", "1"),
    ("NEWT_VEC", "2"), ("NEWT_HOIST_LOADS", "1"), ("NEWT_PID_REMAP", "0"),
    ("NEWT_PID_GROUP", "0"), ("NEWT_PID_GROUP", "2"), ("NEWT_BARE_BARRIER", "1"),
    ("NEWT_WHERE_VERSION", "0"), ("NEWT_NT_LOAD", "1"), ("NEWT_NT_STREAM", "1"),
    ("NEWT_REDUCE_PINGPONG", "0"), ("NEWT_PIPE_CLAMP", "0"), ("NEWT_CSE", "0"),
    ("NEWT_VERSION_BODY", "0"), ("NEWT_PID_LPT", "0"), ("NEWT_PERM16", "0"),
    ("NEWT_PAIR_REDUCE", "0"),
]


def seeded(shape, seed, scale=1.0, mean=0.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale + mean).to(dtype).to("cuda")


def npf(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize("var,value", SWITCHES, ids=[f"{v}={x}" for v, x in SWITCHES])
def test_switch_keeps_results(monkeypatch, var, value):
    import newt_amd as newt
    from newt_amd import workloads as W
    monkeypatch.setenv(var, value)
    print(f"{var}={value}", flush=True)
    for (M, N, K), cfg in (((520, 264, 136), (128, 128, 32, 4, 3)),
                           ((1040, 768, 1056), (256, 256, 32, 4, 4))):
        a = seeded((M, K), 50, scale=K ** -0.5, dtype=torch.float16)
        b = seeded((K, N), 51, scale=K ** -0.5, dtype=torch.float16)
        BM, BN, BK, nw, ns = cfg
        c = W.matmul(a, b, config=newt.Config({"BLOCK_M": BM, "BLOCK_N": BN, "BLOCK_K": BK},
                                             num_warps=nw, num_stages=ns))
        ref = orc.matmul(npf(a), npf(b), "float16")
        assert orc.rel_frobenius(npf(c), ref) <= 1e-2, (M, N, K)
        assert orc.ulp_violations(npf(c), ref, "float16") == 0, (M, N, K)
    q, k, v = (seeded((2, 2, 300, 128), s, dtype=torch.bfloat16) for s in (52, 53, 54))
    for causal in (False, True):
        o = W.attention(q, k, v, causal=causal)
        ref = orc.attention(npf(q), npf(k), npf(v), 128 ** -0.5, causal, p_dtype="bfloat16",
                            out_dtype="bfloat16")
        assert orc.rel_frobenius(npf(o), ref) <= 1e-2, causal
    x = seeded((64, 1000), 55, scale=4.0)
    assert orc.rel_violations(npf(W.softmax(x)), orc.softmax_rows(npf(x)), 1e-5) == 0
    xh = seeded((32, 3000), 56, dtype=torch.float16)
    w = seeded(3000, 57, scale=0.1, mean=1.0, dtype=torch.float16)
    bb = seeded(3000, 58, scale=0.1, dtype=torch.float16)
    y, mean, rstd = W.layernorm(xh, w, bb, 1e-5)
    bad = orc.layernorm_violations(npf(y), npf(mean), npf(rstd), npf(xh), npf(w), npf(bb),
                                   1e-5, "float16")
    assert bad == {"y": 0, "mean": 0, "rstd": 0}, bad
    xa, ya = seeded(12345, 59), seeded(12345, 60)
    assert torch.equal(W.add(xa, ya), xa + ya)


@pytest.mark.parametrize("B,H,S", [(2, 4, 1000), (1, 3, 700), (1, 16, 513)])
def test_heaviest_first_order_is_bit_identical(monkeypatch, B, H, S):
    """The causal examples/05 form runs heaviest first (its key loop grows with
    program_id(0)); the order is a bijection of independent programs, so the
    output equals the hardware order's bit for bit, on head counts that split
    evenly over the 8 XCDs (per-XCD interleave) and that do not (axis 0
    reversed), and matches the oracle."""
    from newt_amd import workloads as W
    print(f"plain causal attention [{B},{H},{S},128] NEWT_PID_LPT on/off", flush=True)
    q, k, v = (seeded((B, H, S, 128), s, dtype=torch.bfloat16) for s in (61, 62, 63))
    outs = []
    for lpt in ("1", "0"):
        monkeypatch.setenv("NEWT_PID_LPT", lpt)
        o = torch.full_like(q, float("nan"))
        W.attention(q, k, v, causal=True, out=o, plain=True, BLOCK_M=128, num_warps=4)
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    ref = orc.attention(npf(q), npf(k), npf(v), 128 ** -0.5, True, p_dtype="bfloat16",
                        out_dtype="bfloat16")
    assert orc.rel_frobenius(npf(outs[0]), ref) <= 1e-2


@pytest.mark.parametrize("tile", ["16x16, 32 rows per wave", "32x32, 64 rows per wave"])
@pytest.mark.parametrize("plain", [False, True])
@pytest.mark.parametrize("causal", [False, True])
def test_paired_lane_reduce_is_bit_identical(monkeypatch, causal, plain, tile):
    """Attention's row statistics with two rows per lane run as
    newt::lane_reduce2 pairs: on the default 16x16x32 accumulator (rows
    reduced over lane bits 4 and 5) and on 32x32x16 with 64 rows per wave
    (lane bit 5 alone). A pair makes the same combines in the same operand
    order as one lane_reduce per row (NEWT_PAIR_REDUCE=0): the outputs are
    equal bit for bit, and match the oracle."""
    from newt_amd import workloads as W
    print(f"attention causal={causal} plain={plain} {tile} NEWT_PAIR_REDUCE on/off", flush=True)
    D = 128 if tile.startswith("16") else 64
    kw = {} if tile.startswith("16") else {"BLOCK_M": 128, "num_warps": 2}
    if not tile.startswith("16"):
        monkeypatch.setenv("NEWT_MFMA", "32")
    q, k, v = (seeded((2, 4, 700, D), s, dtype=torch.bfloat16) for s in (64, 65, 66))
    outs = []
    for pair in ("1", "0"):
        monkeypatch.setenv("NEWT_PAIR_REDUCE", pair)
        o = torch.full_like(q, float("nan"))
        W.attention(q, k, v, causal=causal, out=o, plain=plain, **kw)
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    ref = orc.attention(npf(q), npf(k), npf(v), D ** -0.5, causal, p_dtype="bfloat16",
                        out_dtype="bfloat16")
    assert orc.rel_frobenius(npf(outs[0]), ref) <= 1e-2


@newt.jit
def rowred(x_ptr, s_ptr, mx_ptr, mn_ptr, RB: nl.constexpr, CB: nl.constexpr):
    r = nl.arange(0, RB)
    c = nl.arange(0, CB)
    x = nl.load(x_ptr + r[:, None] * CB + c[None, :])
    nl.store(s_ptr + r, nl.sum(x, axis=1))
    nl.store(mx_ptr + r, nl.max(x, axis=1))
    nl.store(mn_ptr + r, nl.min(x, axis=1))


@pytest.mark.parametrize("R,C,warps", [(8, 1024, 1), (4, 256, 1), (16, 512, 2), (6, 128, 1),
                                        (2, 2048, 1)])
def test_paired_row_reductions(monkeypatch, R, C, warps):
    """Row sums, maxima and minima of blocks whose rows are spread over 32 or
    64 lanes with several rows per lane (their results pair up in
    newt::lane_reduce2, after the lane bits below 16): int32 results equal
    torch's exactly; float results (with signed zeros, infinities and NaNs
    in the rows) equal those of one lane_reduce per row bit for bit."""
    print(f"row reductions [{R},{C}] on {warps} waves", flush=True)
    RB = 1 << (R - 1).bit_length()
    g = torch.Generator().manual_seed(R * C)
    xi = torch.randint(-1000, 1000, (RB, C), generator=g, dtype=torch.int32).cuda()
    xf = (torch.randn(RB, C, generator=g) * 3).cuda()
    xf[0, 5], xf[1, 7], xf[1 % RB, 9] = float("-inf"), float("nan"), -0.0
    xf[2 % RB, :] = -0.0
    xf[3 % RB, 3] = float("inf")
    res = {}
    for pair in ("1", "0"):
        monkeypatch.setenv("NEWT_PAIR_REDUCE", pair)
        for name, x in (("i", xi), ("f", xf)):
            outs = [torch.empty(RB, device="cuda", dtype=x.dtype) for _ in range(3)]
            rowred[(1,)](x, *outs, RB=RB, CB=C, num_warps=warps)
            res[(pair, name)] = outs
    torch.cuda.synchronize()
    s, mx, mn = res[("1", "i")]
    assert torch.equal(s, xi.sum(1, dtype=torch.int32))
    assert torch.equal(mx, xi.max(1).values) and torch.equal(mn, xi.min(1).values)
    for a, b in zip(res[("1", "f")], res[("0", "f")]):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    finite = torch.isfinite(xf).all(1)
    ref = xf[finite].double().sum(1).float()
    torch.testing.assert_close(res[("1", "f")][0][finite], ref, rtol=1e-5, atol=1e-3)
    assert torch.equal(res[("1", "f")][1][finite], xf[finite].max(1).values)
    assert torch.equal(res[("1", "f")][2][finite], xf[finite].min(1).values)
