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
