"""Pinning of the CPU oracle (oracle/newt_oracle.py) - runs without a GPU.

The oracle is only trusted because these checks pass. Each function is held
against: the golden fixtures in tests/golden (written by torch eager in float64,
the reference's own oracle: tests/test_vector_add.py:30,
tests/test_softmax_layernorm.py:47-62, tests/test_matmul.py:52-71,
examples/05_fused_attention.py:67-73); closed forms and invariants; and
brute-force loops on tiny inputs. The last group plants typical mistakes
(a transposed operand, a missing max-subtraction, a dropped causal mask, a
wrong normalisation axis) in copies of the oracle and checks that the same
checks reject them, so the checks are known to discriminate.
"""

import math
import os

import numpy as np
import pytest

from oracle import newt_oracle as orc

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def gold(name):
    return np.load(os.path.join(GOLD, f"{name}.npz"))


# ---------------------------------------------------------------- golden vectors

def test_vector_add_golden():
    g = gold("vector_add_12345")
    assert np.array_equal(orc.vector_add(g["x"], g["y"]), g["out"])


@pytest.mark.parametrize("name", ["softmax_8x128", "softmax_32x781"])
def test_softmax_golden(name):
    g = gold(name)
    np.testing.assert_allclose(orc.softmax_rows(g["x"]), g["out"], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("name", ["layernorm_16x300", "layernorm_8x128"])
def test_layernorm_golden(name):
    g = gold(name)
    y, mean, rstd = orc.layernorm_rows(g["x"], g["w"], g["b"], 1e-5, "float32")
    np.testing.assert_allclose(y, g["out"], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(mean, g["mean"], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(rstd, g["rstd"], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("name", ["matmul_64x64x32", "matmul_300x200x100"])
def test_matmul_golden(name):
    g = gold(name)
    out = orc.matmul(g["a"], g["b"], "float32")
    assert orc.rel_frobenius(out, g["out"]) < 1e-6


@pytest.mark.parametrize("causal", [False, True])
def test_attention_golden(causal):
    g = gold(f"attention_1x2x64x32_{'causal' if causal else 'full'}")
    o = orc.attention(g["q"], g["k"], g["v"], 32 ** -0.5, causal)
    assert orc.rel_frobenius(o, g["out"]) < 1e-6
    # P rounded to bf16 before P@V (what the kernel does) stays well inside the
    # 1e-2 kernel tolerance of the unrounded golden
    ob = orc.attention(g["q"], g["k"], g["v"], 32 ** -0.5, causal, p_dtype="bfloat16")
    assert orc.rel_frobenius(ob, g["out"]) < 5e-3


# ---------------------------------------------------------------- rounding helpers

def test_round_bf16_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 100,
                        np.array([0.0, -0.0, 1e-40, -1e-40, 3.4e38, 65504.0, 1.0 + 2 ** -8,
                                  1.0 + 3 * 2 ** -9, np.inf, -np.inf], np.float32)])
    ref = torch.from_numpy(x).bfloat16().float().numpy()
    got = orc.round_bf16(x)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert np.isnan(orc.round_bf16(np.array([np.nan], np.float32)))[0]


def test_round_fp16_matches_torch():
    torch = pytest.importorskip("torch")
    x = np.random.default_rng(1).standard_normal(5000).astype(np.float32) * 1000
    ref = torch.from_numpy(x).half().float().numpy()
    assert np.array_equal(orc.round_to(x, "float16"), ref)


# ---------------------------------------------------------------- closed forms

def test_vector_add_closed_form():
    x = np.arange(1000, dtype=np.float32)
    assert np.array_equal(orc.vector_add(x, -x), np.zeros(1000, np.float32))
    a, b = np.float32(0.1), np.float32(0.2)
    assert orc.vector_add(np.array([a]), np.array([b]))[0] == np.float32(a + b)


def test_softmax_invariants():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((16, 300)).astype(np.float32) * 4
    p = orc.softmax_rows(x)
    np.testing.assert_allclose(p.sum(axis=1), 1.0, rtol=1e-6)
    # shift invariance along a row
    np.testing.assert_allclose(orc.softmax_rows(x + 7.0), p, rtol=1e-5, atol=1e-7)
    # a constant row is uniform; huge values do not overflow (max subtraction)
    c = np.full((2, 37), 1000.0, np.float32)
    np.testing.assert_allclose(orc.softmax_rows(c), 1.0 / 37, rtol=1e-6)
    # -inf entries (masked columns) get probability 0
    y = x.copy()
    y[:, 5] = -np.inf
    assert np.all(orc.softmax_rows(y)[:, 5] == 0)


def test_softmax_brute_force():
    x = np.random.default_rng(3).standard_normal((3, 11)).astype(np.float32)
    p = orc.softmax_rows(x)
    for i in range(3):
        np.testing.assert_allclose(p[i], orc.softmax_loops([float(v) for v in x[i]]), rtol=1e-6)


def test_layernorm_closed_form():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((8, 500)).astype(np.float32) * 3 + 2
    ones, zeros = np.ones(500, np.float32), np.zeros(500, np.float32)
    y, mean, rstd = orc.layernorm_rows(x, ones, zeros, 1e-5)
    np.testing.assert_allclose(y.mean(axis=1), 0.0, atol=1e-5)
    np.testing.assert_allclose(y.var(axis=1), 1.0 - 1e-5 * rstd ** 2, rtol=1e-4)
    np.testing.assert_allclose(mean, x.astype(np.float64).mean(axis=1), rtol=1e-6)
    np.testing.assert_allclose(rstd, 1 / np.sqrt(x.astype(np.float64).var(axis=1) + 1e-5),
                               rtol=1e-6)
    # affine part: y' = y * w + b exactly as the formula says
    w = rng.standard_normal(500).astype(np.float32)
    b = rng.standard_normal(500).astype(np.float32)
    y2, _, _ = orc.layernorm_rows(x, w, b, 1e-5)
    np.testing.assert_allclose(y2, y * w + b, rtol=1e-4, atol=1e-5)
    # a constant row normalises to b (variance 0 -> rstd = 1/sqrt(eps))
    c = np.full((1, 64), 3.0, np.float32)
    yc, mc, rc = orc.layernorm_rows(c, ones[:64], b[:64], 1e-5)
    np.testing.assert_allclose(yc[0], b[:64], atol=1e-6)
    assert mc[0] == 3.0 and abs(rc[0] - 1 / math.sqrt(1e-5)) < 1e-2


def test_layernorm_brute_force():
    x = np.random.default_rng(5).standard_normal((2, 9)).astype(np.float32)
    w = np.random.default_rng(6).standard_normal(9).astype(np.float32)
    b = np.random.default_rng(7).standard_normal(9).astype(np.float32)
    y, mean, rstd = orc.layernorm_rows(x, w, b, 1e-5)
    for i in range(2):
        row = [float(v) for v in x[i]]
        m = sum(row) / 9
        var = sum((v - m) ** 2 for v in row) / 9
        r = 1 / math.sqrt(var + 1e-5)
        want = [(v - m) * r * float(w[j]) + float(b[j]) for j, v in enumerate(row)]
        np.testing.assert_allclose(y[i], want, rtol=1e-5, atol=1e-6)
        assert abs(mean[i] - m) < 1e-6 and abs(rstd[i] - r) < 1e-5 * r


def test_matmul_brute_force_and_identity():
    rng = np.random.default_rng(8)
    a = rng.standard_normal((5, 7)).astype(np.float32)
    b = rng.standard_normal((7, 3)).astype(np.float32)
    np.testing.assert_allclose(orc.matmul(a, b), orc.matmul_loops(a, b), rtol=1e-5, atol=1e-6)
    eye = np.eye(7, dtype=np.float32)
    np.testing.assert_allclose(orc.matmul(a, eye), a, rtol=0, atol=0)
    # non-square: operand order matters (a transposed operand would not fit)
    assert orc.matmul(a, b).shape == (5, 3)


def test_attention_closed_forms():
    rng = np.random.default_rng(9)
    q = rng.standard_normal((1, 1, 6, 4)).astype(np.float32)
    v = rng.standard_normal((1, 1, 6, 4)).astype(np.float32)
    k_same = np.repeat(rng.standard_normal((1, 1, 1, 4)).astype(np.float32), 6, axis=2)
    # identical keys: uniform attention, output = mean of V
    o = orc.attention(q, k_same, v, 0.5)
    np.testing.assert_allclose(o[0, 0], np.tile(v[0, 0].mean(axis=0), (6, 1)), rtol=1e-5)
    # causal: query row 0 sees only key 0 -> v[0]; row i with identical keys -> mean v[:i+1]
    oc = orc.attention(q, k_same, v, 0.5, causal=True)
    for i in range(6):
        np.testing.assert_allclose(oc[0, 0, i], v[0, 0, :i + 1].mean(axis=0), rtol=1e-5,
                                   atol=1e-6)


def test_attention_brute_force():
    rng = np.random.default_rng(10)
    q, k, v = (rng.standard_normal((1, 1, 5, 3)).astype(np.float32) for _ in range(3))
    for causal in (False, True):
        o = orc.attention(q, k, v, 0.7, causal)
        for i in range(5):
            n = i + 1 if causal else 5
            s = [0.7 * sum(float(q[0, 0, i, d]) * float(k[0, 0, j, d]) for d in range(3))
                 for j in range(n)]
            p = orc.softmax_loops(s)
            want = [sum(p[j] * float(v[0, 0, j, d]) for j in range(n)) for d in range(3)]
            np.testing.assert_allclose(o[0, 0, i], want, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- planted mistakes

def test_checks_reject_planted_mistakes():
    """Mutated copies of the oracle must fail the checks above."""
    sq = gold("matmul_64x64x32")
    a, b = sq["a"], sq["b"]
    wrong = orc.matmul(a[:, ::-1], b)  # wrong K index order
    assert orc.rel_frobenius(wrong, sq["out"]) > 0.5
    wrong = orc.matmul(b.T, a.T)  # operands swapped: (A B)^T instead of A B
    assert orc.rel_frobenius(wrong, sq["out"]) > 0.5
    wrong = orc.matmul(a[:, :-1], b[:-1])  # dropped last K term
    assert orc.rel_frobenius(wrong, sq["out"]) > 1e-3

    s = gold("softmax_32x781")
    x = s["x"].astype(np.float64)
    no_norm = np.exp(x - x.max(axis=1, keepdims=True))
    assert not np.allclose(no_norm, s["out"], rtol=1e-5)
    wrong_axis = np.exp(x - x.max(axis=0, keepdims=True))
    wrong_axis /= wrong_axis.sum(axis=0, keepdims=True)
    assert not np.allclose(wrong_axis, s["out"], rtol=1e-5)

    ln = gold("layernorm_16x300")
    xx = ln["x"].astype(np.float64)
    biased = (xx - xx.mean(1, keepdims=True)) / np.sqrt(xx.var(1, ddof=1, keepdims=True) + 1e-5)
    biased = biased * ln["w"] + ln["b"]
    assert not np.allclose(biased, ln["out"], rtol=1e-5, atol=1e-5)

    at = gold("attention_1x2x64x32_causal")
    full = orc.attention(at["q"], at["k"], at["v"], 32 ** -0.5, causal=False)
    assert orc.rel_frobenius(full, at["out"]) > 0.1
    wrong_scale = orc.attention(at["q"], at["k"], at["v"], 1.0, causal=True)
    assert orc.rel_frobenius(wrong_scale, at["out"]) > 1e-2


# ---------------------------------------------------------------- sampled checks

def test_attention_query_subset_matches_full_rows():
    """q_pos: a subset of query rows, masked by their own positions, gives
    exactly those rows of the full causal result (and of the non-causal one)."""
    at = gold("attention_1x2x64x32_causal")
    q, k, v = at["q"], at["k"], at["v"]
    rows = np.array([0, 5, 31, 32, 63])
    for causal in (False, True):
        full = orc.attention(q, k, v, 32 ** -0.5, causal)
        sub = orc.attention(q[:, :, rows], k, v, 32 ** -0.5, causal, q_pos=rows)
        np.testing.assert_array_equal(sub, full[:, :, rows])
    np.testing.assert_allclose(full, at["out"], rtol=1e-5, atol=1e-6)
    # positions ignored (0..4 assumed) would mask the wrong keys
    wrong = orc.attention(q[:, :, rows], k, v, 32 ** -0.5, True)
    assert orc.rel_frobenius(wrong, full[:, :, rows]) > 0.1


def test_ulp_violations():
    rng = np.random.default_rng(11)
    exact = rng.standard_normal(10000) * 0.02
    for dt, rel in (("float16", 2.0 ** -10), ("bfloat16", 2.0 ** -7)):
        ref = orc.round_to(exact.astype(np.float32), dt)
        assert orc.ulp_violations(ref, ref, dt) == 0
        # one ulp away in either direction (the neighbour in the dtype) passes
        up = ref.astype(np.float64) + np.abs(ref) * rel / 2  # half the binade step
        assert orc.ulp_violations(up, ref, dt) == 0
        # a wrong element, a swapped pair and a NaN are counted
        bad = ref.copy()
        bad[17] *= -1
        bad[[100, 200]] = bad[[200, 100]]
        bad[300] = np.nan
        assert orc.ulp_violations(bad, ref, dt) >= 3
        # three ulps off everywhere is rejected
        assert orc.ulp_violations(ref * (1 + 3 * rel), ref, dt) > 9000
    # fp16 subnormals: the absolute slack covers their fixed 2^-24 spacing
    tiny = np.array([2.0 ** -24, 3 * 2.0 ** -24, 0.0])
    assert orc.ulp_violations(tiny + 2.0 ** -24, tiny, "float16") == 0


def test_panel_rows_cover_every_panel():
    for M, block in ((4096, 64), (8192, 256), (1000, 64), (64, 64), (1, 64)):
        rows = orc.panel_rows(M, block)
        assert rows.min() >= 0 and rows.max() == M - 1
        assert set(rows // block) == set(range((M + block - 1) // block))
        # offsets within the panel vary (not the same wave/lane every time)
        if M // block > 4:
            assert len(set(rows % block)) > 4
    s = orc.spread(128, 8)
    assert s[0] == 0 and s[-1] == 127 and len(s) == 8


# ---------------------------------------------------------------- tolerance checkers

def _bench_like_rows(M, N, seed=0):
    rng = np.random.default_rng(seed)
    return rng.standard_normal((M, N)).astype(np.float16).astype(np.float32)


def _fp32_layernorm(x, w, b, eps, unbiased=False, mean_div=None):
    """A plain fp32 evaluation of examples/03 in a reduction order like a
    GPU's (16 terms per thread, then a tree): what a correct kernel does."""
    M, N = x.shape
    x = x.astype(np.float32)
    part = x.reshape(M, -1, N // 16 if N % 16 == 0 else N).sum(axis=1, dtype=np.float32)
    mean = (part.sum(axis=1, dtype=np.float32) / np.float32(mean_div or N)).astype(np.float32)
    d = (x - mean[:, None]).astype(np.float32)
    sq = (d * d).astype(np.float32).reshape(part.shape[0], -1, part.shape[1])
    var = (sq.sum(axis=1, dtype=np.float32).sum(axis=1, dtype=np.float32)
           / np.float32(N - 1 if unbiased else N)).astype(np.float32)
    rstd = (np.float32(1) / np.sqrt(var + np.float32(eps))).astype(np.float32)
    y = (d * rstd[:, None]).astype(np.float32) * w.astype(np.float32)[None, :] + b.astype(np.float32)
    return y.astype(np.float32), mean, rstd


def test_rel_violations():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((64, 4096)) * 4).astype(np.float32)
    ref = orc.softmax_rows(x)
    # an fp32 evaluation (exp, sum and divide in fp32) is within rtol 1e-5
    e = np.exp(x - x.max(axis=1, keepdims=True)).astype(np.float32)
    fp32 = (e / e.sum(axis=1, keepdims=True, dtype=np.float32)).astype(np.float32)
    assert orc.rel_violations(fp32, ref, 1e-5) == 0
    assert orc.rel_violations(ref * (1 + 0.9e-5), ref, 1e-5) == 0
    # zeroing the probabilities under 1e-6 (which an atol of 1e-6 would pass)
    small = np.where(ref < 1e-6, 0.0, ref)
    assert orc.rel_violations(small, ref, 1e-5) > ref.size // 4
    # a mid-range probability 1e-4 off, an exp with a 2e-5 relative error, a NaN
    bad = ref.copy()
    mid = np.argwhere((ref > 1e-5) & (ref < 1e-3))[0]
    bad[tuple(mid)] *= 1 + 1e-4
    assert orc.rel_violations(bad, ref, 1e-5) == 1
    assert orc.rel_violations(ref * (1 + 2e-5), ref, 1e-5) == ref.size
    bad[-1, -1] = np.nan
    assert tuple(mid) != (63, 4095) and orc.rel_violations(bad, ref, 1e-5) == 2
    # exact zeros of the oracle: an exact zero passes, a nonzero value fails
    assert orc.rel_violations(np.array([0.0, 1e-31]), np.array([0.0, 0.0]), 1e-5) == 0
    assert orc.rel_violations(np.array([1e-20]), np.array([0.0]), 1e-5) == 1


def test_layernorm_violations_accept_fp32_and_reject_mistakes():
    M, N = 256, 8192
    x = _bench_like_rows(M, N)
    rng = np.random.default_rng(5)
    w = (1 + 0.1 * rng.standard_normal(N)).astype(np.float16).astype(np.float32)
    b = (0.1 * rng.standard_normal(N)).astype(np.float16).astype(np.float32)
    y, mean, rstd = _fp32_layernorm(x, w, b, 1e-5)
    for dt in ("float16", "bfloat16", "float32"):
        got = orc.round_to(y, dt)
        assert orc.layernorm_violations(got, mean, rstd, x, w, b, 1e-5, dt) == \
            {"y": 0, "mean": 0, "rstd": 0}
    # the mean divided by N - 1, the unbiased variance, a dropped element
    _, m1, _ = _fp32_layernorm(x, w, b, 1e-5, mean_div=N - 1)
    assert orc.mean_violations(m1, orc.layernorm_rows(x, w, b)[1], x) > M // 2
    _, _, r1 = _fp32_layernorm(x, w, b, 1e-5, unbiased=True)
    assert orc.layernorm_violations(orc.round_to(y, "float16"), mean, r1, x, w, b, 1e-5,
                                    "float16")["rstd"] == M
    x2 = x.copy()
    x2[:, -1] = 0.0
    _, m2, _ = _fp32_layernorm(x2, w, b, 1e-5)
    assert orc.mean_violations(m2, orc.layernorm_rows(x, w, b)[1], x) > M // 2
    # y two fp16 ulps off, one element's sign flipped
    y16 = orc.round_to(y, "float16")
    off = y16 + np.abs(y16) * 2.0 ** -9
    assert orc.layernorm_violations(off, mean, rstd, x, w, b, 1e-5, "float16")["y"] > y.size // 2
    flip = y16.copy()
    flip[3, 5] = -flip[3, 5] if abs(flip[3, 5]) > 1e-3 else 1.0
    assert orc.layernorm_violations(flip, mean, rstd, x, w, b, 1e-5, "float16")["y"] == 1
    # bf16: two ulps off fails
    yb = orc.round_to(y, "bfloat16")
    assert orc.layernorm_violations(yb + np.abs(yb) * 2.0 ** -6, mean, rstd, x, w, b, 1e-5,
                                    "bfloat16")["y"] > y.size // 2
    # fp32 output: the same planted offsets fail the term-scaled rtol
    assert orc.layernorm_violations(y * (1 + 1e-4), mean, rstd, x, w, b, 1e-5,
                                    "float32")["y"] > y.size // 2


def test_attention_sampled_errors_touch_every_program():
    """The sampled attention check passes the oracle's own output and fails
    when any one program's rows are wrong (each (batch, head) x query block
    in turn, on a small launch shaped like the benchmark's)."""
    rng = np.random.default_rng(9)
    B, H, S, D, block = 1, 3, 96, 16, 32
    q, k, v = (orc.round_bf16(rng.standard_normal((B, H, S, D)).astype(np.float32))
               for _ in range(3))
    for causal in (False, True):
        o = orc.attention(q, k, v, D ** -0.5, causal, p_dtype="bfloat16", out_dtype="bfloat16")
        ok = orc.attention_sampled_errors(q, k, v, o, D ** -0.5, causal, block=block,
                                          dense_pairs=2)
        assert ok["worst_row"] < 1e-6 and ok["worst_pair"] < 1e-6
        assert ok["rows"] >= B * H * (S // block)
        for bh in range(B * H):
            for blk in range(S // block):
                bad = o.copy()
                bi, hi = divmod(bh, H)
                # the program's rows taken from another head: plausible values, wrong ones
                bad[bi, hi, blk * block:(blk + 1) * block] = \
                    o[bi, (hi + 1) % H, blk * block:(blk + 1) * block]
                res = orc.attention_sampled_errors(q, k, v, bad, D ** -0.5, causal, block=block,
                                                   dense_pairs=2)
                assert res["worst_row"] > 1e-2, (causal, bh, blk)
