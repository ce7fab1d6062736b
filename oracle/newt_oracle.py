"""CPU oracle for the newt hot path - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker (or as the timed CPU baseline). No product
code path calls it; the HIP extension failing to load is an error, never a
fallback to this file.

Each function restates, in numpy, the algorithm of one kernel the reference
runs on the GPU, in the arithmetic the reference specifies:

  vector_add      examples/01_vector_add.py:14-21      out = x + y (fp32, exact)
  softmax_rows    examples/02_fused_softmax.py:15-24   exp(x - rowmax) / rowsum, fp32
  layernorm_rows  examples/03_layernorm.py:13-27       two-pass mean/var, fp32 math,
                                                       output cast to x.dtype,
                                                       plus saved mean / rstd
  matmul          examples/04_matmul.py:14-45          fp32 accumulation of the
                                                       fp16/bf16 products, cast to C dtype
  attention       examples/05_fused_attention.py:14-48 softmax(q k^T * scale [+ causal
                                                       mask]) v with fp32 softmax state,
                                                       P rounded to the value dtype
                                                       before P @ V, output in q.dtype

Pinning (tests/test_oracle.py): every function is checked against the golden
fixtures in tests/golden (written by torch eager in float64 - the reference's
own oracle), against closed forms (softmax of a constant row, rows summing to
1, layernorm output moments, attention with identical keys returning the mean
of V, causal row 0 returning v[0]) and against brute-force loops on tiny
inputs, so that a dropped term, wrong axis or transposed operand fails.

The checkers below the restatements (ulp_violations, rel_violations,
mean_violations, layernorm_violations, attention_sampled_errors, panel_rows)
hold a kernel's output to the stated tolerance; tests/test_oracle.py checks
that each passes a correct fp32 evaluation and rejects planted mistakes.
"""

import numpy as np

def round_bf16(x):
    """Round float32 values to bfloat16 (round-to-nearest-even), return float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = np.isnan(x)
    lsb = (u >> 16) & 1
    u = (u + 0x7FFF + lsb) & 0xFFFF0000
    out = u.astype(np.uint32).view(np.float32)
    out = np.where(nan, np.float32(np.nan), out)
    return out


def round_to(x, dtype):
    """Round float32 values to `dtype` ('float32' | 'float16' | 'bfloat16')."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "float16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bfloat16":
        return round_bf16(x)
    return x


def vector_add(x, y):
    """examples/01_vector_add.py:14-21: elementwise IEEE fp32 add."""
    return (np.asarray(x, np.float32) + np.asarray(y, np.float32)).astype(np.float32)


def softmax_rows(x):
    """examples/02_fused_softmax.py:15-24: row max, exp(x - max), row sum, divide.
    fp32 throughout (float64 intermediate exp for a tight reference)."""
    x = np.asarray(x, np.float32)
    m = x.max(axis=1, keepdims=True)
    e = np.exp((x - m).astype(np.float64))
    return (e / e.sum(axis=1, keepdims=True)).astype(np.float32)


def layernorm_rows(x, w, b, eps=1e-5, out_dtype="float32"):
    """examples/03_layernorm.py:13-27 (two-pass: mean, then mean of squared
    deviations), fp32 math on upcast inputs; returns (y, mean, rstd) with y
    rounded to out_dtype and mean/rstd in fp32."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    b = np.asarray(b, np.float64)
    n = x.shape[1]
    mean = x.sum(axis=1) / n
    diff = x - mean[:, None]
    var = (diff * diff).sum(axis=1) / n
    rstd = 1.0 / np.sqrt(var + eps)
    y = diff * rstd[:, None] * w[None, :] + b[None, :]
    return (round_to(y.astype(np.float32), out_dtype), mean.astype(np.float32),
            rstd.astype(np.float32))


def matmul(a, b, out_dtype="float32"):
    """examples/04_matmul.py:14-45: C = A @ B with fp32 (here fp64) accumulation
    of the (already fp16/bf16-valued) inputs, rounded to the C dtype."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return round_to((a @ b).astype(np.float32), out_dtype)


def attention(q, k, v, scale, causal=False, p_dtype=None, out_dtype="float32",
              q_pos=None):
    """examples/05_fused_attention.py:14-48 generalised to [B, H, S, D]:
    S = q k^T * scale, optional causal mask (key index <= query index),
    P = softmax(S) (fp32 state), P rounded to the value dtype before P @ V
    (the reference casts p to the MMA dtype), O = P V / rowsum.
    The normalisation uses the unrounded row sums, as the online-softmax
    kernel accumulates l_i from the fp32 probabilities.
    q_pos: sequence positions of q's rows when q holds a subset of them
    (default 0..M-1); the causal mask compares key indices with these."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    s = (q @ np.swapaxes(k, -1, -2)) * scale
    if causal:
        M, N = s.shape[-2:]
        pos = np.arange(M) if q_pos is None else np.asarray(q_pos)
        keep = np.arange(N)[None, :] <= pos[:, None]
        s = np.where(keep, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    p = np.exp(s - m)
    l = p.sum(axis=-1, keepdims=True)
    if p_dtype is not None:
        p = round_to(p.astype(np.float32), p_dtype).astype(np.float64)
    o = (p @ v) / l
    return round_to(o.astype(np.float32), out_dtype)


def rel_frobenius(actual, expected):
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    return float(np.linalg.norm(a - e) / max(np.linalg.norm(e), 1e-30))


# relative spacing of a value's binade: ulp(x) <= REL_ULP * |x| for normal x
REL_ULP = {"float16": 2.0 ** -10, "bfloat16": 2.0 ** -7, "float32": 2.0 ** -23}


def ulp_violations(actual, expected, dtype, atol=1e-6):
    """Number of elements of `actual` farther than one ulp of `dtype` (plus
    atol, for subnormal results) from `expected`, the exact product rounded
    to dtype. A kernel that accumulates in fp32 and rounds once lands within
    one ulp of it; a wrong element (a wrong tile, row or column) does not."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    bad = np.abs(a - e) > REL_ULP[dtype] * np.abs(e) + atol
    return int(np.count_nonzero(bad | np.isnan(a)))


U_FP32 = 2.0 ** -24     # unit roundoff of fp32 (half its relative ulp)
U_FP16_SUB = 2.0 ** -24  # spacing of fp16 subnormals


def rel_violations(actual, expected, rtol, floor=1e-30):
    """Number of elements farther than rtol * |expected| + floor from
    `expected` (NaN counts as a violation). A relative check: the floor
    only keeps an exact zero of the oracle from demanding an exact zero of
    the kernel, so a kernel that writes 0 where the oracle holds a small
    positive value fails."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    ok = np.abs(a - e) <= rtol * np.abs(e) + floor
    return int(np.count_nonzero(~ok))


def mean_violations(actual, expected, x, rtol=1e-5):
    """Rows whose fp32 mean is farther than rtol * |mean| + U_FP32 * mean(|x|)
    from the exact one.

    A mean is an fp32 sum of the N terms of a row: its rounding error in any
    reduction tree of depth D is at most about D * U_FP32 * sum(|x_i|)
    (Higham, Accuracy and Stability of Numerical Algorithms, 2nd ed., 4.2),
    which rtol * |mean| cannot hold where the row's sum cancels. The floor
    U_FP32 * mean(|x|) is 1/D of that worst case (D ~ 30 for 8192 terms: 16
    per thread, 6 lane levels, 8 waves) and ~13x the largest error of fp32
    tree sums over the benchmark rows (N(0,1), N = 8192); it is far below
    the shift of a planted mistake such as dividing by N - 1 (|mean| / N)."""
    a = np.asarray(actual, np.float64).reshape(-1)
    e = np.asarray(expected, np.float64).reshape(-1)
    xs = np.abs(np.asarray(x, np.float64)).mean(axis=1)
    ok = np.abs(a - e) <= rtol * np.abs(e) + U_FP32 * xs
    return int(np.count_nonzero(~ok))


def layernorm_violations(y, mean, rstd, x, w, b, eps=1e-5, out_dtype="float16", rtol=1e-5):
    """Element / row counts of a layernorm result beyond its tolerance, per
    output, against layernorm_rows on the same inputs:
      y     fp16 / bf16 output: within one ulp of the exact result rounded to
            the output dtype (ulp_violations; the absolute slack is the fp16
            subnormal spacing 2^-24, or for bf16 8 fp32 units of the terms'
            magnitude |x - mean| * rstd * |w| + |b|); fp32 output: within rtol
            of that magnitude, since y itself cancels where b meets the
            normalised term
      mean  mean_violations (rtol, floor one fp32 unit of mean(|x|))
      rstd  rtol, relative (a sum of squares does not cancel)"""
    ry, rm, rr = layernorm_rows(x, w, b, eps, out_dtype)
    xf = np.asarray(x, np.float64)
    # magnitude of the terms y is computed from (y itself cancels where b
    # meets the normalised term)
    scale = (np.abs(xf - rm.astype(np.float64)[:, None]) * rr.astype(np.float64)[:, None]
             * np.abs(np.asarray(w, np.float64))[None, :]
             + np.abs(np.asarray(b, np.float64))[None, :])
    if out_dtype == "float16":
        y_bad = ulp_violations(y, ry, out_dtype, atol=U_FP16_SUB)
    elif out_dtype == "bfloat16":
        # bf16 keeps fp32's exponent range: near zero its ulp falls below the
        # fp32 evaluation's own error, bounded by 8 units of the terms' magnitude
        y_bad = ulp_violations(y, ry, out_dtype, atol=8 * U_FP32 * scale)
    else:
        d = np.abs(np.asarray(y, np.float64) - ry)
        y_bad = int(np.count_nonzero(~(d <= rtol * scale)))
    return {"y": y_bad, "mean": mean_violations(mean, rm, x, rtol),
            "rstd": rel_violations(rstd, rr, rtol)}


def panel_rows(M, block=64, extra=(0,), shift=0):
    """Row indices touching every `block`-row panel of an M-row output (one
    row per panel at an offset that cycles through the panel, so different
    waves and lanes are sampled; `shift` moves every offset, so calls for
    different heads or batches sample different lanes), plus M - 1 and
    `extra`."""
    rows = {p * block + (p * 29 + 7 + shift) % block for p in range((M + block - 1) // block)}
    rows = {r for r in rows if r < M} | {M - 1} | {r for r in extra if 0 <= r < M}
    return np.array(sorted(rows))


def attention_sampled_errors(q, k, v, o, scale, causal, block=128, dense_pairs=8,
                             p_dtype="bfloat16", out_dtype="bfloat16"):
    """Relative Frobenius errors of an attention output o [B, H, S, D] against
    `attention` on rows that touch every program of a launch whose programs
    own `block` query rows (or a multiple of them) of one (batch, head):
      sampled  every (batch, head) pair, one row of every `block`-row query
               block, at an offset that cycles through the block and moves
               with the pair (panel_rows with a per-pair shift)
      dense    `dense_pairs` pairs spread over all of them, every row of the
               first, a middle and the last query block
    Returns {"rows": rows checked, "worst_row": the largest per-row error,
    "worst_pair": the largest error over one pair's dense rows}."""
    B, H, S, D = q.shape
    nb = (S + block - 1) // block
    dense = np.concatenate([np.arange(i * block, min(S, (i + 1) * block))
                            for i in sorted({0, nb // 2, nb - 1})])
    dense_set = set(int(i) for i in spread(B * H, dense_pairs))
    worst_row, worst_pair, count = 0.0, 0.0, 0
    for bh in range(B * H):
        bi, hi = divmod(bh, H)
        rows = panel_rows(S, block, extra=(), shift=bh * 13)
        if bh in dense_set:
            rows = np.union1d(rows, dense)
        ref = attention(q[bi, hi, rows], k[bi, hi], v[bi, hi], scale, causal, p_dtype=p_dtype,
                        out_dtype=out_dtype, q_pos=rows)
        got = o[bi, hi, rows]
        num = np.linalg.norm(got.astype(np.float64) - ref, axis=1)
        den = np.maximum(np.linalg.norm(ref.astype(np.float64), axis=1), 1e-30)
        bad = np.isnan(got).any(axis=1)
        worst_row = max(worst_row, float(np.max(np.where(bad, np.inf, num / den))))
        if bh in dense_set:
            sel = np.isin(rows, dense)
            worst_pair = max(worst_pair, rel_frobenius(got[sel], ref[sel]))
        count += len(rows)
    return {"rows": count, "worst_row": worst_row, "worst_pair": worst_pair}


def spread(n, count):
    """`count` indices spread over range(n), always holding 0 and n - 1."""
    if count >= n:
        return np.arange(n)
    return np.unique(np.round(np.linspace(0, n - 1, count)).astype(np.int64))


# -- brute-force forms for tiny inputs (pinning helpers) -------------------------

def matmul_loops(a, b):
    M, K = len(a), len(a[0])
    N = len(b[0])
    return [[sum(float(a[i][kk]) * float(b[kk][j]) for kk in range(K)) for j in range(N)]
            for i in range(M)]


def softmax_loops(row):
    import math
    m = max(row)
    e = [math.exp(v - m) for v in row]
    s = sum(e)
    return [v / s for v in e]
