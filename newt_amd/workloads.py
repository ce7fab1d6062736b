"""The five hot-path workloads written in the newt DSL, with host wrappers.

These are user-level kernels exactly as a newt user writes them (the
reference's examples/01-05), extended to the benchmark configurations:
  add_kernel        examples/01_vector_add.py:14-21 (unchanged)
  copy_kernel       no reference counterpart: a streaming copy that measures
                    the HBM ceiling of a kernel compiled by newt (bench.py)
  softmax_kernel    examples/02_fused_softmax.py:15-24 (unchanged)
  layernorm_kernel  examples/03_layernorm.py:13-27 + stores of the saved
                    per-row mean / rstd (config 3 asks for them)
  matmul_kernel     examples/04_matmul.py:14-45 (unchanged body), autotuned over
                    a configuration space re-derived for gfx950
  attention_kernel  examples/05_fused_attention.py:14-48 generalised to
                    [batch, heads, seq, head_dim] with a batch*head grid axis,
                    strides, an optional causal mask with the loop bound trimmed
                    to the diagonal, p cast to V's dtype before P @ V, and the
                    softmax written on exp2 with log2(e) folded into the scale
                    (exp(x) = exp2(x*log2 e): the same softmax, fewer
                    instructions per element), the exponents referred to each
                    row's first-block maximum (no rescale in the main loops;
                    an online-softmax pass for a program where some row's sum
                    passes 2^80 or the accumulator overflows); launched with
                    waves_per_eu=2 so two waves share each SIMD and one
                    wave's softmax runs while the other's MFMAs do
  attention_plain_kernel
                    examples/05_fused_attention.py:14-48 as written there
                    (nl.exp, qk * scale, a where mask), generalised only by the
                    batch*head axis and the causal mask; also the kernel for a
                    scale <= 0
  dt_matmul         examples/deuteron/01_matmul.py (unchanged body): the tile
                    DSL traced to newt and autotuned against its eager oracle
Everything is compiled by newt_amd's compiler to HIP for gfx950.
"""

import torch

import newt_amd as newt
import newt_amd.language as nl


# ---------------------------------------------------------------------------
# 1. vector add
# ---------------------------------------------------------------------------
@newt.jit
def add_kernel(x_ptr, y_ptr, out_ptr, n, BLOCK: nl.constexpr):
    pid = nl.program_id(0)
    offs = pid * BLOCK + nl.arange(0, BLOCK)
    mask = offs < n
    x = nl.load(x_ptr + offs, mask=mask)
    y = nl.load(y_ptr + offs, mask=mask)
    nl.store(out_ptr + offs, x + y, mask=mask)


def add(x, y, out=None, BLOCK=1024, num_warps=4):
    out = torch.empty_like(x) if out is None else out
    n = x.numel()
    add_kernel[(newt.cdiv(n, BLOCK),)](x, y, out, n, BLOCK=BLOCK, num_warps=num_warps)
    return out


@newt.jit
def copy_kernel(src_ptr, dst_ptr, n, BLOCK: nl.constexpr):
    # a one-read-one-write stream: the HBM ceiling any kernel compiled by
    # newt that reads and writes its bytes once can reach at a given size
    offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
    mask = offs < n
    nl.store(dst_ptr + offs, nl.load(src_ptr + offs, mask=mask), mask=mask)


def copy(src, dst, BLOCK=2048, num_warps=4):
    # 8 fp32 per thread (two 16-byte loads): the fastest shape measured at
    # 128 MiB and 256 MiB moved (BLOCK 1024-16384, 4-16 waves)
    n = src.numel()
    copy_kernel[(newt.cdiv(n, BLOCK),)](src, dst, n, BLOCK=BLOCK, num_warps=num_warps)
    return dst


# ---------------------------------------------------------------------------
# 2. fused row softmax
# ---------------------------------------------------------------------------
@newt.jit
def softmax_kernel(x_ptr, out_ptr, N, stride, BLOCK_N: nl.constexpr):
    row = nl.program_id(0)
    cols = nl.arange(0, BLOCK_N)
    mask = cols < N
    x = nl.load(x_ptr + row * stride + cols, mask=mask, other=float("-inf"))
    x = x - nl.max(x, axis=0)
    num = nl.exp(x)
    den = nl.sum(num, axis=0)
    nl.store(out_ptr + row * stride + cols, num / den, mask=mask)


def softmax_warps(block_n):
    # one row per workgroup, 16 fp32 values (four 16-byte loads) per thread:
    # enough bytes in flight per wave, and several rows per CU to overlap one
    # row's reductions with another's loads (measured best at 1000..8192 cols)
    return max(2, min(16, block_n // 1024))


def softmax(x, out=None, num_warps=None):
    M, N = x.shape
    out = torch.empty_like(x) if out is None else out
    BLOCK_N = newt.next_power_of_2(N)
    nw = num_warps or softmax_warps(BLOCK_N)
    softmax_kernel[(M,)](x, out, N, x.stride(0), BLOCK_N=BLOCK_N, num_warps=nw)
    return out


# ---------------------------------------------------------------------------
# 3. layernorm forward (+ saved mean / rstd)
# ---------------------------------------------------------------------------
@newt.jit
def layernorm_kernel(x_ptr, w_ptr, b_ptr, out_ptr, mean_ptr, rstd_ptr, N, stride, eps,
                     BLOCK_N: nl.constexpr):
    row = nl.program_id(0)
    cols = nl.arange(0, BLOCK_N)
    mask = cols < N
    x = nl.load(x_ptr + row * stride + cols, mask=mask, other=0.0)
    mean = nl.sum(x, axis=0) / N
    diff = nl.where(mask, x - mean, 0.0)
    var = nl.sum(diff * diff, axis=0) / N
    rstd = nl.rsqrt(var + eps)
    w = nl.load(w_ptr + cols, mask=mask)
    b = nl.load(b_ptr + cols, mask=mask)
    y = (x - mean) * rstd * w + b
    nl.store(out_ptr + row * stride + cols, y, mask=mask)
    nl.store(mean_ptr + row, mean)
    nl.store(rstd_ptr + row, rstd)


def layernorm(x, w, b, eps=1e-5, out=None, num_warps=None):
    M, N = x.shape
    out = torch.empty_like(x) if out is None else out
    mean = torch.empty(M, device=x.device, dtype=torch.float32)
    rstd = torch.empty(M, device=x.device, dtype=torch.float32)
    BLOCK_N = newt.next_power_of_2(N)
    # 16 fp16 elements (two 16-byte loads) per thread: a 8192-wide row on 8
    # waves measured ~2% faster than on 4 (fewer registers per wave, and the
    # same bytes in flight per CU); 16 waves per row were 20% slower
    nw = num_warps or max(2, min(8, BLOCK_N // 1024))
    layernorm_kernel[(M,)](x, w, b, out, mean, rstd, N, x.stride(0), eps,
                           BLOCK_N=BLOCK_N, num_warps=nw)
    return out, mean, rstd


# ---------------------------------------------------------------------------
# 4. matmul (fp16 / bf16, fp32 accumulate)
# ---------------------------------------------------------------------------
@newt.jit
def matmul_kernel(a_ptr, b_ptr, c_ptr, M, N, K,
                  sam, sak, sbk, sbn, scm, scn,
                  BLOCK_M: nl.constexpr, BLOCK_N: nl.constexpr, BLOCK_K: nl.constexpr):
    pid_m = nl.program_id(0)
    pid_n = nl.program_id(1)
    offs_m = pid_m * BLOCK_M + nl.arange(0, BLOCK_M)
    offs_n = pid_n * BLOCK_N + nl.arange(0, BLOCK_N)
    offs_k = nl.arange(0, BLOCK_K)
    a_ptrs = a_ptr + offs_m[:, None] * sam + offs_k[None, :] * sak
    b_ptrs = b_ptr + offs_k[:, None] * sbk + offs_n[None, :] * sbn
    acc = nl.zeros((BLOCK_M, BLOCK_N), dtype=nl.float32)
    for k in range(nl.cdiv(K, BLOCK_K)):
        a_mask = (offs_m[:, None] < M) & (offs_k[None, :] < K - k * BLOCK_K)
        b_mask = (offs_k[:, None] < K - k * BLOCK_K) & (offs_n[None, :] < N)
        a = nl.load(a_ptrs, mask=a_mask, other=0.0)
        b = nl.load(b_ptrs, mask=b_mask, other=0.0)
        acc = nl.dot(a, b, acc)
        a_ptrs += BLOCK_K * sak
        b_ptrs += BLOCK_K * sbk
    c_ptrs = c_ptr + offs_m[:, None] * scm + offs_n[None, :] * scn
    c_mask = (offs_m[:, None] < M) & (offs_n[None, :] < N)
    nl.store(c_ptrs, acc.to(c_ptr.dtype.element_ty), mask=c_mask)


# gfx950 search space: 64-wide waves, 160 KB LDS per CU, 256 CUs. The k-loop is
# software-pipelined num_stages deep through distinct LDS stages, so tiles of
# 256x256 with BLOCK_K=32 and 4 stages (128 KB) give each CU one workgroup:
# 4 waves with a 128x128 MFMA sub-tile each (accumulators in AGPRs; half the
# LDS operand reads per flop of 8 waves) or 8 waves with 128x64; smaller tiles
# keep grids of >= 256 workgroups for smaller problems.
MATMUL_CONFIGS = [
    newt.Config({"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": 32}, num_warps=4, num_stages=4),
    newt.Config({"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": 32}, num_warps=8, num_stages=4),
    newt.Config({"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": 64}, num_warps=8, num_stages=2),
    newt.Config({"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": 32}, num_warps=8, num_stages=3),
    newt.Config({"BLOCK_M": 256, "BLOCK_N": 128, "BLOCK_K": 32}, num_warps=8, num_stages=4),
    newt.Config({"BLOCK_M": 128, "BLOCK_N": 256, "BLOCK_K": 32}, num_warps=8, num_stages=4),
    newt.Config({"BLOCK_M": 128, "BLOCK_N": 128, "BLOCK_K": 64}, num_warps=4, num_stages=3),
    # 2048^3 (one 128x128 tile per CU): 64-deep k-steps with 4 stages (128 KB)
    # measured 813 against 799 TFLOP/s for the 32-deep tile below
    newt.Config({"BLOCK_M": 128, "BLOCK_N": 128, "BLOCK_K": 64}, num_warps=4, num_stages=4),
    newt.Config({"BLOCK_M": 128, "BLOCK_N": 128, "BLOCK_K": 32}, num_warps=4, num_stages=4),
    newt.Config({"BLOCK_M": 64, "BLOCK_N": 128, "BLOCK_K": 64}, num_warps=4, num_stages=3),
    # 64x64 tiles give a 1024^3 problem 256 workgroups (one per CU)
    newt.Config({"BLOCK_M": 64, "BLOCK_N": 64, "BLOCK_K": 64}, num_warps=4, num_stages=4),
    newt.Config({"BLOCK_M": 64, "BLOCK_N": 64, "BLOCK_K": 64}, num_warps=4, num_stages=3),
]

matmul_tuned = newt.autotune(configs=MATMUL_CONFIGS, key=["M", "N", "K"])(matmul_kernel)

# fp32 operands run on the fp32 MFMA (v_mfma_f32_32x32x2_f32, full precision;
# gfx950 has no tf32) through the same pipelined k-loop: 16-deep k-steps keep
# 3-4 fp32 stages within the LDS
MATMUL_CONFIGS_FP32 = [
    newt.Config({"BLOCK_M": 256, "BLOCK_N": 256, "BLOCK_K": 16}, num_warps=8, num_stages=3),
    newt.Config({"BLOCK_M": 256, "BLOCK_N": 128, "BLOCK_K": 16}, num_warps=8, num_stages=4),
    newt.Config({"BLOCK_M": 128, "BLOCK_N": 128, "BLOCK_K": 32}, num_warps=4, num_stages=3),
    newt.Config({"BLOCK_M": 128, "BLOCK_N": 128, "BLOCK_K": 16}, num_warps=4, num_stages=4),
]
matmul_tuned_fp32 = newt.autotune(configs=MATMUL_CONFIGS_FP32, key=["M", "N", "K"])(matmul_kernel)


def matmul(a, b, c=None, config=None):
    M, K = a.shape
    K2, N = b.shape
    assert K == K2
    c = torch.empty(M, N, device=a.device, dtype=a.dtype) if c is None else c
    args = (a, b, c, M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1),
            c.stride(0), c.stride(1))
    if config is None:
        grid = lambda meta: (newt.cdiv(M, meta["BLOCK_M"]), newt.cdiv(N, meta["BLOCK_N"]))
        (matmul_tuned_fp32 if a.dtype == torch.float32 else matmul_tuned)[grid](*args)
    else:
        grid = (newt.cdiv(M, config.kwargs["BLOCK_M"]), newt.cdiv(N, config.kwargs["BLOCK_N"]))
        matmul_kernel[grid](*args, **config.kwargs, num_warps=config.num_warps,
                            num_stages=config.num_stages)
    return c


# ---------------------------------------------------------------------------
# 5. flash attention forward
# ---------------------------------------------------------------------------
@newt.jit
def attention_kernel(q_ptr, k_ptr, v_ptr, o_ptr, S, H, scale,
                     sqb, sqh, sqm, skb, skh, skn, svb, svh, svn, sob, soh, som,
                     BLOCK_M: nl.constexpr, BLOCK_N: nl.constexpr, D: nl.constexpr,
                     CAUSAL: nl.constexpr):
    pid = nl.program_id(0)
    bh = nl.program_id(1)
    if CAUSAL:
        # Query block i does i + 1 key blocks: each XCD should start its
        # heaviest programs first, so that the last to start are short ones
        # (longest-processing-time-first order, a short tail). Program ids
        # arrive renumbered so that each XCD runs one contiguous range of
        # lin = pid + nqb * bh in increasing order; when the heads split evenly
        # over the 8 XCDs that range is gh whole heads, which it would run one
        # after another, heaviest to lightest within each. The range is taken
        # in groups of grp = 4 heads (all gh when 4 does not divide gh), and
        # within a group its r-th program becomes weight rank r // grp of head
        # r % grp: every head's heaviest block, then every head's next, and so
        # on, with four heads' keys and values in the XCD's L2 at a time. (Any
        # bijection of the programs computes the same result.)
        nqb = nl.num_programs(0)
        nbh = nl.num_programs(1)
        if nbh % 8 == 0:
            gh = nbh // 8
            grp = gh
            if gh % 4 == 0:
                grp = 4
            lin = pid + nqb * bh
            r = lin % (gh * nqb)
            rr = r % (grp * nqb)
            bh = lin // (gh * nqb) * gh + r // (grp * nqb) * grp + rr % grp
            pid = rr // grp
        pid = nqb - 1 - pid
    bi = bh // H
    hi = bh % H
    q_base = q_ptr + bi * sqb + hi * sqh
    k_base = k_ptr + bi * skb + hi * skh
    v_base = v_ptr + bi * svb + hi * svh
    o_base = o_ptr + bi * sob + hi * soh
    offs_m = pid * BLOCK_M + nl.arange(0, BLOCK_M)
    offs_d = nl.arange(0, D)
    qmask = offs_m[:, None] < S
    q = nl.load(q_base + offs_m[:, None] * sqm + offs_d[None, :], mask=qmask, other=0.0)

    qk_scale = scale * 1.4426950408889634  # log2(e): the softmax runs on exp2
    # The exponents share one reference point per row, m_i: the row's maximum
    # over the first key block, fixed for the rest of the row. O = acc / l_i
    # is the same quotient whatever reference point the exponents share, so
    # the loops never rescale acc: p = exp2(qk * s - m_i) only grows past 1
    # where a later score exceeds the first block's maximum. While every p
    # stays below 2^80, l_i stays far inside fp32's range; a row whose sum l_i
    # passes 2^80 (some score 80 or more above that maximum, in log2 units),
    # or an acc that overflowed, sends the program through the online-softmax
    # loop at the end, which rescales at every block. (A rescale inside the
    # main loops costs a cross-wave maximum, a barrier and a branch per key
    # block.)
    m_i = nl.zeros((BLOCK_M,), dtype=nl.float32)
    l_i = nl.zeros((BLOCK_M,), dtype=nl.float32)
    acc = nl.zeros((BLOCK_M, D), dtype=nl.float32)

    # key blocks wholly inside the sequence (and, causal, wholly below the
    # diagonal of every row of this program) need no mask; the ragged tail and
    # the diagonal blocks run in a second, masked loop. Scores stay unscaled:
    # the scale is applied inside the exponent's fma, and the reference is
    # max(qk) * qk_scale (= max(qk * qk_scale): rounding is monotonic).
    full_n = S // BLOCK_N * BLOCK_N
    end_n = S
    if CAUSAL:
        full_n = nl.minimum(full_n, pid * BLOCK_M // BLOCK_N * BLOCK_N)
        end_n = nl.minimum(S, (pid + 1) * BLOCK_M)
    for start_n in range(0, full_n, BLOCK_N):
        offs_n = start_n + nl.arange(0, BLOCK_N)
        k = nl.load(k_base + offs_n[:, None] * skn + offs_d[None, :])
        qk = nl.dot(q, nl.trans(k))
        if start_n == 0:
            m_i = nl.max(qk, axis=1) * qk_scale
        p = nl.exp2(nl.fma(qk, qk_scale, -m_i[:, None]))
        l_i = l_i + nl.sum(p, axis=1)
        v = nl.load(v_base + offs_n[:, None] * svn + offs_d[None, :])
        acc = nl.dot(p.to(v_ptr.dtype.element_ty), v, acc)
    for start_n in range(full_n, end_n, BLOCK_N):
        offs_n = start_n + nl.arange(0, BLOCK_N)
        nmask = offs_n[:, None] < S
        k = nl.load(k_base + offs_n[:, None] * skn + offs_d[None, :], mask=nmask, other=0.0)
        qk = nl.dot(q, nl.trans(k))
        if CAUSAL:
            qk = nl.where((offs_m[:, None] >= offs_n[None, :]) & (offs_n[None, :] < S),
                          qk, float("-inf"))
        else:
            qk = nl.where(offs_n[None, :] < S, qk, float("-inf"))
        # the first key block has key 0 in it, which no row masks: every row's
        # reference is finite (masked scores are -inf, p = exp2(-inf) = 0)
        if start_n == 0:
            m_i = nl.max(qk, axis=1) * qk_scale
        p = nl.exp2(nl.fma(qk, qk_scale, -m_i[:, None]))
        l_i = l_i + nl.sum(p, axis=1)
        v = nl.load(v_base + offs_n[:, None] * svn + offs_d[None, :], mask=nmask, other=0.0)
        acc = nl.dot(p.to(v_ptr.dtype.element_ty), v, acc)

    # acc <= l_i * max|v|: past the first block's maximum, p grows acc by up
    # to 2^80 more than the per-block rescale's p <= 1 does, so for values
    # above ~2^48 acc can overflow where the rescaled sum stays finite.
    # acc * 0 is NaN exactly where acc holds an inf or NaN (no fast-math:
    # the product is not folded), which makes `peak` NaN and sends the
    # program through the rescaling pass too.
    peak = nl.max(l_i) + nl.sum(acc * 0.0)
    if not (peak <= 1.2089258196146292e24):  # 2^80: start again with a rescale per block
        m_i = nl.full((BLOCK_M,), float("-inf"), dtype=nl.float32)
        l_i = nl.zeros((BLOCK_M,), dtype=nl.float32)
        acc = nl.zeros((BLOCK_M, D), dtype=nl.float32)
        for start_n in range(0, end_n, BLOCK_N):
            offs_n = start_n + nl.arange(0, BLOCK_N)
            nmask = offs_n[:, None] < S
            k = nl.load(k_base + offs_n[:, None] * skn + offs_d[None, :], mask=nmask, other=0.0)
            qk = nl.dot(q, nl.trans(k))
            if CAUSAL:
                qk = nl.where((offs_m[:, None] >= offs_n[None, :]) & (offs_n[None, :] < S),
                              qk, float("-inf"))
            else:
                qk = nl.where(offs_n[None, :] < S, qk, float("-inf"))
            m_new = nl.maximum(m_i, nl.max(qk, axis=1) * qk_scale)
            alpha = nl.exp2(m_i - m_new)
            p = nl.exp2(nl.fma(qk, qk_scale, -m_new[:, None]))
            l_i = l_i * alpha + nl.sum(p, axis=1)
            acc = acc * alpha[:, None]
            v = nl.load(v_base + offs_n[:, None] * svn + offs_d[None, :], mask=nmask, other=0.0)
            acc = nl.dot(p.to(v_ptr.dtype.element_ty), v, acc)
            m_i = m_new

    # one reciprocal per row and a multiply per element instead of a division
    # per element (an IEEE fp32 division is ~10 instructions); the two differ
    # by at most an ulp of fp32, far below the bf16 rounding of the output
    acc = acc * (1.0 / l_i)[:, None]
    nl.store(o_base + offs_m[:, None] * som + offs_d[None, :], acc.to(o_ptr.dtype.element_ty),
             mask=qmask)


@newt.jit
def attention_plain_kernel(q_ptr, k_ptr, v_ptr, o_ptr, S, H, scale,
                           sqb, sqh, sqm, skb, skh, skn, svb, svh, svn, sob, soh, som,
                           BLOCK_M: nl.constexpr, BLOCK_N: nl.constexpr, D: nl.constexpr,
                           CAUSAL: nl.constexpr):
    # examples/05_fused_attention.py:14-48 as written there (one key loop,
    # nl.exp, qk * scale, a where mask, p cast to V's dtype), generalised only
    # by the batch*head grid axis and the causal mask with its loop bound
    pid = nl.program_id(0)
    bh = nl.program_id(1)
    bi = bh // H
    hi = bh % H
    q_base = q_ptr + bi * sqb + hi * sqh
    k_base = k_ptr + bi * skb + hi * skh
    v_base = v_ptr + bi * svb + hi * svh
    o_base = o_ptr + bi * sob + hi * soh
    offs_m = pid * BLOCK_M + nl.arange(0, BLOCK_M)
    offs_d = nl.arange(0, D)
    qmask = offs_m[:, None] < S
    q = nl.load(q_base + offs_m[:, None] * sqm + offs_d[None, :], mask=qmask, other=0.0)

    m_i = nl.full((BLOCK_M,), float("-inf"), dtype=nl.float32)
    l_i = nl.zeros((BLOCK_M,), dtype=nl.float32)
    acc = nl.zeros((BLOCK_M, D), dtype=nl.float32)

    end_n = S
    if CAUSAL:
        end_n = nl.minimum(S, (pid + 1) * BLOCK_M)
    for start_n in range(0, end_n, BLOCK_N):
        offs_n = start_n + nl.arange(0, BLOCK_N)
        nmask = offs_n[:, None] < S
        k = nl.load(k_base + offs_n[:, None] * skn + offs_d[None, :], mask=nmask, other=0.0)
        qk = nl.dot(q, nl.trans(k)) * scale
        if CAUSAL:
            qk = nl.where((offs_n[None, :] < S) & (offs_m[:, None] >= offs_n[None, :]),
                          qk, float("-inf"))
        else:
            qk = nl.where(offs_n[None, :] < S, qk, float("-inf"))
        m_new = nl.maximum(m_i, nl.max(qk, axis=1))
        alpha = nl.exp(m_i - m_new)
        p = nl.exp(qk - m_new[:, None])
        l_i = l_i * alpha + nl.sum(p, axis=1)
        acc = acc * alpha[:, None]
        v = nl.load(v_base + offs_n[:, None] * svn + offs_d[None, :], mask=nmask, other=0.0)
        acc = nl.dot(p.to(v_ptr.dtype.element_ty), v, acc)
        m_i = m_new

    acc = acc / l_i[:, None]
    nl.store(o_base + offs_m[:, None] * som + offs_d[None, :], acc, mask=qmask)


def attention(q, k, v, causal=False, scale=None, out=None, BLOCK_M=None, BLOCK_N=64,
              num_warps=None, num_stages=2, waves_per_eu=2, plain=False):
    """Flash attention forward over [B, H, S, D] tensors (unit stride along D).

    plain=True launches attention_plain_kernel (the examples/05 form). A
    scale <= 0 always does: the default kernel folds the scale into the
    exponent and takes max(qk) * scale as the row maximum, which holds only
    for a positive scale.

    Default tiles: 32 query rows per wave, two waves per SIMD, 256-row
    programs on 8 waves (one workgroup per CU shares each K and V block
    between all 8 waves); causal too, where two 128-row workgroups per CU
    measured 2-3% slower (their register budget spills around the
    online-softmax pass)."""
    if BLOCK_M is None:
        BLOCK_M = 256
    if num_warps is None:
        num_warps = BLOCK_M // 32
    B, H, S, D = q.shape
    for t in (q, k, v):
        if t.stride(3) != 1:
            raise ValueError("attention: q, k and v need unit stride along head_dim")
    out = torch.empty_like(q) if out is None else out
    if out.stride(3) != 1:
        raise ValueError("attention: out needs unit stride along head_dim")
    scale = D ** -0.5 if scale is None else float(scale)
    grid = (newt.cdiv(S, BLOCK_M), B * H)
    if plain or not scale > 0:
        attention_plain_kernel[grid](q, k, v, out, S, H, scale,
                                     q.stride(0), q.stride(1), q.stride(2),
                                     k.stride(0), k.stride(1), k.stride(2),
                                     v.stride(0), v.stride(1), v.stride(2),
                                     out.stride(0), out.stride(1), out.stride(2),
                                     BLOCK_M=BLOCK_M, BLOCK_N=BLOCK_N, D=D, CAUSAL=causal,
                                     num_warps=num_warps, num_stages=num_stages,
                                     waves_per_eu=waves_per_eu)
        return out
    attention_kernel[grid](q, k, v, out, S, H, scale,
                           q.stride(0), q.stride(1), q.stride(2),
                           k.stride(0), k.stride(1), k.stride(2),
                           v.stride(0), v.stride(1), v.stride(2),
                           out.stride(0), out.stride(1), out.stride(2),
                           BLOCK_M=BLOCK_M, BLOCK_N=BLOCK_N, D=D, CAUSAL=causal,
                           num_warps=num_warps, num_stages=num_stages,
                           waves_per_eu=waves_per_eu)
    return out


# ---------------------------------------------------------------------------
# 6. deuteron matmul (examples/deuteron/01_matmul.py, unchanged body)
# ---------------------------------------------------------------------------
from . import deuteron as dt  # noqa: E402


@dt.kernel
def dt_matmul(x, y, out):
    for tile_m, tile_n in dt.tile([x.shape[0], y.shape[1]]):
        acc = dt.zeros([tile_m, tile_n], dtype=dt.float32)
        for tile_k in dt.tile(x.shape[1]):
            acc += x[tile_m, tile_k] @ y[tile_k, tile_n]
        out[tile_m, tile_n] = acc
