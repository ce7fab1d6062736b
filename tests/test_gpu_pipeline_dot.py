"""nl.dot inside loops: the pipelined k-loop's edge cases, and matmul at every
nl.dot dtype, as in the reference's tests/test_pipeline_dot.py and
tests/test_matmul.py:
  two dot loops on one accumulator, the second running zero or one trips :12-50
  an accumulator overwritten after its loop without being read            :53-81
  a configuration whose LDS stages would not fit (fp32, 128x128x64)       :84-110
  a store inside the k-loop                                               :113-142
  matmul fp16 (64x64x32, 256x256x128, 300x200x100), bf16, fp32           test_matmul.py:51-71
Tolerances are the reference's (2e-2, 2e-1 for the fp32 accumulation case).
"""

import pytest
import torch

import newt
import newt.language as nl

pytestmark = pytest.mark.gpu


def rnd(shape, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(shape, device="cuda", generator=g) * 0.3).to(dtype)


@newt.jit
def main_and_tail_k(a_ptr, b_ptr, o_ptr, K, FULL, TAIL,
                    BM: nl.constexpr, BN: nl.constexpr, BK: nl.constexpr):
    rm, rn, rk = nl.arange(0, BM), nl.arange(0, BN), nl.arange(0, BK)
    pa = a_ptr + rm[:, None] * K + rk[None, :]
    pb = b_ptr + rk[:, None] * BN + rn[None, :]
    acc = nl.zeros((BM, BN), dtype=nl.float32)
    for i in range(FULL):
        acc = nl.dot(nl.load(pa), nl.load(pb), acc)
        pa += BK
        pb += BK * BN
    for t in range(TAIL):
        live = (t * BK + rk) < (K - FULL * BK)
        acc = nl.dot(nl.load(pa, mask=live[None, :], other=0.0),
                     nl.load(pb, mask=live[:, None], other=0.0), acc)
    nl.store(o_ptr + rm[:, None] * BN + rn[None, :], acc)


@pytest.mark.parametrize("stages", [1, 2, 3, 4])
@pytest.mark.parametrize("K", [96, 80, 32, 16, 0])
def test_main_loop_then_tail_loop(K, stages):
    BM, BN, BK = 64, 64, 32
    full, rem = K // BK, K % BK
    a = rnd((BM, max(K, 1)), torch.float16, 0)
    b = rnd((max(K, 1), BN), torch.float16, 1)
    o = torch.empty(BM, BN, device="cuda")
    main_and_tail_k[(1,)](a, b, o, K, full, 1 if rem else 0, BM=BM, BN=BN, BK=BK,
                          num_stages=stages)
    want = a[:, :K].float() @ b[:K].float()
    torch.testing.assert_close(o, want, rtol=2e-2, atol=2e-2)


@newt.jit
def overwrite_k(a_ptr, b_ptr, o_ptr, K, BM: nl.constexpr, BN: nl.constexpr, BK: nl.constexpr):
    rm, rn, rk = nl.arange(0, BM), nl.arange(0, BN), nl.arange(0, BK)
    pa = a_ptr + rm[:, None] * K + rk[None, :]
    pb = b_ptr + rk[:, None] * BN + rn[None, :]
    first = nl.dot(nl.load(pa), nl.load(pb))
    acc = nl.zeros((BM, BN), dtype=nl.float32)
    for i in range(K // BK):
        acc = nl.dot(nl.load(pa), nl.load(pb), acc)
        pa += BK
        pb += BK * BN
    acc = first
    nl.store(o_ptr + rm[:, None] * BN + rn[None, :], acc + 0.0)


def test_accumulator_overwritten_unread():
    BM, BN, BK, K = 64, 64, 32, 96
    a, b = rnd((BM, K), torch.float16, 2), rnd((K, BN), torch.float16, 3)
    o = torch.empty(BM, BN, device="cuda")
    overwrite_k[(1,)](a, b, o, K, BM=BM, BN=BN, BK=BK)
    torch.testing.assert_close(o, a[:, :BK].float() @ b[:BK].float(), rtol=2e-2, atol=2e-2)


@newt.jit
def kloop_k(a_ptr, b_ptr, o_ptr, K, BM: nl.constexpr, BN: nl.constexpr, BK: nl.constexpr):
    rm, rn, rk = nl.arange(0, BM), nl.arange(0, BN), nl.arange(0, BK)
    pa = a_ptr + rm[:, None] * K + rk[None, :]
    pb = b_ptr + rk[:, None] * BN + rn[None, :]
    acc = nl.zeros((BM, BN), dtype=nl.float32)
    for i in range(K // BK):
        acc = nl.dot(nl.load(pa), nl.load(pb), acc)
        pa += BK
        pb += BK * BN
    nl.store(o_ptr + rm[:, None] * BN + rn[None, :], acc)


@pytest.mark.parametrize("stages", [3, 8])
def test_stages_beyond_lds_budget_still_compile(stages):
    # fp32 128x128x64 tiles are 64 KiB per stage: 3+ stages exceed the 160 KiB LDS
    BM, BN, BK, K = 128, 128, 64, 128
    a, b = rnd((BM, K), torch.float32, 4), rnd((K, BN), torch.float32, 5)
    o = torch.empty(BM, BN, device="cuda")
    kloop_k[(1,)](a, b, o, K, BM=BM, BN=BN, BK=BK, num_warps=8, num_stages=stages)
    torch.testing.assert_close(o, a @ b, rtol=2e-2, atol=2e-1)


@newt.jit
def store_in_loop_k(a_ptr, b_ptr, o_ptr, dbg_ptr, K,
                    BM: nl.constexpr, BN: nl.constexpr, BK: nl.constexpr):
    rm, rn, rk = nl.arange(0, BM), nl.arange(0, BN), nl.arange(0, BK)
    pa = a_ptr + rm[:, None] * K + rk[None, :]
    pb = b_ptr + rk[:, None] * BN + rn[None, :]
    acc = nl.zeros((BM, BN), dtype=nl.float32)
    for i in range(K // BK):
        acc = nl.dot(nl.load(pa), nl.load(pb), acc)
        nl.store(dbg_ptr + rm, rm.to(nl.float32) + i)
        pa += BK
        pb += BK * BN
    nl.store(o_ptr + rm[:, None] * BN + rn[None, :], acc)


def test_store_inside_kloop():
    BM, BN, BK, K = 64, 64, 32, 128
    a, b = rnd((BM, K), torch.float16, 6), rnd((K, BN), torch.float16, 7)
    o = torch.empty(BM, BN, device="cuda")
    dbg = torch.empty(BM, device="cuda")
    store_in_loop_k[(1,)](a, b, o, dbg, K, BM=BM, BN=BN, BK=BK)
    torch.testing.assert_close(o, a.float() @ b.float(), rtol=2e-2, atol=2e-2)
    assert torch.equal(dbg, torch.arange(BM, device="cuda").float() + K // BK - 1)


@newt.jit
def matmul_k(a_ptr, b_ptr, c_ptr, M, N, K, sam, sak, sbk, sbn, scm, scn,
             BLOCK_M: nl.constexpr, BLOCK_N: nl.constexpr, BLOCK_K: nl.constexpr):
    offs_m = nl.program_id(0) * BLOCK_M + nl.arange(0, BLOCK_M)
    offs_n = nl.program_id(1) * BLOCK_N + nl.arange(0, BLOCK_N)
    offs_k = nl.arange(0, BLOCK_K)
    pa = a_ptr + offs_m[:, None] * sam + offs_k[None, :] * sak
    pb = b_ptr + offs_k[:, None] * sbk + offs_n[None, :] * sbn
    acc = nl.zeros((BLOCK_M, BLOCK_N), dtype=nl.float32)
    for k in range(nl.cdiv(K, BLOCK_K)):
        rest = K - k * BLOCK_K
        a = nl.load(pa, mask=(offs_m[:, None] < M) & (offs_k[None, :] < rest), other=0.0)
        b = nl.load(pb, mask=(offs_k[:, None] < rest) & (offs_n[None, :] < N), other=0.0)
        acc = nl.dot(a, b, acc)
        pa += BLOCK_K * sak
        pb += BLOCK_K * sbk
    nl.store(c_ptr + offs_m[:, None] * scm + offs_n[None, :] * scn,
             acc.to(c_ptr.dtype.element_ty), mask=(offs_m[:, None] < M) & (offs_n[None, :] < N))


def run_matmul(M, N, K, dtype, BM=64, BN=64, BK=32, waves=4):
    g = torch.Generator(device="cuda").manual_seed(M * 7 + N * 3 + K)
    a = (torch.randn(M, K, device="cuda", generator=g) * 0.5).to(dtype)
    b = (torch.randn(K, N, device="cuda", generator=g) * 0.5).to(dtype)
    c = torch.empty(M, N, device="cuda", dtype=dtype)
    matmul_k[(newt.cdiv(M, BM), newt.cdiv(N, BN))](
        a, b, c, M, N, K, a.stride(0), a.stride(1), b.stride(0), b.stride(1),
        c.stride(0), c.stride(1), BLOCK_M=BM, BLOCK_N=BN, BLOCK_K=BK, num_warps=waves)
    return a, b, c


@pytest.mark.parametrize("mnk", [(64, 64, 32), (256, 256, 128), (300, 200, 100)])
def test_matmul_fp16(mnk):
    a, b, c = run_matmul(*mnk, torch.float16)
    newt.testing.assert_close(c, (a.float() @ b.float()).half(), rtol=1e-2, atol=1e-2)


def test_matmul_bf16():
    a, b, c = run_matmul(256, 128, 64, torch.bfloat16)
    newt.testing.assert_close(c, (a.float() @ b.float()).bfloat16(), rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("mnk", [(128, 128, 128), (200, 136, 72)])
def test_matmul_fp32(mnk):
    a, b, c = run_matmul(*mnk, torch.float32)
    newt.testing.assert_close(c, a @ b, rtol=1e-2, atol=1e-2)


def test_matmul_fp32_is_full_precision():
    """fp32 nl.dot runs on the fp32 MFMA (v_mfma_f32_32x32x2_f32): products are
    exact fp32, so it is far closer to an fp64 product than tf32 (10-bit
    mantissa) could be."""
    a, b, c = run_matmul(128, 128, 512, torch.float32)
    want = (a.double() @ b.double())
    rel = ((c.double() - want).norm() / want.norm()).item()
    assert rel < 1e-5



# fp16 A rows whose lane offsets in a 256x32 tile, (sam * 255 + 31) * 2 bytes,
# end just below / just above 2^31 (sam multiple of 16 either way)
SAM_FITS, SAM_TOO_BIG = 4_210_688, 4_300_800


@pytest.mark.parametrize("sam", [SAM_FITS, SAM_TOO_BIG])
@pytest.mark.parametrize("buffer_dma", ["1", "0"])
def test_lane_offsets_near_two_gib(sam, buffer_dma, monkeypatch):
    """Rows of A 8.4 MB apart. Below the limit the fast loop's buffer-form
    copies carry lane offsets up to ~2^31 bytes; above it the entry test
    keeps every iteration on the general loop's 64-bit copies. Either way the
    product is exact (a lane offset that wrapped would read the wrong rows of
    the same allocation)."""
    monkeypatch.setenv("NEWT_BUFFER_DMA", buffer_dma)
    M = N = K = 256
    flat = torch.empty(255 * sam + K, device="cuda", dtype=torch.float16)
    a = flat.as_strided((M, K), (sam, 1))
    a.copy_(rnd((M, K), torch.float16, 10))
    b = rnd((K, N), torch.float16, 11)
    c = torch.empty(M, N, device="cuda")
    kloop_k2[(1, 1)](a, b, c, K, sam, BM=M, BN=N, BK=32, num_warps=4, num_stages=4)
    want = a.float() @ b.float()
    rel = ((c - want).norm() / want.norm()).item()
    del flat, a
    assert rel < 1e-3


@newt.jit
def kloop_k2(a_ptr, b_ptr, o_ptr, K, sam, BM: nl.constexpr, BN: nl.constexpr, BK: nl.constexpr):
    rm, rn, rk = nl.arange(0, BM), nl.arange(0, BN), nl.arange(0, BK)
    pa = a_ptr + rm[:, None] * sam + rk[None, :]
    pb = b_ptr + rk[:, None] * BN + rn[None, :]
    acc = nl.zeros((BM, BN), dtype=nl.float32)
    for i in range(K // BK):
        x = nl.load(pa)
        y = nl.load(pb)
        acc = nl.dot(x, y, acc)
        pa += BK
        pb += BK * BN
    nl.store(o_ptr + rm[:, None] * BN + rn[None, :], acc)


@newt.jit
def chained_dots_k(a_ptr, k_ptr, v_ptr, o_ptr, s_ptr, N, svn, svd,
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


@pytest.mark.parametrize("mfma", ["", "32"])
@pytest.mark.parametrize("v_keys_contiguous", [False, True])
@pytest.mark.parametrize("D", [64, 128])
def test_dot_result_feeds_next_dot(mfma, v_keys_contiguous, D, monkeypatch):
    """A dot's fp16 result as the next dot's A operand inside a pipelined loop
    (attention's P @ V without the softmax). The accumulator registers feed
    the second MFMA in place, and V is read from LDS in the matching permuted
    key order: row-major V (an R-major tile, swizzled for that read) or V
    stored keys-contiguous (a K-major tile). Both on 16x16x32 MFMAs (the
    default for such kernels) and on 32x32x16 (NEWT_MFMA=32). Checked against
    torch in fp32 on the fp16 rounding of the first product; a key order that
    pairs P and V wrongly gives an error of order 1."""
    monkeypatch.setenv("NEWT_MFMA", mfma)
    M, N, BM, BN = 256, 512, 128, 64
    a, k, v = rnd((M, D), torch.float16, 1), rnd((N, D), torch.float16, 2), rnd((N, D), torch.float16, 3)
    vbuf, svn, svd = (v.t().contiguous(), 1, N) if v_keys_contiguous else (v, D, 1)
    o = torch.empty(M, D, device="cuda", dtype=torch.float32)
    s = torch.empty(M, device="cuda", dtype=torch.float32)
    print(f"chained dots: D={D} V keys-contiguous={v_keys_contiguous} NEWT_MFMA={mfma!r}", flush=True)
    chained_dots_k[(M // BM,)](a, k, vbuf, o, s, N, svn, svd, BLOCK_M=BM, BLOCK_N=BN, D=D,
                               num_warps=4, num_stages=2)
    s32 = a.float() @ k.float().t()
    want_o = s32.half().float() @ v.float()
    rel = ((o - want_o).norm() / want_o.norm()).item()
    assert rel < 2e-3, rel
    torch.testing.assert_close(s, s32.sum(1), rtol=1e-4, atol=1e-3)
