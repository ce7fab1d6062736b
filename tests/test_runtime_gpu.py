"""The backend boundary on its own: hipRTC compile + module launch of a
hand-written saxpy, through the C ABI (reference tests/test_runtime_smoke.py:22-48)."""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

SRC = r"""
extern "C" __global__ void saxpy(float a, const float* x, const float* y,
                                 float* out, int n) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = a * x[i] + y[i];
}
"""


def test_saxpy_both_launch_paths():
    from newt_amd.runtime.hip import Kernel, compile_hip, pack_format

    k = Kernel(compile_hip(SRC, "saxpy"), "saxpy")
    n = 1 << 20
    x = torch.randn(n, device="cuda")
    y = torch.randn(n, device="cuda")
    out = torch.empty_like(x)
    stream = torch.cuda.current_stream().cuda_stream
    k.launch(grid=((n + 255) // 256,), block=(256,),
             args=[ctypes.c_float(2.5), ctypes.c_void_p(x.data_ptr()),
                   ctypes.c_void_p(y.data_ptr()), ctypes.c_void_p(out.data_ptr()),
                   ctypes.c_int32(n)], stream=stream)
    torch.cuda.synchronize()
    ref = (2.5 * x.double() + y.double()).float()
    assert torch.allclose(out, ref, atol=1e-5)
    out.zero_()
    buf = pack_format(["f32", "ptr", "ptr", "ptr", "i32"]).pack(
        2.5, x.data_ptr(), y.data_ptr(), out.data_ptr(), n)
    k.launch_packed((n + 255) // 256, 1, 1, 256, stream, buf)
    torch.cuda.synchronize()
    assert torch.allclose(out, ref, atol=1e-5)


def test_timed_launch_records_events_and_computes():
    """newt_launch_packed_timed: same results as launch_packed, the two events
    are recorded by the dispatch (elapsed time positive), a NULL pair is
    accepted, and a ragged 2D grid (work-item counts = grid x block) covers
    every element exactly once."""
    from newt_amd.runtime.hip import Kernel, compile_hip, pack_format

    src = SRC + r"""
extern "C" __global__ void mark(int* out, int nx, int ny) {
    int x = blockIdx.x * blockDim.x + threadIdx.x, y = blockIdx.y;
    if (x < nx && y < ny) atomicAdd(out + y * nx + x, 1);
}
"""
    code = compile_hip(src, "saxpy")
    k = Kernel(code, "saxpy")
    n = (1 << 20) + 77
    x = torch.randn(n, device="cuda")
    y = torch.randn(n, device="cuda")
    out = torch.empty_like(x)
    stream = torch.cuda.current_stream().cuda_stream
    lib = ctypes.CDLL("libamdhip64.so")
    evs = [ctypes.c_void_p(), ctypes.c_void_p()]
    for e in evs:
        assert lib.hipEventCreate(ctypes.byref(e)) == 0
    buf = pack_format(["f32", "ptr", "ptr", "ptr", "i32"]).pack(
        2.5, x.data_ptr(), y.data_ptr(), out.data_ptr(), n)
    k.launch_packed_timed((n + 255) // 256, 1, 1, 256, stream, buf, evs[0].value, evs[1].value)
    torch.cuda.synchronize()
    assert torch.allclose(out, (2.5 * x.double() + y.double()).float(), atol=1e-5)
    ms = ctypes.c_float()
    assert lib.hipEventElapsedTime(ctypes.byref(ms), evs[0], evs[1]) == 0
    assert 0.0 < ms.value < 100.0
    for e in evs:
        lib.hipEventDestroy(e)
    m = Kernel(code, "mark")
    nx, ny = 1000, 3
    hits = torch.zeros(ny * nx, device="cuda", dtype=torch.int32)
    buf = pack_format(["ptr", "i32", "i32"]).pack(hits.data_ptr(), nx, ny)
    m.launch_packed_timed((nx + 127) // 128, ny, 1, 128, stream, buf, None, None)
    torch.cuda.synchronize()
    assert bool((hits == 1).all())


def test_device_is_gfx950():
    from newt_amd.runtime.hip import device_arch, device_limits
    assert device_arch(0).startswith("gfx950")
    cus, lds, ws = device_limits(0)
    assert ws == 64 and cus >= 256 and lds >= 64 * 1024


@pytest.mark.gpu
def test_warm_launches_take_the_c_path():
    """The first launch of a call signature runs in Python and registers a
    plan with the C launcher; later launches with the same signature (other
    tensors and values, same facts) run through it, with the same results."""
    from newt_amd import workloads as W
    from newt_amd.runtime import jit as J
    g = torch.Generator().manual_seed(3)
    x, y = (torch.randn(4096, generator=g).cuda() for _ in range(2))
    W.add(x, y)
    if not J._C_LAUNCH:
        pytest.skip("the C launcher is not built")
    n = len(W.add_kernel._ctable)
    assert n >= 1
    for size in (4096, 4004, 8192):
        a, b = (torch.randn(size, generator=g).cuda() for _ in range(2))
        out = W.add(a, b)
        torch.cuda.synchronize()
        assert torch.equal(out, a + b), size
    # 4004 differs from 4096 in its divisibility (4, not 16), 8192 does not:
    # one new plan
    assert len(W.add_kernel._ctable) == n + 1


import newt_amd as newt  # noqa: E402
import newt_amd.language as nl  # noqa: E402


@newt.jit
def kinds_k(x_ptr, o_ptr, a, n, big, flag, BLOCK: nl.constexpr):
    offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
    m = offs < n
    x = nl.load(x_ptr + offs, mask=m)
    shift = (big >> 36).to(nl.float32)        # an int64 beyond int32's range
    y = a * x + shift
    if flag:
        y = -y
    nl.store(o_ptr + offs, y, mask=m)


@pytest.mark.gpu
def test_c_path_packs_every_argument_kind():
    """A kernel with pointer, fp32, int32, int64 and bool parameters: the
    first launch runs in Python, the second and third through the C launcher
    (same call signature, other values); every launch computes what torch
    computes from the same values."""
    from newt_amd.runtime import jit as J

    g = torch.Generator().manual_seed(5)
    for i, (a, big, flag) in enumerate(((1.5, 3 << 36, True), (-2.0, 5 << 36, False),
                                        (0.25, 7 << 36, True))):
        x = torch.randn(1000, generator=g).cuda()
        o = torch.empty_like(x)
        kinds_k[(4,)](x, o, a, 1000, big, flag, BLOCK=256)
        torch.cuda.synchronize()
        want = a * x + float(big >> 36)
        want = -want if flag else want
        assert torch.equal(o, want), i
    if J._C_LAUNCH:
        assert len(kinds_k._ctable) == 1
