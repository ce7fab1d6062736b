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


def test_device_is_gfx950():
    from newt_amd.runtime.hip import device_arch, device_limits
    assert device_arch(0).startswith("gfx950")
    cus, lds, ws = device_limits(0)
    assert ws == 64 and cus >= 256 and lds >= 64 * 1024
