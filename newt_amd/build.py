"""Build the native parts of newt_amd.

  * libnewt_hip.so - the C-ABI backend boundary (include/newt_hip.h): host C++
    over libamdhip64 + a run-time-loaded hipRTC. No device code, so g++ builds it.
  * _newt_launch - the warm-launch path of @newt.jit in C (a CPython extension
    that calls newt_launch_packed); gcc builds it.
  * device-template check - the gfx950 device header (csrc/device/newt_gfx950.h)
    is compiled offline with hipcc for gfx950, instantiating every template the
    code generator emits, so a broken header fails the build instead of the
    first kernel launch.

Run: python -m newt_amd.build
"""

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIP_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def build_library():
    src = os.path.join(CSRC, "newt_hip.cpp")
    out = os.path.join(CSRC, "libnewt_hip.so")
    tmp = out + ".tmp"
    _run(["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-D__HIP_PLATFORM_AMD__",
          f"-I{ROCM}/include", f"-I{ROOT}/include", src, "-o", tmp, f"-L{ROCM}/lib",
          "-lamdhip64", "-ldl", "-Wl,--no-undefined"])
    os.replace(tmp, out)
    return out


def build_launcher():
    """The warm-launch path of @newt.jit (csrc/newt_pylaunch.c), a CPython
    extension: it resolves newt_launch_packed in libnewt_hip.so at init."""
    import sysconfig
    src = os.path.join(CSRC, "newt_pylaunch.c")
    out = os.path.join(CSRC, "_newt_launch" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out + ".tmp"
    _run(["gcc", "-O2", "-fPIC", "-shared", "-Wall", "-Werror", "-std=c11",
          f"-I{sysconfig.get_paths()['include']}", src, "-o", tmp, "-ldl"])
    os.replace(tmp, out)
    return out


_HEADER_CHECK = r"""
#include <hip/hip_runtime.h>
#include "newt_gfx950.h"
extern "C" __global__ void __launch_bounds__(256) newt_header_check(
    const f16* a, const bf16* b, const float* f, float* o, int n) {
  const int l = threadIdx.x & 63;
  float v[4];
  newt::load_vec<float, 4>(f + 4 * l, v);
  float s = v[0] + v[1] + v[2] + v[3];
  s = newt::lane_reduce<newt::Sum, 63>(s);
  float m = newt::lane_reduce<newt::Max, 63>(v[0]);
  int i = newt::lane_reduce<newt::Min, 63>((int)l);
  f16x8 fa = *(const f16x8*)(a + 8 * l);
  bf16x8 fb = *(const bf16x8*)(b + 8 * l);
  f32x16 c = (f32x16)(0.0f);
  c = newt::mfma_32x32x16(fa, fa, c);
  c = newt::mfma_32x32x16(fb, fb, c);
  f32x4 d = (f32x4)(0.0f);
  d = newt::mfma_16x16x32(fa, fa, d);
  d = newt::mfma_16x16x32(fb, fb, d);
  f16x4 ha = *(const f16x4*)(a + 4 * l);
  bf16x4 hb = *(const bf16x4*)(b + 4 * l);
  c = newt::mfma_32x32x8(ha, ha, c);
  c = newt::mfma_32x32x8(hb, hb, c);
  d = newt::mfma_16x16x16(ha, ha, d);
  d = newt::mfma_16x16x16(hb, hb, d);
  c = newt::mfma_32x32x2(v[1], v[2], c);
  d = newt::mfma_16x16x4(v[1], v[2], d);
  int off = newt::LdsTile<f16, 64>::off(l, 8);
  float r[4] = {s + c[0], m + d[0], (float)i + (float)off, c[15] + d[3]};
  newt::store_vec<float, 4>(o + 4 * threadIdx.x, r);
  newt::atomic_max(o, s);
  newt::atomic_add(o + 1, m);
  if (n > 0 && newt::aligned(o, 16)) o[2] = newt::to_f32(newt::to_bf16(s));
}
"""


def check_device_header():
    """Compile the device header for gfx950 offline (hipcc)."""
    wdir = os.path.join(CSRC, "_build")
    os.makedirs(wdir, exist_ok=True)
    src = os.path.join(wdir, "header_check.hip")
    with open(src, "w") as f:
        f.write(_HEADER_CHECK)
    out = os.path.join(wdir, "header_check.co")
    _run([os.path.join(ROCM, "bin", "hipcc"), "--offload-arch=gfx950", "--genco", "-O3",
          "-std=c++17", *HIP_FLAGS, f"-I{os.path.join(CSRC, 'device')}", src, "-o", out])
    return out


def build(verbose=True):
    lib = build_library()
    if verbose:
        print("built", lib)
    launcher = build_launcher()
    if verbose:
        print("built", launcher)
    co = check_device_header()
    if verbose:
        print("device header compiled for gfx950:", co)
    return lib


if __name__ == "__main__":
    build()
    sys.exit(0)
