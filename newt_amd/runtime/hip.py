"""ctypes binding of libnewt_hip.so (include/newt_hip.h).

This module is the Python side of the backend boundary that replaces the
reference's newt/runtime/cuda.py (NVRTC + CUDA driver over ctypes): hipRTC
compiles HIP source to a gfx950 code object, the HIP module API loads and
launches it on torch's current stream. torch is imported first so that the
library binds to the HIP runtime torch-ROCm already uses (one runtime, one
context, shared streams and device pointers).
"""

import ctypes
import functools
import os
import struct

_HERE = os.path.dirname(os.path.abspath(__file__))
_PKG = os.path.dirname(_HERE)
LIB_PATH = os.path.join(_PKG, "csrc", "libnewt_hip.so")
DEVICE_HEADER = os.path.join(_PKG, "csrc", "device", "newt_gfx950.h")
BACKEND_VERSION = "newt-gfx950-1"
TARGET_ARCH = "gfx950"

# Options for every generated kernel. -ffp-contract=off keeps a*b+c unfused so
# elementwise results are bit-identical to torch eager; packed fp32 VALU ops are
# disabled for robustness on this hardware pool.
COMPILE_OPTIONS = ("-O3", "-std=c++17", "-ffp-contract=off",
                   "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                   "-DNDEBUG")


class HIPError(RuntimeError):
    """A HIP runtime / module error (reference counterpart: CUDAError)."""


class HIPRTCError(RuntimeError):
    """hipRTC compilation failure; message holds the build log
    (reference counterpart: NVRTCError)."""


@functools.cache
def lib():
    import torch  # noqa: F401  (bind to torch's HIP runtime before loading ours)

    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"newt: the HIP backend library {LIB_PATH} is not built; run "
            f"`python -c 'import __graft_entry__ as g; g.build()'` or "
            f"`python -m newt_amd.build`")
    L = ctypes.CDLL(LIB_PATH)
    c_int, c_void_p, c_char_p, c_size_t, c_uint = (ctypes.c_int, ctypes.c_void_p,
                                                   ctypes.c_char_p, ctypes.c_size_t,
                                                   ctypes.c_uint)
    L.newt_abi_version.restype = c_int
    L.newt_error_string.restype = c_char_p
    L.newt_error_string.argtypes = [c_int]
    L.newt_last_error.restype = c_char_p
    L.newt_rtc_compile.restype = c_int
    L.newt_rtc_compile.argtypes = [c_char_p, c_char_p, c_char_p, ctypes.POINTER(c_char_p), c_int,
                                   ctypes.POINTER(c_char_p), ctypes.POINTER(c_char_p), c_int,
                                   ctypes.POINTER(c_void_p), ctypes.POINTER(c_size_t)]
    L.newt_rtc_version.argtypes = [ctypes.POINTER(c_int)]
    L.newt_free.argtypes = [c_void_p]
    L.newt_free.restype = None
    L.newt_module_load.argtypes = [c_void_p, c_size_t, ctypes.POINTER(c_void_p)]
    L.newt_module_get_function.argtypes = [c_void_p, c_char_p, ctypes.POINTER(c_void_p)]
    L.newt_module_unload.argtypes = [c_void_p]
    L.newt_function_set_max_lds.argtypes = [c_void_p, c_int]
    L.newt_function_attributes.argtypes = [c_void_p] + [ctypes.POINTER(c_int)] * 4
    L.newt_launch.argtypes = [c_void_p, c_uint, c_uint, c_uint, c_uint, c_uint, c_void_p,
                              ctypes.POINTER(c_void_p)]
    L.newt_launch_packed.argtypes = [c_void_p, c_uint, c_uint, c_uint, c_uint, c_uint,
                                     c_void_p, c_char_p, c_size_t]
    L.newt_launch_packed_timed.argtypes = [c_void_p, c_uint, c_uint, c_uint, c_uint, c_uint,
                                           c_void_p, c_char_p, c_size_t, c_void_p, c_void_p]
    L.newt_device_arch.argtypes = [c_int, c_char_p, c_size_t]
    L.newt_device_limits.argtypes = [c_int] + [ctypes.POINTER(c_int)] * 3
    if L.newt_abi_version() != 1:
        raise RuntimeError("newt: libnewt_hip.so ABI mismatch; rebuild it")
    return L


def _check(status, what, exc=HIPError):
    if status != 0:
        L = lib()
        detail = (L.newt_last_error() or b"").decode(errors="replace")
        msg = (L.newt_error_string(status) or b"?").decode()
        raise exc(f"{what} failed ({status}: {msg})\n{detail}")


@functools.cache
def device_header():
    with open(DEVICE_HEADER) as f:
        return f.read()


@functools.cache
def rtc_version():
    v = ctypes.c_int()
    _check(lib().newt_rtc_version(ctypes.byref(v)), "hiprtcVersion", HIPRTCError)
    return v.value


def compile_hip(source, name, arch=TARGET_ARCH, extra_opts=()):
    """Compile HIP source with hipRTC to a code object (bytes).
    Replaces compile_cuda (reference newt/runtime/cuda.py:124-154)."""
    L = lib()
    opts = [o.encode() for o in COMPILE_OPTIONS + tuple(extra_opts)]
    c_opts = (ctypes.c_char_p * len(opts))(*opts)
    hdrs = (ctypes.c_char_p * 1)(device_header().encode())
    names = (ctypes.c_char_p * 1)(b"newt_gfx950.h")
    code = ctypes.c_void_p()
    size = ctypes.c_size_t()
    st = L.newt_rtc_compile(source.encode(), f"{name}.hip".encode(), arch.encode(), c_opts,
                            len(opts), hdrs, names, 1, ctypes.byref(code), ctypes.byref(size))
    if st != 0:
        detail = (L.newt_last_error() or b"").decode(errors="replace")
        raise HIPRTCError(f"hipRTC compilation of {name} failed:\n{detail}")
    try:
        return ctypes.string_at(code, size.value)
    finally:
        L.newt_free(code)


@functools.cache
def device_arch(device=0):
    buf = ctypes.create_string_buffer(128)
    _check(lib().newt_device_arch(device, buf, 128), "hipGetDeviceProperties")
    return buf.value.decode()


@functools.cache
def device_limits(device=0):
    cus, lds, ws = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _check(lib().newt_device_limits(device, ctypes.byref(cus), ctypes.byref(lds),
                                    ctypes.byref(ws)), "hipGetDeviceProperties")
    return cus.value, lds.value, ws.value


class Kernel:
    """A loaded gfx950 function (reference counterpart: cuda.Kernel,
    newt/runtime/cuda.py:195-234)."""

    def __init__(self, code, func_name, lds_bytes=0):
        L = lib()
        self._lib = L
        self._code = code  # keep the image alive for the module's lifetime
        self.module = ctypes.c_void_p()
        _check(L.newt_module_load(code, len(code), ctypes.byref(self.module)), "hipModuleLoadData")
        self.func = ctypes.c_void_p()
        _check(L.newt_module_get_function(self.module, func_name.encode(), ctypes.byref(self.func)),
               "hipModuleGetFunction")
        if lds_bytes > 64 * 1024:
            _check(L.newt_function_set_max_lds(self.func, lds_bytes), "set max LDS")
        self.lds_bytes = 0  # the generated kernels declare their LDS statically
        self.name = func_name

    def attributes(self):
        vals = [ctypes.c_int() for _ in range(4)]
        _check(self._lib.newt_function_attributes(self.func, *[ctypes.byref(v) for v in vals]),
               "hipFuncGetAttribute")
        return dict(zip(("num_regs", "lds_bytes", "scratch_bytes", "max_threads"),
                        [v.value for v in vals]))

    def launch(self, grid, block, args, stream=0):
        """args: list of ctypes scalars (c_void_p / c_int32 / c_float ...)."""
        ptrs = (ctypes.c_void_p * max(1, len(args)))(
            *[ctypes.cast(ctypes.byref(a), ctypes.c_void_p) for a in args])
        gx, gy, gz = (list(grid) + [1, 1, 1])[:3]
        bx = block[0] if isinstance(block, (tuple, list)) else block
        _check(self._lib.newt_launch(self.func, gx, gy, gz, bx, self.lds_bytes,
                                     ctypes.c_void_p(stream), ptrs), "hipModuleLaunchKernel")

    def launch_packed(self, gx, gy, gz, block, stream, argbuf):
        st = self._lib.newt_launch_packed(self.func, gx, gy, gz, block, self.lds_bytes,
                                          stream, argbuf, len(argbuf))
        if st != 0:
            _check(st, "hipModuleLaunchKernel")

    def launch_packed_timed(self, gx, gy, gz, block, stream, argbuf, ev_start, ev_stop):
        """launch_packed with two hipEvent_t handles recorded by the dispatch
        itself at the kernel's start and end."""
        st = self._lib.newt_launch_packed_timed(self.func, gx, gy, gz, block, self.lds_bytes,
                                                stream, argbuf, len(argbuf), ev_start, ev_stop)
        if st != 0:
            _check(st, "hipExtModuleLaunchKernel")


# struct codes and alignment of each kernel parameter kind in the packed
# argument segment
_ARG_FMT = {"ptr": ("Q", 8), "i64": ("q", 8), "i32": ("i", 4), "f32": ("f", 4),
            "bool": ("?", 1), "f64": ("d", 8)}


def pack_layout(kinds):
    """(byte offset of each parameter, segment size) of the packed argument
    segment pack_format lays out."""
    offs, off = [], 0
    for k in kinds:
        size = struct.calcsize("=" + _ARG_FMT[k][0])
        off += (-off) % _ARG_FMT[k][1]
        offs.append(off)
        off += size
    return offs, off + (-off) % 8


def pack_format(kinds):
    """struct format (explicit padding) laying out params with natural alignment."""
    fmt = "="
    off = 0
    for k in kinds:
        code, al = _ARG_FMT[k]
        pad = (-off) % al
        if pad:
            fmt += f"{pad}x"
            off += pad
        fmt += code
        off += struct.calcsize("=" + code)
    pad = (-off) % 8
    if pad:
        fmt += f"{pad}x"
    return struct.Struct(fmt)
