"""The JIT's per-launch host path without a GPU (reference counterpart: the
warm launch of newt/runtime/jit.py:166-223).

A launch whose call signature was seen before skips binding, typing and the
specialization lookup: it hashes a signature, reads the parameter values with
one generated expression and hands them to the compiled kernel. These tests
run that path with the device, stream and kernel replaced by stand-ins and
check that it passes the same values as the first (slow) launch, that every
fact the code depends on starts a new entry, and how long it takes.
"""

import statistics
import time

import pytest
import torch

import newt_amd as newt
import newt_amd.language as nl
from newt_amd.compiler import types as tp
from newt_amd.runtime import jit as J


@newt.jit
def saxpy(x_ptr, y_ptr, out_ptr, a, n, FLAG: nl.constexpr, BLOCK: nl.constexpr = 256):
    offs = nl.program_id(0) * BLOCK + nl.arange(0, BLOCK)
    m = offs < n
    nl.store(out_ptr + offs, a * nl.load(x_ptr + offs, mask=m) + nl.load(y_ptr + offs, mask=m),
             mask=m)


class FakeKernel:
    """Stands in for CompiledKernel: records launches."""

    def __init__(self, params):
        self.params = params
        self.launches = []

    def launch(self, grid, values, stream):
        self.launches.append((grid, tuple(values), stream))


@pytest.fixture
def fake(monkeypatch):
    compiled = []

    def type_of(name, val):
        if isinstance(val, torch.Tensor):
            elem = tp.TORCH_TO_NEWT[str(val.dtype)]
            return tp.pointer_type(elem), ("a16" if val.data_ptr() % 16 == 0 else "")
        return REAL_TYPE_OF(name, val)

    def compile_(self, key, constexprs, types, num_warps, num_stages, waves_per_eu=0):
        params = [(n, J.Param(t, n)) for n, (t, _) in types.items()]
        k = FakeKernel(params)
        compiled.append((key, k))
        return k

    monkeypatch.setattr(J._Dev, "device", classmethod(lambda cls: 0))
    monkeypatch.setattr(J._Dev, "stream", staticmethod(lambda d: 1234))
    monkeypatch.setattr(J.JITFunction, "_type_of", staticmethod(type_of))
    monkeypatch.setattr(J.JITFunction, "_compile", compile_)
    saxpy.cache.clear()
    saxpy._fast.clear()
    yield compiled
    saxpy.cache.clear()
    saxpy._fast.clear()


REAL_TYPE_OF = J.JITFunction._type_of


def test_fast_path_passes_the_slow_paths_values(fake):
    x, y, o = torch.zeros(1000), torch.zeros(1000), torch.zeros(1000)
    saxpy[(4,)](x, y, o, 2.5, 1000, FLAG=True)
    saxpy[(4,)](x, y, o, 3.0, 1016, FLAG=True)          # warm: same facts (n divisible by 8)
    saxpy[lambda m: (m["n"] // m["BLOCK"] + 1,)](x, y, o, a=1.0, n=1000, FLAG=True)
    assert len(fake) == 1
    k = fake[0][1]
    ptrs = (x.data_ptr(), y.data_ptr(), o.data_ptr())
    assert k.launches[0] == ((4, 1, 1), ptrs + (2.5, 1000), 1234)
    assert k.launches[1] == ((4, 1, 1), ptrs + (3.0, 1016), 1234)
    # keyword arguments, the default BLOCK and a grid over META reach the
    # same parameter slots
    assert k.launches[2] == ((4, 1, 1), ptrs + (1.0, 1000), 1234)
    # an int where a float was: its own specialization (an int32 parameter)
    saxpy[(4,)](x, y, o, 3, 1000, FLAG=True)
    assert len(fake) == 2 and fake[1][1].launches[0][1][3] == 3


def test_every_specialization_fact_starts_a_new_entry(fake, monkeypatch):
    x, y, o = torch.zeros(1000), torch.zeros(1000), torch.zeros(1000)
    saxpy[(4,)](x, y, o, 2.0, 1000, FLAG=True)
    saxpy[(4,)](x, y, o, 2.0, 1001, FLAG=True)            # n's divisibility changed
    saxpy[(4,)](x, y, o, 2.0, 1, FLAG=True)               # n == 1
    saxpy[(4,)](x, y, o, 2.0, 1000, FLAG=False)           # constexpr value
    saxpy[(4,)](x, y, o, 2.0, 1000, FLAG=1)               # same value, other type
    saxpy[(4,)](x.double(), y, o, 2.0, 1000, FLAG=True)   # dtype
    saxpy[(4,)](x[1:], y, o, 2.0, 1000, FLAG=True)        # 16-byte alignment
    saxpy[(4,)](x, y, o, 2.0, 1000, FLAG=True, num_warps=8)
    assert len(saxpy._fast) == 8
    # a repeated call of any of them adds nothing
    saxpy[(4,)](x, y, o, 2.0, 1001, FLAG=True)
    saxpy[(4,)](x[1:], y, o, 2.0, 1000, FLAG=True)
    assert len(saxpy._fast) == 8
    monkeypatch.setenv("NEWT_VEC", "1")                   # a codegen switch
    saxpy[(4,)](x, y, o, 2.0, 1000, FLAG=True)
    assert len(saxpy._fast) == 9


def test_fast_path_host_cost(fake):
    """The warm launch's host time, without the GPU's own launch call.
    Printed for the record; the bound only catches a path that went slow."""
    x, y, o = torch.zeros(1 << 20), torch.zeros(1 << 20), torch.zeros(1 << 20)
    launch = saxpy[(4096,)]
    for _ in range(100):
        launch(x, y, o, 2.0, 1 << 20, FLAG=True)
    reps = []
    for _ in range(20):
        t0 = time.perf_counter()
        for _ in range(1000):
            launch(x, y, o, 2.0, 1 << 20, FLAG=True)
        reps.append((time.perf_counter() - t0) / 1000 * 1e6)
    us = statistics.median(reps)
    print(f"warm launch host path: {us:.2f} us per launch (median of 20 x 1000)")
    assert len(fake) == 1
    assert us < 40


def test_wrong_device_is_rejected_at_each_launch(fake, monkeypatch):
    """The signature records each tensor's device and the current one: a
    tensor on another device than the current one fails every launch (the
    plan is never stored)."""
    class OnDev1(torch.Tensor):
        def get_device(self):
            return 1

        @property
        def device(self):
            return torch.device("cuda", 1)
    x = torch.zeros(1000).as_subclass(OnDev1)
    y, o = torch.zeros(1000), torch.zeros(1000)
    for _ in range(2):
        with pytest.raises(ValueError, match="current device"):
            saxpy[(4,)](x, y, o, 2.0, 1000, FLAG=True)
    assert not saxpy._fast


# ------------------------------------------------------------------ the C path

_STUB = r"""
#include <stddef.h>
#include <string.h>
static unsigned char last[1024];
static size_t last_size;
static unsigned rec[6];
static void* last_stream;
static void* last_func;
static int calls;
int newt_launch_packed(void* f, unsigned gx, unsigned gy, unsigned gz, unsigned block,
                       unsigned lds, void* stream, const void* buf, size_t size) {
  last_func = f; rec[0] = gx; rec[1] = gy; rec[2] = gz; rec[3] = block; rec[4] = lds;
  last_stream = stream; last_size = size; memcpy(last, buf, size); calls++;
  return 0;
}
int stub_calls(void) { return calls; }
size_t stub_last(unsigned char* out, unsigned* r, void** stream, void** func) {
  memcpy(out, last, last_size); memcpy(r, rec, sizeof rec); *stream = last_stream;
  *func = last_func; return last_size;
}
"""


@pytest.fixture
def c_launch(tmp_path):
    """The C launcher bound to a stand-in newt_launch_packed that records its
    arguments (built here with gcc), device 0 and stream 0x5000."""
    import ctypes
    import importlib.machinery
    import importlib.util
    import os
    import subprocess
    import sysconfig

    from newt_amd.runtime import hip

    path = os.path.join(os.path.dirname(hip.LIB_PATH),
                        "_newt_launch" + sysconfig.get_config_var("EXT_SUFFIX"))
    if not os.path.exists(path):
        pytest.skip("the C launcher is not built")
    src = tmp_path / "stub.c"
    src.write_text(_STUB)
    so = tmp_path / "libstub.so"
    subprocess.run(["gcc", "-O1", "-shared", "-fPIC", str(src), "-o", str(so)], check=True)
    loader = importlib.machinery.ExtensionFileLoader("_newt_launch", path)
    spec = importlib.util.spec_from_file_location("_newt_launch", path, loader=loader)
    mod = importlib.util.module_from_spec(spec)
    loader.exec_module(mod)
    mod.init(str(so), lambda: 0, lambda d: 0x5000, os.environ._data, J._CODEGEN_ENV_B,
             torch.Tensor)
    stub = ctypes.CDLL(str(so))

    def last():
        buf = (ctypes.c_ubyte * 1024)()
        rec = (ctypes.c_uint * 6)()
        stream, func = ctypes.c_void_p(), ctypes.c_void_p()
        n = stub.stub_last(buf, rec, ctypes.byref(stream), ctypes.byref(func))
        return bytes(buf[:n]), tuple(rec[:5]), stream.value, func.value
    yield mod, stub, last
    # the extension's state is per process: if this process set up the real
    # launcher, bind it back to libnewt_hip.so and torch
    if J._C_LAUNCH:
        J._C_LAUNCH = None
        J._c_launcher()


def test_c_launch_packs_what_the_python_path_packs(c_launch):
    mod, stub, last = c_launch
    from newt_amd.runtime import hip
    kinds = ["ptr", "ptr", "ptr", "f32", "i32", "bool", "i64"]
    offs, size = hip.pack_layout(kinds)
    assert size == hip.pack_format(kinds).size
    x, y, o = torch.zeros(100), torch.zeros(100), torch.zeros(100)
    args = (x, y, o, 2.5, 1000, True, 1 << 40, 64)     # the last: a constexpr
    cx = (False,) * 7 + (True,)
    table = {}
    key = mod.run(table, cx, (4, 2), args, {"num_warps": 4})
    assert type(key) is tuple
    table[key] = mod.make_plan(0xABC0, 256, size, tuple(
        (i, J._C_KINDS[k], off) for i, (k, off) in enumerate(zip(kinds, offs))))
    assert mod.run(table, cx, (4, 2), args, {"num_warps": 4}) is None
    buf, rec, stream, func = last()
    want = hip.pack_format(kinds).pack(x.data_ptr(), y.data_ptr(), o.data_ptr(), 2.5, 1000, True,
                                       1 << 40)
    assert buf == want and rec == (4, 2, 1, 256, 0) and stream == 0x5000 and func == 0xABC0
    # same facts, other values: a hit, the new values packed
    args2 = (y, x, o, -1.0, 1016, False, 3 << 40, 64)
    assert mod.run(table, cx, 7, args2, {"num_warps": 4}) is None
    buf, rec, _, _ = last()
    assert buf == hip.pack_format(kinds).pack(y.data_ptr(), x.data_ptr(), o.data_ptr(), -1.0,
                                              1016, False, 3 << 40)
    assert rec[:3] == (7, 1, 1)
    # an empty grid launches nothing
    n = stub.stub_calls()
    assert mod.run(table, cx, (0, 2), args, {"num_warps": 4}) is None
    assert stub.stub_calls() == n


def test_c_launch_key_holds_every_specialization_fact(c_launch, monkeypatch):
    mod, _, _ = c_launch
    x, y, o = torch.zeros(100), torch.zeros(100), torch.zeros(100)
    cx = (False,) * 5 + (True,)
    base = (x, y, o, 2.5, 1000, 64)

    def key(args, kw=None, grid=(4,)):
        return mod.run({}, cx, grid, args, kw or {"num_warps": 4})
    k0 = key(base)
    assert key((y, x, o, -3.0, 1016, 64)) == k0          # values only
    assert key(base, grid=(8, 8)) == k0                   # the grid is not specialized on
    variants = [
        (x.double(), y, o, 2.5, 1000, 64),                # dtype
        (x[1:], y, o, 2.5, 1000, 64),                     # 16-byte alignment
        (x, y, o, 2.5, 1001, 64),                         # divisibility
        (x, y, o, 2.5, 1, 64),                            # == 1
        (x, y, o, 2.5, 1 << 33, 64),                      # int64
        (x, y, o, 2, 1000, 64),                           # int where a float was
        (x, y, o, 2.5, 1000, 128),                        # constexpr value
        (x, y, o, 2.5, 1000, 64.0),                       # constexpr type
    ]
    keys = {key(v) for v in variants}
    assert len(keys) == len(variants) and k0 not in keys
    assert key(base, {"num_warps": 8}) != k0              # launch options
    monkeypatch.setenv("NEWT_VEC", "1")                   # codegen switches
    assert key(base) != k0
    # shapes this path leaves to Python: a callable grid, an unknown argument type
    assert mod.run({}, cx, lambda m: (1,), base, {}) is False
    assert mod.run({}, cx, (4,), (x, y, o, 2.5, "s", 64), {}) is False
    assert mod.run({}, cx, (4,), (x, y, o, 2.5, 1 << 70, 64), {}) is False
    with pytest.raises(TypeError):                        # an unhashable constexpr
        mod.run({}, cx, (4,), (x, y, o, 2.5, 1000, [64]), {})


def test_c_launch_host_cost(c_launch):
    """Host time of a warm launch through the C path (the launch call itself
    is the stand-in): printed for the record."""
    mod, _, _ = c_launch
    from newt_amd.runtime import hip
    kinds = ["ptr", "ptr", "ptr", "i32"]
    offs, size = hip.pack_layout(kinds)
    x, y, o = torch.zeros(1 << 20), torch.zeros(1 << 20), torch.zeros(1 << 20)
    args, cx, kw = (x, y, o, 1 << 20), (False,) * 4 + (True,), {"BLOCK": 1024, "num_warps": 4}
    table = {}
    key = mod.run(table, cx, (1024,), args, kw)
    table[key] = mod.make_plan(1, 256, size, tuple((i, J._C_KINDS[k], off)
                                                   for i, (k, off) in enumerate(zip(kinds, offs))))
    reps = []
    for _ in range(20):
        t0 = time.perf_counter()
        for _ in range(1000):
            mod.run(table, cx, (1024,), args, {"BLOCK": 1024, "num_warps": 4})
        reps.append((time.perf_counter() - t0) / 1000 * 1e6)
    us = statistics.median(reps)
    print(f"C warm launch host path: {us:.2f} us per launch (median of 20 x 1000)")
    assert us < 20
