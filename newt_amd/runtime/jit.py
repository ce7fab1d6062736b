"""@newt.jit: compile-on-first-call kernel wrapper for MI355X.

Surface and behaviour follow the reference (newt/runtime/jit.py:72-229):
arguments bind like a Python call; constexpr parameters are compile-time;
tensors become pointers (they must be on the current GPU), bools int1, ints
int32/int64 by range, floats fp32; grids are a tuple, an int, or a callable
over META (runtime args + constexprs + num_warps); an empty grid is a no-op;
launches go on torch's current stream and nothing is synchronized.

What differs is the backend: `num_warps` counts wave64s (64 threads each, so at
most 16); an optional `waves_per_eu=N` launch option (as in Triton's ROCm
backend) asks the register allocator to leave room for N waves per SIMD;
kernels are specialized, as Triton does, on integer arguments equal to 1 and on
the power-of-two divisibility (up to 16) of integers and of pointer addresses;
code objects come from hipRTC and are cached on disk under ~/.newt/cache
(NEWT_CACHE_DIR) keyed by the HIP source, the device-template header, the
target, the hipRTC version and this backend's version; launches pass one packed
argument buffer through hipModuleLaunchKernel.
"""

import ast
import functools
import hashlib
import inspect
import os
import textwrap

from ..compiler import Param, compile_fn
from ..compiler import types as tp
from ..compiler.codegen import _CKEYWORDS
from . import hip as _hip


# environment switches that change generated code (part of the specialization key)
# Timing hook: None, or a callable returning the (start, stop) hipEvent_t
# handles that the next launch's dispatch records at the kernel's start and end
# (a benchmark sets it around its timed launches). It is process-wide: while it
# is set, every newt launch from any thread takes a pair, so set it only
# around launches the timing code makes itself.
launch_events = None

_CODEGEN_ENV = ("NEWT_VEC", "NEWT_PIPELINE_DOT", "NEWT_LDS_DMA", "NEWT_MFMA", "NEWT_PID_REMAP",
                "NEWT_PIPE_VERSION", "NEWT_PLR", "NEWT_SCHED", "NEWT_HOIST_LOADS", "NEWT_PID_GROUP", "NEWT_IGLP",
                "NEWT_BUFFER_DMA", "NEWT_NT_STORE", "NEWT_BARE_BARRIER", "NEWT_WHERE_VERSION", "NEWT_NT_LOAD", "NEWT_NT_STREAM",
                "NEWT_REDUCE_PINGPONG", "NEWT_PIPE_CLAMP", "NEWT_CSE", "NEWT_VERSION_BODY",
                "NEWT_PID_LPT", "NEWT_PERM16",
                "NEWT_PAIR_REDUCE")
_CODEGEN_ENV_B = tuple(k.encode() for k in _CODEGEN_ENV)


class _Dev:
    """The current device and stream, read the way a launch needs them: the
    first call goes through torch.cuda (which initialises the runtime), later
    ones through torch's raw accessors (no Stream object per launch)."""

    ready = False

    @classmethod
    def device(cls):
        import torch
        if cls.ready:
            return torch._C._cuda_getDevice()
        d = torch.cuda.current_device()
        cls.ready = True
        return d

    @staticmethod
    def stream(device):
        import torch
        return torch._C._cuda_getCurrentRawStream(device)


# the warm-launch path in C (csrc/newt_pylaunch.c): None until first use, then
# the module, or False where it is not built (launches then stay in Python)
_C_LAUNCH = None
_C_KINDS = {"ptr": 0, "f32": 1, "i32": 2, "i64": 3, "bool": 4}


def _c_launcher():
    global _C_LAUNCH
    if _C_LAUNCH is None:
        _C_LAUNCH = False
        if os.environ.get("NEWT_C_LAUNCH", "1") == "0":
            return False
        import importlib.machinery
        import importlib.util
        import sysconfig

        import torch
        path = os.path.join(os.path.dirname(_hip.LIB_PATH),
                            "_newt_launch" + sysconfig.get_config_var("EXT_SUFFIX"))
        if not os.path.exists(path):
            return False
        _hip.lib()   # the backend library first: the launcher resolves its entry point
        loader = importlib.machinery.ExtensionFileLoader("_newt_launch", path)
        spec = importlib.util.spec_from_file_location("_newt_launch", path, loader=loader)
        mod = importlib.util.module_from_spec(spec)
        loader.exec_module(mod)
        mod.init(_hip.LIB_PATH, torch._C._cuda_getDevice, torch._C._cuda_getCurrentRawStream,
                 os.environ._data, _CODEGEN_ENV_B, torch.Tensor)
        _C_LAUNCH = mod
    return _C_LAUNCH


def _env_snapshot():
    """The codegen switches as a tuple, read without os.environ's per-key
    string encoding (a launch reads it on every call)."""
    data = getattr(os.environ, "_data", None)
    if isinstance(data, dict):
        return tuple(map(data.get, _CODEGEN_ENV_B))
    return tuple(os.environ.get(k) for k in _CODEGEN_ENV)


def _cache_dir():
    d = os.environ.get("NEWT_CACHE_DIR") or os.path.join(os.path.expanduser("~"), ".newt", "cache")
    os.makedirs(d, exist_ok=True)
    return d


def _is_constexpr_ann(ann):
    from .. import language as nl

    if ann is nl.constexpr or isinstance(ann, nl.constexpr):
        return True
    return isinstance(ann, str) and "constexpr" in ann


def _pow2_div(v, cap=16):
    v = abs(int(v))
    if v == 0:
        return cap
    return min(v & -v, cap)


@functools.cache
def _arch():
    """gfx target of the current device (the compiler only targets gfx950)."""
    import torch

    if not torch.cuda.is_available():
        return _hip.TARGET_ARCH
    name = _hip.device_arch(torch.cuda.current_device()).split(":")[0]
    if name != _hip.TARGET_ARCH:
        raise RuntimeError(f"newt_amd generates code for {_hip.TARGET_ARCH} (MI355X) only; "
                           f"the current device is {name}")
    return name


def cache_key(source):
    """Disk-cache key of a kernel's code object: the generated HIP source,
    the device-template header it includes, the target, the hipRTC version,
    this backend's version and the compile options."""
    key_src = "\n".join([source, _hip.device_header(), _arch(), str(_hip.rtc_version()),
                         _hip.BACKEND_VERSION, " ".join(_hip.COMPILE_OPTIONS)])
    return hashlib.sha256(key_src.encode()).hexdigest()[:32]


def _write_atomic(path, data):
    tmp = f"{path}.{os.getpid()}.tmp"
    with open(tmp, "wb") as f:
        f.write(data)
    os.replace(tmp, path)


def _cached_image(path):
    """The code object at `path` if the sha256 recorded beside it (`.sha256`)
    matches its bytes and it is an ELF image; None when the file is missing,
    truncated, corrupted or has no digest (the caller then recompiles)."""
    try:
        with open(path, "rb") as f:
            code = f.read()
        with open(path[:-len(".hsaco")] + ".sha256") as f:
            want = f.read().strip()
    except OSError:
        return None
    if code[:4] != b"\x7fELF" or hashlib.sha256(code).hexdigest() != want:
        return None
    return code


def code_object(source, name):
    """hipRTC-compile (or fetch from the disk cache) a kernel's code object.

    Cache entries under NEWT_CACHE_DIR (default ~/.newt/cache) are
    <key>.hsaco (the image hipModuleLoadData receives), <key>.sha256 (its
    digest, checked on the host before the image is used) and <key>.hip (the
    source, for inspection). An entry that fails the check is rebuilt."""
    key = cache_key(source)
    base = os.path.join(_cache_dir(), key)
    code = _cached_image(base + ".hsaco")
    if code is not None:
        return code
    try:
        code = _hip.compile_hip(source, name, _arch())
    except _hip.HIPRTCError as e:
        lined = "\n".join(f"{i + 1:4d} | {ln}" for i, ln in enumerate(source.splitlines()))
        raise _hip.HIPRTCError(f"{e}\n--- generated source ---\n{lined}") from None
    _write_atomic(base + ".hsaco", code)
    _write_atomic(base + ".sha256", hashlib.sha256(code).hexdigest().encode())
    _write_atomic(base + ".hip", source.encode())
    return code


class CompiledKernel:
    def __init__(self, name, source, lds_bytes, num_warps, params):
        self.name = name
        self.source = source
        self.lds_bytes = lds_bytes
        self.num_warps = num_warps
        self.params = params  # list of (name, Param)
        self.param_names = [n for n, _ in params]
        self.kinds = []
        for _, p in params:
            if isinstance(p.dtype, tp.pointer_type):
                self.kinds.append("ptr")
            elif p.dtype == tp.int1:
                self.kinds.append("bool")
            elif p.dtype == tp.int64:
                self.kinds.append("i64")
            elif p.dtype.is_int:
                self.kinds.append("i32")
            else:
                self.kinds.append("f32")
        self.packer = _hip.pack_format(self.kinds)
        self.code = code_object(source, name)
        self.kernel = _hip.Kernel(self.code, name, lds_bytes)

    def launch(self, grid, values, stream):
        """grid: (gx, gy, gz) workgroups; values: the parameters in order."""
        gx, gy, gz = grid
        ev = launch_events
        if ev is None:
            self.kernel.launch_packed(gx, gy, gz, 64 * self.num_warps, stream,
                                      self.packer.pack(*values))
        else:
            self.kernel.launch_packed_timed(gx, gy, gz, 64 * self.num_warps, stream,
                                            self.packer.pack(*values), *ev())


class JITFunction:
    def __init__(self, fn):
        functools.update_wrapper(self, fn)
        self.fn = fn
        src = textwrap.dedent(inspect.getsource(fn))
        tree = ast.parse(src)
        self.fndef = tree.body[0]
        assert isinstance(self.fndef, ast.FunctionDef)
        sig = inspect.signature(fn)
        self.param_names = list(sig.parameters)
        self.constexpr_names = [n for n, p in sig.parameters.items()
                                if _is_constexpr_ann(p.annotation)]
        self.defaults = {n: p.default for n, p in sig.parameters.items()
                         if p.default is not inspect.Parameter.empty}
        self.cache = {}
        # launch fast path: call signature -> (CompiledKernel, argument plan)
        self._fast = {}
        # the C launcher's plans: its call key -> plan
        self._ctable = {}
        self._cx_pos = tuple(n in self.constexpr_names for n in self.param_names)

    def __getitem__(self, grid):
        return functools.partial(self._run, grid)

    def __call__(self, *args, **kwargs):
        raise RuntimeError(
            f"@newt.jit kernel '{self.fn.__name__}' must be launched with a grid: "
            f"kernel[grid](...)")

    def _classify(self, args, kwargs):
        """(constexprs, runtime values) from a call (reference jit.py:99-123)."""
        if len(args) > len(self.param_names):
            raise TypeError(f"{self.fn.__name__}() takes {len(self.param_names)} arguments "
                            f"but {len(args)} were given")
        bound = dict(zip(self.param_names, args))
        for name, val in kwargs.items():
            if name in self.param_names:
                if name in bound:
                    raise TypeError(f"duplicate argument {name}")
                bound[name] = val
        unknown = [k for k in kwargs if k not in self.param_names]
        if unknown:
            raise TypeError(f"unknown kernel arguments: {unknown}")
        for name, d in self.defaults.items():
            bound.setdefault(name, d)
        missing = [n for n in self.param_names if n not in bound]
        if missing:
            raise TypeError(f"missing kernel arguments: {missing}")
        constexprs = {n: bound[n] for n in self.constexpr_names}
        runtime = {n: bound[n] for n in self.param_names if n not in self.constexpr_names}
        return constexprs, runtime

    @staticmethod
    def _type_of(name, val):
        """(dtype, specialization facts) of a runtime argument (reference jit.py:125-144)."""
        import torch

        if isinstance(val, torch.Tensor):
            if not val.is_cuda:
                raise TypeError(f"argument '{name}' must be a GPU tensor")
            elem = tp.TORCH_TO_NEWT.get(str(val.dtype))
            if elem is None:
                raise TypeError(f"unsupported tensor dtype {val.dtype} for '{name}'")
            return tp.pointer_type(elem), ("a16" if val.data_ptr() % 16 == 0 else "")
        if isinstance(val, bool):
            return tp.int1, ""
        if isinstance(val, int):
            if not -(2 ** 63) <= val < 2 ** 63:
                raise TypeError(f"integer argument '{name}'={val} does not fit int64")
            t = tp.int32 if -(2 ** 31) <= val < 2 ** 31 else tp.int64
            return t, ("1" if val == 1 else f"d{_pow2_div(val)}")
        if isinstance(val, float):
            return tp.float32, ""
        raise TypeError(f"unsupported kernel argument type {type(val)} for '{name}'")

    def _compile(self, key, constexprs, runtime_types, num_warps, num_stages, waves_per_eu=0):
        params = []
        for name in self.param_names:
            if name in self.constexpr_names:
                continue
            t, spec = runtime_types[name]
            cname = f"g_{name}" if name in _CKEYWORDS else name
            params.append((name, Param(t, cname, eq1=(spec == "1"),
                                       div=int(spec[1:]) if spec.startswith("d") else 1,
                                       aligned16=(spec == "a16"))))
        khash = hashlib.sha256(repr(key).encode()).hexdigest()[:8]
        kname = f"{self.fn.__name__}_{khash}"
        source, lds = compile_fn(self.fndef, self.fn.__globals__, params, constexprs,
                                 num_warps, kname, num_stages=num_stages,
                                 waves_per_eu=waves_per_eu)
        if os.environ.get("NEWT_DEBUG"):
            print(f"=== newt: {kname} (lds={lds}b, waves={num_warps}) ===")
            print(source)
        return CompiledKernel(kname, source, lds, num_warps, params)

    def specialize(self, *args, num_warps=4, num_stages=3, waves_per_eu=0, **kwargs):
        """Compile (without launching) for these arguments; returns the
        CompiledKernel (source, code object, resource usage)."""
        constexprs, runtime = self._classify(args, kwargs)
        types = {n: self._type_of(n, v) for n, v in runtime.items()}
        key = self._key(constexprs, types, num_warps, num_stages, waves_per_eu)
        # a code object is loaded into the current device: one entry per device
        key = key + (_Dev.device(),)
        ck = self.cache.get(key)
        if ck is None:
            ck = self._compile(key[:-1], constexprs, types, num_warps, num_stages, waves_per_eu)
            self.cache[key] = ck
        return ck

    @staticmethod
    def _key(constexprs, types, num_warps, num_stages, waves_per_eu=0):
        env = tuple(os.environ.get(k, "") for k in _CODEGEN_ENV)
        return (tuple(sorted((k, repr(v)) for k, v in constexprs.items())),
                tuple((n, t.name, s) for n, (t, s) in types.items()),
                num_warps, num_stages, waves_per_eu, env)

    def _call_signature(self, args, kwargs, opts):
        """A cheap, hashable summary of everything a launch specializes on:
        the launch options and current device (opts), the codegen switches,
        and per argument its dtype, 16-byte alignment and device (tensors),
        ==1, power-of-two divisibility and int32 range (ints), or type and
        value (constexprs). Raises TypeError for an unhashable constexpr."""
        import torch

        Tensor = torch.Tensor
        cx = self._cx_pos
        ncx = len(cx)
        out = [opts, _env_snapshot()]
        append = out.append
        for i, v in enumerate(args):
            if i < ncx and cx[i]:
                append((type(v), v))
                continue
            t = type(v)
            if t is int:
                append((v == 1, min(v & -v, 16) if v else 16, -2147483648 <= v < 2147483648))
            elif t is float:
                append(float)
            elif t is Tensor or isinstance(v, Tensor):
                # dtypes are singletons: their id stands for them (cheaper to
                # hash); get_device() is the device index (-1 on the CPU)
                append((id(v.dtype), not v.data_ptr() & 15, v.get_device()))
            else:
                append((t, v))
        for k, v in kwargs.items():
            append((k, (type(v), v) if k in self.constexpr_names else _arg_sig(v, torch)))
        sig = tuple(out)
        hash(sig)
        return sig

    def _plan(self, ck, args, kwargs, device):
        """The fast launch of this call signature: the compiled kernel and a
        function from (args, kwargs) to the kernel's parameter values, in the
        kernel's parameter order. Every tensor argument is checked here to be
        on the current device: the signature records each tensor's device and
        the current one, so a launch that reuses the plan needs no check."""
        import torch

        bound = dict(zip(self.param_names, args))
        bound.update(kwargs)
        for name, v in bound.items():
            if isinstance(v, torch.Tensor) and v.device.index not in (None, device):
                raise ValueError(f"tensor '{name}' is on {v.device} but the current device is "
                                 f"cuda:{device}; newt launches on the current device")
        pos = {n: i for i, n in enumerate(self.param_names[:len(args)])}
        items, consts = [], {}
        for name, p in ck.params:
            if name in pos:
                src = f"a[{pos[name]}]"
            elif name in kwargs:
                src = f"k[{name!r}]"
            else:
                consts[f"_d{len(consts)}"] = self.defaults[name]
                src = f"_d{len(consts) - 1}"
            if isinstance(p.dtype, tp.pointer_type):
                items.append(f"{src}.data_ptr()")
            elif p.dtype == tp.float32:
                items.append(f"float({src})")
            else:
                items.append(src)
        # one generated expression instead of a loop over the parameters
        values = eval(f"lambda a, k: ({', '.join(items)}{',' if len(items) == 1 else ''})",
                      consts)
        return ck, values

    def _run(self, grid, *args, **kwargs):
        ckey = None
        C = _C_LAUNCH if _C_LAUNCH is not None else _c_launcher()
        if C and not _Dev.ready:
            try:
                _Dev.device()       # initialises the runtime once, through torch
            except (RuntimeError, AssertionError):
                pass                # no GPU: the Python path reports what is wrong
        if C and _Dev.ready and launch_events is None:
            try:
                r = C.run(self._ctable, self._cx_pos, grid, args, kwargs)
            except TypeError:     # an unhashable constexpr: the Python path reports it
                r = False
            if r is None:
                return
            if type(r) is int:
                _hip._check(r, "hipModuleLaunchKernel")
            if type(r) is tuple:
                ckey = r
        num_warps = kwargs.pop("num_warps", 4)
        num_stages = kwargs.pop("num_stages", 3)
        waves_per_eu = kwargs.pop("waves_per_eu", 0)
        try:
            device = _Dev.device()
        except (RuntimeError, AssertionError):
            device = None   # no GPU: the slow path reports argument errors first
        try:
            csig = self._call_signature(args, kwargs, (num_warps, num_stages, waves_per_eu,
                                                       device))
        except TypeError:
            csig = None
        fast = self._fast.get(csig) if csig is not None else None
        if fast is None:
            fast = self._slow_path(args, kwargs, num_warps, num_stages, waves_per_eu, device)
            if csig is not None:
                self._fast[csig] = fast
        ck, values = fast
        if callable(grid):
            meta = dict(self.defaults)
            meta.update(zip(self.param_names, args))
            meta.update(kwargs)
            meta["num_warps"] = num_warps
            grid = grid(meta)
        if type(grid) is not tuple:
            grid = (grid,) if isinstance(grid, int) else tuple(grid)
        if len(grid) == 1:
            g = (int(grid[0]), 1, 1)
        else:
            g = (tuple(int(x) for x in grid) + (1, 1))[:3]
        if g[0] <= 0 or g[1] <= 0 or g[2] <= 0:
            return  # empty grid: no-op
        ck.launch(g, values(args, kwargs), _Dev.stream(device))
        if ckey is not None:
            self._register_c_plan(ckey, ck, args)

    def _register_c_plan(self, ckey, ck, args):
        """Hand the C launcher a plan for this call signature when every
        kernel parameter comes from a positional argument."""
        pos = {n: i for i, n in enumerate(self.param_names[:len(args)])}
        func = getattr(getattr(ck, "kernel", None), "func", None)
        if not (func and func.value) or any(n not in pos for n, _ in ck.params):
            return
        offs, size = _hip.pack_layout(ck.kinds)
        slots = tuple((pos[n], _C_KINDS[k], o) for (n, _), k, o in zip(ck.params, ck.kinds, offs))
        self._ctable[ckey] = _C_LAUNCH.make_plan(func.value, 64 * ck.num_warps, size, slots)

    def _slow_path(self, args, kwargs, num_warps, num_stages, waves_per_eu, device):
        """First launch of a call signature: option checks, binding, types,
        the specialization (compiled on a cache miss) and its launch plan."""
        waves_per_eu = int(waves_per_eu)
        if not 0 <= waves_per_eu <= 8:
            raise ValueError(f"waves_per_eu must be in 0..8 (0 = no request), got {waves_per_eu}")
        if num_warps not in (1, 2, 4, 8, 16):
            raise ValueError(f"num_warps must be a power of two <= 16 (wave64s per "
                             f"workgroup, at most 1024 threads), got {num_warps}")
        if not 1 <= num_stages <= 8:
            raise ValueError(f"num_stages must be in 1..8, got {num_stages}")
        constexprs, runtime = self._classify(args, kwargs)
        types = {n: self._type_of(n, v) for n, v in runtime.items()}
        if device is None:
            import torch
            device = torch.cuda.current_device()   # raises the runtime's own error
        key = self._key(constexprs, types, num_warps, num_stages, waves_per_eu) + (device,)
        ck = self.cache.get(key)
        if ck is None:
            ck = self._compile(key[:-1], constexprs, types, num_warps, num_stages, waves_per_eu)
            self.cache[key] = ck
        return self._plan(ck, args, kwargs, device)


def _arg_sig(v, torch):
    """_call_signature's entry for a runtime argument passed by keyword."""
    t = type(v)
    if t is int:
        return ("i", v == 1, _pow2_div(v), -(2 ** 31) <= v < 2 ** 31)
    if t is float:
        return "f"
    if t is bool:
        return "b"
    if isinstance(v, torch.Tensor):
        return (id(v.dtype), v.data_ptr() % 16 == 0, v.get_device())
    return ("?", t, v)


def jit(fn=None):
    if fn is None:
        return jit
    return JITFunction(fn)
