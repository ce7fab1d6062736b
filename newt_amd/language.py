"""newt.language (`nl`) - the kernel DSL surface, unchanged from the reference.

Every symbol mirrors newt/language.py:1-256 of the reference: `constexpr` with
host-side arithmetic, the dtypes, and device-only stubs tagged `_newt_builtin`
that the compiler resolves by name. Calling a stub from ordinary Python raises.
"""

from .compiler.types import (  # noqa: F401  (re-exported dtypes)
    bfloat16,
    float16,
    float32,
    float64,
    int1,
    int8,
    int16,
    int32,
    int64,
    uint8,
    uint32,
)


class constexpr:
    """Annotation for compile-time constant kernel parameters
    (reference newt/language.py:23-75)."""

    def __init__(self, value=None):
        self.value = value

    def __class_getitem__(cls, item):
        return cls

    @staticmethod
    def _v(other):
        return other.value if isinstance(other, constexpr) else other

    def __add__(self, o):
        return constexpr(self.value + self._v(o))

    def __radd__(self, o):
        return constexpr(self._v(o) + self.value)

    def __sub__(self, o):
        return constexpr(self.value - self._v(o))

    def __rsub__(self, o):
        return constexpr(self._v(o) - self.value)

    def __mul__(self, o):
        return constexpr(self.value * self._v(o))

    def __rmul__(self, o):
        return constexpr(self._v(o) * self.value)

    def __floordiv__(self, o):
        return constexpr(self.value // self._v(o))

    def __eq__(self, o):
        return self.value == self._v(o)

    def __lt__(self, o):
        return self.value < self._v(o)

    def __le__(self, o):
        return self.value <= self._v(o)

    def __gt__(self, o):
        return self.value > self._v(o)

    def __ge__(self, o):
        return self.value >= self._v(o)

    def __hash__(self):
        return hash(self.value)

    def __index__(self):
        return int(self.value)

    def __int__(self):
        return int(self.value)

    def __bool__(self):
        return bool(self.value)

    def __repr__(self):
        return f"constexpr[{self.value!r}]"


def _device_only(fn):
    name = fn.__name__

    def stub(*args, **kwargs):
        raise RuntimeError(
            f"nl.{name} can only be called inside a @newt.jit kernel "
            f"(or via the interpreter with NEWT_INTERPRET=1)")

    stub.__name__ = name
    stub.__doc__ = fn.__doc__
    stub._newt_builtin = name
    return stub


# -- core ---------------------------------------------------------------------

@_device_only
def program_id(axis):
    """Index of the current program instance along grid axis 0-2."""


@_device_only
def num_programs(axis):
    """Number of program instances along a grid axis."""


@_device_only
def arange(start, end):
    """1D int32 block [start, end); end - start must be a power of two."""


@_device_only
def zeros(shape, dtype=float32):
    """Block of zeros. Each dim must be a power of two."""


@_device_only
def full(shape, value, dtype=float32):
    """Block filled with a scalar value."""


@_device_only
def load(pointer, mask=None, other=None):
    """Load a block from memory. Masked-off lanes yield `other` (default 0)."""


@_device_only
def store(pointer, value, mask=None):
    """Store a block to memory."""


# -- shape manipulation ---------------------------------------------------------

@_device_only
def expand_dims(x, axis):
    """Insert a size-1 dimension (same as x[:, None])."""


@_device_only
def broadcast_to(x, shape):
    """Broadcast a block to a larger shape."""


@_device_only
def reshape(x, shape):
    """Reshape, preserving the element count (row-major)."""


@_device_only
def trans(x):
    """Transpose a 2D block."""


@_device_only
def cast(x, dtype):
    """Elementwise cast (same as x.to(dtype))."""


# -- reductions -----------------------------------------------------------------

@_device_only
def sum(x, axis=None):
    """Sum along an axis (or all axes). fp16/bf16 reduce in fp32."""


@_device_only
def max(x, axis=None):
    """Maximum along an axis (or all axes)."""


@_device_only
def min(x, axis=None):
    """Minimum along an axis (or all axes)."""


# -- linear algebra ---------------------------------------------------------------

@_device_only
def dot(a, b, acc=None, out_dtype=float32):
    """Block matmul a[M,K] @ b[K,N] -> [M,N] float32 on the matrix cores (MFMA).

    fp16/bf16 inputs use the fp16/bf16 MFMA instructions, fp32 inputs the fp32
    MFMA. Pass `acc` to accumulate across loop iterations. M and N must be
    multiples of 16; K a multiple of 16 (8 for fp32).
    """


# -- elementwise math ---------------------------------------------------------------

@_device_only
def exp(x): ...


@_device_only
def exp2(x): ...


@_device_only
def log(x): ...


@_device_only
def log2(x): ...


@_device_only
def sqrt(x): ...


@_device_only
def rsqrt(x): ...


@_device_only
def sin(x): ...


@_device_only
def cos(x): ...


@_device_only
def tanh(x): ...


@_device_only
def erf(x): ...


@_device_only
def sigmoid(x): ...


@_device_only
def abs(x): ...


@_device_only
def floor(x): ...


@_device_only
def ceil(x): ...


@_device_only
def maximum(a, b): ...


@_device_only
def minimum(a, b): ...


@_device_only
def where(cond, a, b):
    """Elementwise select."""


@_device_only
def fma(a, b, c):
    """a * b + c, fused."""


# -- atomics --------------------------------------------------------------------------

@_device_only
def atomic_add(pointer, value, mask=None): ...


@_device_only
def atomic_max(pointer, value, mask=None): ...


# -- misc --------------------------------------------------------------------------------

@_device_only
def cdiv(a, b):
    """Ceiling division."""


@_device_only
def multiple_of(x, value):
    """Compiler hint: x is a multiple of value."""


@_device_only
def max_contiguous(x, value):
    """Compiler hint (accepted for Triton compatibility)."""


@_device_only
def static_assert(cond, msg=""):
    """Compile-time assertion on constexpr values."""


@_device_only
def static_print(*args):
    """Print constexpr values at compile time."""
