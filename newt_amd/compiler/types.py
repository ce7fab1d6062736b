"""Scalar dtypes, pointer types and the promotion rules of the newt DSL.

Semantics follow newt/compiler/types.py:4-117 of the reference (names, itemsizes,
kinds, numpy-flavoured promotion, broadcasting); the device type names are HIP's
native clang types for gfx950 (`_Float16`, `__bf16`) instead of CUDA's
`__half` / `__nv_bfloat16`.
"""


class dtype:
    """A scalar element type. `ctype` is the HIP C++ spelling used by codegen."""

    def __init__(self, name, ctype, itemsize, kind):
        self.name = name
        self.ctype = ctype
        self.itemsize = itemsize
        self.kind = kind  # 'f' float, 'i' signed int, 'u' unsigned int, 'b' bool
        self.torch_name = name

    @property
    def is_floating(self):
        return self.kind == "f"

    @property
    def is_int(self):
        return self.kind in ("i", "u", "b")

    @property
    def is_signed(self):
        return self.kind == "i"

    @property
    def bits(self):
        return self.itemsize * 8

    def __repr__(self):
        return f"nl.{self.name}"

    def __eq__(self, other):
        return isinstance(other, dtype) and self.name == other.name

    def __hash__(self):
        return hash(self.name)


float64 = dtype("float64", "double", 8, "f")
float32 = dtype("float32", "float", 4, "f")
float16 = dtype("float16", "_Float16", 2, "f")
bfloat16 = dtype("bfloat16", "__bf16", 2, "f")
int64 = dtype("int64", "long long", 8, "i")
int32 = dtype("int32", "int", 4, "i")
int16 = dtype("int16", "short", 2, "i")
int8 = dtype("int8", "signed char", 1, "i")
uint32 = dtype("uint32", "unsigned int", 4, "u")
uint8 = dtype("uint8", "unsigned char", 1, "u")
int1 = dtype("int1", "bool", 1, "b")

ALL_DTYPES = [float64, float32, float16, bfloat16, int64, int32, int16, int8, uint32,
              uint8, int1]
BY_NAME = {d.name: d for d in ALL_DTYPES}

# torch dtype string -> newt dtype (reference newt/compiler/types.py:45-57)
TORCH_TO_NEWT = {
    "torch.uint32": uint32,
    "torch.float32": float32,
    "torch.float64": float64,
    "torch.float16": float16,
    "torch.bfloat16": bfloat16,
    "torch.int64": int64,
    "torch.int32": int32,
    "torch.int16": int16,
    "torch.int8": int8,
    "torch.uint8": uint8,
    "torch.bool": int1,
}


class pointer_type:
    """Pointer to global memory holding `element`s."""

    def __init__(self, element):
        self.element = element
        self.element_ty = element  # Triton-compatible alias: ptr.dtype.element_ty
        self.name = f"pointer<{element.name}>"

    @property
    def ctype(self):
        return f"{self.element.ctype}*"

    @property
    def is_floating(self):
        return False

    @property
    def is_int(self):
        return False

    def __repr__(self):
        return self.name

    def __eq__(self, other):
        return isinstance(other, pointer_type) and self.element == other.element

    def __hash__(self):
        return hash(("ptr", self.element))


_ORDER = ["int1", "int8", "uint8", "int16", "int32", "uint32", "int64",
          "float16", "bfloat16", "float32", "float64"]


def promote(a, b):
    """Binary promotion: floats beat ints, wider beats narrower, and
    float16 with bfloat16 gives float32 (reference types.py:86-99)."""
    if a == b:
        return a
    if a.is_floating != b.is_floating:
        return a if a.is_floating else b
    if a.is_floating and {a.name, b.name} == {"float16", "bfloat16"}:
        return float32
    return a if _ORDER.index(a.name) >= _ORDER.index(b.name) else b


def broadcast_shapes(s1, s2):
    """Numpy broadcasting over compile-time shapes (reference types.py:102-117)."""
    s1, s2 = tuple(s1), tuple(s2)
    if s1 == ():
        return s2
    if s2 == ():
        return s1
    n = max(len(s1), len(s2))
    a = (1,) * (n - len(s1)) + s1
    b = (1,) * (n - len(s2)) + s2
    out = []
    for x, y in zip(a, b):
        if x == y or x == 1 or y == 1:
            out.append(max(x, y))
        else:
            raise TypeError(f"incompatible block shapes {s1} and {s2}")
    return tuple(out)


def is_half(d):
    return d in (float16, bfloat16)


def compute_dtype(d):
    """fp16/bf16 arithmetic is carried out in fp32 and rounded per op."""
    return float32 if is_half(d) else d
