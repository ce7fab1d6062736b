"""Compile-time values of the newt compiler.

    Const    a Python value known at compile time (constexpr parameters, literals,
             dtypes, shapes, ...)
    Scalar   a uniform C value (same in every thread of the program): kernel
             parameters, program ids, reduction results, loop counters
    Block    a [power-of-two shape] value spread over the workgroup:
               Affine   lazy integer block  base + sum_d coef_d * index_d
                        (aranges and the pointer-offset arithmetic built on them)
               Lazy     lazy elementwise expression over Affine / Fill / Scalar
                        leaves (index arithmetic, masks, casts of indices)
               Fill     lazy block holding one scalar everywhere (zeros/full)
               PtrBlock pointer block: uniform base pointer + integer offset block
               LazyLoad a load not yet emitted (a dot may stage it straight to LDS)
               Reg      values materialized in registers under a Layout

Affine offsets are what let the code generator prove contiguity and alignment
of global accesses at compile time and turn masks like `offs < n` into one
uniform "whole tile in bounds" test, instead of the reference's per-group
runtime checks on materialized offset arrays (newt/compiler/codegen.py:1631-1680).
"""

from . import types as tp

BIG_DIV = 1 << 30


def _pow2_div(v):
    v = abs(int(v))
    if v == 0:
        return BIG_DIV
    return min(v & -v, BIG_DIV)


class Sym:
    """A uniform integer term: C expression, optional compile-time value, and a
    known power-of-two divisor (for alignment proofs)."""

    __slots__ = ("expr", "const", "div")

    def __init__(self, expr, const=None, div=1):
        self.expr = expr
        self.const = const
        self.div = div

    @staticmethod
    def c(v):
        v = int(v)
        return Sym(str(v) if v >= 0 else f"({v})", v, _pow2_div(v))

    def __repr__(self):
        return f"Sym({self.expr}, div={self.div})"

    @property
    def is_const(self):
        return self.const is not None


def s_add(a, b):
    if a.is_const and b.is_const:
        return Sym.c(a.const + b.const)
    if a.is_const and a.const == 0:
        return b
    if b.is_const and b.const == 0:
        return a
    return Sym(f"({a.expr} + {b.expr})", None, min(a.div, b.div))


def s_neg(a):
    if a.is_const:
        return Sym.c(-a.const)
    return Sym(f"(-{a.expr})", None, a.div)


def s_sub(a, b):
    return s_add(a, s_neg(b))


def s_mul(a, b):
    if a.is_const and b.is_const:
        return Sym.c(a.const * b.const)
    for x, y in ((a, b), (b, a)):
        if x.is_const:
            if x.const == 0:
                return Sym.c(0)
            if x.const == 1:
                return y
    return Sym(f"({a.expr} * {b.expr})", None, min(a.div * b.div, BIG_DIV))


class Val:
    kind = "?"


class Const(Val):
    kind = "const"

    def __init__(self, pyval):
        self.pyval = pyval

    def __repr__(self):
        return f"Const({self.pyval!r})"


class Scalar(Val):
    """Uniform value. `expr` is a C identifier or expression of immutable terms.
    For integer scalars `sym` carries the affine-friendly view (divisibility)."""

    kind = "scalar"

    def __init__(self, dtype, expr, sym=None, aligned16=False):
        self.dtype = dtype
        self.expr = expr
        self.sym = sym
        self.aligned16 = aligned16  # pointer scalars: base known 16-byte aligned

    @property
    def is_ptr(self):
        return isinstance(self.dtype, tp.pointer_type)

    def as_sym(self):
        if self.sym is not None:
            return self.sym
        return Sym(self.expr, None, 1)

    def __repr__(self):
        return f"Scalar({self.dtype}, {self.expr})"


class Block(Val):
    kind = "block"
    dtype = None
    shape = ()

    @property
    def numel(self):
        n = 1
        for d in self.shape:
            n *= d
        return n

    @property
    def is_ptr(self):
        return isinstance(self.dtype, tp.pointer_type)


class Affine(Block):
    """base + sum_d coefs[d] * index_d  (int32 or int64)."""

    def __init__(self, dtype, shape, base, coefs):
        self.dtype = dtype
        self.shape = tuple(shape)
        self.base = base                      # Sym
        self.coefs = dict(coefs)              # axis -> Sym (non-zero only)

    def __repr__(self):
        return f"Affine({self.shape}, {self.base}, {self.coefs})"


class Fill(Block):
    def __init__(self, dtype, shape, value):
        self.dtype = dtype
        self.shape = tuple(shape)
        self.value = value  # Const or Scalar (already of `dtype` semantics)

    def __repr__(self):
        return f"Fill({self.dtype}, {self.shape}, {self.value})"


class Lazy(Block):
    """Elementwise expression evaluated per element on demand.
    fn(list of C expressions of the operands) -> C expression."""

    def __init__(self, dtype, shape, fn, args, size=1):
        self.dtype = dtype
        self.shape = tuple(shape)
        self.fn = fn
        self.args = args
        self.size = size  # node count, to bound re-evaluation cost

    def __repr__(self):
        return f"Lazy({self.dtype}, {self.shape})"


class PtrBlock(Block):
    def __init__(self, base, offset):
        self.base = base          # Scalar (pointer)
        self.offset = offset      # Block of ints (Affine / Lazy / Reg)
        self.dtype = base.dtype
        self.shape = offset.shape

    @property
    def elem(self):
        return self.dtype.element

    def __repr__(self):
        return f"PtrBlock({self.base.expr}, {self.offset})"


class LazyLoad(Block):
    def __init__(self, ptr, mask, other, node):
        self.ptr = ptr
        self.mask = mask
        self.other = other
        self.node = node
        self.dtype = ptr.elem
        self.shape = ptr.shape
        self.consumed = False   # staged by a dot
        self.poisoned = False   # consumed, then a flush point passed
        self.result = None      # Reg once materialized

    def __repr__(self):
        return f"LazyLoad({self.ptr})"


class Reg(Block):
    """Materialized block: C array `var` of layout.nslots elements; if `vec` is
    nonzero the array holds ext-vectors of `vec` elements (MFMA accumulators)."""

    def __init__(self, dtype, shape, layout, var, vec=0, storage=False):
        self.dtype = dtype
        self.shape = tuple(shape)
        self.layout = layout
        self.var = var
        self.vec = vec
        self.storage = storage

    def at(self, s):
        """C lvalue of slot s (int or C expression)."""
        if self.vec:
            if isinstance(s, int):
                return f"{self.var}[{s // self.vec}][{s % self.vec}]"
            return f"{self.var}[({s}) / {self.vec}][({s}) % {self.vec}]"
        return f"{self.var}[{s}]"

    def __repr__(self):
        return f"Reg({self.dtype}, {self.shape}, {self.var}, {self.layout.tag})"


class Staged(Block):
    """A dot operand tile resident in one LDS stage of a pipelined loop.

    rec is the staged load's record (shape and dtype as loaded, LDS format,
    byte offset inside the stage); slot the stage index; trans a transposed
    view (nl.trans of the loaded block). Only nl.dot consumes these."""

    def __init__(self, rec, slot, trans=False):
        self.rec = rec
        self.slot = slot
        self.trans = trans
        self.dtype = rec["dt"]
        r0, r1 = rec["shape"]
        self.shape = (r1, r0) if trans else (r0, r1)

    def __repr__(self):
        return f"Staged({self.rec['name']}, slot={self.slot}, trans={self.trans})"
