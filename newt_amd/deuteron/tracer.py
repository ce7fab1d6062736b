"""deuteron tracer: a @dt.kernel function -> the source of one @newt.jit kernel.

Behaviour follows the reference generator (deuteron/codegen.py:51-484): the
outermost `for ... in dt.tile(...)` loop is the launch grid (one program per
tile, up to 3 axes), inner dt.tile loops run sequentially over tiles, a
tensor subscripted by tiles (or `:`, a whole dimension sized to the next power
of two) is a masked load or store, `acc += a @ b` accumulates a dot, padded
lanes never reach a reduction, and every tile size is a constexpr so one
source serves every configuration the autotuner tries.

The design is this backend's own, in two phases:

  1. Tracing builds a small typed IR. Every expression node knows its axes
     (a tuple of tile dimensions, None for a size-1 axis made by `[:, None]`)
     and which of those axes may hold padded lanes. Broadcasting follows
     numpy's right-aligned rule; two whole-dimension axes that meet (x[t, :]
     * w[:]) are unified, become one constexpr, and the launch checks that
     their sizes agree. A reduction masks exactly the padded axes it folds;
     a dot whose contracted axis may be padded in both operands masks one of
     them to zero.
  2. Rendering prints the IR as newt source. Each tensor read is its own
     statement, so a k-loop `acc += x[m, k] @ y[k, n]` renders as the plain
     load / load / dot loop newt's compiler software-pipelines, with masks
     that are conjunctions of `index < extent` tests (which the compiler
     turns into one uniform in-bounds test per tile).
"""

import ast

from . import language as dl


class TraceError(Exception):
    pass


# --------------------------------------------------------------------------- dims

class Dim:
    """One tiled axis. role: 'grid' (a launch-grid axis), 'loop' (an inner
    tile loop) or 'whole' (a `:` subscript: the whole dimension in one tile).
    Whole dims that meet in an expression are merged (union-find)."""

    _created = 0

    def __init__(self, var, extent, role, const):
        Dim._created += 1
        self.order = Dim._created
        self.var = var          # stem of the rendered names (<var>_idx, <var>_in)
        self.extent = extent    # runtime size: "x_d1", a scalar parameter or an int literal
        self.role = role
        self.const = const      # constexpr holding the tile size
        self._parent = None
        self.members = [self]   # whole dims merged into this representative

    def find(self):
        d = self
        while d._parent is not None:
            d = d._parent
        return d

    def __repr__(self):
        return f"Dim({self.var}, {self.extent}, {self.role})"


def _merge(a, b, node, tracer):
    """The axis two operands share: a None axis broadcasts, equal dims are
    the same axis, two whole dims are unified, anything else is an error."""
    if a is None:
        return b
    if b is None:
        return a
    a, b = a.find(), b.find()
    if a is b:
        return a
    if a.role == "whole" and b.role == "whole":
        if b.order < a.order:
            a, b = b, a         # the dim seen first names the merged one
        b._parent = a
        a.members.extend(b.members)
        return a
    tracer.fail(node, f"tiles {a.var} and {b.var} cannot be combined elementwise")


def _broadcast(shapes, node, tracer):
    rank = max((len(s) for s in shapes), default=0)
    out = [None] * rank
    for s in shapes:
        for i, d in enumerate(s):
            pos = rank - len(s) + i
            out[pos] = _merge(out[pos], d, node, tracer)
    return tuple(out)


# --------------------------------------------------------------------------- IR

class Node:
    """An IR expression: `axes` (Dim or None per axis), `padded` (the dims
    whose out-of-range lanes may hold arbitrary values) and `zero_padded`
    (out-of-range lanes are known to be zero)."""

    axes = ()
    padded = frozenset()
    zero_padded = False

    def live_padded(self):
        return {d.find() for d in self.padded}

    def folded_padded(self, axis):
        """The padded dims a reduction over `axis` (None: every axis) folds:
        their out-of-range lanes must become the reduction's identity."""
        folded = self.axes if axis is None else (self.axes[axis],)
        live = self.live_padded()
        out = []
        for d in folded:
            if d is not None and d.find() in live and d.find() not in out:
                out.append(d.find())
        return out


class Const(Node):
    def __init__(self, text):
        self.text = text


class Ref(Node):
    """A named value: a local variable, a scalar parameter or a size symbol."""

    def __init__(self, text, axes=(), padded=frozenset(), zero_padded=False):
        self.text, self.axes, self.padded, self.zero_padded = text, axes, padded, zero_padded


class Load(Node):
    def __init__(self, tensor, dims, is_int):
        self.tensor, self.dims, self.is_int = tensor, dims, is_int
        self.axes = tuple(dims)
        self.padded = frozenset(dims)
        self.zero_padded = True


class Op(Node):
    """An elementwise operator or nl.* call over broadcast operands."""

    def __init__(self, fmt, operands, axes, padded):
        self.fmt, self.operands, self.axes, self.padded = fmt, operands, axes, padded


class Fill(Node):
    def __init__(self, dims, dtype, value):
        self.dims, self.dtype, self.value = dims, dtype, value
        self.axes = tuple(dims)
        self.zero_padded = value is None


class Dot(Node):
    def __init__(self, a, b, acc, mask_a, mask_b):
        self.a, self.b, self.acc = a, b, acc
        self.mask_a, self.mask_b = mask_a, mask_b
        self.axes = (a.axes[0], b.axes[1])
        pad = {d for d in a.live_padded() if d is a.axes[0].find()}
        pad |= {d for d in b.live_padded() if d is b.axes[1].find()}
        if acc is not None:
            pad |= acc.live_padded()
        self.padded = frozenset(pad)


class Reduce(Node):
    def __init__(self, fn, identity, value, axis, divide_by=None):
        self.fn, self.identity, self.value, self.axis = fn, identity, value, axis
        self.divide_by = divide_by
        if axis is None:
            self.axes = ()
            self.padded = frozenset()
        else:
            self.axes = value.axes[:axis] + value.axes[axis + 1:]
            self.padded = frozenset(value.live_padded() - {value.axes[axis].find()})


class Reshape(Node):
    """`v[:, None]`-style subscripts: `pattern` holds ':' and None entries."""

    def __init__(self, value, pattern):
        self.value, self.pattern = value, pattern
        it = iter(value.axes)
        self.axes = tuple(next(it) if p == ":" else None for p in pattern)
        self.padded = value.padded


class Assign:
    def __init__(self, name, node):
        self.name, self.node = name, node


class Store:
    def __init__(self, tensor, dims, node):
        self.tensor, self.dims, self.node = tensor, dims, node


class Loop:
    def __init__(self, dim, body):
        self.dim, self.body = dim, body


class Traced:
    """What the runtime needs to launch the generated kernel.

    name, source   the @newt.jit function's name and module source
    args           [('tensor', name, ndim) | ('scalar', name)] in call order;
                   a tensor passes (pointer, sizes..., strides...)
    grid           Dims of the launch grid, axis order
    tunable        constexprs the autotuner chooses (tile loops, in order)
    spans          [(constexpr, [extent symbols])]: whole-dimension tiles,
                   sized to the next power of two of extents that must agree
    writes         tensor parameters the kernel stores to
    has_dot        whether the kernel contracts tiles with a dot
    """

    def __init__(self, name, source, args, grid, tunable, spans, writes, has_dot):
        self.name, self.source, self.args, self.grid = name, source, args, grid
        self.tunable, self.spans, self.writes, self.has_dot = tunable, spans, writes, has_dot


# --------------------------------------------------------------------------- phase 1

_ARITH = {ast.Add: "+", ast.Sub: "-", ast.Mult: "*", ast.Div: "/", ast.FloorDiv: "//",
          ast.Mod: "%", ast.Pow: "**"}
_COMPARE = {ast.Eq: "==", ast.NotEq: "!=", ast.Lt: "<", ast.LtE: "<=", ast.Gt: ">",
            ast.GtE: ">="}
_INPLACE = {ast.Add: "+", ast.Sub: "-", ast.Mult: "*", ast.Div: "/"}


class _Tracer:
    def __init__(self, fn, fndef, args):
        import torch

        self.fn, self.fndef = fn, fndef
        names = [a.arg for a in fndef.args.args]
        if len(names) != len(args):
            raise TraceError(f"{fndef.name} takes {len(names)} arguments, called with {len(args)}")
        self.order = names
        self.tensors = {}       # name -> (ndim, dtype)
        self.scalars = set()
        for name, value in zip(names, args):
            if torch.is_tensor(value):
                if value.dtype not in dl.NL_DTYPES:
                    raise TraceError(f"tensor argument '{name}' has unsupported dtype {value.dtype}")
                self.tensors[name] = (value.dim(), value.dtype)
            elif isinstance(value, (bool, int, float)):
                self.scalars.add(name)
            else:
                raise TraceError(f"argument '{name}' must be a tensor or a Python number, "
                                 f"not {type(value).__name__}")
        self.tiles = {}         # tile variable -> Dim
        self.tile_order = []    # grid and loop Dims in order of appearance
        self.wholes = {}        # (tensor, axis) -> Dim
        self.grid = []
        self.env = {}           # local variable -> Ref
        self.writes = set()
        self.has_dot = False

    def fail(self, node, msg):
        raise TraceError(f"{self.fndef.name}:{getattr(node, 'lineno', '?')}: {msg}")

    def _is_dt(self, func, attr=None):
        if not (isinstance(func, ast.Attribute) and isinstance(func.value, ast.Name)):
            return False
        mod = getattr(self.fn.__globals__.get(func.value.id), "__name__", "")
        ok = mod in ("deuteron", "newt_amd.deuteron") or mod.endswith("deuteron.language")
        return ok and (attr is None or func.attr == attr)

    # ---- sizes and tiles
    def extent(self, node):
        if (isinstance(node, ast.Subscript) and isinstance(node.value, ast.Attribute)
                and node.value.attr == "shape" and isinstance(node.value.value, ast.Name)
                and node.value.value.id in self.tensors):
            if not (isinstance(node.slice, ast.Constant) and isinstance(node.slice.value, int)):
                self.fail(node, "index .shape with an integer literal")
            t, axis = node.value.value.id, node.slice.value
            if not 0 <= axis < self.tensors[t][0]:
                self.fail(node, f"'{t}' has no axis {axis}")
            return f"{t}_d{axis}"
        if isinstance(node, ast.Constant) and isinstance(node.value, int):
            return str(node.value)
        if isinstance(node, ast.Name) and node.id in self.scalars:
            return node.id
        self.fail(node, "a tile extent is tensor.shape[i], an integer literal or a scalar argument")

    def tile_extents(self, it):
        if not (isinstance(it, ast.Call) and self._is_dt(it.func, "tile") and len(it.args) == 1
                and not it.keywords):
            self.fail(it, "loops in a deuteron kernel iterate dt.tile(extent) or "
                          "dt.tile([extents])")
        a = it.args[0]
        return [self.extent(e) for e in (a.elts if isinstance(a, (ast.List, ast.Tuple)) else [a])]

    def new_tile(self, node, name, extent, role):
        if name in self.tiles:
            self.fail(node, f"tile variable '{name}' is bound twice")
        d = Dim(name, extent, role, f"BLOCK_{name.upper()}")
        self.tiles[name] = d
        self.tile_order.append(d)
        return d

    def whole(self, tensor, axis):
        d = self.wholes.get((tensor, axis))
        if d is None:
            d = Dim(f"{tensor}_all{axis}", f"{tensor}_d{axis}", "whole",
                    f"SPAN_{tensor.upper()}_{axis}")
            self.wholes[(tensor, axis)] = d
        return d

    # ---- statements
    def top(self):
        body = list(self.fndef.body)
        if body and isinstance(body[0], ast.Expr) and isinstance(body[0].value, ast.Constant):
            body = body[1:]
        loops = [s for s in body if isinstance(s, ast.For)]
        if len(loops) != len(body) or len(loops) != 1:
            bad = next((s for s in body if not isinstance(s, ast.For)), body[-1] if body else
                       self.fndef)
            self.fail(bad, "top level of a deuteron kernel must be exactly one "
                           "`for ... in dt.tile(...)` loop (the launch grid)")
        grid_loop = loops[0]
        if grid_loop.orelse:
            self.fail(grid_loop, "for/else is not supported")
        extents = self.tile_extents(grid_loop.iter)
        targets = self.loop_targets(grid_loop, len(extents))
        if len(targets) > 3:
            self.fail(grid_loop, "the launch grid has at most 3 tile axes")
        for name, ext in zip(targets, extents):
            self.grid.append(self.new_tile(grid_loop, name, ext, "grid"))
        return self.block(grid_loop.body)

    def loop_targets(self, node, count):
        targets = node.target.elts if isinstance(node.target, ast.Tuple) else [node.target]
        if not all(isinstance(t, ast.Name) for t in targets):
            self.fail(node, "tile loop targets must be plain names")
        if len(targets) != count:
            self.fail(node, f"{len(targets)} tile variables for {count} extents")
        return [t.id for t in targets]

    def block(self, stmts):
        out = []
        for s in stmts:
            self.statement(s, out)
        return out

    def statement(self, s, out):
        if isinstance(s, ast.For):
            if s.orelse:
                self.fail(s, "for/else is not supported")
            extents = self.tile_extents(s.iter)
            if len(extents) != 1:
                self.fail(s, "an inner tile loop walks one extent")
            (name,) = self.loop_targets(s, 1)
            dim = self.new_tile(s, name, extents[0], "loop")
            out.append(Loop(dim, self.block(s.body)))
            return
        if isinstance(s, ast.Expr) and isinstance(s.value, ast.Constant):
            return
        if isinstance(s, ast.Assign):
            if len(s.targets) != 1:
                self.fail(s, "one assignment target per statement")
            target = s.targets[0]
            if isinstance(target, ast.Subscript):
                out.append(self.store(s, target, self.expr(s.value)))
                return
            if isinstance(target, ast.Name):
                out.append(self.bind(target.id, self.expr(s.value)))
                return
            self.fail(s, "assign to a name or to a tensor subscript")
        if isinstance(s, ast.AugAssign):
            if not isinstance(s.target, ast.Name):
                self.fail(s, "augmented assignment updates a local variable")
            cur = self.env.get(s.target.id)
            if cur is None:
                self.fail(s, f"'{s.target.id}' is updated before it is assigned")
            v = s.value
            if isinstance(s.op, ast.Add) and isinstance(v, ast.BinOp) and isinstance(v.op, ast.MatMult):
                node = self.dot(s, self.expr(v.left), self.expr(v.right), cur)
            elif type(s.op) in _INPLACE:
                node = self.arith(s, _INPLACE[type(s.op)], cur, self.expr(v))
            else:
                self.fail(s, f"augmented {type(s.op).__name__} is not supported")
            out.append(self.bind(s.target.id, node))
            return
        if isinstance(s, ast.Expr):
            self.fail(s, "a bare expression has no effect in a deuteron kernel")
        self.fail(s, f"{type(s).__name__} statements are not supported")

    def bind(self, name, node):
        ref = Ref(f"v_{name}", node.axes, node.padded, node.zero_padded)
        self.env[name] = ref
        return Assign(ref.text, node)

    # ---- tensor accesses
    def access(self, node, sub):
        t = sub.value.id
        ndim = self.tensors[t][0]
        idx = sub.slice.elts if isinstance(sub.slice, ast.Tuple) else [sub.slice]
        if len(idx) != ndim:
            self.fail(node, f"'{t}' has {ndim} dims, indexed with {len(idx)}")
        if ndim not in (1, 2):
            self.fail(node, "tensor accesses are 1D or 2D")
        dims = []
        for axis, e in enumerate(idx):
            if isinstance(e, ast.Name) and e.id in self.tiles:
                dims.append(self.tiles[e.id])
            elif isinstance(e, ast.Slice) and e.lower is None and e.upper is None and e.step is None:
                dims.append(self.whole(t, axis))
            else:
                self.fail(node, "subscript a tensor with tile variables or ':'")
        return t, dims

    def store(self, node, target, value):
        if not (isinstance(target.value, ast.Name) and target.value.id in self.tensors):
            self.fail(node, "stores write to a tensor argument")
        t, dims = self.access(node, target)
        _broadcast([tuple(dims), value.axes], node, self)
        self.writes.add(t)
        return Store(t, dims, value)

    # ---- expressions
    def arith(self, node, sym, a, b):
        return Op("({0} " + sym + " {1})", [a, b], _broadcast([a.axes, b.axes], node, self),
                  a.padded | b.padded)

    def dot(self, node, a, b, acc=None):
        if len(a.axes) != 2 or len(b.axes) != 2 or None in a.axes + b.axes:
            self.fail(node, "@ contracts two 2D tiles")
        _merge(a.axes[1], b.axes[0], node, self)
        k = a.axes[1].find() if a.axes[1] is not None else None
        # an operand whose padded k lanes may hold anything (a computed value:
        # exp, log, a reciprocal of the zero a load put there) is zeroed there,
        # whatever the other operand holds: 0 * inf is NaN, so a zero-padded
        # load on the other side does not make the product safe
        unsafe = lambda v: k is not None and not v.zero_padded and k in v.live_padded()
        self.has_dot = True
        if acc is not None:
            _broadcast([(a.axes[0], b.axes[1]), acc.axes], node, self)
        return Dot(a, b, acc, mask_a=unsafe(a), mask_b=unsafe(b))

    def expr(self, node):
        if isinstance(node, ast.Constant):
            if not isinstance(node.value, (bool, int, float)):
                self.fail(node, f"constant {node.value!r} is not a number")
            return Const(repr(node.value))
        if isinstance(node, ast.Name):
            if node.id in self.env:
                return self.env[node.id]
            if node.id in self.scalars:
                return Ref(node.id)
            if node.id in self.tiles:
                self.fail(node, f"tile '{node.id}' is only an index or a dt.zeros/dt.full size")
            self.fail(node, f"name '{node.id}' is not defined in the kernel")
        if isinstance(node, ast.UnaryOp) and isinstance(node.op, (ast.USub, ast.UAdd)):
            v = self.expr(node.operand)
            return v if isinstance(node.op, ast.UAdd) else Op("(-{0})", [v], v.axes, v.padded)
        if isinstance(node, ast.BinOp):
            a, b = self.expr(node.left), self.expr(node.right)
            if isinstance(node.op, ast.MatMult):
                return self.dot(node, a, b)
            if type(node.op) not in _ARITH:
                self.fail(node, f"operator {type(node.op).__name__} is not supported")
            return self.arith(node, _ARITH[type(node.op)], a, b)
        if isinstance(node, ast.Compare):
            if len(node.ops) != 1:
                self.fail(node, "chained comparisons are not supported")
            return self.arith(node, _COMPARE[type(node.ops[0])], self.expr(node.left),
                              self.expr(node.comparators[0]))
        if isinstance(node, ast.Subscript):
            return self.subscript(node)
        if isinstance(node, ast.Call):
            return self.call(node)
        self.fail(node, f"{type(node).__name__} expressions are not supported")

    def subscript(self, node):
        v = node.value
        if isinstance(v, ast.Name) and v.id in self.tensors:
            t, dims = self.access(node, node)
            return Load(t, dims, not self.tensors[t][1].is_floating_point)
        if (isinstance(v, ast.Attribute) and v.attr == "shape" and isinstance(v.value, ast.Name)
                and v.value.id in self.tensors):
            return Ref(self.extent(node))
        base = self.expr(v)
        idx = node.slice.elts if isinstance(node.slice, ast.Tuple) else [node.slice]
        pattern = []
        for e in idx:
            if isinstance(e, ast.Constant) and e.value is None:
                pattern.append(None)
            elif isinstance(e, ast.Slice) and e.lower is None and e.upper is None and e.step is None:
                pattern.append(":")
            else:
                self.fail(node, "computed tiles take only ':' and None subscripts")
        if pattern.count(":") != len(base.axes):
            self.fail(node, f"{len(base.axes)}-D value subscripted with {pattern.count(':')} ':'")
        return Reshape(base, pattern)

    def call(self, node):
        f = node.func
        if self._is_dt(f):
            if f.attr in ("zeros", "full"):
                return self.fill(node, f.attr)
            fmt = dl.NL_CALLS.get(f.attr)
            if fmt is None:
                self.fail(node, f"dt.{f.attr} is not supported in compiled kernels")
            ops = [self.expr(a) for a in node.args]
            pad = frozenset().union(*(o.padded for o in ops)) if ops else frozenset()
            return Op(fmt, ops, _broadcast([o.axes for o in ops], node, self), pad)
        if (isinstance(f, ast.Name) and f.id in ("float", "int") and len(node.args) == 1
                and isinstance(node.args[0], ast.Constant)):
            return Const(f"{f.id}({node.args[0].value!r})")
        if isinstance(f, ast.Attribute):
            base = self.expr(f.value)
            if f.attr in dl.REDUCE_METHODS or f.attr == "mean":
                return self.reduce(node, base, f.attr)
            if f.attr == "to":
                self.fail(node, "casts with .to() are not traced: give dt.zeros / dt.full a dtype; "
                                "stores convert to the tensor's dtype")
        self.fail(node, "unsupported call")

    def fill(self, node, kind):
        if not node.args:
            self.fail(node, f"dt.{kind} needs a shape")
        shape = node.args[0]
        dims = []
        for e in (shape.elts if isinstance(shape, (ast.List, ast.Tuple)) else [shape]):
            if isinstance(e, ast.Name) and e.id in self.tiles:
                dims.append(self.tiles[e.id])
            else:
                self.fail(node, f"dt.{kind} shapes are lists of tile variables")
        dtype = "nl.float32"
        for kw in node.keywords:
            if kw.arg != "dtype":
                continue
            try:
                value = eval(compile(ast.Expression(kw.value), "<dtype>", "eval"),
                             self.fn.__globals__)
            except Exception:
                value = None
            dtype = dl.NL_DTYPES.get(value)
            if dtype is None:
                self.fail(node, "unsupported dtype")
        fill = None
        if kind == "full":
            if len(node.args) < 2:
                self.fail(node, "dt.full needs a fill value")
            fill = self.expr(node.args[1])
            if fill.axes:
                self.fail(node, "dt.full fills with a scalar")
        return Fill(dims, dtype, fill)

    def reduce(self, node, base, method):
        axis = None
        if node.args:
            if not isinstance(node.args[0], ast.Constant):
                self.fail(node, "reduction axes are integer literals")
            axis = node.args[0].value
        for kw in node.keywords:
            if kw.arg in ("axis", "dim"):
                if not isinstance(kw.value, ast.Constant):
                    self.fail(node, "reduction axes are integer literals")
                axis = kw.value.value
        rank = len(base.axes)
        if axis is not None:
            if not -rank <= axis < rank:
                self.fail(node, f"axis {axis} out of range for a {rank}-D value")
            axis %= rank
            if base.axes[axis] is None:
                self.fail(node, "reducing a size-1 axis")
        if method == "mean":
            folded = [d for d in (base.axes if axis is None else (base.axes[axis],)) if d]
            if any(d.find().role != "whole" for d in folded):
                self.fail(node, "mean() folds whole dimensions (':' subscripts) only: a tile "
                                "holds part of its dimension")
            sizes = " * ".join(d.find().extent for d in folded)
            return Reduce("nl.sum", "0.0", base, axis, divide_by=sizes or "1")
        fn, identity = dl.REDUCE_METHODS[method]
        return Reduce(fn, identity, base, axis)


# --------------------------------------------------------------------------- phase 2

def _mask_text(dims, axes):
    """`<d>_in` tests of `dims`, expanded to a value of `axes`."""
    terms = []
    for d in dims:
        pos = [a.find() if a is not None else None for a in axes].index(d)
        name = f"{d.var}_in"
        if len(axes) > 1:
            name += "[" + ", ".join(":" if i == pos else "None" for i in range(len(axes))) + "]"
        terms.append(name)
    return " & ".join(terms)


def _address(t, dims):
    dims = [d.find() for d in dims]
    if len(dims) == 1:
        return f"{t}_ptr + {dims[0].var}_idx * {t}_s0", f"{dims[0].var}_in"
    r, c = dims
    return (f"{t}_ptr + {r.var}_idx[:, None] * {t}_s0 + {c.var}_idx[None, :] * {t}_s1",
            f"{r.var}_in[:, None] & {c.var}_in[None, :]")


class _Renderer:
    def __init__(self):
        self.lines = []
        self.ntemp = 0

    def emit(self, depth, text):
        self.lines.append("    " * depth + text)

    def temp(self, depth, text):
        self.ntemp += 1
        name = f"_t{self.ntemp}"
        self.emit(depth, f"{name} = {text}")
        return name

    def expr(self, n, depth):
        if isinstance(n, (Const, Ref)):
            return n.text
        if isinstance(n, Load):
            addr, mask = _address(n.tensor, n.dims)
            other = "0" if n.is_int else "0.0"
            return self.temp(depth, f"nl.load({addr}, mask={mask}, other={other})")
        if isinstance(n, Op):
            return n.fmt.format(*[self.expr(o, depth) for o in n.operands])
        if isinstance(n, Fill):
            shape = "(" + ", ".join(d.find().const for d in n.dims) + ",)"
            if n.value is None:
                return f"nl.zeros({shape}, dtype={n.dtype})"
            return f"nl.full({shape}, {self.expr(n.value, depth)}, dtype={n.dtype})"
        if isinstance(n, Reshape):
            pat = ", ".join(":" if p == ":" else "None" for p in n.pattern)
            return f"({self.expr(n.value, depth)})[{pat}]"
        if isinstance(n, Dot):
            a, b = self.expr(n.a, depth), self.expr(n.b, depth)
            if n.mask_a:
                k = n.a.axes[1].find()
                a = self.temp(depth, f"nl.where({_mask_text([k], n.a.axes)}, {a}, 0.0)")
            if n.mask_b:
                k = n.b.axes[0].find()
                b = self.temp(depth, f"nl.where({_mask_text([k], n.b.axes)}, {b}, 0.0)")
            if n.acc is None:
                return f"nl.dot({a}, {b})"
            return f"nl.dot({a}, {b}, {self.expr(n.acc, depth)})"
        if isinstance(n, Reduce):
            v = self.expr(n.value, depth)
            masked = n.value.folded_padded(n.axis)
            if masked:
                v = f"nl.where({_mask_text(masked, n.value.axes)}, {v}, {n.identity})"
            axis = "" if n.axis is None else f", axis={n.axis}"
            out = f"{n.fn}({v}{axis})"
            return f"({out} / ({n.divide_by}))" if n.divide_by else out
        raise TraceError(f"cannot render {type(n).__name__}")

    def dim_header(self, depth, d, start):
        self.emit(depth, f"{d.var}_idx = {start}nl.arange(0, {d.const})")
        self.emit(depth, f"{d.var}_in = {d.var}_idx < {d.extent}")

    def body(self, stmts, depth):
        for s in stmts:
            if isinstance(s, Assign) and isinstance(s.node, Load):
                addr, mask = _address(s.node.tensor, s.node.dims)
                other = "0" if s.node.is_int else "0.0"
                self.emit(depth, f"{s.name} = nl.load({addr}, mask={mask}, other={other})")
            elif isinstance(s, Assign):
                self.emit(depth, f"{s.name} = {self.expr(s.node, depth)}")
            elif isinstance(s, Store):
                addr, mask = _address(s.tensor, s.dims)
                self.emit(depth, f"nl.store({addr}, {self.expr(s.node, depth)}, mask={mask})")
            else:
                d = s.dim
                self.emit(depth, f"for {d.var}_step in range(nl.cdiv({d.extent}, {d.const})):")
                self.dim_header(depth + 1, d, f"{d.var}_step * {d.const} + ")
                self.body(s.body, depth + 1)


def generate(fn, fndef, args):
    """Trace fn for example arguments (only ranks and dtypes matter) into the
    source of one @newt.jit kernel; returns a Traced."""
    tr = _Tracer(fn, fndef, args)
    body = tr.top()
    spans = []
    for d in tr.wholes.values():
        rep = d.find()
        if rep is d:
            spans.append(rep)
    r = _Renderer()
    for axis, d in enumerate(tr.grid):
        r.dim_header(1, d, f"nl.program_id({axis}) * {d.const} + ")
    for d in spans:
        r.dim_header(1, d, "")
    r.body(body, 1)

    sig, plan = [], []
    for name in tr.order:
        if name in tr.tensors:
            nd = tr.tensors[name][0]
            sig += [f"{name}_ptr"] + [f"{name}_d{i}" for i in range(nd)] + \
                   [f"{name}_s{i}" for i in range(nd)]
            plan.append(("tensor", name, nd))
        else:
            sig.append(name)
            plan.append(("scalar", name))
    sig += [f"{d.const}: nl.constexpr" for d in tr.tile_order]
    sig += [f"{d.const}: nl.constexpr" for d in spans]
    kname = f"{fndef.name}__tiles"
    text = ["import newt", "import newt.language as nl", "", "", "@newt.jit",
            f"def {kname}({', '.join(sig)}):"] + r.lines
    return Traced(kname, "\n".join(text) + "\n", plan, list(tr.grid),
                  [d.const for d in tr.tile_order],
                  [(d.const, [m.extent for m in d.members]) for d in spans],
                  set(tr.writes), tr.has_dot)
