"""deuteron tracer: a @dt.kernel function's AST -> the source of a @newt.jit kernel.

Semantics follow the reference generator (deuteron/codegen.py:51-484): the
outermost `for ... in dt.tile(...)` becomes the launch grid (one program per
tile, at most 3 dims), inner dt.tile loops become sequential loops over tiles,
`tensor[tile, ...]` becomes pointer arithmetic on (ptr, dims, strides) with a
bounds mask, `:` spans a whole dimension (BLOCK = next power of two of it),
`acc += a @ b` accumulates into the dot, masks travel with values so that
reductions fill padded lanes with their identity, and every tile size is a
constexpr so one source serves every autotuner configuration.

The emitted code is shaped for this backend: each tensor read is its own
`_ldN = nl.load(...)` statement, so a k-loop `acc += x[..] @ y[..]` is a
plain load/load/dot loop that the compiler software-pipelines (direct-to-LDS
stages), and masks are built from `offs < size` comparisons the compiler turns
into one uniform in-bounds test per tile.
"""

import ast

from . import language as dl


class TraceError(Exception):
    pass


class TileDim:
    def __init__(self, name, size, kind, block):
        self.name = name      # tile variable name in the kernel function
        self.size = size      # runtime size symbol ("x_d1") or an int literal string
        self.kind = kind      # 'grid' | 'loop' | 'full'
        self.block = block    # constexpr parameter name ("BLOCK_TILE_M")

    @property
    def offs(self):
        return f"offs_{self.name}"

    @property
    def mask(self):
        return f"mask_{self.name}"


class Val:
    """A traced expression: newt source text, the mask of its padded lanes
    (or None when every lane is real) and its rank."""

    def __init__(self, code, mask=None, ndim=0):
        self.code = code
        self.mask = mask
        self.ndim = ndim


class KernelSource:
    def __init__(self, name, source, params, tiles, grid, tunable, stores):
        self.name = name          # @newt.jit function name in `source`
        self.source = source
        self.params = params      # [('tensor', name) | ('scalar', name)] in call order
        self.tile_vars = tiles    # every TileDim (grid, loop, full)
        self.grid_tiles = grid    # TileDims of the launch grid, axis order
        self.tunable = tunable    # constexpr names the autotuner chooses
        self.store_params = stores  # tensor parameters the kernel writes


_BINOPS = {ast.Add: "+", ast.Sub: "-", ast.Mult: "*", ast.Div: "/", ast.FloorDiv: "//",
           ast.Mod: "%", ast.Pow: "**"}
_CMPS = {ast.Eq: "==", ast.NotEq: "!=", ast.Lt: "<", ast.LtE: "<=", ast.Gt: ">", ast.GtE: ">="}


class Tracer:
    def __init__(self, fn, fndef, args):
        import torch

        self.fn = fn
        self.fndef = fndef
        names = [a.arg for a in fndef.args.args]
        if len(names) != len(args):
            raise TraceError(f"{fndef.name}: expected {len(names)} args, got {len(args)}")
        self.tensors = {}   # name -> (ndim, dtype)
        self.scalars = []
        for nm, v in zip(names, args):
            if torch.is_tensor(v):
                self.tensors[nm] = (v.dim(), v.dtype)
            elif isinstance(v, (bool, int, float)):
                self.scalars.append(nm)
            else:
                raise TraceError(f"unsupported argument type for '{nm}': {type(v).__name__}")
        self.params = names
        self.lines = []
        self.depth = 1
        self.tiles = {}
        self.full_tiles = {}
        self.grid = []
        self.env = {}
        self.stores = set()
        self.ntmp = 0

    # ------------------------------------------------------------ helpers
    def fail(self, node, msg):
        raise TraceError(f"{self.fndef.name}:{getattr(node, 'lineno', '?')}: {msg}")

    def emit(self, line):
        self.lines.append("    " * self.depth + line)

    def temp(self, code):
        self.ntmp += 1
        nm = f"_ld{self.ntmp}"
        self.emit(f"{nm} = {code}")
        return nm

    def is_dt(self, func, attr=None):
        """`func` is dt.<attr> for the module the kernel imported as dt."""
        if not (isinstance(func, ast.Attribute) and isinstance(func.value, ast.Name)):
            return False
        mod = self.fn.__globals__.get(func.value.id)
        modname = getattr(mod, "__name__", "")
        if modname not in ("deuteron", "newt_amd.deuteron") and not modname.endswith(
                "deuteron.language"):
            return False
        return attr is None or func.attr == attr

    # ------------------------------------------------------------- tiles
    def size_symbol(self, node):
        if (isinstance(node, ast.Subscript) and isinstance(node.value, ast.Attribute)
                and node.value.attr == "shape" and isinstance(node.value.value, ast.Name)
                and node.value.value.id in self.tensors):
            if not isinstance(node.slice, ast.Constant):
                self.fail(node, "shape index must be a literal")
            return f"{node.value.value.id}_d{node.slice.value}"
        if isinstance(node, ast.Constant) and isinstance(node.value, int):
            return str(node.value)
        if isinstance(node, ast.Name) and node.id in self.scalars:
            return node.id
        self.fail(node, "tile sizes must be x.shape[i], an int literal, or a scalar param")

    def tile_sizes(self, it):
        if not (isinstance(it, ast.Call) and self.is_dt(it.func, "tile")) or len(it.args) != 1:
            self.fail(it, "expected dt.tile(size) or dt.tile([sizes])")
        a = it.args[0]
        return [self.size_symbol(e) for e in (a.elts if isinstance(a, (ast.List, ast.Tuple))
                                              else [a])]

    def trace_for(self, node):
        if node.orelse:
            self.fail(node, "for/else not supported")
        sizes = self.tile_sizes(node.iter)
        targets = node.target.elts if isinstance(node.target, ast.Tuple) else [node.target]
        if len(targets) != len(sizes):
            self.fail(node, f"{len(targets)} tile vars but {len(sizes)} sizes")
        if not all(isinstance(t, ast.Name) for t in targets):
            self.fail(node, "tile targets must be plain names")
        names = [t.id for t in targets]
        if not self.grid:
            if len(names) > 3:
                self.fail(node, "grid tile loops support at most 3 dimensions")
            for axis, (nm, size) in enumerate(zip(names, sizes)):
                td = TileDim(nm, size, "grid", f"BLOCK_{nm.upper()}")
                self.tiles[nm] = td
                self.grid.append(td)
                self.emit(f"pid_{axis} = nl.program_id({axis})")
                self.emit(f"{td.offs} = pid_{axis} * {td.block} + nl.arange(0, {td.block})")
                self.emit(f"{td.mask} = {td.offs} < {size}")
            for s in node.body:
                self.trace_stmt(s)
            return
        if len(names) != 1:
            self.fail(node, "inner tile loops iterate one dimension at a time")
        nm, size = names[0], sizes[0]
        td = TileDim(nm, size, "loop", f"BLOCK_{nm.upper()}")
        self.tiles[nm] = td
        self.emit(f"for _i_{nm} in range(0, nl.cdiv({size}, {td.block})):")
        self.depth += 1
        self.emit(f"{td.offs} = _i_{nm} * {td.block} + nl.arange(0, {td.block})")
        self.emit(f"{td.mask} = {td.offs} < {size}")
        for s in node.body:
            self.trace_stmt(s)
        self.depth -= 1

    # -------------------------------------------------------- statements
    def trace_stmt(self, s):
        if isinstance(s, ast.For):
            return self.trace_for(s)
        if isinstance(s, ast.Expr) and isinstance(s.value, ast.Constant):
            return  # docstring / stray literal
        if isinstance(s, ast.Assign):
            if len(s.targets) != 1:
                self.fail(s, "single assignment targets only")
            t = s.targets[0]
            if isinstance(t, ast.Subscript):
                return self.store(s, t, self.expr(s.value))
            if isinstance(t, ast.Name):
                v = self.expr(s.value)
                self.emit(f"{t.id} = {v.code}")
                self.env[t.id] = Val(t.id, v.mask, v.ndim)
                return
            self.fail(s, "unsupported assignment target")
        if isinstance(s, ast.AugAssign):
            if not isinstance(s.target, ast.Name):
                self.fail(s, "augmented assignment needs a plain name target")
            nm = s.target.id
            cur = self.env.get(nm)
            if cur is None:
                self.fail(s, f"'{nm}' not defined before augmented assignment")
            v = s.value
            if isinstance(s.op, ast.Add) and isinstance(v, ast.BinOp) and isinstance(v.op, ast.MatMult):
                a, b = self.expr(v.left), self.expr(v.right)
                self.emit(f"{nm} = nl.dot({a.code}, {b.code}, {nm})")
                self.env[nm] = Val(nm, None, 2)
                return
            sym = {ast.Add: "+", ast.Sub: "-", ast.Mult: "*", ast.Div: "/"}.get(type(s.op))
            if sym is None:
                self.fail(s, "unsupported augmented operator")
            e = self.expr(v)
            self.emit(f"{nm} = {nm} {sym} ({e.code})")
            self.env[nm] = Val(nm, cur.mask or e.mask, max(cur.ndim, e.ndim))
            return
        if isinstance(s, ast.Expr):
            self.fail(s, "expression statements have no effect in deuteron kernels")
        self.fail(s, f"unsupported statement: {type(s).__name__}")

    # --------------------------------------------------- tensor accesses
    def index_tiles(self, node, sub):
        pname = sub.value.id
        ndim = self.tensors[pname][0]
        idx = sub.slice.elts if isinstance(sub.slice, ast.Tuple) else [sub.slice]
        if len(idx) != ndim:
            self.fail(node, f"'{pname}' has {ndim} dims but {len(idx)} indices given")
        tiles = []
        for d, e in enumerate(idx):
            if isinstance(e, ast.Name) and e.id in self.tiles:
                tiles.append(self.tiles[e.id])
            elif isinstance(e, ast.Slice) and e.lower is None and e.upper is None and e.step is None:
                sym = f"{pname}_d{d}"
                td = self.full_tiles.get(sym)
                if td is None:
                    k = len(self.full_tiles)
                    td = TileDim(f"full{k}", sym, "full", f"BLOCK_FULL{k}")
                    self.full_tiles[sym] = td
                tiles.append(td)
            else:
                self.fail(node, "tensor indices must be tile variables or ':'")
        return pname, tiles

    def address(self, node, sub):
        pname, tiles = self.index_tiles(node, sub)
        if len(tiles) == 1:
            t = tiles[0]
            return pname, f"{pname}_ptr + {t.offs} * {pname}_s0", t.mask, 1
        if len(tiles) == 2:
            a, b = tiles
            return (pname, f"{pname}_ptr + {a.offs}[:, None] * {pname}_s0 + "
                           f"{b.offs}[None, :] * {pname}_s1",
                    f"{a.mask}[:, None] & {b.mask}[None, :]", 2)
        self.fail(node, "only 1D and 2D tensor accesses are supported")

    def store(self, node, t, value):
        if not (isinstance(t.value, ast.Name) and t.value.id in self.tensors):
            self.fail(node, "stores must target a tensor parameter")
        pname, ptr, mask, _ = self.address(node, t)
        self.stores.add(pname)
        self.emit(f"nl.store({ptr}, {value.code}, mask={mask})")

    # ------------------------------------------------------- expressions
    def expr(self, node):
        if isinstance(node, ast.Constant):
            return Val(repr(node.value))
        if isinstance(node, ast.Name):
            if node.id in self.env:
                return self.env[node.id]
            if node.id in self.scalars:
                return Val(node.id)
            if node.id in self.tiles:
                self.fail(node, f"tile '{node.id}' can only be used as an index or size")
            self.fail(node, f"unknown name '{node.id}'")
        if isinstance(node, ast.UnaryOp) and isinstance(node.op, ast.USub):
            e = self.expr(node.operand)
            return Val(f"(-{e.code})", e.mask, e.ndim)
        if isinstance(node, ast.BinOp):
            a, b = self.expr(node.left), self.expr(node.right)
            if isinstance(node.op, ast.MatMult):
                return Val(f"nl.dot({a.code}, {b.code})", None, 2)
            sym = _BINOPS.get(type(node.op))
            if sym is None:
                self.fail(node, f"unsupported operator {type(node.op).__name__}")
            return Val(f"({a.code} {sym} {b.code})", a.mask or b.mask, max(a.ndim, b.ndim))
        if isinstance(node, ast.Compare):
            if len(node.ops) != 1:
                self.fail(node, "chained comparisons not supported")
            a, b = self.expr(node.left), self.expr(node.comparators[0])
            return Val(f"({a.code} {_CMPS[type(node.ops[0])]} {b.code})", a.mask or b.mask,
                       max(a.ndim, b.ndim))
        if isinstance(node, ast.Subscript):
            return self.subscript(node)
        if isinstance(node, ast.Call):
            return self.call(node)
        self.fail(node, f"unsupported expression: {type(node).__name__}")

    def subscript(self, node):
        import torch

        if isinstance(node.value, ast.Name) and node.value.id in self.tensors:
            pname, ptr, mask, ndim = self.address(node, node)
            other = "0" if self.tensors[pname][1] in (torch.int32, torch.int64) else "0.0"
            return Val(self.temp(f"nl.load({ptr}, mask={mask}, other={other})"), mask, ndim)
        if (isinstance(node.value, ast.Attribute) and node.value.attr == "shape"
                and isinstance(node.value.value, ast.Name) and node.value.value.id in self.tensors):
            return Val(self.size_symbol(node))
        base = self.expr(node.value)
        idx = node.slice.elts if isinstance(node.slice, ast.Tuple) else [node.slice]
        parts, added = [], 0
        for e in idx:
            if isinstance(e, ast.Constant) and e.value is None:
                parts.append("None")
                added += 1
            elif isinstance(e, ast.Slice) and e.lower is None and e.upper is None:
                parts.append(":")
            else:
                self.fail(node, "only ':' and None subscripts on computed values")
        sub = ", ".join(parts)
        mask = f"({base.mask})[{sub}]" if base.mask and added else base.mask
        return Val(f"({base.code})[{sub}]", mask, base.ndim + added)

    def call(self, node):
        if self.is_dt(node.func):
            fname = node.func.attr
            if fname in ("zeros", "full"):
                return self.fill(node, fname)
            tmpl = dl.NL_CALLS.get(fname)
            if tmpl is None:
                self.fail(node, f"dt.{fname} is not supported in compiled kernels")
            args = [self.expr(a) for a in node.args]
            mask = next((a.mask for a in args if a.mask), None)
            return Val(tmpl.format(*[a.code for a in args]), mask,
                       max((a.ndim for a in args), default=0))
        if isinstance(node.func, ast.Name) and node.func.id in ("float", "int") \
                and len(node.args) == 1 and isinstance(node.args[0], ast.Constant):
            return Val(f"{node.func.id}({node.args[0].value!r})")
        if isinstance(node.func, ast.Attribute):
            meth = node.func.attr
            base = self.expr(node.func.value)
            if meth in dl.REDUCE_METHODS or meth == "mean":
                return self.reduce(node, base, meth)
            if meth == "to":
                self.fail(node, "use dt.zeros(..., dtype=...) / implicit store casts instead of .to()")
        self.fail(node, f"unsupported call {ast.dump(node.func)[:60]}")

    def fill(self, node, fname):
        shape = node.args[0]
        elts = shape.elts if isinstance(shape, (ast.List, ast.Tuple)) else [shape]
        dims = []
        for e in elts:
            if isinstance(e, ast.Name) and e.id in self.tiles:
                dims.append(self.tiles[e.id].block)
            elif isinstance(e, ast.Constant) and isinstance(e.value, int):
                dims.append(str(e.value))
            else:
                self.fail(node, "dt.zeros/dt.full shapes hold tile variables or int literals")
        dtype = "nl.float32"
        for kw in node.keywords:
            if kw.arg == "dtype":
                try:
                    val = eval(compile(ast.Expression(kw.value), "<dtype>", "eval"),
                               self.fn.__globals__)
                except Exception:
                    val = None
                dtype = dl.NL_DTYPES.get(val)
                if dtype is None:
                    self.fail(node, "unsupported dtype")
        shp = f"({', '.join(dims)},)"
        if fname == "zeros":
            return Val(f"nl.zeros({shp}, dtype={dtype})", None, len(dims))
        return Val(f"nl.full({shp}, {self.expr(node.args[1]).code}, dtype={dtype})", None,
                   len(dims))

    def reduce(self, node, base, meth):
        axis = None
        if node.args and isinstance(node.args[0], ast.Constant):
            axis = node.args[0].value
        for kw in node.keywords:
            if kw.arg in ("axis", "dim") and isinstance(kw.value, ast.Constant):
                axis = kw.value.value
        if axis is not None and axis < 0:
            if base.ndim <= 0:
                self.fail(node, "cannot resolve a negative axis here; use a non-negative one")
            axis += base.ndim
        if meth == "mean":
            self.fail(node, "mean() is not supported yet; use .sum(axis) / explicit size")
        fn, identity = dl.REDUCE_METHODS[meth]
        inner = f"nl.where({base.mask}, {base.code}, {identity})" if base.mask else base.code
        ax = "" if axis is None else f", axis={axis}"
        return Val(f"{fn}({inner}{ax})", None, 0 if axis is None else max(0, base.ndim - 1))

    # -------------------------------------------------------------- output
    def source(self):
        body = self.fndef.body
        if body and isinstance(body[0], ast.Expr) and isinstance(body[0].value, ast.Constant):
            body = body[1:]
        for s in body:
            if not isinstance(s, ast.For):
                self.fail(s, "top level of a deuteron kernel must be `for ... in dt.tile(...)`")
            self.trace_for(s)
        # full-dimension tiles are discovered while tracing; their offsets go first
        head = []
        for td in self.full_tiles.values():
            head.append(f"    {td.offs} = nl.arange(0, {td.block})")
            head.append(f"    {td.mask} = {td.offs} < {td.size}")
        sig, launch = [], []
        for nm in self.params:
            if nm in self.tensors:
                nd = self.tensors[nm][0]
                sig += [f"{nm}_ptr"] + [f"{nm}_d{d}" for d in range(nd)] + \
                       [f"{nm}_s{d}" for d in range(nd)]
                launch.append(("tensor", nm))
            else:
                sig.append(nm)
                launch.append(("scalar", nm))
        tiles = list(self.tiles.values()) + list(self.full_tiles.values())
        sig += [f"{td.block}: nl.constexpr" for td in tiles]
        kname = f"{self.fndef.name}_newt"
        src = ["import newt", "import newt.language as nl", "", "", "@newt.jit",
               f"def {kname}({', '.join(sig)}):"] + head + self.lines
        return KernelSource(kname, "\n".join(src) + "\n", launch, tiles, list(self.grid),
                            [td.block for td in self.tiles.values()], set(self.stores))


def generate(fn, fndef, args):
    """Trace fn for these example arguments (ranks, dtypes) -> KernelSource."""
    return Tracer(fn, fndef, args).source()
