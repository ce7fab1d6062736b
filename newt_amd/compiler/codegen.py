"""The newt compiler for MI355X: Python kernel AST -> HIP C++ for gfx950.

Execution model (the reference's, newt/compiler/codegen.py:1-13, re-derived for
CDNA4): one program = one workgroup of 64 * num_warps threads (num_warps counts
wave64s); block values live in registers under a bit `Layout`
(layouts.py); reductions run in-thread, then across lanes with DPP/ds_swizzle
butterflies, then across waves through LDS; `nl.dot` runs on the MFMA matrix
cores from XOR-swizzled LDS tiles, with loop-carried accumulators in MFMA
registers and a global->LDS prefetch pipeline across loop iterations.

Index arithmetic (aranges, pointer offsets, masks) stays symbolic (`Affine`,
`Lazy`) until an access needs it, so contiguity, alignment and "whole tile in
bounds" are decided at compile time or by one uniform test, and per-element
offsets are recomputed from lane/slot coordinates instead of being held in
offset arrays.

Layout decisions that depend on later uses (the layout a loop-carried value
should live in, the layout a load should land in) are learned by compiling,
recording "hints" whenever a value had to be converted, and compiling again
with the hints applied (compile_fn drives this fixed point).

Language semantics (promotion, constant typing, per-op fp16 rounding, C integer
division, reduction identities, masked-load `other`, scalar-pointer atomics
once per program, control-flow and error rules) follow the reference; the
relevant reference lines are cited at each operation.
"""

import ast
import builtins
import math
import os
import re

from . import layouts as lo
from . import types as tp
from .values import (Affine, Block, Const, Fill, Lazy, LazyLoad, PtrBlock, Reg, Scalar,
                     Staged, Sym, s_add, s_mul, s_neg)


class CompileError(Exception):
    pass


_CKEYWORDS = {
    "auto", "bool", "break", "case", "char", "const", "continue", "default", "do",
    "double", "else", "enum", "extern", "float", "for", "goto", "if", "int", "long",
    "register", "return", "short", "signed", "sizeof", "static", "struct", "switch",
    "template", "this", "typedef", "union", "unsigned", "void", "volatile", "while",
    "half", "bool",
}

_BIN = {ast.Add: "+", ast.Sub: "-", ast.Mult: "*", ast.BitAnd: "&", ast.BitOr: "|",
        ast.BitXor: "^", ast.LShift: "<<", ast.RShift: ">>"}
_CMP = {ast.Eq: "==", ast.NotEq: "!=", ast.Lt: "<", ast.LtE: "<=", ast.Gt: ">",
        ast.GtE: ">="}

_MATH = {  # name -> (fp32 fn, fp64 fn)
    # fp32 exp2 is the hardware v_exp_f32 (1 ulp); results below 2**-126 flush
    # to zero instead of taking the library's denormal-scaling path, which
    # would cost a compare, two selects and an ldexp per element. fp32 exp is
    # exp2(x * log2 e) on the same unit (newt::exp_f32: relative error under
    # 8e-6 over the whole range, within the reference's 1e-5 for exp)
    "exp": ("newt::exp_f32", "exp"), "exp2": ("__builtin_amdgcn_exp2f", "exp2"), "log": ("logf", "log"),
    "log2": ("log2f", "log2"), "sqrt": ("sqrtf", "sqrt"), "rsqrt": ("rsqrtf", "rsqrt"),
    "sin": ("sinf", "sin"), "cos": ("cosf", "cos"), "tanh": ("tanhf", "tanh"),
    "erf": ("erff", "erf"), "floor": ("floorf", "floor"), "ceil": ("ceilf", "ceil"),
}

MAX_LDS = 160 * 1024
LAZY_LIMIT = 48  # max node count of a lazy expression before it is materialized


def _pow2(n):
    return n > 0 and (n & (n - 1)) == 0


# ---------------------------------------------------------------------------
# Storage of names that outlive a control-flow statement
# ---------------------------------------------------------------------------


class Storage:
    """A variable with persistent C storage (loop-carried or defined inside a
    branch/loop and read after it)."""

    def __init__(self, name, kind, cvar, dtype=None, shape=(), layout=None, base=None,
                 coefs=None, key=None, vec=0):
        self.name = name
        self.kind = kind      # 'scalar' | 'reg' | 'affine' | 'ptraffine' | 'ptrreg'
        self.cvar = cvar
        self.dtype = dtype
        self.shape = tuple(shape)
        self.layout = layout
        self.base = base      # pointer Scalar for ptr* kinds
        self.coefs = coefs    # affine kinds: axis -> Sym
        self.key = key        # hint key
        self.vec = vec


class _Prepass:
    """Names assigned inside each compound statement, and names read after it."""

    @staticmethod
    def assigned(node):
        out = set()
        for n in ast.walk(node):
            if isinstance(n, ast.Assign):
                for t in n.targets:
                    for e in ([t] if not isinstance(t, ast.Tuple) else t.elts):
                        if isinstance(e, ast.Name):
                            out.add(e.id)
            elif isinstance(n, (ast.AugAssign, ast.AnnAssign)):
                if isinstance(n.target, ast.Name):
                    out.add(n.target.id)
            elif isinstance(n, ast.For) and isinstance(n.target, ast.Name):
                out.add(n.target.id)
        return out

    @staticmethod
    def read(nodes):
        out = set()
        for node in nodes:
            for n in ast.walk(node):
                if isinstance(n, ast.Name) and isinstance(n.ctx, ast.Load):
                    out.add(n.id)
        return out

    @staticmethod
    def exposed(stmts):
        """Names whose value on entry to `stmts` may be read: read before an
        assignment that certainly runs first. Assignments inside loops and
        branches are not certain to run; a loop body's own exposed reads are
        exposed for the loop (except its target)."""
        rd = _Prepass.read
        live, defined = set(), set()
        for st in stmts:
            if isinstance(st, ast.Assign):
                live |= rd([st.value] + st.targets) - defined
                for t in st.targets:
                    defined |= {e.id for e in ast.walk(t)
                                if isinstance(e, ast.Name) and isinstance(e.ctx, ast.Store)}
            elif isinstance(st, (ast.AugAssign, ast.AnnAssign)):
                tgt = st.target.id if isinstance(st.target, ast.Name) else None
                vals = [st.value] if st.value is not None else []
                reads = rd(vals)
                if isinstance(st, ast.AugAssign) and tgt is not None:
                    reads |= {tgt}
                live |= reads - defined
                if tgt is not None:
                    defined.add(tgt)
            elif isinstance(st, ast.For):
                inner = _Prepass.exposed(st.body)
                if isinstance(st.target, ast.Name):
                    inner = inner - {st.target.id}
                live |= (rd([st.iter]) | inner | _Prepass.exposed(st.orelse)) - defined
            elif isinstance(st, ast.While):
                live |= (rd([st.test]) | _Prepass.exposed(st.body)
                         | _Prepass.exposed(st.orelse)) - defined
            elif isinstance(st, ast.If):
                live |= (rd([st.test]) | _Prepass.exposed(st.body)
                         | _Prepass.exposed(st.orelse)) - defined
            else:
                live |= rd([st]) - defined
        return live


class Codegen(ast.NodeVisitor):
    def __init__(self, fndef, fn_globals, params, constexprs, num_warps, kernel_name,
                 num_stages=3, hints=None, waves_per_eu=0):
        """params: list of (name, Param) for runtime parameters in signature order."""
        self.fndef = fndef
        self.globals = fn_globals
        self.W = num_warps
        self.T = 64 * num_warps
        self.name = kernel_name
        self.num_stages = num_stages
        self.waves_per_eu = waves_per_eu
        self.hints = dict(hints or {})
        self.new_hints = {}
        self.lines = []
        self.prologue = []
        self._blocks = []       # ids of the open C blocks, outermost first
        self._block_seq = 0
        self.cse = {}           # binop key -> (operands, result Reg, C block path)
        self.cse_on = os.environ.get("NEWT_CSE", "1") != "0"
        self.indent = 1
        self.tmpc = 0
        self.locals = {}
        self.storages = {}
        self.pending_loads = []
        self.coord_consts = {}
        self.lds_dedicated = 0
        self.lds_regions = []
        self.arena_bytes = 0
        self.loop_depth = 0
        self.pending_hoist = []
        self.body_stack = []
        self.dot_state = {}
        self.lds_arrays = []      # (name, bytes): distinct __shared__ arrays (pipeline stages)
        self.lds_pool = []        # indices of lds_arrays freed by finished pipelined loops
        self.pipe_records = []
        self.pipe_active = None   # pipeline state while its loop body compiles
        self.pid_remap = False
        self.group_pids = False   # set by compile_fn for matmul-shaped kernels
        self.remap_pids = True    # compile_fn: False when no data is shared by a subset of programs
        self.lpt_pids = False     # compile_fn: True when a program's work grows with program_id(0)
        self.params = params
        vec = 1
        for _, p in params:
            if isinstance(p.dtype, tp.pointer_type):
                vec = max(vec, 16 // p.dtype.element.itemsize)
        self.VEC = min(vec, 8)
        env = os.environ.get("NEWT_VEC")
        if env:
            self.VEC = int(env)
        for name, p in params:
            if p.eq1:
                self.locals[name] = Const(1)
            elif isinstance(p.dtype, tp.pointer_type):
                self.locals[name] = Scalar(p.dtype, p.cname, aligned16=p.aligned16)
            elif p.dtype.is_int and p.dtype != tp.int1:
                self.locals[name] = Scalar(p.dtype, p.cname, Sym(p.cname, None, p.div))
            else:
                self.locals[name] = Scalar(p.dtype, p.cname)
        for name, v in constexprs.items():
            self.locals[name] = Const(v)

    # ------------------------------------------------------------------ infra
    @property
    def indent(self):
        return len(self._blocks)

    @indent.setter
    def indent(self, depth):
        """Every increase opens a new C block (a fresh id), every decrease
        closes the innermost ones; `} else {` therefore gets an id of its own."""
        del self._blocks[depth:]
        while len(self._blocks) < depth:
            self._block_seq += 1
            self._blocks.append(self._block_seq)

    def cse_lookup(self, key, operands):
        """A register block computed earlier from the same operand objects by
        the same operation, if its C declaration is visible here."""
        hit = self.cse.get(key)
        if hit is None:
            return None
        ops, res, path = hit
        if len(ops) != len(operands) or any(x is not y for x, y in zip(ops, operands)):
            return None
        if tuple(self._blocks[:len(path)]) != path:
            return None
        return res

    def cse_store(self, key, operands, res):
        """Remember res for reuse: only materialized, immutable register
        blocks whose operands are not loop-carried storage (storage is
        rewritten in place; every read of it is a new object anyway)."""
        if not isinstance(res, Reg) or res.storage or not self.cse_on:
            return
        if any(isinstance(o, Reg) and o.storage for o in operands):
            return
        self.cse[key] = (tuple(operands), res, tuple(self._blocks))

    def err(self, node, msg):
        line = getattr(node, "lineno", "?")
        raise CompileError(f"{self.fndef.name}:{line}: {msg}")

    def emit(self, s):
        self.lines.append("  " * self.indent + s)

    def fresh(self, p="t"):
        self.tmpc += 1
        return f"_{p}{self.tmpc}"

    def barrier(self):
        self.emit("__syncthreads();")

    def lds_alloc(self, nbytes, align=16):
        """Dedicated LDS region (for the whole kernel); returns C byte offset expr."""
        off = (self.lds_dedicated + align - 1) // align * align
        self.lds_dedicated = off + nbytes
        name = f"_LDS{len(self.lds_regions)}"
        self.lds_regions.append((name, off))
        return name

    def lds_arena(self, nbytes):
        """Shared scratch region; the caller must barrier before writing it."""
        self.arena_bytes = max(self.arena_bytes, (nbytes + 15) // 16 * 16)
        return "_LDSA"

    # --------------------------------------------------------- literals/types
    def cdtype(self, v):
        if isinstance(v, Const):
            p = v.pyval
            if isinstance(p, bool):
                return tp.int1
            if isinstance(p, int):
                return tp.int32 if -2**31 <= p < 2**31 else tp.int64
            if isinstance(p, float):
                return tp.float32
            raise CompileError(f"constexpr {p!r} has no device type")
        return v.dtype

    def literal(self, pyval, dtype):
        if dtype is None:
            dtype = tp.float32 if isinstance(pyval, float) else tp.int32
        if isinstance(dtype, tp.pointer_type):
            raise CompileError("pointer literal")
        if dtype == tp.int1:
            return "true" if pyval else "false"
        if dtype.is_int:
            v = int(pyval)
            if dtype == tp.int64:
                if v == -2**63:
                    return "(-9223372036854775807LL - 1)"
                return f"{v}LL" if v >= 0 else f"({v}LL)"
            if dtype == tp.uint32:
                return f"{v & 0xffffffff}u"
            if v == -2**31:
                return "(-2147483647 - 1)"
            return str(v) if v >= 0 else f"({v})"
        f = float(pyval)
        if math.isinf(f) or math.isnan(f):
            bits = "0x7f800000u" if f > 0 else "0xff800000u"
            if math.isnan(f):
                bits = "0x7fc00000u"
            core = f"newt::bits_f32({bits})"
            if dtype == tp.float64:
                core = f"((double){core})"
        else:
            core = repr(f) + ("f" if dtype != tp.float64 else "")
            if core.startswith("-"):
                core = f"({core})"
        if dtype == tp.float16:
            return f"((f16){core})"
        if dtype == tp.bfloat16:
            return f"((bf16){core})"
        return core

    def conv(self, e, src, dst):
        """C conversion of expression e from dtype src to dst."""
        if src == dst or dst is None or src is None:
            return e
        if isinstance(src, tp.pointer_type) or isinstance(dst, tp.pointer_type):
            return e
        if dst in (tp.float16, tp.bfloat16):
            if src not in (tp.float32,):
                e = self.conv(e, src, tp.float32)
            return f"(({dst.ctype})({e}))"
        if src in (tp.float16, tp.bfloat16):
            e = f"((float)({e}))"
            return e if dst == tp.float32 else f"(({dst.ctype})({e}))"
        return f"(({dst.ctype})({e}))"

    def scalar_expr(self, v, dtype=None):
        """C expression of a Const/Scalar, optionally converted to dtype."""
        if isinstance(v, Const):
            return self.literal(v.pyval, dtype or self.cdtype(v))
        if dtype is None:
            return v.expr
        return self.conv(v.expr, v.dtype, dtype)

    def new_scalar(self, dtype, expr, sym=None):
        t = self.fresh()
        self.emit(f"const {dtype.ctype} {t} = {expr};")
        if sym is None and dtype.is_int and dtype != tp.int1:
            sym = Sym(t, None, 1)
        elif sym is not None:
            sym = Sym(t, sym.const, sym.div)
        return Scalar(dtype, t, sym)

    # ------------------------------------------------------------ coordinates
    def default_layout(self, shape):
        return lo.blocked(tuple(shape), self.W, self.VEC)

    def lane_part(self, L, d):
        key = (L.key(), d)
        name = self.coord_consts.get(key)
        if name is None:
            terms = L.hw_coord_terms(d)
            if not terms:
                name = ""
            else:
                name = f"_c{len(self.coord_consts)}"
                self.prologue.append(f"const int {name} = {' | '.join(terms)};")
            self.coord_consts[key] = name
        return name

    def coord(self, L, d, s):
        """C expression of the coordinate along dim d of slot s (int) in L."""
        if L.shape[d] == 1:
            return "0"
        lp = self.lane_part(L, d)
        rp = L.reg_coord(s, d)
        if lp and rp:
            return f"({lp} + {rp})"
        if lp:
            return lp
        return str(rp)

    def canon_cond(self, L):
        conds = []
        lm, wm = L.lane_rep_mask(), L.wave_rep_mask()
        if lm:
            conds.append(f"((_lane & {lm}) == 0)")
        if wm:
            conds.append(f"((_wave & {wm}) == 0)")
        return " && ".join(conds) if conds else None

    # ------------------------------------------------------------ shape utils
    def expand_to_rank(self, v, rank):
        while isinstance(v, Block) and len(v.shape) < rank:
            v = self.expand_dims(v, 0)
        return v

    def expand_dims(self, v, axis):
        if isinstance(v, (Const, Scalar)):
            return v
        if isinstance(v, LazyLoad):
            v = self.materialize_load(v)
        if axis < 0:
            axis += len(v.shape) + 1
        shape = list(v.shape)
        shape.insert(axis, 1)
        if isinstance(v, Affine):
            coefs = {(a + (a >= axis)): c for a, c in v.coefs.items()}
            return Affine(v.dtype, shape, v.base, coefs)
        if isinstance(v, Fill):
            return Fill(v.dtype, shape, v.value)
        if isinstance(v, Lazy):
            args = [self.expand_dims(a, axis) if isinstance(a, Block) and len(a.shape) == len(v.shape)
                    else self._expand_lower(a, axis, len(v.shape)) for a in v.args]
            out = Lazy(v.dtype, shape, v.fn, args, v.size)
            out.meta = getattr(v, "meta", None) and self._meta_expand(v.meta, axis)
            return out
        if isinstance(v, PtrBlock):
            return PtrBlock(v.base, self.expand_dims(v.offset, axis))
        if isinstance(v, Reg):
            return Reg(v.dtype, shape, v.layout.expand_dims(axis), v.var, v.vec)
        raise CompileError(f"cannot expand {v}")

    def _expand_lower(self, a, axis, rank):
        if not isinstance(a, Block):
            return a
        a = self.expand_to_rank(a, rank)
        return self.expand_dims(a, axis)

    def _meta_expand(self, meta, axis):
        kind = meta[0]
        if kind == "cmp":
            return ("cmp", meta[1], self.expand_dims(meta[2], axis))
        if kind == "and":
            return ("and", [self._meta_expand(m, axis) for m in meta[1]])
        return None

    def permute(self, v, perm):
        if isinstance(v, (Const, Scalar)):
            return v
        if isinstance(v, Staged):
            return Staged(v.rec, v.slot, not v.trans)
        if isinstance(v, LazyLoad):
            ptr = self.permute(v.ptr, perm)
            mask = self.permute(v.mask, perm) if isinstance(v.mask, Block) else v.mask
            other = self.permute(v.other, perm) if isinstance(v.other, Block) else v.other
            out = LazyLoad(ptr, mask, other, v.node)
            out.src = v
            self.pending_loads.append(out)
            v.transposed_alias = out
            return out
        shape = [v.shape[p] for p in perm]
        inv = {old: new for new, old in enumerate(perm)}
        if isinstance(v, Affine):
            return Affine(v.dtype, shape, v.base, {inv[a]: c for a, c in v.coefs.items()})
        if isinstance(v, Fill):
            return Fill(v.dtype, shape, v.value)
        if isinstance(v, Lazy):
            args = [self.permute(self.expand_to_rank(a, len(perm)), perm) if isinstance(a, Block) else a
                    for a in v.args]
            out = Lazy(v.dtype, shape, v.fn, args, v.size)
            out.meta = None
            return out
        if isinstance(v, PtrBlock):
            return PtrBlock(v.base, self.permute(v.offset, perm))
        if isinstance(v, Reg):
            return Reg(v.dtype, shape, v.layout.permute(perm), v.var, v.vec)
        raise CompileError(f"cannot permute {v}")

    def reshape(self, node, v, shape):
        if isinstance(v, LazyLoad):
            v = self.materialize_load(v)
        if isinstance(v, Fill):
            return Fill(v.dtype, shape, v.value)
        if isinstance(v, PtrBlock):
            return PtrBlock(v.base, self.reshape(node, v.offset, shape))
        if isinstance(v, (Affine, Lazy)):
            v = self.to_reg(v)
        if isinstance(v, Reg):
            return Reg(v.dtype, shape, v.layout.reshape(shape), v.var, v.vec)
        self.err(node, "cannot reshape this value")

    # ------------------------------------------------------------- evaluation
    def lazy_size(self, v):
        if isinstance(v, Lazy):
            return v.size
        return 1

    def ev(self, v, L, s):
        """C expression of value v at slot s of layout L (v's shape broadcasts
        to L.shape, same rank). Reg leaves must already be slot-compatible."""
        if isinstance(v, Const):
            return self.literal(v.pyval, self.cdtype(v))
        if isinstance(v, Scalar):
            return v.expr
        if isinstance(v, Fill):
            return self.scalar_expr(v.value, v.dtype)
        if isinstance(v, Affine):
            terms = [] if (v.base.is_const and v.base.const == 0) else [v.base.expr]
            for a, c in sorted(v.coefs.items()):
                if v.shape[a] == 1:
                    continue
                cd = self.coord(L, a, s)
                if cd == "0":
                    continue
                if c.is_const and c.const == 1:
                    terms.append(cd)
                else:
                    terms.append(f"{c.expr} * {cd}")
            if not terms:
                return "0"
            e = " + ".join(terms)
            if v.dtype == tp.int64:
                return f"((long long)({e}))" if len(terms) > 1 else f"((long long){e})"
            return f"({e})"
        if isinstance(v, Lazy):
            return v.fn([self.ev(a, L, s) for a in v.args])
        if isinstance(v, Reg):
            if v.layout == L:
                return v.at(s)
            f = lo.slot_map(v.layout, L)
            if f is None:
                raise CompileError("internal: incompatible layout in ev")
            return v.at(f(s))
        if isinstance(v, LazyLoad):
            r = self.materialize_load(v, L)
            return self.ev(r, L, s)
        raise CompileError(f"internal: cannot evaluate {v}")

    def prepare(self, v, L):
        """Make every Reg inside v evaluable in layout L (converting through
        LDS when the layouts are incompatible)."""
        if isinstance(v, Reg):
            if v.layout == L or lo.slot_map(v.layout, L) is not None:
                return v
            return self.convert(v, L)
        if isinstance(v, LazyLoad):
            return self.materialize_load(v, L if v.shape == L.shape else None)
        if isinstance(v, Lazy):
            args = [self.prepare(a, L) if isinstance(a, Block) else a for a in v.args]
            if all(a is b for a, b in zip(args, v.args)):
                return v
            out = Lazy(v.dtype, v.shape, v.fn, args, v.size)
            out.meta = getattr(v, "meta", None)
            return out
        return v

    def new_reg(self, dtype, shape, L, vec=0):
        var = self.fresh("r")
        n = L.nslots
        if vec:
            vt = {16: "f32x16", 4: "f32x4"}[vec]
            self.emit(f"{vt} {var}[{n // vec}];")
        else:
            self.emit(f"{dtype.ctype} {var}[{n}];")
        return Reg(dtype, shape, L, var, vec)

    def to_reg(self, v, L=None, dtype=None):
        """Materialize a block value into registers (layout L or default)."""
        if isinstance(v, Reg) and (L is None or v.layout == L):
            return v if dtype is None or dtype == v.dtype else self.cast_block(v, dtype)
        if isinstance(v, LazyLoad):
            r = self.materialize_load(v, L)
            return self.to_reg(r, L, dtype)
        if isinstance(v, PtrBlock):
            raise CompileError("pointer blocks cannot be materialized as values")
        if L is None:
            L = self.default_layout(v.shape)
        if isinstance(v, Reg):
            f = lo.slot_map(v.layout, L)
            if f is None:
                return self.to_reg(self.convert(v, L), L, dtype)
        v = self.prepare(v, L)
        dt = dtype or v.dtype
        out = self.new_reg(dt, L.shape, L)
        for s in range(L.nslots):
            self.emit(f"{out.at(s)} = {self.conv(self.ev(v, L, s), v.dtype, dt)};")
        return out

    def convert(self, r, L):
        """Move a Reg into layout L (shape of r broadcastable to L.shape)."""
        if r.layout == L:
            return r
        f = lo.slot_map(r.layout, L)
        if f is not None:
            out = self.new_reg(r.dtype, L.shape, L)
            for s in range(L.nslots):
                self.emit(f"{out.at(s)} = {r.at(f(s))};")
            return out
        origin = getattr(r, "origin", None)
        hinted = False
        if origin is not None and origin not in self.hints and r.shape == L.shape:
            self.new_hints[origin] = L
            hinted = True
        # LDS round trip: write source elements at their row-major index
        Ls = r.layout
        esz = 4 if r.dtype == tp.int1 else max(r.dtype.itemsize, 1)
        ct = "int" if r.dtype == tp.int1 else r.dtype.ctype
        nbytes = r.numel * esz
        if nbytes > MAX_LDS:
            if hinted:
                raise _Retry()
            raise CompileError(f"layout conversion of {r.shape} needs {nbytes} bytes of LDS")
        area = self.lds_arena(nbytes)
        buf = self.fresh("cv")
        self.barrier()
        self.emit(f"{ct}* {buf} = ({ct}*)(_lds + {area});")
        strides = self._strides(r.shape)
        canon = self.canon_cond(Ls)
        if canon:
            self.emit(f"if ({canon}) {{")
            self.indent += 1
        for s in range(Ls.nslots):
            if not Ls.slot_is_canonical(s):
                continue
            idx = self._flat_index(Ls, s, strides)
            self.emit(f"{buf}[{idx}] = ({ct}){r.at(s)};")
        if canon:
            self.indent -= 1
            self.emit("}")
        self.barrier()
        out = self.new_reg(r.dtype, L.shape, L)
        for s in range(L.nslots):
            idx = self._flat_index(L, s, strides, src_shape=r.shape)
            self.emit(f"{out.at(s)} = ({r.dtype.ctype}){buf}[{idx}];")
        return out

    @staticmethod
    def _strides(shape):
        st = [1] * len(shape)
        for d in range(len(shape) - 2, -1, -1):
            st[d] = st[d + 1] * shape[d + 1]
        return st

    def _flat_index(self, L, s, strides, src_shape=None):
        terms = []
        for d in range(len(L.shape)):
            if src_shape is not None and src_shape[d] == 1:
                continue
            c = self.coord(L, d, s)
            if c == "0":
                continue
            terms.append(c if strides[d] == 1 else f"{c} * {strides[d]}")
        return " + ".join(terms) if terms else "0"

    # --------------------------------------------------------- elementwise core
    def pick_layout(self, operands, shape):
        """Layout for an elementwise result: a register operand's layout if one
        has the full result shape (preferring layouts that come from an MFMA
        accumulator, so row statistics and accumulators stay where the matrix
        cores put them and loop-carried state learns that layout), else one
        broadcastable into it, else default."""
        full = [o for o in operands if isinstance(o, Reg) and o.shape == tuple(shape)]
        for o in full:
            if o.layout.tag.startswith("mfma") and not o.layout.tag.startswith("mfmaop"):
                return o.layout
        if full:
            return full[0].layout
        for o in operands:
            if isinstance(o, Reg):
                L = o.layout.broadcast_into(tuple(shape))
                if L is not None and L.nslots <= max(self.default_layout(shape).nslots, 1):
                    return L
        return self.default_layout(shape)

    def elementwise(self, node, operands, rdtype, fn, meta=None, fast=None):
        """Apply fn (list of C exprs -> C expr) elementwise over broadcast operands.
        fast=(uniform C condition, fn2): when the result lands in registers,
        fn2 replaces fn under the condition (a scalar branch per block)."""
        shape = ()
        for o in operands:
            if isinstance(o, Block):
                shape = tp.broadcast_shapes(shape, o.shape)
        if shape == ():
            exprs = [self.scalar_expr(o) for o in operands]
            return self.new_scalar(rdtype, fn(exprs))
        ops = [self.expand_to_rank(o, len(shape)) if isinstance(o, Block) else o for o in operands]
        # a load an earlier statement already brought into registers takes
        # part as those registers, so its layout can be the result's; left as
        # a load, a broadcast operand (a row statistic) would choose the
        # layout and the whole loaded block would go through LDS to meet it
        ops = [o.result if isinstance(o, LazyLoad) and o.result is not None else o for o in ops]
        regs = [o for o in ops if isinstance(o, (Reg, LazyLoad))]
        if not regs:
            size = 1 + sum(self.lazy_size(o) for o in ops)
            if size <= LAZY_LIMIT:
                out = Lazy(rdtype, shape, fn, ops, size)
                out.meta = meta
                return out
        L = self.pick_layout(ops, shape)
        if any(isinstance(o, LazyLoad) for o in ops):
            ops = [self.materialize_load(o, L if o.shape == L.shape else None)
                   if isinstance(o, LazyLoad) else o for o in ops]
            L = self.pick_layout(ops, shape)
        ops = [self.prepare(o, L) if isinstance(o, Block) else o for o in ops]
        out = self.new_reg(rdtype, shape, L)
        if fast is not None:
            self.emit(f"if ({fast[0]}) {{")
            self.indent += 1
            for s in range(L.nslots):
                self.emit(f"{out.at(s)} = {fast[1]([self.ev(o, L, s) for o in ops])};")
            self.indent -= 1
            self.emit("} else {")
            self.indent += 1
        for s in range(L.nslots):
            exprs = [self.ev(o, L, s) for o in ops]
            self.emit(f"{out.at(s)} = {fn(exprs)};")
        if fast is not None:
            self.indent -= 1
            self.emit("}")
        return out

    def cast_block(self, v, dt):
        src = v.dtype
        return self.elementwise(None, [v], dt, lambda es: self.conv(es[0], src, dt))

    # ----------------------------------------------------------------- compile
    def compile(self):
        self.visit_body(self.fndef.body)
        self.flush_loads()
        return self.assemble()

    def assemble(self):
        lds_total = self.lds_dedicated
        arena_off = (lds_total + 15) // 16 * 16
        lds_total = arena_off + self.arena_bytes
        lds_all = lds_total + sum(b for _, b in self.lds_arrays)
        if lds_all > MAX_LDS:
            # layouts learned in this pass remove conversions (and their LDS)
            # in the next one: try that before a pipeline gives anything up
            if any(self.hints.get(k) != v for k, v in self.new_hints.items()
                   if isinstance(v, lo.Layout)):
                raise _Retry()
            # a dot pipeline that does not fit gives up a stage (down to 2), then
            # falls back to synchronous staging, before the kernel is rejected
            for rec in self.pipe_records:
                key = rec["node"].lineno
                if rec["S"] > 2:
                    self.new_hints[("pipe_stages", key)] = rec["S"] - 1
                    raise _Retry()
                if not self.hints.get(("nopipe", key)):
                    self.new_hints[("nopipe", key)] = True
                    raise _Retry()
            raise CompileError(f"kernel needs {lds_all} bytes of LDS (max {MAX_LDS}); "
                               f"use smaller block sizes")
        sig = []
        for name, p in self.params:
            if isinstance(p.dtype, tp.pointer_type):
                sig.append(f"{p.dtype.element.ctype}* __restrict__ {p.cname}")
            else:
                sig.append(f"{p.dtype.ctype} {p.cname}")
        out = ['#include "newt_gfx950.h"', ""]
        for nm, off in self.lds_regions:
            out.append(f"#define {nm} {off}")
        out.append(f"#define _LDSA {arena_off}")
        out.append("")
        # waves_per_eu > 0 asks for that many waves per SIMD: the register
        # allocator then keeps each wave within 512 / waves_per_eu registers
        occ = (f"__attribute__((amdgpu_waves_per_eu({self.waves_per_eu}))) "
               if self.waves_per_eu else "")
        out.append(f'extern "C" __global__ void __launch_bounds__({self.T}) {occ}'
                   f'{self.name}({", ".join(sig)}) {{')
        if lds_total:
            out.append(f"  __shared__ __attribute__((aligned(16))) unsigned char _lds[{lds_total}];")
        for nm, nb in self.lds_arrays:
            out.append(f"  __shared__ __attribute__((aligned(16))) unsigned char {nm}[{nb}];")
        body = ["  const int _tid = (int)threadIdx.x;",
                "  const int _lane = _tid & 63;",
                "  const int _wave = __builtin_amdgcn_readfirstlane(_tid >> 6);",
                "  (void)_lane; (void)_wave;"]
        body += ["  " + p for p in self.prologue]
        out += self.version_body(body + self.lines)
        out.append("}")
        self.lds_total = lds_all
        return "\n".join(out) + "\n"

    _CIDENT = re.compile(r"[A-Za-z_]\w*")
    _BRANCH = re.compile(r"^\s*if \((.*)\) \{$")
    # hipRTC's time grows faster than the body: a 4,700-line body took 4.7 s,
    # its two copies 29.5 s
    VERSION_MAX_LINES = 1200

    def version_body(self, lines):
        """Version a small, loop-free kernel body once on its uniform "tile in
        bounds" test. Masked loads, stores and `where`s each branch on such a
        test; when one test over scalar kernel arguments only guards two or
        more of them, the whole body is emitted twice: `if (test) { body, test
        folded to true } else { body }`. The first copy is straight-line code
        the scheduler can order freely; the second is the body as generated.
        Both compute the same values, so results are identical. The lane
        index arithmetic of the prologue goes into both copies too (measured
        1.5% faster than computing it once before the test). On layernorm
        4096x8192: 20.9 against 23.1 us back to back, 28.1 against 29.0 us
        flushed. Tests over per-program values (vector add's) are left
        alone: versioning the body after the values they read measured 1.3%
        slower. So are bodies with loops (the dot pipeline versions its own
        loops) and bodies over VERSION_MAX_LINES. NEWT_VERSION_BODY=0 turns it
        off."""
        if os.environ.get("NEWT_VERSION_BODY", "1") == "0" or len(lines) > self.VERSION_MAX_LINES:
            return lines
        text = "\n".join(lines)
        if re.search(r"\b(for|while|do|goto)\b", text):
            return lines
        params = {p.cname for _, p in self.params}
        counts = {}
        for ln in lines:
            m = self._BRANCH.match(ln)
            if m:
                counts[m.group(1)] = counts.get(m.group(1), 0) + 1
        for cond, n in sorted(counts.items(), key=lambda kv: -kv[1]):
            if n < 2:
                break
            names = set(self._CIDENT.findall(cond)) - {"true", "false"}
            if not names or not names <= params:
                continue
            # an argument the body assigns would not keep the test's value
            if any(re.search(rf"\b{nm}\s*([-+*/%&|^]|<<|>>)?=(?!=)", text)
                   or re.search(rf"(\+\+|--)\s*{nm}\b|\b{nm}\s*(\+\+|--)", text)
                   for nm in names):
                continue
            # only whole `if (test) {` lines are rewritten: the test's text may
            # also occur inside a longer expression that means something else
            branch = f"if ({cond}) {{"
            fast = ["  " + (ln.replace(branch, "if ((true)) {") if self._BRANCH.match(ln) else ln)
                    for ln in lines]
            slow = ["  " + ln for ln in lines]
            return [f"  if ({cond}) {{"] + fast + ["  } else {"] + slow + ["  }"]
        return lines

    # -------------------------------------------------------------- statements
    def visit_Expr(self, node):
        if isinstance(node.value, ast.Constant):
            return
        self.visit_expr(node.value)

    def visit_Assign(self, node):
        if len(node.targets) != 1:
            self.err(node, "chained assignment not supported")
        tgt = node.targets[0]
        if isinstance(tgt, ast.Tuple):
            if not (isinstance(node.value, ast.Tuple) and len(node.value.elts) == len(tgt.elts)
                    and all(isinstance(t, ast.Name) for t in tgt.elts)):
                self.err(node, "tuple unpacking only supports `a, b = expr1, expr2`")
            vals = [self.visit_expr(v) for v in node.value.elts]
            for t, v in zip(tgt.elts, vals):
                self.bind(node, t.id, v)
            return
        if not isinstance(tgt, ast.Name):
            self.err(node, "can only assign to plain names")
        v = self.visit_expr(node.value)
        if getattr(node, "_newt_prefetch", False) and isinstance(v, LazyLoad) and not self.loop_depth:
            # a load moved ahead of independent work: issue it here, after the
            # loads that precede it in the program
            self.flush_loads()
            self.materialize_load(v)
        self.bind(node, tgt.id, v)

    def visit_AnnAssign(self, node):
        if node.value is None:
            return
        self.bind(node, node.target.id, self.visit_expr(node.value))

    def visit_AugAssign(self, node):
        cur = self.lookup(node, node.target.id)
        rhs = self.visit_expr(node.value)
        self.bind(node, node.target.id, self.binop(node, type(node.op), cur, rhs))

    def visit_Pass(self, node):
        pass

    def visit_Assert(self, node):
        pass  # host asserts are ignored on device (reference codegen.py:1104-1105)

    def visit_Return(self, node):
        if node.value is not None:
            self.err(node, "kernels cannot return values")
        self.flush_loads()
        self.drain_dots()
        self.emit("return;")

    def visit_Break(self, node):
        self.flush_loads()
        self.emit("break;")

    def visit_Continue(self, node):
        self.flush_loads()
        self.emit("continue;")

    def generic_visit(self, node):
        if isinstance(node, ast.stmt):
            self.err(node, f"unsupported statement: {type(node).__name__}")
        super().generic_visit(node)

    def visit_body(self, stmts):
        for i, st in enumerate(stmts):
            self.body_stack.append((stmts, i))
            try:
                self.visit(st)
            finally:
                self.body_stack.pop()

    def _read_after(self):
        """Names whose current values may be read after the current statement,
        in any enclosing body (reads preceded by a reassignment that certainly
        runs first do not count)."""
        out = set()
        for stmts, i in self.body_stack:
            out |= _Prepass.exposed(stmts[i + 1:])
        return out

    def _enter_compound(self, node):
        """Create storage for names that the statement reassigns (loop-carried)
        and register placeholders for names it defines and that are read later.
        A for loop's target is not loop-carried: the loop header rebinds it on
        every trip (an earlier binding of the name, e.g. the target of a
        previous loop, is not its initial value)."""
        assigned = _Prepass.assigned(node)
        if isinstance(node, ast.For) and isinstance(node.target, ast.Name):
            assigned = assigned - {node.target.id}
        for name in sorted(assigned):
            if name in self.locals:
                v = self.locals[name]
                if isinstance(v, Const) and name not in self.storages and self._is_param_const(name):
                    continue
                if name not in self.storages:
                    if isinstance(v, Const) and not isinstance(v.pyval, (int, float, bool)):
                        continue
                    self.make_storage(node, name, v)
        after = self._read_after()
        hoist = {n for n in assigned if n not in self.locals and n in after}
        if isinstance(node, ast.For) and isinstance(node.target, ast.Name):
            hoist.discard(node.target.id)
        rec = {"names": hoist, "index": len(self.lines), "indent": self.indent, "node": node,
               "pre": set(self.locals) | set(self.storages)}
        self.pending_hoist.append(rec)
        return rec

    def _is_param_const(self, name):
        return False

    def _exit_compound(self, rec):
        """Names first defined inside the statement and not read after it are
        scoped to its C block: drop their bindings, so a later statement that
        assigns the same name starts fresh instead of carrying a stale value."""
        self.pending_hoist.remove(rec)
        for name in _Prepass.assigned(rec["node"]) - rec["pre"] - rec["names"]:
            # a storage such a name got inside the statement (a loop nested in
            # it carried the name) is declared in the same C block, so it goes
            # out of scope with it as well
            self.storages.pop(name, None)
            self.locals.pop(name, None)

    def visit_For(self, node):
        self.flush_loads()
        if node.orelse:
            self.err(node, "for/else not supported")
        if not (isinstance(node.iter, ast.Call) and self._callee(node.iter.func) == "range"):
            self.err(node, "only `for i in range(...)` loops are supported")
        if not isinstance(node.target, ast.Name):
            self.err(node, "loop target must be a name")
        args = [self.visit_expr(a) for a in node.iter.args]
        if len(args) == 1:
            lo_, hi, st = Const(0), args[0], Const(1)
        elif len(args) == 2:
            lo_, hi, st = args[0], args[1], Const(1)
        elif len(args) == 3:
            lo_, hi, st = args
        else:
            self.err(node, "range() takes 1-3 arguments")
        for a in (lo_, hi, st):
            if not isinstance(a, (Const, Scalar)):
                self.err(node, "range bounds must be scalars")
        idt = tp.int64 if any(self.cdtype(a) == tp.int64 for a in (lo_, hi, st)) else tp.int32
        if isinstance(st, Const) and isinstance(st.pyval, int) and st.pyval > 0:
            plan = self.pipeline_plan(node)
            if plan is not None:
                return self.pipelined_for(node, plan, lo_, hi, st, idt)
        rec = self._enter_compound(node)
        self.drain_dots_for_loop(node)
        ivar = self.fresh("i")
        all_const = all(isinstance(a, Const) for a in (lo_, hi, st))
        neg = isinstance(st, Const) and st.pyval < 0
        if all_const and len(range(lo_.pyval, hi.pyval, st.pyval)) <= 64:
            self.emit("#pragma unroll")
        cmp = ">" if neg else "<"
        self.emit(f"for ({idt.ctype} {ivar} = {self.scalar_expr(lo_, idt)}; "
                  f"{ivar} {cmp} {self.scalar_expr(hi, idt)}; {ivar} += {self.scalar_expr(st, idt)}) {{")
        self.indent += 1
        self.loop_depth += 1
        div = 1
        if isinstance(lo_, Const) and isinstance(st, Const):
            div = min(lo.log2i(1) if False else _gcd_pow2(lo_.pyval, st.pyval), 1 << 30)
        self.locals[node.target.id] = Scalar(idt, ivar, Sym(ivar, None, div))
        self.visit_body(node.body)
        self.flush_loads()
        self.loop_backedge(node)
        self.loop_depth -= 1
        self.indent -= 1
        self.emit("}")
        self._exit_compound(rec)
        self.end_loop_target(node)
        self.after_loop(node)

    def end_loop_target(self, node):
        """The loop counter is scoped to the C loop; after the loop the target
        name is unbound (reading it is an undefined-name error)."""
        self.locals.pop(node.target.id, None)

    def visit_While(self, node):
        self.flush_loads()
        if node.orelse:
            self.err(node, "while/else not supported")
        # a constexpr-false condition drops the loop (reference codegen.py:1054-1058)
        start = len(self.lines)
        save_tmp = self.tmpc
        rec = self._enter_compound(node)
        self.emit("while (true) {")
        self.indent += 1
        self.loop_depth += 1
        cond = self.visit_expr(node.test)
        if isinstance(cond, Const):
            if not cond.pyval:
                del self.lines[start:]
                self.indent -= 1
                self.loop_depth -= 1
                self._exit_compound(rec)
                self.tmpc = save_tmp
                return
        elif not isinstance(cond, Scalar):
            self.err(node, "while condition must be a scalar")
        else:
            self.emit(f"if (!({cond.expr})) break;")
        self.visit_body(node.body)
        self.flush_loads()
        self.loop_backedge(node)
        self.loop_depth -= 1
        self.indent -= 1
        self.emit("}")
        self._exit_compound(rec)
        self.after_loop(node)

    def visit_If(self, node):
        self.flush_loads()
        cond = self.visit_expr(node.test)
        if isinstance(cond, Const):
            # constexpr condition prunes the dead branch (reference codegen.py:1070-1074)
            self.visit_body(node.body if cond.pyval else node.orelse)
            return
        if not isinstance(cond, Scalar):
            self.err(node, "if condition must be a scalar (use nl.where for blocks)")
        rec = self._enter_compound(node)
        self.drain_dots()
        self.emit(f"if ({cond.expr}) {{")
        self.indent += 1
        self.visit_body(node.body)
        self.flush_loads()
        self.drain_dots()
        self.indent -= 1
        if node.orelse:
            self.emit("} else {")
            self.indent += 1
            self.visit_body(node.orelse)
            self.flush_loads()
            self.drain_dots()
            self.indent -= 1
        self.emit("}")
        self._exit_compound(rec)

    # ------------------------------------------------------------- name binding
    def lookup(self, node, name):
        if name in self.storages:
            return self.read_storage(self.storages[name])
        if name in self.locals:
            return self.locals[name]
        if name in self.globals:
            return Const(self.globals[name])
        if hasattr(builtins, name):
            return Const(getattr(builtins, name))
        self.err(node, f"undefined name '{name}'")

    def make_storage(self, node, name, v, decl_at=None, hint_node=None):
        """Create persistent storage for `name` initialised from v."""
        key = ((hint_node or node).lineno, (hint_node or node).col_offset, name)
        cvar = f"v_{name}_{self.fresh('')[1:]}"
        hint = self.hints.get(key)
        emit_decl = self.emit if decl_at is None else (lambda s: self._insert_decl(decl_at, s))
        if isinstance(v, LazyLoad):
            v = self.materialize_load(v, hint if isinstance(hint, lo.Layout) and hint.shape == v.shape else None)
        if isinstance(v, (Const, Scalar)):
            dt = self.cdtype(v)
            if isinstance(dt, tp.pointer_type):
                emit_decl(f"{dt.element.ctype}* {cvar};")
            else:
                emit_decl(f"{dt.ctype} {cvar};")
            st = Storage(name, "scalar", cvar, dt, (), key=key)
            st.aligned16 = getattr(v, "aligned16", False)
        elif isinstance(v, Affine) and hint != "reg":
            emit_decl(f"{v.dtype.ctype} {cvar};")
            st = Storage(name, "affine", cvar, v.dtype, v.shape, coefs=dict(v.coefs), key=key)
        elif isinstance(v, PtrBlock) and isinstance(v.offset, Affine) and hint != "reg":
            off = v.offset
            emit_decl(f"{off.dtype.ctype} {cvar};")
            st = Storage(name, "ptraffine", cvar, off.dtype, off.shape, base=v.base,
                         coefs=dict(off.coefs), key=key)
            st.base_div = off.base.div
        elif isinstance(v, PtrBlock):
            offdt = v.offset.dtype
            L = hint if isinstance(hint, lo.Layout) and hint.shape == v.shape else (
                v.offset.layout if isinstance(v.offset, Reg) else self.default_layout(v.shape))
            emit_decl(f"{offdt.ctype} {cvar}[{L.nslots}];")
            st = Storage(name, "ptrreg", cvar, offdt, v.shape, layout=L, base=v.base, key=key)
        elif isinstance(v, Block):
            if isinstance(hint, lo.Layout) and hint.shape == v.shape:
                L = hint
            elif isinstance(v, Reg):
                L = v.layout
            else:
                L = self.default_layout(v.shape)
            vec = 0
            mi = lo.mfma_tag_instr(L.tag)
            if mi is not None and v.dtype == tp.float32:
                vec = lo.INSTR[mi[0]][4]
            if vec:
                vt = {16: "f32x16", 4: "f32x4"}[vec]
                emit_decl(f"{vt} {cvar}[{L.nslots // vec}];")
            else:
                emit_decl(f"{v.dtype.ctype} {cvar}[{L.nslots}];")
            st = Storage(name, "reg", cvar, v.dtype, v.shape, layout=L, key=key, vec=vec)
        else:
            self.err(node, f"cannot keep {type(v).__name__} in loop-carried storage")
        self.storages[name] = st
        self.locals[name] = st
        self.write_storage(node, st, v)
        return st

    def _insert_decl(self, rec, line):
        self.lines.insert(rec["index"], "  " * rec["indent"] + line)
        # later hoist records that point after this index shift by one
        for r in self.pending_hoist:
            if r is not rec and r["index"] >= rec["index"]:
                r["index"] += 1
        rec["index"] += 1

    def read_storage(self, st):
        if st.kind == "scalar":
            t = self.fresh()
            if isinstance(st.dtype, tp.pointer_type):
                self.emit(f"{st.dtype.element.ctype}* const {t} = {st.cvar};")
                return Scalar(st.dtype, t, aligned16=getattr(st, "aligned16", False))
            self.emit(f"const {st.dtype.ctype} {t} = {st.cvar};")
            sym = Sym(t, None, 1) if st.dtype.is_int and st.dtype != tp.int1 else None
            return Scalar(st.dtype, t, sym)
        if st.kind == "affine":
            t = self.fresh()
            self.emit(f"const {st.dtype.ctype} {t} = {st.cvar};")
            return Affine(st.dtype, st.shape, Sym(t, None, 1), st.coefs)
        if st.kind == "ptraffine":
            t = self.fresh()
            self.emit(f"const {st.dtype.ctype} {t} = {st.cvar};")
            return PtrBlock(st.base, Affine(st.dtype, st.shape, Sym(t, None, st.base_div), st.coefs))
        if st.kind == "ptrreg":
            return PtrBlock(st.base, Reg(st.dtype, st.shape, st.layout, st.cvar))
        self.flush_dot(st)
        r = Reg(st.dtype, st.shape, st.layout, st.cvar, st.vec, storage=True)
        r.origin = st.key
        return r

    def write_storage(self, node, st, v):
        if st.kind == "scalar":
            if isinstance(v, Block):
                self.err(node, f"loop-carried variable '{st.name}' changed from scalar to block")
            vd = self.cdtype(v)
            if isinstance(st.dtype, tp.dtype) and st.dtype.is_int and isinstance(vd, tp.dtype) and vd.is_floating:
                self.err(node, f"loop-carried scalar '{st.name}' was created as {st.dtype} but "
                               f"updated with {vd}; initialize it as a float (e.g. `s = 0.0`)")
            if isinstance(st.dtype, tp.pointer_type) and st.dtype != vd:
                self.err(node, f"loop-carried pointer '{st.name}' changed type")
            self.emit(f"{st.cvar} = {self.scalar_expr(v, st.dtype) if not isinstance(st.dtype, tp.pointer_type) else v.expr};")
            if isinstance(st.dtype, tp.pointer_type):
                st.aligned16 = getattr(st, "aligned16", False) and getattr(v, "aligned16", False)
            return
        if st.kind == "affine":
            if isinstance(v, (Const, Scalar)) and st.shape == ():
                self.err(node, "internal: scalar in affine storage")
            if not (isinstance(v, Affine) and self._same_coefs(v.coefs, st.coefs)
                    and tuple(v.shape) == st.shape):
                self.new_hints[st.key] = "reg"
                self.err_retry(node)
            self.emit(f"{st.cvar} = {self.conv(v.base.expr, None, None)};")
            return
        if st.kind == "ptraffine":
            if not isinstance(v, PtrBlock):
                self.err(node, f"loop-carried pointer block '{st.name}' assigned a non-pointer")
            if v.base.expr != st.base.expr:
                self.err(node, "a loop-carried pointer block cannot switch its base tensor; "
                               "use separate pointer variables")
            if not (isinstance(v.offset, Affine) and self._same_coefs(v.offset.coefs, st.coefs)
                    and tuple(v.shape) == st.shape):
                self.new_hints[st.key] = "reg"
                self.err_retry(node)
            st.base_div = min(getattr(st, "base_div", 1), v.offset.base.div)
            self.emit(f"{st.cvar} = {v.offset.base.expr};")
            return
        if st.kind == "ptrreg":
            if not isinstance(v, PtrBlock):
                self.err(node, f"loop-carried pointer block '{st.name}' assigned a non-pointer")
            if v.base.expr != st.base.expr:
                self.err(node, "a loop-carried pointer block cannot switch its base tensor; "
                               "use separate pointer variables")
            off = self.expand_to_rank(v.offset, len(st.shape))
            off = self.prepare(off, st.layout)
            vals = [self.ev(off, st.layout, s) for s in range(st.layout.nslots)]
            for s, e in enumerate(vals):
                self.emit(f"{st.cvar}[{s}] = {e};")
            return
        # reg storage
        if isinstance(v, (Const, Scalar)):
            v = Fill(self.cdtype(v), st.shape, v)
        if not isinstance(v, Block) or isinstance(v, PtrBlock):
            self.err(node, f"loop-carried variable '{st.name}' changed kind")
        if tuple(v.shape) != st.shape:
            if v.numel == math.prod(st.shape) and isinstance(v, Reg):
                v = Reg(v.dtype, st.shape, v.layout.reshape(st.shape), v.var, v.vec)
            else:
                try:
                    tp.broadcast_shapes(v.shape, st.shape)
                except TypeError:
                    self.err(node, f"loop-carried variable '{st.name}' changed shape "
                                   f"{st.shape} -> {v.shape}")
        if isinstance(v, Reg) and v.var == st.cvar:
            return
        if isinstance(v, LazyLoad):
            v = self.materialize_load(v, st.layout if v.shape == st.shape else None)
        if isinstance(v, Reg) and v.layout != st.layout and v.shape == st.shape:
            if st.key not in self.hints or self.hints.get(st.key) != v.layout:
                self.new_hints[st.key] = v.layout
        v = self.expand_to_rank(v, len(st.shape))
        v = self.prepare(v, st.layout)
        tmp = []
        for s in range(st.layout.nslots):
            tmp.append(self.conv(self.ev(v, st.layout, s), v.dtype, st.dtype))
        target = Reg(st.dtype, st.shape, st.layout, st.cvar, st.vec)
        for s, e in enumerate(tmp):
            self.emit(f"{target.at(s)} = {e};")

    def err_retry(self, node):
        raise _Retry()

    @staticmethod
    def _same_coefs(a, b):
        if set(a) != set(b):
            return False
        return all(a[k].expr == b[k].expr for k in a)

    def bind(self, node, name, v):
        if isinstance(v, Const) and v.pyval is None:
            self.locals[name] = v
            return
        if name in self.storages:
            st = self.storages[name]
            self.flush_loads()
            self.flush_dot(st)
            self.write_storage(node, st, v)
            return
        for rec in reversed(self.pending_hoist):
            if name in rec["names"]:
                self.flush_loads()
                self.make_storage(node, name, v, decl_at=rec, hint_node=rec["node"])
                return
        # aliasing loop-carried register storage must snapshot it
        if isinstance(v, Reg) and v.storage:
            v = self.copy_reg(v)
        self.locals[name] = v

    def copy_reg(self, r):
        out = self.new_reg(r.dtype, r.shape, r.layout, r.vec)
        if r.vec:
            for i in range(r.layout.nslots // r.vec):
                self.emit(f"{out.var}[{i}] = {r.var}[{i}];")
        else:
            for s in range(r.layout.nslots):
                self.emit(f"{out.at(s)} = {r.at(s)};")
        return out

    # hooks for the dot pipeline (dot.py overrides)
    def drain_dots(self):
        pass

    def drain_dots_for_loop(self, node):
        pass

    def loop_backedge(self, node):
        pass

    def after_loop(self, node):
        pass

    def flush_dot(self, st):
        pass

    # -------------------------------------------------------------- expressions
    def visit_expr(self, node):
        m = getattr(self, f"expr_{type(node).__name__}", None)
        if m is None:
            self.err(node, f"unsupported expression: {type(node).__name__}")
        return m(node)

    def expr_Name(self, node):
        return self.lookup(node, node.id)

    def expr_Constant(self, node):
        return Const(node.value)

    def expr_Tuple(self, node):
        vals = [self.visit_expr(e) for e in node.elts]
        if all(isinstance(v, Const) for v in vals):
            return Const(tuple(v.pyval for v in vals))
        self.err(node, "tuples of runtime values are not supported")

    expr_List = expr_Tuple

    def expr_Attribute(self, node):
        base = self.visit_expr(node.value)
        if isinstance(base, Const):
            try:
                return Const(getattr(base.pyval, node.attr))
            except AttributeError:
                self.err(node, f"no attribute {node.attr!r}")
        if node.attr == "shape":
            return Const(tuple(getattr(base, "shape", ())))
        if node.attr == "dtype":
            return Const(base.dtype)
        if node.attr == "T" and isinstance(base, Block):
            return self.op_trans(node, base)
        self.err(node, f"unsupported attribute access .{node.attr}")

    def expr_UnaryOp(self, node):
        v = self.visit_expr(node.operand)
        if isinstance(v, Const):
            import operator
            ops = {ast.USub: operator.neg, ast.UAdd: operator.pos, ast.Invert: operator.invert,
                   ast.Not: operator.not_}
            return Const(ops[type(node.op)](v.pyval))
        d = self.cdtype(v)
        if isinstance(node.op, ast.USub):
            if isinstance(v, Affine):
                return Affine(v.dtype, v.shape, s_neg(v.base), {a: s_neg(c) for a, c in v.coefs.items()})
            if tp.is_half(d):
                return self.elementwise(node, [v], d, lambda e: self.conv(
                    f"(-{self.conv(e[0], d, tp.float32)})", tp.float32, d))
            return self.elementwise(node, [v], d, lambda e: self._wrap_int(f"(-{e[0]})", d))
        if isinstance(node.op, ast.Not):
            return self.elementwise(node, [v], tp.int1, lambda e: f"(!{e[0]})")
        if isinstance(node.op, ast.Invert):
            return self.elementwise(node, [v], d, lambda e: self._wrap_int(f"(~{e[0]})", d))
        return v

    def _wrap_int(self, e, d):
        if isinstance(d, tp.dtype) and d.is_int and (d.itemsize < 4 or d == tp.int1 or d == tp.uint32):
            return f"(({d.ctype})({e}))"
        return e

    def expr_BinOp(self, node):
        a = self.visit_expr(node.left)
        b = self.visit_expr(node.right)
        return self.binop(node, type(node.op), a, b)

    def _result_dtype(self, a, b):
        """Promotion with Python constants adopting the typed operand's dtype
        (reference codegen.py:1211-1221)."""
        da, db = self.cdtype(a), self.cdtype(b)
        if isinstance(a, Const) and not isinstance(b, Const):
            return tp.promote(tp.float32, db) if isinstance(a.pyval, float) and db.is_int else db
        if isinstance(b, Const) and not isinstance(a, Const):
            return tp.promote(da, tp.float32) if isinstance(b.pyval, float) and da.is_int else da
        return tp.promote(da, db)

    def to_compute(self, e, operand, cd, vd=None):
        """Operand expression converted to the compute dtype; constants are
        rounded to the value dtype first (fp16 * 0.1 uses fp16(0.1))."""
        if isinstance(operand, Const):
            vd = vd or cd
            return self.conv(self.literal(operand.pyval, vd), vd, cd)
        return self.conv(e, operand.dtype, cd)

    def binop(self, node, op, a, b):
        if isinstance(a, Const) and isinstance(b, Const):
            import operator
            ops = {ast.Add: operator.add, ast.Sub: operator.sub, ast.Mult: operator.mul,
                   ast.Div: operator.truediv, ast.FloorDiv: operator.floordiv,
                   ast.Mod: operator.mod, ast.Pow: operator.pow, ast.BitAnd: operator.and_,
                   ast.BitOr: operator.or_, ast.BitXor: operator.xor,
                   ast.LShift: operator.lshift, ast.RShift: operator.rshift}
            if op not in ops:
                self.err(node, f"unsupported operator {op.__name__}")
            return Const(ops[op](a.pyval, b.pyval))
        if isinstance(a, LazyLoad) and isinstance(b, LazyLoad):
            a = self.materialize_load(a)
        if (isinstance(a, (Scalar, Block)) and a.is_ptr) or (isinstance(b, (Scalar, Block)) and b.is_ptr):
            return self.ptr_arith(node, op, a, b)
        rd = self._result_dtype(a, b)
        if op in (ast.Add, ast.Sub, ast.Mult) and rd in (tp.int32, tp.int64):
            r = self.affine_arith(op, a, b, rd)
            if r is not None:
                return r
            A, B = self.as_affine(a, rd), self.as_affine(b, rd)
            if A is not None and B is not None and not A.shape and not B.shape:
                # uniform integer arithmetic keeps its divisibility facts
                f = {ast.Add: lambda x, y: s_add(x, y), ast.Sub: lambda x, y: s_add(x, s_neg(y)),
                     ast.Mult: s_mul}[op]
                sym = f(A.base, B.base)
                if sym.is_const:
                    return self.new_scalar(rd, self.literal(sym.const, rd), sym)
                return self.new_scalar(rd, self.conv(sym.expr, None, None), sym)
        # the same operation on the same operand objects reuses the earlier
        # register block: `(x - mean)` written twice (layernorm's variance and
        # output) is computed once, and x need not stay live for the second
        key = ("bin", op, rd, id(a), id(b))
        hit = self.cse_lookup(key, (a, b))
        if hit is not None:
            return hit
        r = self._binop_values(node, op, a, b, rd)
        self.cse_store(key, (a, b), r)
        return r

    def _binop_values(self, node, op, a, b, rd):
        half = tp.is_half(rd)
        cd = tp.compute_dtype(rd)

        def wrap(fn):
            if not half:
                return lambda es: self._wrap_int(fn(es), rd)
            return lambda es: self.conv(fn(es), tp.float32, rd)

        def emit(fn, x=a, y=b):
            return self.elementwise(node, [x, y], rd, lambda es: fn(
                [self.to_compute(es[0], x, cd, rd), self.to_compute(es[1], y, cd, rd)]))

        if op in _BIN:
            sym = _BIN[op]
            if sym in ("&", "|", "^", "<<", ">>") and rd.is_floating:
                self.err(node, f"bitwise {sym} on floats")
            r = emit(wrap(lambda es: f"({es[0]} {sym} {es[1]})"))
            if sym == "&" and rd == tp.int1 and isinstance(r, Lazy):
                r.meta = self._and_meta(a, b)
            return r
        if op == ast.Div:
            return emit(wrap(lambda es: f"({es[0]} / {es[1]})"))
        if op == ast.FloorDiv:
            if rd.is_int:
                return emit(wrap(lambda es: f"({es[0]} / {es[1]})"))
            f = "floorf" if cd != tp.float64 else "floor"
            return emit(wrap(lambda es: f"{f}({es[0]} / {es[1]})"))
        if op == ast.Mod:
            if rd.is_int:
                return emit(wrap(lambda es: f"({es[0]} % {es[1]})"))
            f = "fmodf" if cd != tp.float64 else "fmod"
            return emit(wrap(lambda es: f"{f}({es[0]}, {es[1]})"))
        if op == ast.Pow:
            if isinstance(b, Const) and b.pyval == 2:
                return self.elementwise(node, [a], rd, lambda es: wrap(
                    lambda xs: f"({xs[0]} * {xs[0]})")([self.to_compute(es[0], a, cd, rd)]))
            if rd.is_int:
                self.err(node, "integer ** requires a constexpr exponent of 2")
            f = "powf" if cd != tp.float64 else "pow"
            return emit(wrap(lambda es: f"{f}({es[0]}, {es[1]})"))
        self.err(node, f"unsupported operator {op.__name__}")

    def _and_meta(self, a, b):
        parts = []
        for x in (a, b):
            m = getattr(x, "meta", None) if isinstance(x, Lazy) else None
            if m is None:
                return None
            parts += m[1] if m[0] == "and" else [m]
        return ("and", parts)

    def as_affine(self, v, rd):
        if isinstance(v, Affine):
            return v
        if isinstance(v, Const) and isinstance(v.pyval, int) and not isinstance(v.pyval, bool):
            return Affine(rd, (), Sym.c(v.pyval), {})
        if isinstance(v, Scalar) and v.dtype in (tp.int32, tp.int64):
            return Affine(rd, (), v.as_sym(), {})
        return None

    def affine_arith(self, op, a, b, rd):
        A, B = self.as_affine(a, rd), self.as_affine(b, rd)
        if A is None or B is None:
            return None
        if not isinstance(a, Affine) and not isinstance(b, Affine):
            return None  # scalar op scalar: plain scalar arithmetic
        shape = tp.broadcast_shapes(A.shape, B.shape)
        A = self.expand_to_rank(A, len(shape)) if A.shape else A
        B = self.expand_to_rank(B, len(shape)) if B.shape else B
        if op == ast.Mult:
            if A.coefs and B.coefs:
                return None
            if B.coefs:
                A, B = B, A
            k = B.base
            return Affine(rd, shape, s_mul(A.base, k), {ax: s_mul(c, k) for ax, c in A.coefs.items()})
        if op == ast.Sub:
            B = Affine(rd, B.shape, s_neg(B.base), {ax: s_neg(c) for ax, c in B.coefs.items()})
        coefs = dict(A.coefs)
        for ax, c in B.coefs.items():
            coefs[ax] = s_add(coefs[ax], c) if ax in coefs else c
        coefs = {ax: c for ax, c in coefs.items() if not (c.is_const and c.const == 0)}
        return Affine(rd, shape, s_add(A.base, B.base), coefs)

    def ptr_arith(self, node, op, a, b):
        if isinstance(b, (Scalar, Block)) and b.is_ptr and not (isinstance(a, (Scalar, Block)) and a.is_ptr):
            if op == ast.Sub:
                self.err(node, "int - pointer is not supported")
            a, b = b, a
        if op not in (ast.Add, ast.Sub):
            self.err(node, "only + and - on pointers")
        if isinstance(b, (Scalar, Block)) and b.is_ptr:
            self.err(node, "pointer - pointer not supported")
        if isinstance(b, LazyLoad):
            b = self.materialize_load(b)
        bd = self.cdtype(b)
        if not bd.is_int:
            self.err(node, "pointer offsets must be integers")
        if op == ast.Sub:
            b = self.expr_neg(node, b)
        if isinstance(a, Scalar):
            if isinstance(b, (Const, Scalar)):
                sym = b.as_sym() if isinstance(b, Scalar) else Sym.c(b.pyval)
                esz = a.dtype.element.itemsize
                al = a.aligned16 and (sym.div * esz) % 16 == 0
                t = self.fresh("p")
                self.emit(f"{a.dtype.element.ctype}* const {t} = {a.expr} + ({sym.expr});")
                return Scalar(a.dtype, t, aligned16=al)
            return PtrBlock(a, b)
        # pointer block +- int
        off = self.binop(node, ast.Add, a.offset, b)
        return PtrBlock(a.base, off)

    def expr_neg(self, node, v):
        if isinstance(v, Const):
            return Const(-v.pyval)
        if isinstance(v, Affine):
            return Affine(v.dtype, v.shape, s_neg(v.base), {a: s_neg(c) for a, c in v.coefs.items()})
        if isinstance(v, Scalar):
            return self.new_scalar(v.dtype, f"(-{v.expr})", s_neg(v.as_sym()))
        d = v.dtype
        return self.elementwise(node, [v], d, lambda e: f"(-{e[0]})")

    def expr_Compare(self, node):
        if len(node.ops) != 1:
            self.err(node, "chained comparisons not supported")
        a = self.visit_expr(node.left)
        b = self.visit_expr(node.comparators[0])
        return self.compare(node, type(node.ops[0]), a, b)

    def compare(self, node, op, a, b):
        if isinstance(a, Const) and isinstance(b, Const):
            import operator
            ops = {ast.Eq: operator.eq, ast.NotEq: operator.ne, ast.Lt: operator.lt,
                   ast.LtE: operator.le, ast.Gt: operator.gt, ast.GtE: operator.ge}
            return Const(ops[op](a.pyval, b.pyval))
        sym = _CMP.get(op)
        if sym is None:
            self.err(node, f"unsupported comparison {op.__name__}")
        cd = tp.compute_dtype(tp.promote(self.cdtype(a), self.cdtype(b)))
        meta = None
        if cd in (tp.int32, tp.int64):
            A, B = self.as_affine(a, cd), self.as_affine(b, cd)
            if A is not None and B is not None and (A.coefs or B.coefs):
                diff = self.affine_arith(ast.Sub, A, B, cd)
                if diff is not None:
                    meta = ("cmp", sym, diff)
        r = self.elementwise(node, [a, b], tp.int1, lambda es: (
            f"({self.to_compute(es[0], a, cd)} {sym} {self.to_compute(es[1], b, cd)})"), meta=meta)
        if isinstance(r, Lazy) and meta is not None:
            r.meta = ("and", [meta])
        return r

    def expr_BoolOp(self, node):
        vals = [self.visit_expr(v) for v in node.values]
        if all(isinstance(v, Const) for v in vals):
            out = vals[0].pyval
            for v in vals[1:]:
                out = (out and v.pyval) if isinstance(node.op, ast.And) else (out or v.pyval)
            return Const(out)
        if any(isinstance(v, Block) for v in vals):
            self.err(node, "use & / | for elementwise boolean ops on blocks")
        sym = "&&" if isinstance(node.op, ast.And) else "||"
        return self.new_scalar(tp.int1, "(" + f" {sym} ".join(
            self.scalar_expr(v, tp.int1) if isinstance(v, Const) else f"({v.expr})" for v in vals) + ")")

    def expr_IfExp(self, node):
        c = self.visit_expr(node.test)
        if isinstance(c, Const):
            return self.visit_expr(node.body if c.pyval else node.orelse)
        return self.op_where(node, c, self.visit_expr(node.body), self.visit_expr(node.orelse))

    def expr_Subscript(self, node):
        base = self.visit_expr(node.value)
        if isinstance(base, Const):
            idx = self.visit_expr(node.slice)
            if not isinstance(idx, Const):
                self.err(node, "runtime indexing of constexpr values")
            return Const(base.pyval[idx.pyval])
        elts = node.slice.elts if isinstance(node.slice, ast.Tuple) else [node.slice]
        out = base
        di = 0
        for e in elts:
            if isinstance(e, ast.Constant) and e.value is None:
                out = self.expand_dims(out, di)
                di += 1
            elif isinstance(e, ast.Slice) and e.lower is None and e.upper is None and e.step is None:
                if di >= len(out.shape):
                    self.err(node, "too many indices")
                di += 1
            else:
                self.err(node, "only x[:, None]-style indexing is supported on blocks")
        return out

    def _callee(self, func):
        if isinstance(func, ast.Name):
            return func.id
        if isinstance(func, ast.Attribute):
            return func.attr
        return None

    def _resolve(self, func):
        try:
            if isinstance(func, ast.Name):
                v = self.locals.get(func.id)
                if isinstance(v, Const):
                    return v.pyval
                if v is not None:
                    return None
                if func.id in self.globals:
                    return self.globals[func.id]
                return getattr(builtins, func.id, None)
            if isinstance(func, ast.Attribute):
                base = self._resolve(func.value)
                if base is not None:
                    return getattr(base, func.attr, None)
        except Exception:
            return None
        return None

    def expr_Call(self, node):
        if isinstance(node.func, ast.Attribute) and node.func.attr == "to":
            base = self.visit_expr(node.func.value)
            if not isinstance(base, Const):
                dt = self.visit_expr(node.args[0])
                return self.cast(node, base, dt.pyval)
        name = self._callee(node.func)
        target = self._resolve(node.func)
        if target is not None and hasattr(target, "_newt_builtin"):
            name = target._newt_builtin
            handler = getattr(self, f"op_{name}", None)
            args = [self.visit_expr(a) for a in node.args]
            kwargs = {kw.arg: self.visit_expr(kw.value) for kw in node.keywords}
            if handler is None:
                self.err(node, f"nl.{name} is not supported")
            try:
                return handler(node, *args, **kwargs)
            except TypeError as e:
                if "positional argument" in str(e) or "unexpected keyword" in str(e):
                    self.err(node, f"bad arguments to nl.{name}: {e}")
                raise
        args = [self.visit_expr(a) for a in node.args]
        kwargs = {kw.arg: self.visit_expr(kw.value) for kw in node.keywords}
        if target is not None and all(isinstance(v, Const) for v in args) and all(
                isinstance(v, Const) for v in kwargs.values()):
            try:
                return Const(target(*[v.pyval for v in args],
                                    **{k: v.pyval for k, v in kwargs.items()}))
            except Exception as e:
                self.err(node, f"constexpr call failed: {e}")
        if name in ("min", "max") and len(args) == 2:
            return (self.op_minimum if name == "min" else self.op_maximum)(node, *args)
        if name == "abs" and len(args) == 1:
            return self.op_abs(node, args[0])
        self.err(node, f"unknown function '{name}' (newt kernels can only call nl.* builtins)")

    # ------------------------------------------------------------ builtin ops
    def _cx(self, node, v, what):
        if not isinstance(v, Const):
            self.err(node, f"{what} must be a compile-time constant")
        return v.pyval

    def op_program_id(self, node, axis):
        """Program ids are a bijection of the hardware workgroup ids, chosen
        for MI355X's 8 XCDs: the dispatcher hands consecutive workgroups to
        XCDs round-robin, so the linear id b is renumbered to
        (b % 8) * (nb / 8) + b / 8 (for b below the largest multiple of 8) and
        each XCD runs one contiguous range of programs. Neighbouring programs
        then share an L2, and a grid whose work varies along axis 0 (causal
        attention) is spread evenly over the XCDs instead of giving one XCD
        every eighth, heaviest block. Programs are independent, so any
        bijection keeps the language's semantics (NEWT_PID_REMAP=0: identity).
        Kernels whose programs share no data with a subset of the others
        (remap_pids False: streaming row kernels) keep the hardware order.

        In a kernel where program (i, j) reads row panel i of one dot operand
        and column panel j of the other (group_pids), each XCD's range is
        further walked in groups of G values of axis 0 with axis 1 varying
        inside a group: the 32 or so programs an XCD runs at once then share
        G row panels and about 32/G column panels instead of needing every
        row panel, which keeps an 8192^3 fp16 matmul's operands in L2/MALL
        (NEWT_PID_GROUP=G, default 4; 0 turns grouping off).

        In a kernel whose work grows with program_id(0) (lpt_pids: a causal
        attention's key loop ends at its query block's diagonal), the
        programs run heaviest first, the longest-processing-time-first order
        that keeps short programs for the end of the launch. When the grid's
        other axes split evenly over the 8 XCDs, each XCD's range holds gh
        whole rows of axis 0 (gh heads), taken in groups of G = 4 rows (all gh
        when 4 does not divide gh): within a group, the r-th program becomes
        weight rank r / G of row r % G, counted from the heaviest, so every
        row's heaviest program starts first, then every row's next. Groups of
        4 keep four heads' keys and values in the XCD's L2 at a time, which
        measured 3% faster than interleaving all gh heads. Otherwise axis 0 is
        reversed within each row (NEWT_PID_LPT=0 turns this off)."""
        ax = self._cx(node, axis, "program_id axis")
        if os.environ.get("NEWT_PID_REMAP", "1") == "0" or not self.remap_pids:
            return self.new_scalar(tp.int32, f"(int)blockIdx.{'xyz'[ax]}")
        if not self.pid_remap:
            self.pid_remap = True
            self.prologue += [
                "const unsigned _nbx = gridDim.x, _nby = gridDim.y;",
                "const unsigned _nb = _nbx * _nby * gridDim.z;",
                "unsigned _pb = blockIdx.x + _nbx * (blockIdx.y + _nby * blockIdx.z);",
                "{ const unsigned _full = _nb & ~7u;",
                "  if (_pb < _full) _pb = (_pb & 7u) * (_full >> 3) + (_pb >> 3); }",
            ]
            G = int(os.environ.get("NEWT_PID_GROUP", "4")) if self.group_pids else 0
            if G == 0 and self.lpt_pids and os.environ.get("NEWT_PID_LPT", "1") != "0":
                self.prologue += [
                    "{ const unsigned _nh = _nb / _nbx;",
                    "  if (_nh % 8u == 0u) {",
                    "    const unsigned _gh = _nh >> 3, _per = _gh * _nbx, _base = _pb / _per * _per, "
                    "_r = _pb - _base;",
                    "    const unsigned _G = _gh % 4u == 0u ? 4u : _gh, _g = _r / (_G * _nbx), "
                    "_rr = _r % (_G * _nbx);",
                    "    _pb = _base + (_g * _G + _rr % _G) * _nbx + (_nbx - 1u - _rr / _G);",
                    "  } else {",
                    "    const unsigned _p0 = _pb % _nbx;",
                    "    _pb = _pb - _p0 + (_nbx - 1u - _p0);",
                    "  } }",
                ]
            if G > 0:
                self.prologue += [
                    f"const unsigned _q = _pb % (_nbx * _nby), _gw = {G}u * _nby;",
                    f"const unsigned _g0 = (_q / _gw) * {G}u;",
                    f"const unsigned _gn = _nbx - _g0 < {G}u ? _nbx - _g0 : {G}u;",
                    "const int _pid0 = (int)(_g0 + (_q % _gw) % _gn);",
                    "const int _pid1 = (int)((_q % _gw) / _gn);",
                ]
            else:
                self.prologue += [
                    "const int _pid0 = (int)(_pb % _nbx);",
                    "const int _pid1 = (int)((_pb / _nbx) % _nby);",
                ]
            self.prologue.append("const int _pid2 = (int)(_pb / (_nbx * _nby));")
        return Scalar(tp.int32, f"_pid{ax}", Sym(f"_pid{ax}", None, 1))

    def op_num_programs(self, node, axis):
        ax = self._cx(node, axis, "num_programs axis")
        return self.new_scalar(tp.int32, f"(int)gridDim.{'xyz'[ax]}")

    def op_arange(self, node, start, end):
        s = self._cx(node, start, "arange start")
        e = self._cx(node, end, "arange end")
        n = e - s
        if not _pow2(n):
            self.err(node, f"arange size must be a positive power of two, got {n}")
        return Affine(tp.int32, (n,), Sym.c(s), {0: Sym.c(1)})

    def _shape(self, node, shape):
        sh = self._cx(node, shape, "block shape")
        if isinstance(sh, int):
            sh = (sh,)
        sh = tuple(int(x) for x in sh)
        for d in sh:
            if not _pow2(d):
                self.err(node, f"block dims must be powers of two, got {sh}")
        return sh

    def op_zeros(self, node, shape, dtype=None):
        sh = self._shape(node, shape)
        dt = dtype.pyval if dtype is not None else tp.float32
        return Fill(dt, sh, Const(0))

    def op_full(self, node, shape, value, dtype=None):
        sh = self._shape(node, shape)
        dt = dtype.pyval if dtype is not None else tp.float32
        if isinstance(value, Block):
            self.err(node, "full() value must be a scalar")
        if isinstance(value, Scalar):
            value = self.new_scalar(dt, self.scalar_expr(value, dt))
        return Fill(dt, sh, value)

    def op_expand_dims(self, node, x, axis):
        return self.expand_dims(x, self._cx(node, axis, "axis"))

    def op_broadcast_to(self, node, x, shape):
        sh = self._shape(node, shape)
        if isinstance(x, (Const, Scalar)):
            return Fill(self.cdtype(x), sh, x)
        x = self.expand_to_rank(x, len(sh))
        tp.broadcast_shapes(x.shape, sh)
        if isinstance(x, (Affine, Lazy, Fill)):
            return self._rebroadcast(x, sh)
        if isinstance(x, LazyLoad):
            x = self.materialize_load(x)
        if isinstance(x, Reg):
            if x.shape == sh:
                return x
            L = x.layout.broadcast_into(sh)
            if L is not None:
                return self.to_reg(x, L)
            return self.convert(x, self.default_layout(sh))
        self.err(node, "cannot broadcast this value")

    def _rebroadcast(self, x, sh):
        if isinstance(x, Affine):
            return Affine(x.dtype, sh, x.base, x.coefs)
        if isinstance(x, Fill):
            return Fill(x.dtype, sh, x.value)
        out = Lazy(x.dtype, sh, x.fn, x.args, x.size)
        out.meta = getattr(x, "meta", None)
        return out

    def op_reshape(self, node, x, shape):
        sh = self._shape(node, shape)
        if isinstance(x, (Const, Scalar)):
            return Fill(self.cdtype(x), sh, x)
        if math.prod(sh) != x.numel:
            self.err(node, f"reshape {x.shape} -> {sh} changes element count")
        return self.reshape(node, x, sh)

    def op_trans(self, node, x):
        if not isinstance(x, Block) or len(x.shape) != 2:
            self.err(node, "trans expects a 2D block")
        return self.permute(x, (1, 0))

    def cast(self, node, x, dt):
        if not isinstance(dt, tp.dtype):
            self.err(node, f"invalid dtype {dt!r}")
        if isinstance(x, Const):
            return x
        if x.dtype == dt:
            return x
        if isinstance(x, Scalar):
            return self.new_scalar(dt, self.conv(x.expr, x.dtype, dt))
        src = x.dtype
        if isinstance(x, Fill):
            return Fill(dt, x.shape, self.cast(node, x.value, dt) if isinstance(x.value, Scalar) else x.value)
        return self.elementwise(node, [x], dt, lambda es: self.conv(es[0], src, dt))

    def op_cast(self, node, x, dtype):
        return self.cast(node, x, dtype.pyval)

    # math (reference codegen.py:2011-2153)
    def _math1(self, node, x, name):
        if isinstance(x, Const):
            x = Scalar(self.cdtype(x), self.literal(x.pyval, self.cdtype(x)))
        d = x.dtype
        if not d.is_floating:
            x = self.cast(node, x, tp.float32)
            d = tp.float32
        cd = tp.compute_dtype(d)
        f32, f64 = _MATH[name]
        fn = f64 if cd == tp.float64 else f32

        def expr(es):
            r = f"{fn}({self.conv(es[0], d, cd)})"
            return self.conv(r, cd, d)

        return self.elementwise(node, [x], d, expr)

    def op_exp(self, node, x): return self._math1(node, x, "exp")
    def op_exp2(self, node, x): return self._math1(node, x, "exp2")
    def op_log(self, node, x): return self._math1(node, x, "log")
    def op_log2(self, node, x): return self._math1(node, x, "log2")
    def op_sqrt(self, node, x): return self._math1(node, x, "sqrt")
    def op_rsqrt(self, node, x): return self._math1(node, x, "rsqrt")
    def op_sin(self, node, x): return self._math1(node, x, "sin")
    def op_cos(self, node, x): return self._math1(node, x, "cos")
    def op_tanh(self, node, x): return self._math1(node, x, "tanh")
    def op_erf(self, node, x): return self._math1(node, x, "erf")
    def op_floor(self, node, x): return self._math1(node, x, "floor")
    def op_ceil(self, node, x): return self._math1(node, x, "ceil")

    def op_sigmoid(self, node, x):
        d = self.cdtype(x)
        cd = tp.compute_dtype(d)
        one = "1.0" if cd == tp.float64 else "1.0f"
        ex = "exp" if cd == tp.float64 else "newt::exp_f32"
        return self.elementwise(node, [x], d, lambda es: self.conv(
            f"({one} / ({one} + {ex}(-({self.conv(es[0], d, cd)}))))", cd, d))

    def op_abs(self, node, x):
        if isinstance(x, Const):
            return Const(abs(x.pyval))
        d = self.cdtype(x)
        if d.is_floating:
            cd = tp.compute_dtype(d)
            fn = "fabs" if cd == tp.float64 else "fabsf"
            return self.elementwise(node, [x], d, lambda es: self.conv(
                f"{fn}({self.conv(es[0], d, cd)})", cd, d))
        return self.elementwise(node, [x], d, lambda es: self._wrap_int(
            f"(({es[0]}) < 0 ? -({es[0]}) : ({es[0]}))", d))

    def _math2(self, node, a, b, ffn, iop):
        rd = tp.promote(self.cdtype(a), self.cdtype(b))
        cd = tp.compute_dtype(rd)
        if rd.is_int:
            return self.elementwise(node, [a, b], rd, lambda es: (
                f"(({self.to_compute(es[0], a, cd)}) {iop} ({self.to_compute(es[1], b, cd)}) ? "
                f"({self.to_compute(es[0], a, cd)}) : ({self.to_compute(es[1], b, cd)}))"))
        fn = ffn if cd != tp.float64 else ffn.rstrip("f")
        return self.elementwise(node, [a, b], rd, lambda es: self.conv(
            f"{fn}({self.to_compute(es[0], a, cd)}, {self.to_compute(es[1], b, cd)})", cd, rd))

    def op_maximum(self, node, a, b):
        return self._math2(node, a, b, "fmaxf", ">")

    def op_minimum(self, node, a, b):
        return self._math2(node, a, b, "fminf", "<")

    def op_fma(self, node, a, b, c):
        rd = tp.promote(self.cdtype(a), tp.promote(self.cdtype(b), self.cdtype(c)))
        cd = tp.compute_dtype(rd)
        fn = "fma" if cd == tp.float64 else "fmaf"
        ops = (a, b, c)
        return self.elementwise(node, [a, b, c], rd, lambda es: self.conv(
            f"{fn}({', '.join(self.to_compute(e, o, cd) for e, o in zip(es, ops))})", cd, rd))

    def op_where(self, node, cond, a, b):
        if isinstance(cond, Const):
            return a if cond.pyval else b
        rd = tp.promote(self.cdtype(a), self.cdtype(b))
        st = self.pipe_active
        if st is not None and st.get("fast") and id(node) in st.get("true_wheres", ()):
            # the branch-free copy of a pipelined loop runs only iterations in
            # which this mask is all-true (its entry test proved it)
            return self.elementwise(node, [cond, a, b], rd,
                                    lambda es: self.to_compute(es[1], a, rd))
        fast = None
        if isinstance(cond, Block):
            # a mask that one uniform test proves all-true (interior tiles of a
            # bounds or causal mask) selects `a` without per-element compares
            full = self.mask_all_true(cond, cond.shape)
            if full not in (None, "true", "false"):
                fast = (full, lambda es: self.to_compute(es[1], a, rd))
        return self.elementwise(node, [cond, a, b], rd, lambda es: (
            f"(({es[0]}) ? ({self.to_compute(es[1], a, rd)}) : ({self.to_compute(es[2], b, rd)}))"),
            fast=fast)

    def op_cdiv(self, node, a, b):
        if isinstance(a, Const) and isinstance(b, Const):
            return Const(-(-a.pyval // b.pyval))
        rd = tp.promote(self.cdtype(a), self.cdtype(b))
        return self.elementwise(node, [a, b], rd, lambda es: (
            f"(({self.to_compute(es[0], a, rd)} + {self.to_compute(es[1], b, rd)} - 1) / "
            f"{self.to_compute(es[1], b, rd)})"))

    def op_multiple_of(self, node, x, value=None):
        if isinstance(x, Scalar) and isinstance(value, Const) and x.sym is not None:
            v = int(value.pyval)
            d = v & -v if v else 1
            return Scalar(x.dtype, x.expr, Sym(x.sym.expr, x.sym.const, max(x.sym.div, d)))
        return x

    def op_max_contiguous(self, node, x, value=None):
        return x

    def op_static_assert(self, node, cond, msg=None):
        c = self._cx(node, cond, "static_assert condition")
        if not c:
            m = msg.pyval if msg is not None else ""
            self.err(node, f"static_assert failed: {m}")
        return Const(None)

    def op_static_print(self, node, *args):
        print("[newt static_print]", *[a.pyval if isinstance(a, Const) else a for a in args])
        return Const(None)


class _Retry(Exception):
    """Raised when a storage decision was wrong; compile again with new hints."""


def _gcd_pow2(a, b):
    d = 1 << 30
    for v in (a, b):
        v = abs(int(v))
        if v:
            d = min(d, v & -v)
    return d
