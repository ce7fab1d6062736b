"""The newt compiler for gfx950: kernel AST -> HIP C++ source."""

import ast
import copy
import os

from .codegen import CompileError, Codegen, _Retry
from .ops_dot import DotOps
from .ops_memory import MemoryOps
from .ops_pipeline import DotPipeline
from .ops_reduce import ReduceOps


class Param:
    """A runtime kernel parameter as specialized by the JIT: its dtype (or
    pointer type), C name, and the value facts compiled into the kernel
    (integer == 1, power-of-two divisor up to 16, pointer 16-byte aligned)."""

    def __init__(self, dtype, cname, eq1=False, div=1, aligned16=False):
        self.dtype = dtype
        self.cname = cname
        self.eq1 = eq1
        self.div = div
        self.aligned16 = aligned16

    def __repr__(self):
        return f"Param({self.dtype}, {self.cname}, eq1={self.eq1}, div={self.div}, a16={self.aligned16})"


class Compiler(DotPipeline, DotOps, ReduceOps, MemoryOps, Codegen):
    pass


def _has_row_reduction(fndef):
    import ast
    for n in ast.walk(fndef):
        if isinstance(n, ast.Call):
            name = n.func.attr if isinstance(n.func, ast.Attribute) else getattr(n.func, "id", None)
            if name in ("sum", "max", "min"):
                for kw in n.keywords:
                    if kw.arg == "axis" and isinstance(kw.value, ast.Constant) and kw.value.value in (1, -1):
                        return True
                if len(n.args) >= 2 and isinstance(n.args[1], ast.Constant) and n.args[1].value in (1, -1):
                    return True
    return False


def _chained_dots(fndef):
    """True when some nl.dot's first operand is computed from another dot's
    result (attention's P @ V after S = Q K^T). Names are followed through
    assignments anywhere in the function, to a fixed point, so loop-carried
    dependences count."""
    import ast
    assigns = [n for n in ast.walk(fndef) if isinstance(n, (ast.Assign, ast.AugAssign))]

    def reads(e):
        return {x.id for x in ast.walk(e) if isinstance(x, ast.Name) and isinstance(x.ctx, ast.Load)}

    fed = set()
    changed = True
    while changed:
        changed = False
        for a in assigns:
            tgts = a.targets if isinstance(a, ast.Assign) else [a.target]
            names = {t.id for t in tgts if isinstance(t, ast.Name)}
            if names <= fed:
                continue
            if any(_callee_name(x) == "dot" for x in ast.walk(a.value)) or reads(a.value) & fed:
                fed |= names
                changed = True
    return any(_callee_name(n) == "dot" and n.args and reads(n.args[0]) & fed
               for n in ast.walk(fndef))


def _split_dot_axes(fndef):
    """True when some nl.dot's first operand depends on program axis 0 but not
    axis 1 and its second on axis 1 but not axis 0 (or the reverse): the tiled
    matmul pattern, in which program (i, j) reads row panel i of one operand
    and column panel j of the other. Dependence is followed through
    assignments by name (an over-approximation: it only ever adds axes, so an
    unclear case is not matched)."""
    _, axes = _pid_taint(fndef)
    for n in ast.walk(fndef):
        if _callee_name(n) == "dot" and len(n.args) >= 2:
            a, b = axes(n.args[0]), axes(n.args[1])
            if -1 in a or -1 in b:
                continue
            if ({0, 1} & a, {0, 1} & b) in (({0}, {1}), ({1}, {0})):
                return True
    return False


def _pid_taint(fndef):
    """Name -> set of program axes its value depends on (-1: an axis not
    known at compile time), followed through assignments by name; returns
    (taint, axes) where axes(expr) is the set for an expression."""
    taint = {}

    def axes(expr):
        out = set()
        for n in ast.walk(expr):
            if _callee_name(n) == "program_id":
                arg = n.args[0] if n.args else next((k.value for k in n.keywords if k.arg == "axis"), None)
                out.add(arg.value if isinstance(arg, ast.Constant) else -1)
            elif isinstance(n, ast.Name) and n.id in taint:
                out |= taint[n.id]
        return out

    changed = True
    while changed:
        changed = False
        for n in ast.walk(fndef):
            if isinstance(n, ast.Assign):
                targets, value = n.targets, n.value
            elif isinstance(n, (ast.AugAssign, ast.AnnAssign)) and n.value is not None:
                targets, value = [n.target], n.value
            elif isinstance(n, ast.For):
                targets, value = [n.target], n.iter
                # a range's end bound sets how many values the target takes,
                # not which: only its start and step carry dependence
                if _callee_name(value) == "range" and 1 <= len(value.args) <= 3:
                    parts = [] if len(value.args) == 1 else [value.args[0]] + list(value.args[2:])
                    value = ast.Tuple(elts=parts, ctx=ast.Load())
            else:
                continue
            t = axes(value)
            for tg in targets:
                for e in ast.walk(tg):
                    if isinstance(e, ast.Name) and not t <= taint.get(e.id, set()):
                        taint[e.id] = taint.get(e.id, set()) | t
                        changed = True
    return taint, axes


def _streamed(fndef, kinds):
    """ids of the top-level calls named in `kinds` (nl.load / nl.store) that
    touch data no other program touches: the address depends on every
    program axis the kernel uses (one row per program, as in softmax or
    layernorm), the call is inside no loop, at any depth (no re-reads), and a load's value
    does not feed nl.dot (dot operands are shared by the programs of a row or
    column of tiles). Their lines need not stay in the caches, so they take
    the non-temporal hint; data shared by all programs (a layernorm's weight
    and bias) keeps the caches to itself."""
    taint, axes = _pid_taint(fndef)
    used = set()
    for n in ast.walk(fndef):
        if _callee_name(n) in ("program_id", "num_programs"):
            arg = n.args[0] if n.args else next((k.value for k in n.keywords if k.arg == "axis"), None)
            used.add(arg.value if isinstance(arg, ast.Constant) else -1)
    if not used or -1 in used:
        return set()
    dot_names = {a.id for n in ast.walk(fndef) if _callee_name(n) == "dot"
                 for a in ast.walk(n) if isinstance(a, ast.Name)}
    in_loops = {id(n) for st in ast.walk(fndef) if isinstance(st, (ast.For, ast.While))
                for n in ast.walk(st)}
    out = set()
    for st in fndef.body:
        if isinstance(st, (ast.For, ast.While)):
            continue
        for n in ast.walk(st):
            if _callee_name(n) not in kinds or not n.args or id(n) in in_loops:
                continue
            if isinstance(st, ast.Assign) and any(isinstance(t, ast.Name) and t.id in dot_names
                                                  for t in st.targets):
                continue
            if used <= axes(n.args[0]):
                out.add(id(n))
    return out


def _shares_across_programs(fndef):
    """False only for streaming kernels: every load outside any loop, each
    either private to its program (the address depends on every program axis
    the kernel uses: a row of softmax) or common to all programs (no program
    axis: a layernorm's weights). Otherwise some data may be read by a subset
    of the programs (a matmul's row panel, one attention head's keys and
    values), and renumbering programs so that each XCD runs a contiguous
    range keeps that data in one L2. Streaming kernels gain nothing from the
    renumbering and measured 2-4% slower with it (the hardware's round-robin
    order spreads a stream over the HBM channels better)."""
    taint, axes = _pid_taint(fndef)
    used = set()
    for n in ast.walk(fndef):
        if _callee_name(n) in ("program_id", "num_programs"):
            arg = n.args[0] if n.args else next((k.value for k in n.keywords if k.arg == "axis"), None)
            used.add(arg.value if isinstance(arg, ast.Constant) else -1)
    if -1 in used:
        return True
    in_loops = {id(n) for st in ast.walk(fndef) if isinstance(st, (ast.For, ast.While))
                for n in ast.walk(st)}
    for n in ast.walk(fndef):
        if _callee_name(n) == "load" and n.args:
            dep = axes(n.args[0])
            if id(n) in in_loops or -1 in dep or (dep & used and not used <= dep):
                return True
    return False


def _work_grows_along_axis0(fndef, constexprs):
    """True when a program's work grows with its program_id(0): the trip
    count of some outermost for-loop is a non-decreasing function of axis 0
    that depends on it (a causal attention's key loop, bounded by its query
    block's diagonal), every other outermost loop's count is independent of
    axis 0, and the kernel has no atomics (so the order in which programs run
    cannot be observed). Such a grid is best run heaviest first: every
    program that starts late is then a short one.

    An abstract interpretation over the statements in order gives each name
    'C' (independent of axis 0), 'I' (non-decreasing in it and dependent on
    it), 'D' (non-increasing) or 'U' (unknown). Constexpr ifs take their live
    branch, a runtime if joins its branches, and names assigned inside a loop
    are 'U' after it."""

    def const_value(e):
        # compile-time value of an expression over literals and constexprs
        if isinstance(e, ast.Constant) and isinstance(e.value, (int, float, bool)):
            return e.value
        if isinstance(e, ast.Name) and e.id in constexprs:
            v = constexprs[e.id]
            return getattr(v, "value", v)
        if isinstance(e, ast.UnaryOp):
            v = const_value(e.operand)
            if v is None:
                return None
            return {ast.USub: lambda: -v, ast.Not: lambda: not v, ast.UAdd: lambda: v}.get(
                type(e.op), lambda: None)()
        if isinstance(e, ast.BinOp):
            a, b = const_value(e.left), const_value(e.right)
            if a is None or b is None:
                return None
            ops = {ast.Add: lambda: a + b, ast.Sub: lambda: a - b, ast.Mult: lambda: a * b,
                   ast.FloorDiv: lambda: a // b if b else None, ast.Mod: lambda: a % b if b else None}
            return ops.get(type(e.op), lambda: None)()
        if isinstance(e, ast.BoolOp):
            vs = [const_value(x) for x in e.values]
            if any(v is None for v in vs):
                return None
            return all(vs) if isinstance(e.op, ast.And) else any(vs)
        if isinstance(e, ast.Compare) and len(e.ops) == 1:
            a, b = const_value(e.left), const_value(e.comparators[0])
            if a is None or b is None:
                return None
            ops = {ast.Eq: a == b, ast.NotEq: a != b, ast.Lt: a < b, ast.LtE: a <= b,
                   ast.Gt: a > b, ast.GtE: a >= b}
            return ops.get(type(e.ops[0]))
        return None

    def positive(e):
        v = const_value(e)
        return isinstance(v, (int, float)) and not isinstance(v, bool) and v > 0

    def add(a, b):
        if a == "C":
            return b
        if b == "C":
            return a
        return a if a == b and a in ("I", "D") else "U"

    neg = {"C": "C", "I": "D", "D": "I", "U": "U"}
    atomics = [False]

    def ev(e, env):
        name = _callee_name(e) if isinstance(e, ast.Call) else None
        if name == "program_id":
            arg = e.args[0] if e.args else next((k.value for k in e.keywords if k.arg == "axis"), None)
            ax = const_value(arg) if arg is not None else None
            return "I" if ax == 0 else ("C" if ax in (1, 2) else "U")
        if name in ("minimum", "maximum", "min", "max") and len(e.args) == 2 and not e.keywords:
            a, b = ev(e.args[0], env), ev(e.args[1], env)
            return add(a, b) if "U" not in (a, b) else "U"
        if name == "cdiv" and len(e.args) == 2 and positive(e.args[1]):
            return ev(e.args[0], env)
        if isinstance(e, ast.Name):
            return env.get(e.id, "C")
        if isinstance(e, ast.Constant):
            return "C"
        if isinstance(e, ast.UnaryOp) and isinstance(e.op, ast.USub):
            return neg[ev(e.operand, env)]
        if isinstance(e, ast.BinOp):
            a, b = ev(e.left, env), ev(e.right, env)
            if isinstance(e.op, ast.Add):
                return add(a, b)
            if isinstance(e.op, ast.Sub):
                return add(a, neg[b])
            if isinstance(e.op, ast.Mult):
                if a == "C" and b == "C":
                    return "C"
                if a == "C" and positive(e.left):
                    return b
                if b == "C" and positive(e.right):
                    return a
                return "U"
            if isinstance(e.op, ast.FloorDiv) and b == "C" and positive(e.right):
                return a
            return "C" if a == b == "C" else "U"
        # anything else is independent of axis 0 only if all of its parts are
        parts = [x for x in ast.iter_child_nodes(e) if isinstance(x, ast.expr)]
        return "C" if all(ev(x, env) == "C" for x in parts) else "U"

    def assigned(stmts):
        out = set()
        for st in stmts:
            for n in ast.walk(st):
                if isinstance(n, (ast.Assign, ast.AugAssign, ast.AnnAssign, ast.For)):
                    tgts = n.targets if isinstance(n, ast.Assign) else [n.target]
                    for t in tgts:
                        out |= {x.id for x in ast.walk(t) if isinstance(x, ast.Name)}
        return out

    counts = []

    def walk(stmts, env):
        for st in stmts:
            for n in ast.walk(st):
                if _callee_name(n) in ("atomic_add", "atomic_max", "atomic_min"):
                    atomics[0] = True
            if isinstance(st, ast.Assign):
                v = ev(st.value, env)
                for t in st.targets:
                    names = [x.id for x in ast.walk(t) if isinstance(x, ast.Name)]
                    for nm in names:
                        env[nm] = v if isinstance(t, ast.Name) else "U"
            elif isinstance(st, ast.AugAssign) and isinstance(st.target, ast.Name):
                env[st.target.id] = ev(ast.BinOp(left=ast.Name(id=st.target.id, ctx=ast.Load()),
                                                 op=st.op, right=st.value), env)
            elif isinstance(st, ast.AnnAssign) and isinstance(st.target, ast.Name) and st.value:
                env[st.target.id] = ev(st.value, env)
            elif isinstance(st, ast.If):
                c = const_value(st.test)
                if c is not None:
                    walk(st.body if c else st.orelse, env)
                else:
                    e1, e2 = dict(env), dict(env)
                    walk(st.body, e1)
                    walk(st.orelse, e2)
                    for k in set(e1) | set(e2):
                        a, b = e1.get(k, "C"), e2.get(k, "C")
                        env[k] = a if a == b else "U"
            elif isinstance(st, (ast.For, ast.While)):
                cnt = "U"
                if (isinstance(st, ast.For) and _callee_name(st.iter) == "range"
                        and 1 <= len(st.iter.args) <= 3 and not st.iter.keywords):
                    a = st.iter.args
                    lo, hi = (ast.Constant(0), a[0]) if len(a) == 1 else (a[0], a[1])
                    if len(a) < 3 or positive(a[2]):
                        cnt = add(ev(hi, env), neg[ev(lo, env)])
                counts.append(cnt)
                for nm in assigned([st]):
                    env[nm] = "U"
            else:
                for nm in assigned([st]):
                    env[nm] = "U"

    walk(fndef.body, {})
    return not atomics[0] and "I" in counts and all(c in ("C", "I") for c in counts)


_MEM_WRITES = {"store", "atomic_add", "atomic_max", "atomic_min"}


def _callee_name(node):
    if not isinstance(node, ast.Call):
        return None
    f = node.func
    return f.attr if isinstance(f, ast.Attribute) else getattr(f, "id", None)


def hoist_loads(fndef):
    """Move each top-level `name = nl.load(...)` up to just after the last
    statement it depends on, so independent loads are issued before earlier
    reductions and their barriers (layernorm's weight and bias loads then
    overlap the row statistics instead of following them). A load never moves
    across a store or atomic, another load, a compound statement, or a
    statement that reads or writes its target; loads feeding nl.dot keep their place (their layout
    is chosen by the dot). The moved statements are marked for immediate
    issue. Returns a new FunctionDef; the argument is not modified."""
    body = list(fndef.body)
    dot_names = {a.id for n in ast.walk(fndef) if _callee_name(n) == "dot"
                 for a in ast.walk(n) if isinstance(a, ast.Name)}

    def writes(st):
        out = set()
        for n in ast.walk(st):
            if isinstance(n, ast.Assign):
                for t in n.targets:
                    out |= {e.id for e in ast.walk(t) if isinstance(e, ast.Name)}
            elif isinstance(n, (ast.AugAssign, ast.AnnAssign, ast.For)):
                t = n.target
                out |= {e.id for e in ast.walk(t) if isinstance(e, ast.Name)}
        return out

    def reads(st):
        return {n.id for n in ast.walk(st) if isinstance(n, ast.Name) and isinstance(n.ctx, ast.Load)}

    def barrier_to(st):
        # loads keep their relative order (vmcnt waits are in issue order)
        return (not isinstance(st, (ast.Assign, ast.AugAssign, ast.AnnAssign, ast.Expr, ast.Pass))
                or any(_callee_name(n) in _MEM_WRITES | {"load"} for n in ast.walk(st)))

    moved = False
    out = []
    for st in body:
        is_load = (isinstance(st, ast.Assign) and len(st.targets) == 1
                   and isinstance(st.targets[0], ast.Name) and _callee_name(st.value) == "load"
                   and st.targets[0].id not in dot_names)
        if not is_load:
            out.append(st)
            continue
        tgt, need = st.targets[0].id, reads(st.value)
        pos = len(out)
        while pos > 0:
            prev = out[pos - 1]
            if barrier_to(prev) or (writes(prev) & (need | {tgt})) or tgt in reads(prev):
                break
            pos -= 1
        if pos < len(out):
            st = copy.copy(st)
            st._newt_prefetch = True
            moved = True
        out.insert(pos, st)
    if not moved:
        return fndef
    new = copy.copy(fndef)
    new.body = out
    return new


def compile_fn(fndef, fn_globals, params, constexprs, num_warps, kernel_name, num_stages=3,
               max_passes=10, waves_per_eu=0):
    """Compile a kernel. Returns (hip_source, lds_bytes).

    params: list of (name, Param) for the runtime parameters in signature order.
    waves_per_eu: 0, or the number of waves per SIMD the register allocation
    must allow (an occupancy request, as Triton's ROCm backend takes it).
    Mirrors the reference boundary compile_fn(...) -> (source, smem)
    (newt/compiler/codegen.py:2758-2765); layout hints learned by one pass are
    fed to the next until no new hint appears."""
    hints = {}
    prefer_rows = _has_row_reduction(fndef)
    chained_dots = _chained_dots(fndef)
    group_pids = _split_dot_axes(fndef)
    remap_pids = _shares_across_programs(fndef)
    lpt_pids = _work_grows_along_axis0(fndef, constexprs)
    # NEWT_NT_LOAD=1 / NEWT_NT_STREAM=1 read / write program-private streams
    # with the non-temporal hint. Measured on streaming kernels of 32-256 MB:
    # loads +2-4% under XCD-renumbered program order but 1-4% slower in the
    # hardware order these kernels now keep; stores 10-15% slower at
    # 128-256 MiB (19% faster at 32 MB). Both stay off by default.
    stream_loads = (_streamed(fndef, ("load",)) if os.environ.get("NEWT_NT_LOAD", "0") == "1"
                    else set())
    stream_stores = (_streamed(fndef, ("store",)) if os.environ.get("NEWT_NT_STREAM", "0") == "1"
                     else set())
    # off by default: on memory-bound kernels the registers held by early loads
    # cost more occupancy than the overlap gains (layernorm 4096x8192: 86 -> 109
    # VGPRs, 5 -> 4 waves per SIMD, 7% slower)
    if os.environ.get("NEWT_HOIST_LOADS", "0") == "1":
        fndef = hoist_loads(fndef)
    last = None
    for _ in range(max_passes):
        cg = Compiler(fndef, fn_globals, params, constexprs, num_warps, kernel_name,
                      num_stages=num_stages, hints=hints, waves_per_eu=waves_per_eu)
        cg.prefer_rows = prefer_rows
        cg.chained_dots = chained_dots
        cg.group_pids = group_pids
        cg.stream_loads = stream_loads
        cg.remap_pids = remap_pids
        cg.lpt_pids = lpt_pids
        cg.stream_stores = stream_stores
        try:
            src = cg.compile()
        except _Retry:
            hints.update(cg.new_hints)
            continue
        fresh = {k: v for k, v in cg.new_hints.items() if hints.get(k) != v}
        last = (src, cg.lds_total)
        if not fresh:
            return last
        hints.update(fresh)
    if last is None:
        raise CompileError(f"{fndef.name}: layout assignment did not converge")
    return last


__all__ = ["CompileError", "Param", "compile_fn", "Compiler"]
