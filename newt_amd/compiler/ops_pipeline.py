"""Software pipeline for loops whose loads feed nl.dot.

The reference stages dot operands through a cp.async ring of `num_stages`
shared-memory slots with deferred consumption (newt/compiler/codegen.py:
2279-2369, :2560-2654). This is the gfx950 design of the same idea, for any
loop whose tiles come from nl.load and go only into nl.dot (the matmul k-loop,
the K and V tiles of flash attention):

  * the loop is rotated: a prologue issues the staged tiles of the first
    num_stages-1 iterations, and iteration i issues those of iteration i+S-1
    before it computes iteration i, so global latency hides behind S-1
    iterations of work;
  * every stage is its own __shared__ array and the main loop is unrolled by S,
    so each stage is a distinct LDS object - the compiler can see that
    direct-to-LDS writes into one stage do not alias reads of another and waits
    for exactly the right loads (s_waitcnt vmcnt(N)) instead of draining all
    of them before each LDS read;
  * a tile that is contiguous along one dim, 16-byte aligned and proven in
    bounds by a uniform test is copied global -> LDS with
    global_load_lds_dwordx4 (no VGPR staging, no ds_write); other tiles
    (ragged edges, strided operands) take a register path with the masked
    loads' `other` fill, written with ds_write and hinted cold;
  * a tile is stored with its memory-contiguous dim contiguous in LDS: when
    that dim is the dot's reduction dim it is an XOR-swizzled K-major tile read
    with ds_read_b128, otherwise an R-major tile read with ds_read_b64_tr_b16
    (B of a row-major A @ B, V of attention) - nothing is transposed through
    registers;
  * operands that do not change in the loop (attention's Q) are loaded once,
    before the loop, straight into MFMA operand registers; a dot operand that
    is the fp16/bf16 cast of another dot's row-per-lane accumulator
    (attention's P) feeds the MFMA from registers, with the other operand read
    from LDS in the matching permuted k order;
  * each iteration has one barrier: after it, every wave's copies of the stage
    to be read are complete and every wave is done reading the stage about to
    be overwritten.

What is pipelined (else the loop compiles unchanged with synchronous staging):
a `for k in range(lo, hi, step)` with a positive constant step whose body has
only assignments (constexpr `if`s are resolved first) and no stores, atomics,
nested loops or early exits; a staged tile is `x = nl.load(...)` used exactly
once, as an operand of one nl.dot (directly or through nl.trans / .T), whose
pointer and mask depend only on the loop variable, loop invariants,
temporaries computed from those, and pointers advanced by a loop-invariant
increment after their last use. Advanced pointers and staged names must not be
read after the loop (the advances run S-1 iterations ahead).
"""

import ast
import os

from . import layouts as lo
from . import types as tp
from .values import Affine, Block, Const, LazyLoad, Reg, Scalar, Staged, Sym

_SIDE_EFFECTS = {"store", "atomic_add", "atomic_max", "atomic_min"}


def _callee(node):
    if not isinstance(node, ast.Call):
        return None
    f = node.func
    return f.attr if isinstance(f, ast.Attribute) else getattr(f, "id", None)


def _names_read(node):
    return {n.id for n in ast.walk(node) if isinstance(n, ast.Name) and isinstance(n.ctx, ast.Load)}


def _target(s):
    if isinstance(s, ast.Assign) and len(s.targets) == 1 and isinstance(s.targets[0], ast.Name):
        return s.targets[0].id
    if isinstance(s, (ast.AugAssign, ast.AnnAssign)) and isinstance(s.target, ast.Name):
        return s.target.id
    return None


def _targets(s):
    """Names a statement of a pipelined body assigns (a runtime `if` assigns
    those of both branches)."""
    if isinstance(s, ast.If):
        out = set()
        for x in s.body + s.orelse:
            out |= _targets(x)
        return out
    nm = _target(s)
    return {nm} if nm is not None else set()


def _operand_name(a):
    """(name, transposed) of a dot operand written `x`, `nl.trans(x)` or `x.T`."""
    trans = False
    if _callee(a) == "trans" and len(a.args) == 1:
        a, trans = a.args[0], True
    elif isinstance(a, ast.Attribute) and a.attr == "T":
        a, trans = a.value, True
    return (a.id, trans) if isinstance(a, ast.Name) else (None, trans)


def _kform(e, kinds):
    """How expression e depends on the loop variable: 'c' not at all, 'a' affinely
    (sums, differences, products with an invariant factor), 'b' as a conjunction
    of comparisons between such terms (a condition that holds on an interval of
    iterations), None in any other way. kinds maps loop-defined names to their
    form (None for names of unknown form)."""
    if isinstance(e, ast.Name):
        return kinds.get(e.id, "c")
    if isinstance(e, ast.Constant):
        return "c"
    if isinstance(e, ast.Subscript):
        f = _kform(e.value, kinds)
        return f if _kform(e.slice, kinds) == "c" else None
    if isinstance(e, (ast.Tuple, ast.Slice)):
        parts = [p for p in ast.iter_child_nodes(e) if isinstance(p, ast.expr)]
        return "c" if all(_kform(p, kinds) == "c" for p in parts) else None
    if isinstance(e, ast.UnaryOp):
        f = _kform(e.operand, kinds)
        if isinstance(e.op, (ast.USub, ast.UAdd)) and f != "b":
            return f
        return "c" if f == "c" else None
    if isinstance(e, ast.BinOp):
        fl, fr = _kform(e.left, kinds), _kform(e.right, kinds)
        if fl is None or fr is None:
            return None
        if fl == "c" and fr == "c":
            return "c"
        if isinstance(e.op, ast.BitAnd):
            return "b" if {fl, fr} <= {"b", "c"} else None
        if "b" in (fl, fr):
            return None
        if isinstance(e.op, (ast.Add, ast.Sub)):
            return "a"
        if isinstance(e.op, ast.Mult) and "c" in (fl, fr):
            return "a"
        return None
    if isinstance(e, ast.Compare):
        forms = [_kform(x, kinds) for x in [e.left] + list(e.comparators)]
        if all(f == "c" for f in forms):
            return "c"
        if (len(e.ops) == 1 and isinstance(e.ops[0], (ast.Lt, ast.LtE, ast.Gt, ast.GtE))
                and all(f in ("a", "c") for f in forms)):
            return "b"
        return None
    if isinstance(e, ast.BoolOp) and isinstance(e.op, ast.And):
        forms = [_kform(x, kinds) for x in e.values]
        if all(f == "c" for f in forms):
            return "c"
        return "b" if all(f in ("b", "c") for f in forms) else None
    if isinstance(e, (ast.Call, ast.Attribute)):
        parts = [p for p in ast.walk(e) if isinstance(p, ast.Name)]
        return "c" if all(kinds.get(p.id, "c") == "c" for p in parts) else None
    return None


class DotPipeline:
    # ------------------------------------------------------------ detection
    def _const_test(self, test):
        """Compile-time value of a constexpr `if` test, or None."""
        if isinstance(test, ast.Constant):
            return bool(test.value)
        if isinstance(test, ast.Name):
            v = self.locals.get(test.id)
            if isinstance(v, Const) and test.id not in self.storages:
                return bool(v.pyval)
            return None
        if isinstance(test, ast.UnaryOp) and isinstance(test.op, ast.Not):
            v = self._const_test(test.operand)
            return None if v is None else not v
        return None

    def _branch_ok(self, stmts):
        """A runtime `if` inside a pipelined body holds plain assignments (and
        such `if`s) only: no load, dot or side effect, so the stages' copies
        and the dots' operands never depend on the branch taken."""
        for s in stmts:
            if isinstance(s, ast.If):
                if not (self._branch_ok(s.body) and self._branch_ok(s.orelse)):
                    return False
            elif isinstance(s, (ast.Assign, ast.AugAssign, ast.AnnAssign)):
                if _target(s) is None or getattr(s, "value", None) is None:
                    return False
            elif not isinstance(s, ast.Pass):
                return False
            if any(_callee(n) in _SIDE_EFFECTS | {"load", "dot"} for n in ast.walk(s)):
                return False
        return True

    def _flatten(self, stmts):
        out = []
        for s in stmts:
            if isinstance(s, ast.If):
                v = self._const_test(s.test)
                if v is None:
                    # a runtime branch stays one statement of the body
                    if not self._branch_ok([s]):
                        return None
                    out.append(s)
                    continue
                sub = self._flatten(s.body if v else s.orelse)
                if sub is None:
                    return None
                out += sub
            elif isinstance(s, (ast.Assign, ast.AugAssign, ast.AnnAssign)):
                if _target(s) is None or getattr(s, "value", None) is None:
                    return None
                out.append(s)
            elif isinstance(s, ast.Pass):
                continue
            else:
                return None
        return out

    def pipeline_plan(self, node):
        if self.num_stages < 2 or os.environ.get("NEWT_PIPELINE_DOT", "1") == "0":
            return None
        if self.hints.get(("nopipe", node.lineno)):
            return None
        flat = self._flatten(node.body)
        if not flat:
            return None
        kname = node.target.id
        for s in flat:
            if any(_callee(n) in _SIDE_EFFECTS for n in ast.walk(s)):
                return None
        assigned = {}
        for i, s in enumerate(flat):
            for nm in _targets(s):
                assigned.setdefault(nm, []).append(i)
        if kname in assigned:
            return None
        # names the body computes from a dot result (directly or through others)
        dot_fed = set()
        for s in flat:
            nm = _target(s)
            if nm is not None and (any(_callee(n) == "dot" for n in ast.walk(s))
                                   or _names_read(s) & dot_fed):
                dot_fed.add(nm)
        uses = {}
        acc_fed = set()
        for s in flat:
            for n in ast.walk(s):
                if _callee(n) != "dot":
                    continue
                args = list(n.args)[:2]
                for role, a in zip(("A", "B"), args):
                    nm, trans = _operand_name(a)
                    if nm is not None:
                        uses.setdefault(nm, []).append((role, trans))
                        if role == "B" and len(args) == 2 and _names_read(args[0]) & dot_fed:
                            acc_fed.add(nm)
        reads = {}
        for s in flat:
            for n in ast.walk(s):
                if isinstance(n, ast.Name) and isinstance(n.ctx, ast.Load):
                    reads[n.id] = reads.get(n.id, 0) + 1

        def invariant(nm):
            return nm not in assigned and nm != kname

        # pointers advanced by a loop-invariant increment after their last read
        carried = set()
        for nm, idx in assigned.items():
            if len(idx) != 1 or not isinstance(flat[idx[0]], ast.AugAssign):
                continue
            s = flat[idx[0]]
            if not all(invariant(r) for r in _names_read(s.value)):
                continue
            if any(nm in _names_read(t) for t in flat[idx[0] + 1:]):
                continue
            if nm in self.locals or nm in self.storages:
                carried.add(nm)
        # temporaries that are pure functions of the loop variable and invariants
        konly = set()
        for s in flat:
            nm = _target(s)
            if nm is None or nm in carried or len(assigned[nm]) != 1 or not isinstance(s, ast.Assign):
                continue
            if any(_callee(n) in ("load", "dot") for n in ast.walk(s.value)):
                continue
            if all(r == kname or invariant(r) or r in konly or r in carried
                   for r in _names_read(s.value)):
                konly.add(nm)
        staged = {}
        for i, s in enumerate(flat):
            nm = _target(s)
            if not (isinstance(s, ast.Assign) and _callee(s.value) == "load"):
                continue
            if len(assigned[nm]) != 1 or len(uses.get(nm, [])) != 1 or reads.get(nm) != 1:
                continue
            if nm in self.locals or nm in self.storages:
                continue
            if not all(r == kname or invariant(r) or r in konly or r in carried
                       for r in _names_read(s.value)):
                continue
            role, trans = uses[nm][0]
            # reduction dim of the tile as loaded: A [M,K] -> 1, B [K,N] -> 0
            kdim = (1 if role == "A" else 0) ^ (1 if trans else 0)
            staged[nm] = {"name": nm, "index": i, "kdim": kdim, "acc_fed": nm in acc_fed}
        if not staged:
            return None
        # the statements computing the staged tiles' pointers and masks
        need = set()
        for rec in staged.values():
            need |= _names_read(flat[rec["index"]].value)
        slice_idx = set(rec["index"] for rec in staged.values())
        changed = True
        while changed:
            changed = False
            for i, s in enumerate(flat):
                nm = _target(s)
                if nm in konly and nm in need and i not in slice_idx:
                    slice_idx.add(i)
                    need |= _names_read(s.value)
                    changed = True
        # advanced pointers may only be read by the slice
        for nm in sorted(carried):
            readers = [i for i, s in enumerate(flat) if nm in _names_read(s)
                       and i != assigned[nm][0]]
            if any(i not in slice_idx for i in readers):
                return None
        if (carried | set(staged)) & self._read_after():
            return None
        # temporaries of the loop are recomputed each iteration, so they must
        # not be defined before it
        if any(t in self.locals or t in self.storages for t in konly):
            return None
        # form of each staged mask in the loop variable: conjunctions of affine
        # comparisons hold on an interval of iterations, which lets the loop be
        # versioned on a test of its first and last iterations
        kinds = {kname: "a"}
        for nm in carried:
            kinds[nm] = None
        for s in flat:
            nm = _target(s)
            if nm in konly:
                kinds[nm] = _kform(s.value, kinds)
        fast_ok = True
        for rec in staged.values():
            call = flat[rec["index"]].value
            masks = [k.value for k in call.keywords if k.arg == "mask"] + list(call.args[1:2])
            if any(_kform(m, kinds) not in ("b", "c") for m in masks):
                fast_ok = False
        # where() masks of the loop body whose condition is also such a
        # conjunction (bounds and causal masks): the branch-free copy can run
        # only iterations where they are all-true and select without them
        advance_idx = set(assigned[nm][0] for nm in carried)
        staged_idx = set(rec["index"] for rec in staged.values())
        wheres, wneed = [], set()
        for i, st_ in enumerate(flat):
            if i in slice_idx or i in advance_idx or i in staged_idx:
                continue
            for nd in ast.walk(st_):
                if (_callee(nd) == "where" and len(nd.args) == 3 and not nd.keywords
                        and _kform(nd.args[0], kinds) == "b"):
                    wheres.append(nd)
                    wneed |= _names_read(nd.args[0])
        where_deps = set()
        changed = True
        while changed:
            changed = False
            for i, st_ in enumerate(flat):
                nm = _target(st_)
                if nm in konly and nm in wneed and i not in where_deps:
                    where_deps.add(i)
                    wneed |= _names_read(st_.value)
                    changed = True
        return {"flat": flat, "staged": staged, "slice": sorted(slice_idx),
                "advance": sorted(advance_idx), "konly": konly,
                "kname": kname, "node": node, "fast_ok": fast_ok,
                "wheres": wheres, "where_deps": sorted(where_deps)}

    # ----------------------------------------------------------- emission
    def pipelined_for(self, node, plan, lo_, hi, st, idt):
        S = int(self.hints.get(("pipe_stages", node.lineno), self.num_stages))
        flat, staged, kname = plan["flat"], plan["staged"], plan["kname"]
        slice_stmts = [flat[i] for i in plan["slice"]]
        advance = [flat[i] for i in plan["advance"]]
        skip = set(plan["advance"]) | set(rec["index"] for rec in staged.values())
        temps = plan["konly"] | set(staged) | {kname}
        stv = int(st.pyval)
        lo_e = self.scalar_expr(lo_, idt)
        hi_e = self.scalar_expr(hi, idt)
        n = self.new_scalar(idt, f"((({hi_e}) > ({lo_e})) ? ((({hi_e}) - ({lo_e}) + {stv - 1}) "
                                 f"/ {stv}) : 0)")
        state = {"node": node, "S": S, "recs": None, "plan": plan}
        compute = [x for i, x in enumerate(flat) if i not in skip and i not in plan["slice"]]
        ndots = sum(1 for x in compute for nd in ast.walk(x) if _callee(nd) == "dot")
        # a k-loop that only accumulates one dot (matmul) reads the first k-step
        # of the next stage's operands into registers before the barrier
        simple = len(compute) == 1 and ndots == 1
        plr_env = os.environ.get("NEWT_PLR", "auto")
        state["plr"] = S >= 3 and (plr_env == "1" or (plr_env == "auto" and simple))
        state["simple"] = simple
        # a loop body with a dot and an exponential (flash attention) takes
        # LLVM's exp/MFMA interleave strategy in its branch-free copy
        state["exp_mix"] = ndots > 0 and any(_callee(nd) in ("exp", "exp2")
                                             for x in compute for nd in ast.walk(x))
        state["pf"] = {}
        self.pipe_records.append(state)
        for s in range(S - 1):
            self.locals[kname] = self.new_scalar(idt, f"({lo_e} + {s * stv})")
            self.visit_body(slice_stmts)
            self.pipe_issue(state, s, f"({s} < {n.expr})")
            self.visit_body(advance)
            for t in temps:
                self.locals.pop(t, None)
        self.pipe_hoist_operands(state)
        rec = self._enter_compound(node)
        self.drain_dots_for_loop(node)
        it0 = self.fresh("it")
        self.emit(f"{idt.ctype} {it0} = 0;")
        mark = len(self.lines)
        ctx = (node, state, S, n, lo_e, stv, idt, slice_stmts, advance, skip, temps, kname, flat)
        state["clamp"] = os.environ.get("NEWT_PIPE_CLAMP", "1") != "0"
        state["clamp_n"] = n
        if plan["fast_ok"] and os.environ.get("NEWT_PIPE_VERSION", "1") != "0":
            state["fast_emitted"] = True
            # leading iterations whose every tile is a whole in-bounds copy run
            # in a copy of the loop with no per-iteration tests at all; its
            # copies take the buffer form (32-bit lane offsets) when every
            # tile's lane offsets fit, which joins the entry test
            state["bufdma"] = os.environ.get("NEWT_BUFFER_DMA", "1") != "0"
            nf = self._fast_count(ctx)
            self.emit(f"for (; {it0} + {2 * S - 2} < {nf.expr}; {it0} += {S}) {{")
            self._pipe_iterations(ctx, it0, fast=True)
            self.emit("}")
            if state["clamp"]:
                # when every iteration is fast, one more branch-free trip runs
                # S of the last iterations: its copies past the end repeat the
                # last tile into stages no iteration reads again, so every
                # sub-iteration keeps the same copies in flight and the same
                # waits (the general loop ran these ~1.5x slower). The loop
                # above stays as it was: clamping there lengthened the scalar
                # work ahead of every copy.
                self.emit(f"if ((({nf.expr}) == ({n.expr})) && {it0} + {S - 1} < {n.expr}) {{")
                state["clamp_trip"] = True
                self._pipe_iterations(ctx, it0, fast=True)
                state["clamp_trip"] = False
                self.emit(f"  {it0} += {S};")
                self.emit("}")
        self.emit(f"for (; {it0} < {n.expr}; {it0} += {S}) {{")
        self._pipe_iterations(ctx, it0, fast=False)
        self.emit("}")
        if state.get("clamp") and state.get("fast_emitted"):
            # repeated copies may still be in flight: drain them before the
            # stages' LDS is reused or the workgroup ends
            self.emit("newt::wait_vmcnt<0>();")
        if state["plr"]:
            self._insert_lines(mark, self._plr_preamble(state, n))
        self._exit_compound(rec)
        self.end_loop_target(node)
        self.after_loop(node)
        if state["recs"] is not None:
            self.lds_pool.extend(state["lds_idx"])

    def _insert_lines(self, index, lines):
        ind = "  " * self.indent
        self.lines[index:index] = [ind + ln for ln in lines]
        for r in self.pending_hoist:
            if r["index"] >= index:
                r["index"] += len(lines)

    def _plr_preamble(self, state, n):
        """Declarations of the prefetched fragments and their first fill from
        stage 0, once iterations 0 and 1 have landed."""
        S, ops = state["S"], state["ops"]
        out = []
        for d, frags in sorted(state["pf"].items()):
            for var, _ in frags:
                out.append(f"i16x8 {var};")
        deep = (S - 3) * ops
        if deep:
            out.append(f"if ({S - 2} < {n.expr}) newt::wait_vmcnt<{deep}>(); else newt::wait_vmcnt<0>();")
        else:
            out.append("newt::wait_vmcnt<0>();")
        out.append("__syncthreads();")
        for d, frags in sorted(state["pf"].items()):
            for var, fn in frags:
                out.append(f"{var} = {fn(0)};")
        return out

    def _plr_fill(self, state, slot):
        for d, frags in sorted(state["pf"].items()):
            for var, fn in frags:
                self.emit(f"{var} = {fn(slot)};")

    def _sched_hints(self, state):
        """Interleave, in the straight-line fast loop, each k-step's MFMAs with
        the LDS reads of the next k-step (the last k-step with the prefetch of
        the next stage) and the first k-step's MFMAs with the stage copies."""
        info = state.get("sched")
        if not info:
            return
        reads, mfmas = info["reads"], info["mfmas"]
        nks = len(reads)
        fills = []
        for t in range(nks):
            f = [("0x100", 1)] * (reads[t + 1] if t + 1 < nks else reads[0])
            if t == 0:
                dma = [("0x020", 1)] * state["ops"]
                # alternate copies and reads so neither queue starves
                mixed = []
                while f or dma:
                    if dma:
                        mixed.append(dma.pop(0))
                    if f:
                        mixed.append(f.pop(0))
                f = mixed
            fills.append(f)
        # the fill items of a k-step are spaced evenly over its MFMAs (item j
        # after MFMA j * m / n): with one 32-deep k-step per stage the 64
        # MFMAs of a 128x128 wave tile carry 8 copies and 24 fragment reads,
        # and packing them one per MFMA into the first half measured ~2% slower
        for t in range(nks):
            f = fills[t]
            m = mfmas[t]
            slots = [[] for _ in range(m)]
            for j, item in enumerate(f):
                slots[min(m - 1, j * m // len(f))].append(item)
            for i in range(m):
                self.emit("__builtin_amdgcn_sched_group_barrier(0x008, 1, 0);")
                for mask, cnt in slots[i]:
                    self.emit(f"__builtin_amdgcn_sched_group_barrier({mask}, {cnt}, 0);")

    def _fast_count(self, ctx):
        """Number of leading iterations j (from 0) whose DMA tiles are all
        whole, in-bounds copies. Each such condition is a conjunction of
        comparisons affine in j, so it holds on an interval: it holds for every
        j < m+1 when it holds at j = 0 and at j = m. m = n-1 covers divisible
        loops, m = n-2 a ragged last tile; otherwise no iteration is fast."""
        node, state, S, n, lo_e, stv, idt, slice_stmts, advance, skip, temps, kname, flat = ctx
        if state["plan"]["wheres"] and os.environ.get("NEWT_WHERE_VERSION", "1") != "0":
            return self._fast_prefix(ctx)
        conds = []
        for j in ("0", f"({n.expr} - 1)", f"({n.expr} - 2)"):
            self.locals[kname] = self.new_scalar(idt, f"({lo_e} + {j} * {stv})")
            self.visit_body(slice_stmts)
            conds.append(self.pipe_dma_condition(state))
            for t in temps:
                self.locals.pop(t, None)
        c0, c1, c2 = conds
        return self.new_scalar(idt, f"(({c0}) ? (({c1}) ? {n.expr} : (({c2}) ? ({n.expr} - 1) : 0)) : 0)")

    def _fast_prefix(self, ctx):
        """Number of leading iterations j in which every DMA tile is a whole
        in-bounds copy and every versioned where() mask is all-true. Each
        condition is a conjunction of comparisons affine in j, so the set of
        iterations where all of them hold is an interval; when it holds at
        j = 0 that interval is a prefix, whose length a binary search finds
        (a causal mask ends it at the diagonal, not at the last iteration).
        Records which where() masks the branch-free copy may drop."""
        node, state, S, n, lo_e, stv, idt, slice_stmts, advance, skip, temps, kname, flat = ctx
        plan = state["plan"]
        in_slice = set(plan["slice"])
        deps = [flat[i] for i in plan["where_deps"] if i not in in_slice]
        dep_names = {_target(x) for x in deps}

        def cond_at(j):
            self.locals[kname] = self.new_scalar(idt, f"({lo_e} + ({j}) * {stv})")
            self.visit_body(slice_stmts)
            parts = [self.pipe_dma_condition(state)]
            self.visit_body(deps)
            proven = []
            for nd in plan["wheres"]:
                v = self.visit_expr(nd.args[0])
                full = self.mask_all_true(v, v.shape) if isinstance(v, Block) else None
                if full is not None and full != "false":
                    parts.append(f"({full})")
                    proven.append(id(nd))
            for t in temps | dep_names:
                self.locals.pop(t, None)
            return " && ".join(p for p in parts if p != "true") or "true", proven

        c0, proven = cond_at("0")
        state["true_wheres"] = set(proven)
        fm, lo, hi, mid = (self.fresh(x) for x in ("fm", "lo", "hi", "mid"))
        self.emit(f"int {fm} = 0;")
        self.emit(f"if ({n.expr} > 0 && ({c0})) {{")
        self.indent += 1
        self.emit(f"int {lo} = 1, {hi} = {n.expr};")
        self.emit(f"while ({lo} < {hi}) {{")
        self.indent += 1
        self.emit(f"const int {mid} = ({lo} + {hi}) >> 1;")
        cm, _ = cond_at(mid)
        self.emit(f"if ({cm}) {lo} = {mid} + 1; else {hi} = {mid};")
        self.indent -= 1
        self.emit("}")
        self.emit(f"{fm} = {lo};")
        self.indent -= 1
        self.emit("}")
        return Scalar(idt, fm, Sym(fm, None, 1))

    def pipe_dma_condition(self, state):
        """Uniform condition under which every DMA tile of the slice just
        visited is a whole in-bounds copy; consumes the slice's loads."""
        if state["recs"] is None:
            self._init_recs(state)
        conds = []
        for r in state["recs"].values():
            X = self.locals.get(r["name"])
            if not isinstance(X, LazyLoad) or X.result is not None or tuple(X.shape) != r["shape"]:
                self._no_pipe(state)
            if r["dma"]:
                full = self.mask_all_true(X.mask, X.shape)
                if full is not None and full != "true":
                    conds.append(f"({full})")
                if full is not None and state.get("bufdma"):
                    V = X if r["kdim"] == 1 else self.permute(X, (1, 0))
                    conds.append(f"({self._lane_bytes_fit(V, r['R'], r['K'], r['dt'])})")
                    if V is not X:
                        V.consumed = True
                        if V in self.pending_loads:
                            self.pending_loads.remove(V)
            X.consumed = True
            if X in self.pending_loads:
                self.pending_loads.remove(X)
        return " && ".join(conds) if conds else "true"

    def _pipe_iterations(self, ctx, it0, fast):
        """One trip of the main loop: S sub-iterations, sub-iteration s computing
        from stage s and issuing iteration it+S-1 into stage (s+S-1)%S. In the
        fast copy every sub-iteration is known to run, to wait for exactly the
        copies of S-2 later iterations, and to issue whole in-bounds tiles."""
        node, state, S, n, lo_e, stv, idt, slice_stmts, advance, skip, temps, kname, flat = ctx
        self.indent += 1
        self.loop_depth += 1
        ops = state["ops"]
        self.pipe_active = state
        plr = state["plr"]
        state["fast"] = fast
        for s in range(S):
            it = f"({it0} + {s})"
            if s and not fast:
                self.emit(f"if ({it} >= {n.expr}) break;")
            # with prefetching, iteration it+1 must also have landed: its first
            # k-step is read before the next barrier
            deep = (S - 3 if plr else S - 2) * ops
            if deep and fast:
                self.emit(f"newt::wait_vmcnt<{deep}>();")
            elif deep:
                self.emit(f"if ({it} + {S - 2} < {n.expr}) newt::wait_vmcnt<{deep}>(); "
                          f"else newt::wait_vmcnt<0>();")
            else:
                self.emit("newt::wait_vmcnt<0>();")
            if fast and os.environ.get("NEWT_BARE_BARRIER", "0") == "1":
                self.emit("newt::barrier_nofence();")
            else:
                self.emit("__syncthreads();")
            self.emit("__builtin_amdgcn_sched_barrier(0);")
            if fast and state["exp_mix"] and os.environ.get("NEWT_IGLP", "1") != "0":
                self.emit("__builtin_amdgcn_iglp_opt(2);")
            # issue iteration it+S-1 into the stage that iteration it-1 read
            issue = f"({it} + {S - 1})"
            clamp = fast and state.get("clamp_trip", False)
            if clamp:
                # past the last iteration the branch-free copy repeats the last
                # tile, and the carried pointers stay on it
                last = f"({n.expr} - 1)"
                self.locals[kname] = self.new_scalar(
                    idt, f"({lo_e} + (({issue} < {last}) ? {issue} : {last}) * {stv})")
            else:
                self.locals[kname] = self.new_scalar(idt, f"({lo_e} + {issue} * {stv})")
            self.visit_body(slice_stmts)
            self.pipe_issue(state, (s + S - 1) % S, f"({issue} < {n.expr})", fast=fast)
            if clamp and advance:
                self.emit(f"if ({issue} < {n.expr} - 1) {{")
                self.indent += 1
                self.visit_body(advance)
                self.indent -= 1
                self.emit("}")
            else:
                self.visit_body(advance)
            for t in temps:
                self.locals.pop(t, None)
            # compute iteration it from stage s
            self.locals[kname] = self.new_scalar(idt, f"({lo_e} + {it} * {stv})")
            for nm, r in state["recs"].items():
                self.locals[nm] = Staged(r, s)
            state["pf_d"] = 0
            state["sched"] = None
            self.visit_body([x for i, x in enumerate(flat) if i not in skip])
            for t in temps:
                self.locals.pop(t, None)
            if plr:
                self._plr_fill(state, (s + 1) % S)
            if fast and state["simple"] and os.environ.get("NEWT_SCHED", "1") != "0":
                self._sched_hints(state)
        self.pipe_active = None
        self.flush_loads()
        self.loop_backedge(node)
        self.loop_depth -= 1
        self.indent -= 1

    def _no_pipe(self, state):
        self.new_hints[("nopipe", state["node"].lineno)] = True
        from .codegen import _Retry
        raise _Retry()

    # --------------------------------------------------------------- staging
    def _tile_format(self, X, kdim):
        """LDS format of a staged tile: 'k' when its unit-stride dim is the
        reduction dim (or neither dim is unit-stride), 'r' when it is the row
        dim."""
        off = X.ptr.offset
        R = X.shape[1 - kdim]
        K = X.shape[kdim]
        if isinstance(off, Affine):
            ck, cr = off.coefs.get(kdim), off.coefs.get(1 - kdim)
            if ck is not None and ck.is_const and ck.const == 1 and K % 8 == 0:
                return "k"
            if cr is not None and cr.is_const and cr.const == 1 and R % 32 == 0:
                return "r"
        return "k"

    def _dma_ok(self, X, fmt, R, K, dt):
        """Compile-time conditions for global_load_lds of whole 16-byte chunks
        (X is the [R, K] view)."""
        off = X.ptr.offset
        if not isinstance(off, Affine) or not X.ptr.base.aligned16:
            return False
        epc = 16 // dt.itemsize
        cdim, odim = (1, 0) if fmt == "k" else (0, 1)
        c, o = off.coefs.get(cdim), off.coefs.get(odim)
        if c is None or not c.is_const or c.const != 1:
            return False
        if (R if fmt == "r" else K) % epc:
            return False
        if o is not None and off.shape[odim] > 1 and o.div % epc:
            return False
        if off.base.div % epc:
            return False
        return (R * K // epc) % self.T == 0

    def _r_tile_swizzle_bit(self, info, fmt, R, K, dt):
        """Swizzle bit of a 16-bit R-major tile: 2 when its dot will most
        likely read it with the accumulator-ordered 16-row fragments (a B
        operand whose A is computed from another dot's result in a
        row-oriented kernel, with 16x16x32 MFMAs), else 3. Writer and readers
        both take it from the record, so the guess only affects bank
        conflicts, never results."""
        if fmt != "r" or dt == tp.float32 or not info.get("acc_fed") or self.dot_orient() != "row":
            return 3
        return 2 if self.pick_instr(32, R, K, dt) == "16x16x32" else 3

    def _init_recs(self, state):
        recs = {}
        off = 0
        ops = 0
        for nm, info in sorted(state["plan"]["staged"].items(), key=lambda kv: kv[1]["index"]):
            X = self.locals.get(nm)
            if not isinstance(X, LazyLoad) or X.result is not None or len(X.shape) != 2:
                self._no_pipe(state)
            dt = X.dtype
            if dt not in (tp.float16, tp.bfloat16, tp.float32):
                self._no_pipe(state)
            kdim = info["kdim"]
            V = X if kdim == 1 else self.permute(X, (1, 0))   # [R, K] view
            R, K = V.shape
            if K % (8 if dt == tp.float32 else 16) or R % 16:
                self._no_pipe(state)
            fmt = self._tile_format(X, kdim)
            if dt == tp.float32:
                # fp32 fragments are read four k at a time (fragment prefetch
                # holds 16-bit fragments only); R-major fp32 tiles need >= 64 rows
                state["plr"] = False
                if fmt == "r" and R % 64:
                    self._no_pipe(state)
            nbytes = self.tile_bytes(R, K, dt)
            dma = self._dma_ok(V, fmt, R, K, dt) and os.environ.get("NEWT_LDS_DMA", "1") != "0"
            epc = 16 // dt.itemsize
            if dma:
                ops += R * K // epc // self.T
            recs[nm] = {"name": nm, "shape": tuple(X.shape), "dt": dt, "kdim": kdim, "R": R,
                        "K": K, "fmt": fmt, "off": off, "dma": dma,
                        "sb": self._r_tile_swizzle_bit(info, fmt, R, K, dt)}
            off += (nbytes + 15) // 16 * 16
            if V is not X:
                V.consumed = True
                if V in self.pending_loads:
                    self.pending_loads.remove(V)
        # stage arrays of a pipelined loop that has finished are reused (a
        # later loop never needs them at the same time); a barrier first lets
        # every wave finish reading them before this loop's copies land. A loop
        # nested in another rewrites its stages on each outer trip: same barrier
        names, idx = [], []
        reused = False
        for _ in range(state["S"]):
            if self.lds_pool:
                i = self.lds_pool.pop(0)
                nm, sz = self.lds_arrays[i]
                self.lds_arrays[i] = (nm, max(sz, off))
                reused = True
            else:
                i = len(self.lds_arrays)
                nm = f"_ldsP{i}"
                self.lds_arrays.append((nm, off))
            names.append(nm)
            idx.append(i)
        if reused or self.loop_depth > 0:
            self.emit("__syncthreads();")
        state.update(recs=recs, ops=ops, names=names, lds_idx=idx)

    def pipe_issue(self, state, slot, valid, fast=False):
        if state["recs"] is None:
            self._init_recs(state)
        base = state["names"][slot]
        # register-path tiles first: their (synchronous) loads must not drain
        # the asynchronous copies issued for this stage
        order = sorted(state["recs"].values(), key=lambda r: (r["dma"], r["off"]))
        self.emit("{")
        self.indent += 1
        for r in order:
            X = self.locals.get(r["name"])
            if not isinstance(X, LazyLoad) or X.result is not None or tuple(X.shape) != r["shape"]:
                self._no_pipe(state)
            V = X if r["kdim"] == 1 else self.permute(X, (1, 0))
            dt, R, K, fmt = r["dt"], r["R"], r["K"], r["fmt"]
            tile = f"(({dt.ctype}*)({base} + {r['off']}))"
            full = self.mask_all_true(X.mask, X.shape) if r["dma"] else None
            if r["dma"] and full is not None and fast:
                self._dma_stage(V, base, r["off"], fmt, R, K, dt, buffer=state.get("bufdma", False),
                                sb=r["sb"])
            elif fast:
                self._reg_stage(V, tile, fmt, R, K, dt, sb=r["sb"])
            elif r["dma"] and full is not None:
                cond = valid if full == "true" else f"{valid} && ({full})"
                # the in-bounds copy is the hot path; the hint moves the masked
                # register path out of the loop's straight-line code
                self.emit(f"if (__builtin_expect({cond}, 1)) {{")
                self.indent += 1
                self._dma_stage(V, base, r["off"], fmt, R, K, dt, sb=r["sb"])
                self.indent -= 1
                if full != "true":
                    self.emit(f"}} else if ({valid}) {{")
                    self.indent += 1
                    self._reg_stage(V, tile, fmt, R, K, dt, sb=r["sb"])
                    self.indent -= 1
                self.emit("}")
            else:
                self.emit(f"if ({valid}) {{")
                self.indent += 1
                self._reg_stage(V, tile, fmt, R, K, dt, sb=r["sb"])
                self.indent -= 1
                self.emit("}")
            for ld in (X, V):
                ld.consumed = True
                if ld in self.pending_loads:
                    self.pending_loads.remove(ld)
        self.indent -= 1
        self.emit("}")

    def _lane_bytes_fit(self, V, R, K, dt):
        """Uniform condition under which every lane's part of a DMA tile's
        offset (c0 * r + c1 * k over the [R, K] view, without the tile's
        uniform start) is a non-negative byte count below 2^31, as the buffer
        form of the copy needs."""
        off = V.ptr.offset
        parts, conds = [], []
        for c, ext in ((off.coefs.get(0), R - 1), (off.coefs.get(1), K - 1)):
            if c is None:
                continue
            if c.is_const:
                if c.const < 0:
                    return "false"
                parts.append(f"{c.const * ext}LL")
            else:
                conds.append(f"({c.expr}) >= 0")
                parts.append(f"(long long)({c.expr}) * {ext}")
        conds.append(f"({' + '.join(parts) if parts else '0LL'}) < {(1 << 31) // dt.itemsize}LL")
        return " && ".join(conds)

    def _dma_stage(self, X, base, boff, fmt, R, K, dt, buffer=False, sb=3):
        """Direct-to-LDS copies of one [R, K] tile. buffer: the branch-free
        fast loop's form, a scalar descriptor on the tile's uniform start and
        a 32-bit lane offset (the entry test guarantees it fits)."""
        off = X.ptr.offset
        T = dt.ctype
        epc = 16 // dt.itemsize
        rounds = R * K // epc // self.T
        c0, c1 = off.coefs.get(0), off.coefs.get(1)
        gb = X.ptr.base.expr
        for i in range(rounds):
            self.emit("{")
            self.indent += 1
            self.emit(f"const int _s = {i * self.T} + _tid;")
            self.emit("int _r, _k;")
            if fmt == "k":
                self.emit(f"newt::lds_tile_slot<{T}, {K}>(_s, _r, _k);")
            elif dt == tp.float32:
                self.emit(f"newt::LdsTileR32<{R}>::slot(_s, _k, _r);")
            else:
                self.emit(f"newt::LdsTileR<{T}, {R}, {sb}>::slot(_s, _k, _r);")
            ubase = None if (off.base.is_const and off.base.const == 0) else off.base.expr
            lane = []
            for c, v in ((c0, "_r"), (c1, "_k")):
                if c is None:
                    continue
                lane.append(v if c.is_const and c.const == 1 else f"{c.expr} * {v}")
            dst = f"(void*)({base} + {boff} + {16 * i * self.T} + _wave * 1024)"
            if buffer:
                tb = f"({gb} + ({ubase}))" if ubase else gb
                lb = f"(unsigned)(({' + '.join(lane) if lane else '0'}) * {dt.itemsize})"
                self.emit(f"newt::lds_dma16_buf({tb}, {lb}, {dst});")
            else:
                terms = ([ubase] if ubase else []) + lane
                gaddr = f"({gb} + {' + '.join(terms) if terms else '0'})"
                self.emit(f"newt::lds_dma16({gaddr}, {dst});")
            self.indent -= 1
            self.emit("}")

    def _reg_stage(self, X, tile, fmt, R, K, dt, sb=3):
        if fmt == "k":
            L = self.staging_layout(X)
        else:
            v = 16 // dt.itemsize
            L = lo.blocked((K, R), self.W, min(v, R)).permute((1, 0))
        r = self.emit_load(X, L)
        if r.dtype != dt:
            r = self.to_reg(r, r.layout, dt)
        self.write_tile_to(r, tile, dt, fmt, sb)

    def write_tile_to(self, r, tile, dt, fmt, sb=3):
        """Write register block r ([R, K] view) into an LDS tile of format fmt
        (sb: swizzle bit of a 16-bit R-major tile)."""
        L = r.layout
        R, K = L.shape
        T = dt.ctype
        epc = 16 // dt.itemsize
        cdim = 1 if fmt == "k" else 0
        kb = 0
        while kb < len(L.reg) and L.reg[kb] == (cdim, kb):
            kb += 1
        chunk = max(1, min(1 << kb, epc))
        canon = self.canon_cond(L)
        if canon:
            self.emit(f"if ({canon}) {{")
            self.indent += 1
        for s in range(0, L.nslots, chunk):
            if not L.slot_is_canonical(s):
                continue
            rr = self.coord(L, 0, s)
            kk = self.coord(L, 1, s)
            o = (f"newt::LdsTile<{T}, {K}>::off({rr}, {kk})" if fmt == "k"
                 else f"newt::LdsTileR32<{R}>::off({kk}, {rr})" if dt == tp.float32
                 else f"newt::LdsTileR<{T}, {R}, {sb}>::off({kk}, {rr})")
            if chunk > 1:
                self.emit(f"newt::store_vec<{T}, {chunk}>({tile} + {o}, {r.var} + {s});")
            else:
                self.emit(f"{tile}[{o}] = {r.at(s)};")
        if canon:
            self.indent -= 1
            self.emit("}")

    def _staged_dot_f32(self, node, a, b, acc, M, N, K, instr, wm, wn, rep, state):
        """fp32 nl.dot from pipeline stages on the 32x32x2 MFMA. Within each
        group of 8 k, MFMA t contracts k = kk + t (lanes 0-31) and kk + 4 + t
        (lanes 32-63): a lane's four k of one row are contiguous, one 16-byte
        read of a K-major tile (four 4-byte reads of an R-major one) feeds four
        MFMAs, and both operands use the same order."""
        if rep > 1 or instr != "32x32x2" or K % 8:
            self._no_pipe(state)
        Bt = Staged(b.rec, b.slot, not b.trans) if isinstance(b, Staged) else None
        if not isinstance(a, Staged) or Bt is None:
            self._no_pipe(state)
        Lc = self.mfma_layout(M, N, instr, wm, wn, 1)
        RM, RN = M // wm // 32, N // wn // 32
        orient = self.dot_orient()
        accv = self.init_acc(node, acc, Lc, M, N)
        self.emit("{")
        self.indent += 1
        self.emit(f"const int _ra = (_wave & {wm - 1}) * {M // wm};")
        self.emit(f"const int _rb = ((_wave >> {lo.log2i(wm)}) & {wn - 1}) * {N // wn};")
        self.emit("const int _kh = 4 * (_lane >> 5);")
        tiles = []
        for idx, X in enumerate((a, Bt)):
            nm = f"_pt{idx}"
            self.emit(f"const float* {nm} = (const float*)({state['names'][X.slot]} + "
                      f"{X.rec['off']});")
            tiles.append(nm)

        def group(idx, X, r0, kk):
            # the record describes the tile's [R, K] view (R = M for A, N for B)
            rec, tile = X.rec, tiles[idx]
            if rec["fmt"] == "k":
                return f"newt::lds_frag_k32f<{rec['K']}>({tile}, {r0}, {kk}, _lane)"
            c = f"({r0} + (_lane & 31))"
            els = ", ".join(f"{tile}[newt::LdsTileR32<{rec['R']}>::off({kk} + _kh + {t}, {c})]"
                            for t in range(4))
            return f"f32x4{{{els}}}"

        for g in range(K // 8):
            kk = 8 * g
            for i in range(RM):
                self.emit(f"const f32x4 _fa{g}_{i} = {group(0, a, f'_ra + {i * 32}', kk)};")
            for j in range(RN):
                self.emit(f"const f32x4 _fb{g}_{j} = {group(1, Bt, f'_rb + {j * 32}', kk)};")
            for t in range(4):
                for i in range(RM):
                    for j in range(RN):
                        fa_, fb_ = f"_fa{g}_{i}[{t}]", f"_fb{g}_{j}[{t}]"
                        x, y = (fb_, fa_) if orient == "row" else (fa_, fb_)
                        v = f"{accv.var}[{j + RN * i}]"
                        self.emit(f"{v} = newt::mfma_{instr}({x}, {y}, {v});")
        state["sched"] = None
        self.indent -= 1
        self.emit("}")
        return accv

    # ------------------------------------------------- loop-invariant operands
    def _dot_operand_shape(self, a, state):
        """(shape, name) of a dot operand expression, without emitting code;
        name is None for transposed or non-name operands."""
        nm, trans = _operand_name(a)
        if nm is None:
            return None, None
        if nm in state["recs"]:
            sh = state["recs"][nm]["shape"]
        else:
            sh = getattr(self.locals.get(nm), "shape", None)
            if sh is None or len(sh) != 2:
                return None, None
        sh = tuple(sh)
        return (sh[::-1] if trans else sh), (None if trans else nm)

    def pipe_hoist_operands(self, state):
        """Load A operands that do not change in the loop into MFMA operand
        registers once, before it."""
        plan = state["plan"]
        assigned = set().union(*(_targets(s) for s in plan["flat"]))
        for s in plan["flat"]:
            for nd in ast.walk(s):
                if _callee(nd) != "dot" or len(nd.args) < 2:
                    continue
                sa, na = self._dot_operand_shape(nd.args[0], state)
                sb, _ = self._dot_operand_shape(nd.args[1], state)
                if sa is None or sb is None or sa[1] != sb[0]:
                    continue
                if na is None or na in assigned or na in state["recs"] or na in self.storages:
                    continue
                v = self.locals.get(na)
                if not isinstance(v, (LazyLoad, Reg)) or v.dtype not in (tp.float16, tp.bfloat16):
                    continue
                geo = self._geometry_of(sa[0], sb[1], sa[1], v.dtype)
                if geo is None:
                    continue
                instr, wm, wn = geo
                L = lo.mfma_operand(sa[0], sa[1], instr, wm, wn, other_first=False)
                if isinstance(v, Reg) and v.layout == L:
                    continue
                self.locals[na] = self.to_reg(v, L)

    def _geometry_of(self, M, N, K, dt):
        if M % 16 or N % 16 or K % 16 or M < 16 or N < 16:
            return None
        instr = self.pick_instr(M, N, K, dt)
        if lo.INSTR[instr][3] != 8:
            return None
        wm, wn, rep = self.wave_grid(M, N, instr)
        if rep > 1:
            return None
        return instr, wm, wn

    # ------------------------------------------------------------- the dot
    @staticmethod
    def _slot_for(L, coords):
        """Register slot of L that holds the element whose in-thread
        coordinate parts are `coords` (dim -> value, lane/wave parts excluded)."""
        s = 0
        want = dict(coords)
        for i, b in enumerate(L.reg):
            if b is None:
                continue
            d, bit = b
            if (want.get(d, 0) >> bit) & 1:
                s |= 1 << i
                want[d] = want[d] & ~(1 << bit)
        if any(want.values()):
            raise ValueError("coordinate not held in registers")
        return s

    def staged_dot(self, node, a, b, acc):
        """nl.dot with at least one operand resident in a pipeline stage."""
        M, N, K, dt, instr, wm, wn, rep = self.dot_geometry(node, a, b)
        MI, NI, KI, kpl, nacc = lo.INSTR[instr]
        state = getattr(self, "pipe_active", None)
        if dt == tp.float32 and state is not None:
            return self._staged_dot_f32(node, a, b, acc, M, N, K, instr, wm, wn, rep, state)
        if rep > 1 or kpl != 8 or dt not in (tp.float16, tp.bfloat16) or state is None:
            if state is not None:
                self._no_pipe(state)
            self.err(node, "internal: staged operand in an unsupported dot")
        Lc = self.mfma_layout(M, N, instr, wm, wn, 1)
        T = dt.ctype
        Bt = Staged(b.rec, b.slot, not b.trans) if isinstance(b, Staged) else self.permute(b, (1, 0))
        RM, RN = M // wm // MI, N // wn // NI
        nks = K // KI
        orient = self.dot_orient()
        # an accumulator-layout A operand (fp16/bf16 cast of a row-per-lane dot
        # result) is used in place, with B read in the permuted k order: the
        # k-slot e of a lane maps to the column its accumulator register holds
        # (32x32: kk + 8*(e/4) + 4h + e%4 for lane half h; 16x16: kk +
        # 16*(e/4) + 4g + e%4 for lane group g, two accumulator tiles per MFMA)
        # (an [M, K] accumulator of this instruction exists only when K is a
        # multiple of its tile width: a 16-wide P never is one of 32x32x16)
        perm = (orient == "row" and isinstance(a, Reg) and isinstance(Bt, Staged)
                and wn == 1 and K % MI == 0 and a.layout == lo.mfma_c(M, K, instr, wm, 1, "row")
                and (MI == 32 or os.environ.get("NEWT_PERM16", "1") != "0"))
        srcs = []
        for role, X in (("A", a), ("B", Bt)):
            if isinstance(X, Staged):
                srcs.append(("lds", X))
            elif role == "A" and perm:
                srcs.append(("acc", X))
            else:
                if role == "A":
                    L = lo.mfma_operand(M, K, instr, wm, wn, other_first=False)
                else:
                    L = lo.mfma_operand(N, K, instr, wn, wm, other_first=True)
                r = X if isinstance(X, Reg) and X.layout == L and not X.vec else self.to_reg(X, L)
                if r.dtype != dt:
                    r = self.to_reg(r, r.layout, dt)
                srcs.append(("op", r))
        accv = self.init_acc(node, acc, Lc, M, N)
        self.emit("{")
        self.indent += 1
        self.emit(f"const int _ra = (_wave & {wm - 1}) * {M // wm};")
        self.emit(f"const int _rb = ((_wave >> {lo.log2i(wm)}) & {wn - 1}) * {N // wn};")
        tiles = {}
        for idx, (kind, X) in enumerate(srcs):
            if kind == "lds":
                nm = f"_pt{idx}"
                self.emit(f"const {T}* {nm} = (const {T}*)({state['names'][X.slot]} + "
                          f"{X.rec['off']});")
                tiles[idx] = nm

        def frag(idx, i, ks, tile=None, r0=None):
            kind, X = srcs[idx]
            kk = ks * KI
            if kind == "lds":
                rec, tile = X.rec, tile or tiles[idx]
                r0 = r0 or f"{'_ra' if idx == 0 else '_rb'} + {i * MI}"
                if rec["fmt"] == "k":
                    fn, targs = ((f"lds_frag_k_perm{MI}", f"{T}, {rec['K']}") if perm else
                                 ("lds_frag_k", f"{T}, {rec['K']}, {MI}"))
                else:
                    fn, targs = ((f"lds_frag_r_perm{MI}", f"{T}, {rec['R']}, {rec['sb']}") if perm
                                 else ("lds_frag_r", f"{T}, {rec['R']}, {MI}, {rec['sb']}"))
                return f"newt::{fn}<{targs}>({tile}, {r0}, {kk}, _lane)"
            if kind == "acc":
                step = 8 if MI == 32 else 16
                slots = [self._slot_for(X.layout, {0: i * MI, 1: kk + step * (e // 4) + (e % 4)})
                         for e in range(8)]
            else:
                slots = [self._slot_for(X.layout, {0: i * MI, 1: kk + e}) for e in range(8)]
            return f"newt::pack8<{T}>({', '.join(X.at(s) for s in slots)})"

        plr = state.get("plr")
        pf = {}
        if plr:
            d = state["pf_d"]
            state["pf_d"] += 1
            woff = {0: f"((_wave & {wm - 1}) * {M // wm})",
                    1: f"(((_wave >> {lo.log2i(wm)}) & {wn - 1}) * {N // wn})"}
            frags = []
            for idx, cnt, tag in ((0, RM, "a"), (1, RN, "b")):
                kind, X = srcs[idx]
                if kind != "lds":
                    continue
                for i in range(cnt):
                    var = f"_pf{d}{tag}{i}"

                    def fn(slot, idx=idx, i=i, X=X):
                        tile = f"((const {T}*)({state['names'][slot]} + {X.rec['off']}))"
                        return frag(idx, i, 0, tile=tile, r0=f"{woff[idx]} + {i * MI}")
                    frags.append((var, fn))
                    pf[(idx, i)] = var
            state["pf"][d] = frags

        def n_reads(idx):
            kind, X = srcs[idx]
            if kind != "lds":
                return 0
            return 1 if (X.rec["fmt"] == "k" and not perm) else 2

        def emit_frags(ks):
            for i in range(RM):
                src = pf.get((0, i)) if ks == 0 else None
                self.emit(f"const i16x8 _fa{ks}_{i} = {src or frag(0, i, ks)};")
            for j in range(RN):
                src = pf.get((1, j)) if ks == 0 else None
                self.emit(f"const i16x8 _fb{ks}_{j} = {src or frag(1, j, ks)};")

        emit_frags(0)
        for ks in range(nks):
            if ks + 1 < nks:
                emit_frags(ks + 1)
            for i in range(RM):
                for j in range(RN):
                    fa_ = f"newt::as_frag<{T}>(_fa{ks}_{i})"
                    fb_ = f"newt::as_frag<{T}>(_fb{ks}_{j})"
                    x, y = (fb_, fa_) if orient == "row" else (fa_, fb_)
                    v = f"{accv.var}[{j + RN * i}]"
                    self.emit(f"{v} = newt::mfma_{instr}({x}, {y}, {v});")
        per_ks = RM * n_reads(0) + RN * n_reads(1)
        state["sched"] = {"reads": [per_ks] * nks, "mfmas": [RM * RN] * nks}
        self.indent -= 1
        self.emit("}")
        return accv
