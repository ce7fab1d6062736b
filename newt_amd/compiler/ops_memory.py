"""Global memory access: nl.load / nl.store / nl.atomic_* lowering.

Semantics follow the reference (newt/compiler/codegen.py:1538-1801): masked-off
elements of a load yield `other` (default 0) converted to the element type; a
scalar pointer cannot take a block mask; a store or atomic first materializes
every deferred load (they must observe pre-store memory); an atomic through a
scalar pointer fires once per program.

The access strategy is this backend's own. The element offsets of a pointer
block are symbolic (`Affine`), so for each register layout the code generator
knows at compile time which runs of register slots are contiguous in memory
and whether a run's first address is 16-byte aligned; those runs become single
global_load_dwordx4 / global_store_dwordx4 transactions. Masks built from
comparisons of affine indices with scalars are reduced to one uniform
"whole tile in bounds" condition that selects an unmasked fast path; other
tiles take a per-run path (vector access when the run is fully valid,
predicated element accesses otherwise).
"""

import os

from . import layouts as lo
from . import types as tp
from .codegen import CompileError
from .values import Affine, Block, Const, Lazy, LazyLoad, PtrBlock, Reg, Scalar


class MemoryOps:
    # ------------------------------------------------------------------ loads
    def op_load(self, node, pointer, mask=None, other=None):
        if isinstance(mask, LazyLoad):
            mask = self.materialize_load(mask)
        if isinstance(other, LazyLoad):
            other = self.materialize_load(other)
        if isinstance(pointer, Scalar):
            if not pointer.is_ptr:
                self.err(node, "load() expects a pointer block")
            if isinstance(mask, Block):
                self.err(node, "a scalar pointer cannot take a block mask "
                               "(broadcast the pointer with `ptr + offsets` first)")
            elem = pointer.dtype.element
            if mask is None or (isinstance(mask, Const) and mask.pyval):
                return self.new_scalar(elem, f"*({pointer.expr})")
            oexpr = self.scalar_expr(other, elem) if other is not None else self.literal(0, elem)
            if isinstance(mask, Const):
                return self.new_scalar(elem, oexpr)
            return self.new_scalar(elem, f"(({mask.expr}) ? *({pointer.expr}) : {oexpr})")
        if not isinstance(pointer, PtrBlock):
            self.err(node, "load() expects a pointer block")
        shape = pointer.shape
        for v in (mask, other):
            if isinstance(v, Block):
                shape = tp.broadcast_shapes(shape, v.shape)
        rank = len(shape)
        ptr = PtrBlock(pointer.base, self.expand_to_rank(pointer.offset, rank))
        mask = self.expand_to_rank(mask, rank) if isinstance(mask, Block) else mask
        other = self.expand_to_rank(other, rank) if isinstance(other, Block) else other
        ld = LazyLoad(ptr, mask, other, node)
        ld.shape = tuple(shape)
        self.pending_loads.append(ld)
        return ld

    def flush_loads(self):
        """Emit every deferred load not yet staged by a dot; loads a dot has
        consumed become unusable (their pointers may now be stale)."""
        for ld in list(self.pending_loads):
            if ld.result is not None:
                continue
            if ld.consumed:
                ld.poisoned = True
            else:
                self.materialize_load(ld)
        self.pending_loads = []

    def materialize_load(self, ld, L=None):
        if ld.result is not None:
            if L is None or ld.result.layout == L:
                return ld.result
            return self.convert(ld.result, L)
        if ld.poisoned:
            raise CompileError(
                "a value from nl.load was consumed by nl.dot and then used after "
                "a store/loop boundary; load it into a separate variable first")
        key = ("load", ld.node.lineno, ld.node.col_offset, getattr(ld, "src", None) is not None)
        if L is None:
            h = self.hints.get(key)
            L = h if isinstance(h, lo.Layout) and h.shape == ld.shape else self.default_layout(ld.shape)
        r = self.emit_load(ld, L)
        r.origin = key
        ld.result = r
        if ld in self.pending_loads:
            self.pending_loads.remove(ld)
        return r

    # --------------------------------------------------------- access analysis
    def contiguous_bits(self, L, off):
        """Number of leading register bits of L that walk consecutive elements
        (offset coefficient 1 along that dim)."""
        if not isinstance(off, Affine) or not L.reg or L.reg[0] is None:
            return 0
        d = L.reg[0][0]
        c = off.coefs.get(d)
        if c is None or not c.is_const or c.const != 1 or off.shape[d] == 1:
            return 0
        n = 0
        while n < len(L.reg) and L.reg[n] == (d, n):
            n += 1
        return n

    def offset_div(self, L, off, gbits):
        """Power-of-two divisor of the offset at the first slot of every run of
        2**gbits slots."""
        if not isinstance(off, Affine):
            return 1
        div = off.base.div
        for a, c in off.coefs.items():
            if off.shape[a] == 1:
                continue
            # lowest coordinate bit of dim a that a run start can have set
            low = None
            for bits, skip in ((L.reg, gbits), (L.lane, 0), (L.wave, 0)):
                for i, b in enumerate(bits):
                    if bits is L.reg and i < skip:
                        continue
                    if b is not None and b[0] == a:
                        low = b[1] if low is None else min(low, b[1])
            cd = (1 << low) if low is not None else (1 << 30)
            div = min(div, min(c.div * cd, 1 << 30))
        return div

    def mask_all_true(self, mask, shape):
        """Uniform C condition under which `mask` is true everywhere, or None."""
        if mask is None:
            return "true"
        if isinstance(mask, Const):
            return "true" if mask.pyval else "false"
        if isinstance(mask, Scalar):
            return f"({mask.expr})"
        meta = getattr(mask, "meta", None) if isinstance(mask, Lazy) else None
        if not meta or meta[0] != "and":
            return None
        conds = []
        for part in meta[1]:
            if part is None or part[0] != "cmp":
                return None
            _, sym, aff = part
            hi, lo_ = [], []
            for a, c in aff.coefs.items():
                n = shape[a] if a < len(shape) else 1
                if aff.shape[a] == 1 or n == 1:
                    continue
                if not c.is_const:
                    return None
                v = c.const * (n - 1)
                (hi if v > 0 else lo_).append(v)
            base = aff.base.expr
            if sym in ("<", "<="):
                ext = sum(hi)
            elif sym in (">", ">="):
                ext = sum(lo_)
            else:
                return None
            e = f"({base} + {ext})" if ext else f"({base})"
            conds.append(f"({e} {sym} 0)")
        return " && ".join(conds) if conds else "true"

    # ------------------------------------------------------------ emission
    def emit_load(self, ld, L):
        ptr, mask, other = ld.ptr, ld.mask, ld.other
        elem = ptr.elem
        esz = elem.itemsize
        off = self.prepare(ptr.offset, L)
        mask = self.prepare(mask, L) if isinstance(mask, Block) else mask
        other = self.prepare(other, L) if isinstance(other, Block) else other
        out = self.new_reg(elem, L.shape, L)
        base = ptr.base.expr
        gb = self.contiguous_bits(L, off)
        run = 1 << gb
        chunk = max(1, min(run, 16 // esz))
        cbits = chunk.bit_length() - 1
        div = self.offset_div(L, off, cbits)
        proven = ptr.base.aligned16 and div % chunk == 0
        all_true = self.mask_all_true(mask, L.shape)
        nt = id(ld.node) in getattr(self, "stream_loads", ())
        rd = (lambda e: f"__builtin_nontemporal_load(&{e})") if nt else (lambda e: e)

        def oth(s):
            if other is None:
                return self.literal(0, elem)
            return self.conv(self.ev(other, L, s), self.cdtype(other), elem)

        def body(masked):
            for g in range(0, L.nslots, chunk):
                o = self.ev(off, L, g)
                if chunk > 1:
                    addr = f"({base} + {o})"
                    self.emit("{")
                    self.indent += 1
                    if masked:
                        ms = [f"({self.ev(mask, L, g + i)})" for i in range(chunk)]
                        for i, m in enumerate(ms):
                            self.emit(f"const bool _m{i} = {m};")
                        cond = " && ".join(f"_m{i}" for i in range(chunk))
                    else:
                        cond = ""
                    if not proven:
                        al = f"newt::aligned({addr}, {chunk * esz})"
                        cond = f"{cond} && {al}" if cond else al
                    vec = (f"newt::load_vec{'_nt' if nt else ''}<{elem.ctype}, {chunk}>({addr}, "
                           f"{out.var} + {g});")
                    if not cond:
                        self.emit(vec)
                    else:
                        self.emit(f"if ({cond}) {{ {vec} }} else {{")
                        self.indent += 1
                        for i in range(chunk):
                            e = rd(f"{base}[{o} + {i}]")
                            if masked:
                                self.emit(f"{out.at(g + i)} = _m{i} ? {e} : {oth(g + i)};")
                            else:
                                self.emit(f"{out.at(g + i)} = {e};")
                        self.indent -= 1
                        self.emit("}")
                    self.indent -= 1
                    self.emit("}")
                else:
                    e = rd(f"{base}[{o}]")
                    if masked:
                        m = self.ev(mask, L, g)
                        self.emit(f"{out.at(g)} = ({m}) ? {e} : {oth(g)};")
                    else:
                        self.emit(f"{out.at(g)} = {e};")

        def scoped(masked):
            self.emit("{")
            self.indent += 1
            body(masked)
            self.indent -= 1
            self.emit("}")

        if all_true == "true":
            scoped(False)
        elif all_true is None:
            scoped(True)
        else:
            self.emit(f"if ({all_true}) {{")
            self.indent += 1
            body(False)
            self.indent -= 1
            self.emit("} else {")
            self.indent += 1
            body(True)
            self.indent -= 1
            self.emit("}")
        return out

    # ----------------------------------------------------------------- stores
    def op_store(self, node, pointer, value, mask=None):
        if isinstance(value, LazyLoad):
            value = self.materialize_load(value)
        if isinstance(mask, LazyLoad):
            mask = self.materialize_load(mask)
        if isinstance(pointer, Scalar):
            if not pointer.is_ptr:
                self.err(node, "store() expects a pointer block")
            if isinstance(mask, Block):
                self.err(node, "a scalar pointer cannot take a block mask")
            if isinstance(value, Block):
                self.err(node, "cannot store a block through a scalar pointer")
            elem = pointer.dtype.element
            src = self.scalar_expr(value, elem)
            self.flush_loads()
            self.drain_dots()
            if isinstance(mask, Const):
                if not mask.pyval:
                    return Const(None)
                mask = None
            cond = "_tid == 0" + (f" && ({mask.expr})" if isinstance(mask, Scalar) else "")
            self.emit(f"if ({cond}) *({pointer.expr}) = {src};")
            return Const(None)
        if not isinstance(pointer, PtrBlock):
            self.err(node, "store() expects a pointer block")
        elem = pointer.elem
        if (isinstance(value, Block) and value.dtype != elem and value.dtype.is_floating
                and elem.is_floating):
            # convert the block first, as value.to(elem) would: the same
            # rounding, and the registers of a wide accumulator are released
            # in one pass instead of staying live across the narrowing stores
            value = self.cast(node, value, elem)
        shape = pointer.shape
        for v in (value, mask):
            if isinstance(v, Block):
                shape = tp.broadcast_shapes(shape, v.shape)
        rank = len(shape)
        value = self.expand_to_rank(value, rank) if isinstance(value, Block) else value
        mask = self.expand_to_rank(mask, rank) if isinstance(mask, Block) else mask
        off = self.expand_to_rank(pointer.offset, rank)
        if isinstance(value, Reg) and value.shape == tuple(shape):
            L = value.layout
        elif isinstance(value, Reg):
            L = value.layout.broadcast_into(tuple(shape)) or self.default_layout(shape)
        else:
            L = self.default_layout(shape)
        value = self.prepare(value, L) if isinstance(value, Block) else value
        mask = self.prepare(mask, L) if isinstance(mask, Block) else mask
        off = self.prepare(off, L)
        self.flush_loads()
        self.drain_dots()
        self.emit_store(L, pointer.base, off, value, mask, elem,
                        stream=id(node) in getattr(self, "stream_stores", ()))
        return Const(None)

    def emit_store(self, L, pbase, off, value, mask, elem, stream=False):
        esz = elem.itemsize
        base = pbase.expr
        gb = self.contiguous_bits(L, off)
        chunk = max(1, min(1 << gb, 16 // esz))
        cbits = chunk.bit_length() - 1
        div = self.offset_div(L, off, cbits)
        proven = pbase.aligned16 and div % chunk == 0
        all_true = self.mask_all_true(mask, L.shape)
        vd = self.cdtype(value)
        # a matmul's C tile (a column-oriented dot accumulator: the kernel has
        # no row reductions) is stored once, by every workgroup at about the
        # same time, after its k-loop: the non-temporal hint keeps that burst
        # from displacing operands that workgroups still in their k-loops read
        # through L2 (4096^3 fp16: +0.3-4%). Attention's O (row-oriented,
        # written as workgroups finish) measured 5-7% slower with it, and
        # streaming row kernels slower too, so they keep plain stores.
        acc = lo.mfma_tag_instr(L.tag)
        nt = acc is not None and acc[1] == "col" and os.environ.get("NEWT_NT_STORE", "1") != "0"
        nt = nt or stream

        def val(s):
            return self.conv(self.ev(value, L, s), vd, elem)

        def scalar_store(o, v):
            if nt:
                return f"__builtin_nontemporal_store(({elem.ctype})({v}), &{base}[{o}]);"
            return f"{base}[{o}] = {v};"

        def body(masked):
            for g in range(0, L.nslots, chunk):
                if not L.slot_is_canonical(g):
                    continue
                o = self.ev(off, L, g)
                if chunk > 1:
                    addr = f"({base} + {o})"
                    self.emit("{")
                    self.indent += 1
                    self.emit(f"{elem.ctype} _w[{chunk}];")
                    for i in range(chunk):
                        self.emit(f"_w[{i}] = {val(g + i)};")
                    conds = []
                    if masked:
                        for i in range(chunk):
                            self.emit(f"const bool _m{i} = {self.ev(mask, L, g + i)};")
                        conds.append(" && ".join(f"_m{i}" for i in range(chunk)))
                    if not proven:
                        conds.append(f"newt::aligned({addr}, {chunk * esz})")
                    vec = f"newt::store_vec{'_nt' if nt else ''}<{elem.ctype}, {chunk}>({addr}, _w);"
                    if conds:
                        self.emit(f"if ({' && '.join(conds)}) {{ {vec} }} else {{")
                        self.indent += 1
                        for i in range(chunk):
                            st = scalar_store(f"{o} + {i}", f"_w[{i}]")
                            self.emit(f"if (_m{i}) {st}" if masked else st)
                        self.indent -= 1
                        self.emit("}")
                    else:
                        self.emit(vec)
                    self.indent -= 1
                    self.emit("}")
                else:
                    st = scalar_store(o, val(g))
                    if masked:
                        self.emit(f"if ({self.ev(mask, L, g)}) {st}")
                    else:
                        self.emit(st)

        canon = self.canon_cond(L)
        if canon:
            self.emit(f"if ({canon}) {{")
            self.indent += 1
        if all_true == "true":
            body(False)
        elif all_true is None:
            body(True)
        else:
            self.emit(f"if ({all_true}) {{")
            self.indent += 1
            body(False)
            self.indent -= 1
            self.emit("} else {")
            self.indent += 1
            body(True)
            self.indent -= 1
            self.emit("}")
        if canon:
            self.indent -= 1
            self.emit("}")

    # ---------------------------------------------------------------- atomics
    def _atomic(self, node, fn, pointer, value, mask):
        if isinstance(value, LazyLoad):
            value = self.materialize_load(value)
        if isinstance(mask, LazyLoad):
            mask = self.materialize_load(mask)
        if isinstance(pointer, Scalar):
            if not pointer.is_ptr:
                self.err(node, "atomic ops expect a pointer block")
            if isinstance(value, Block):
                self.err(node, "scalar-pointer atomic with a block value; reduce it first")
            if isinstance(mask, Block):
                self.err(node, "scalar-pointer atomic cannot take a block mask")
            elem = pointer.dtype.element
            self.flush_loads()
            self.drain_dots()
            conds = ["_tid == 0"]  # once per program (reference codegen.py:1773-1777)
            if isinstance(mask, Scalar):
                conds.append(f"({mask.expr})")
            elif isinstance(mask, Const) and not mask.pyval:
                return Const(None)
            self.emit(f"if ({' && '.join(conds)}) {fn}({pointer.expr}, {self.scalar_expr(value, elem)});")
            return Const(None)
        if not isinstance(pointer, PtrBlock):
            self.err(node, "atomic ops expect a pointer block")
        elem = pointer.elem
        shape = pointer.shape
        for v in (value, mask):
            if isinstance(v, Block):
                shape = tp.broadcast_shapes(shape, v.shape)
        rank = len(shape)
        value = self.expand_to_rank(value, rank) if isinstance(value, Block) else value
        mask = self.expand_to_rank(mask, rank) if isinstance(mask, Block) else mask
        off = self.expand_to_rank(pointer.offset, rank)
        L = value.layout if isinstance(value, Reg) and value.shape == tuple(shape) else self.default_layout(shape)
        value = self.prepare(value, L) if isinstance(value, Block) else value
        mask = self.prepare(mask, L) if isinstance(mask, Block) else mask
        off = self.prepare(off, L)
        self.flush_loads()
        self.drain_dots()
        vd = self.cdtype(value)
        canon = self.canon_cond(L)
        if canon:
            self.emit(f"if ({canon}) {{")
            self.indent += 1
        for s in range(L.nslots):
            if not L.slot_is_canonical(s):
                continue
            line = f"{fn}(&{pointer.base.expr}[{self.ev(off, L, s)}], {self.conv(self.ev(value, L, s), vd, elem)});"
            if mask is not None and not (isinstance(mask, Const) and mask.pyval):
                if isinstance(mask, Const):
                    continue
                self.emit(f"if ({self.ev(mask, L, s)}) {line}")
            else:
                self.emit(line)
        if canon:
            self.indent -= 1
            self.emit("}")
        return Const(None)

    def op_atomic_add(self, node, pointer, value, mask=None):
        return self._atomic(node, "newt::atomic_add", pointer, value, mask)

    def op_atomic_max(self, node, pointer, value, mask=None):
        return self._atomic(node, "newt::atomic_max", pointer, value, mask)
