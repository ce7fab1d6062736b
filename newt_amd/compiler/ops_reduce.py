"""nl.sum / nl.max / nl.min lowering.

Semantics (reference newt/compiler/codegen.py:1883-1999): fp16/bf16 reduce to an
fp32 result, a bool block reduces to an int32 count (sum) or "any" (max);
identities are 0, -inf/+inf, INT_MIN/INT_MAX; float max/min are fmaxf/fminf.

Lowering (this backend's own): the reduced dimension's logical bits are split
by the hardware index that carries them in the operand's layout -
  register bits -> combined in-thread,
  lane bits     -> wave64 butterfly (newt::lane_reduce: DPP quad_perm for
                   xor 1/2, DPP row mirrors (or ds_swizzle) for xor 4/8,
                   v_permlane16/32_swap for xor 16/32; newt::lane_reduce2
                   reduces two results held by the same lanes at once),
  wave bits     -> one LDS exchange + barrier.
Replicated hardware bits are never combined (they hold copies). The result of
an axis reduction keeps the operand's layout minus the reduced bits, so a row
statistic of an MFMA tile stays one-row-per-lane and broadcasts back for free.
"""

import math
import os

from . import types as tp
from .values import Const, LazyLoad, Reg, Scalar

_OPS = {"sum": "newt::Sum", "max": "newt::Max", "min": "newt::Min"}


class ReduceOps:
    def _identity(self, op, dt):
        if op == "sum":
            return self.literal(0, dt)
        if dt.is_floating:
            return self.literal(float("-inf") if op == "max" else float("inf"), dt)
        if dt == tp.int64:
            return "(-9223372036854775807LL - 1)" if op == "max" else "9223372036854775807LL"
        if dt == tp.uint32:
            return "0u" if op == "max" else "4294967295u"
        return "(-2147483647 - 1)" if op == "max" else "2147483647"

    def _combine(self, op, a, b):
        return f"{_OPS[op]}::op({a}, {b})"

    def _reduce(self, node, x, axis, op):
        if isinstance(x, (Const, Scalar)):
            return x
        if isinstance(x, LazyLoad):
            x = self.materialize_load(x)
        rt = tp.float32 if tp.is_half(x.dtype) else x.dtype
        if rt == tp.int1:
            rt = tp.int32
        x = self.to_reg(x) if not isinstance(x, Reg) else x
        if axis is not None:
            ax = self._cx(node, axis, "axis") if not isinstance(axis, int) else axis
            if ax < 0:
                ax += len(x.shape)
            if ax >= len(x.shape):
                self.err(node, f"axis {ax} out of range for shape {x.shape}")
            if len(x.shape) > 1:
                return self._reduce_axis(x, ax, op, rt)
        return self._reduce_full(x, op, rt)

    def _lds_for_reduce(self, nbytes):
        """LDS offset (a C expression) for one reduction site's cross-wave
        partials. Outside loops the site has one region. Inside a loop it runs
        again, so a write must not overtake a slower wave's reads of the last
        partials: the site alternates between two regions, and the barrier
        that follows each write (which a wave reaches only after reading the
        site's previous partials, in program order) then separates every
        write from the reads of the same region two executions back, with no
        barrier before the write. Large partial sets keep one region and a
        barrier before the write."""
        if not self.loop_depth:
            return self.lds_alloc(nbytes)
        if nbytes > 4096 or os.environ.get("NEWT_REDUCE_PINGPONG", "1") == "0":
            self.barrier()
            return self.lds_alloc(nbytes)
        stride = (nbytes + 15) // 16 * 16
        region = self.lds_alloc(2 * stride)
        par = self.fresh("rpar")
        self.prologue.append(f"unsigned {par} = 0u;")
        self.emit(f"{par} ^= 1u;")
        return f"({region} + {par} * {stride}u)"

    def _reduce_full(self, x, op, rt):
        L = x.layout
        p = self.fresh("rp")
        first = True
        for s in range(L.nslots):
            if not L.slot_is_canonical(s):
                continue
            e = self.conv(x.at(s), x.dtype, rt)
            if first:
                self.emit(f"{rt.ctype} {p} = {e};")
                first = False
            else:
                self.emit(f"{p} = {self._combine(op, p, e)};")
        lmask = sum(1 << i for i, b in enumerate(L.lane) if b is not None)
        if lmask:
            self.emit(f"{p} = newt::lane_reduce<{_OPS[op]}, {lmask}>({p});")
        wbits = [i for i, b in enumerate(L.wave) if b is not None]
        if wbits:
            n = 1 << len(wbits)
            region = self._lds_for_reduce(n * max(rt.itemsize, 4))
            buf = self.fresh("rb")
            self.emit(f"{rt.ctype}* {buf} = ({rt.ctype}*)(_lds + {region});")
            idx = " | ".join(f"(((_wave >> {w}) & 1) << {k})" for k, w in enumerate(wbits))
            rep = L.wave_rep_mask()
            cond = "_lane == 0" + (f" && (_wave & {rep}) == 0" if rep else "")
            self.emit(f"if ({cond}) {buf}[{idx}] = {p};")
            self.barrier()
            self.emit(f"{p} = {buf}[0];")
            for i in range(1, n):
                self.emit(f"{p} = {self._combine(op, p, f'{buf}[{i}]')};")
        return Scalar(rt, p)

    def _reduce_axis(self, x, axis, op, rt):
        L = x.layout
        Lr = L.reduce(axis)
        keep = [i for i, b in enumerate(L.reg) if b is None or b[0] != axis]
        out = self.new_reg(rt, Lr.shape, Lr)
        seen = set()
        for s in range(L.nslots):
            if not L.slot_is_canonical(s):
                continue  # replicated register copy
            t = 0
            for k, i in enumerate(keep):
                if (s >> i) & 1:
                    t |= 1 << k
            e = self.conv(x.at(s), x.dtype, rt)
            if t not in seen:
                self.emit(f"{out.at(t)} = {e};")
                seen.add(t)
            else:
                self.emit(f"{out.at(t)} = {self._combine(op, out.at(t), e)};")
        lmask = sum(1 << i for i, b in enumerate(L.lane) if b is not None and b[0] == axis)
        if lmask:
            slots = [t for t in range(Lr.nslots) if Lr.slot_is_canonical(t)]
            # results held two or more to a lane (a 16x16 MFMA tile's rows)
            # share the permlane steps of lane bits 4 and 5 in pairs
            if lmask & 48 and os.environ.get("NEWT_PAIR_REDUCE", "1") != "0":
                while len(slots) >= 2:
                    t0, t1 = slots.pop(0), slots.pop(0)
                    self.emit(f"newt::lane_reduce2<{_OPS[op]}, {lmask}>({out.at(t0)}, "
                              f"{out.at(t1)});")
            for t in slots:
                self.emit(f"{out.at(t)} = newt::lane_reduce<{_OPS[op]}, {lmask}>({out.at(t)});")
        wbits = [i for i, b in enumerate(L.wave) if b is not None and b[0] == axis]
        if wbits:
            n = 1 << len(wbits)
            numel = math.prod(Lr.shape) if Lr.shape else 1
            region = self._lds_for_reduce(n * numel * max(rt.itemsize, 4))
            buf = self.fresh("rb")
            self.emit(f"{rt.ctype}* {buf} = ({rt.ctype}*)(_lds + {region});")
            widx = " | ".join(f"(((_wave >> {w}) & 1) << {k})" for k, w in enumerate(wbits))
            strides = self._strides(Lr.shape)
            for t in range(Lr.nslots):
                if not Lr.slot_is_canonical(t):
                    continue
                flat = self._flat_index(Lr, t, strides)
                self.emit(f"{buf}[({widx}) * {numel} + {flat}] = {out.at(t)};")
            self.barrier()
            for t in range(Lr.nslots):
                if not Lr.slot_is_canonical(t):
                    continue
                flat = self._flat_index(Lr, t, strides)
                self.emit(f"{out.at(t)} = {buf}[{flat}];")
                for i in range(1, n):
                    self.emit(f"{out.at(t)} = {self._combine(op, out.at(t), f'{buf}[{i * numel} + {flat}]')};")
        rmask = Lr.reg_rep_mask()
        for t in range(Lr.nslots):
            if t & rmask:
                self.emit(f"{out.at(t)} = {out.at(t & ~rmask)};")
        return out

    def op_sum(self, node, x, axis=None):
        return self._reduce(node, x, axis, "sum")

    def op_max(self, node, x, axis=None):
        return self._reduce(node, x, axis, "max")

    def op_min(self, node, x, axis=None):
        return self._reduce(node, x, axis, "min")
