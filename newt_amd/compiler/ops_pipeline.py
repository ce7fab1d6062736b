"""Software pipeline for k-loops that feed nl.dot from nl.load.

The reference stages dot operands through a cp.async ring of `num_stages`
shared-memory slots with deferred consumption (newt/compiler/codegen.py:
2279-2369, :2560-2654). This is the gfx950 design of the same idea:

  * the loop is rotated: a prologue issues the operand tiles of the first
    num_stages-1 iterations, and iteration i issues iteration i+S-1 before it
    runs the MFMAs of iteration i, so global latency hides behind S-1
    iterations of matrix work;
  * every stage is its own __shared__ array, and the main loop is unrolled by
    S, so each stage is addressed through a distinct LDS object - that lets the
    compiler see that direct-to-LDS writes into one stage do not alias reads of
    another and wait for exactly the right loads (s_waitcnt vmcnt(N)) instead
    of draining everything before each LDS read;
  * a tile whose rows (or k) are contiguous, 16-byte aligned and proven in
    bounds by a uniform test is copied global -> LDS with
    global_load_lds_dwordx4 (no VGPR staging, no ds_write); other tiles
    (ragged edges, strided operands) take a register path with the masked
    loads' `other` fill, written with ds_write;
  * an operand contiguous along k lands in an XOR-swizzled K-major tile read
    with ds_read_b128; an operand contiguous along its rows (B of a row-major
    A @ B) lands R-major and is read with ds_read_b64_tr_b16, so nothing is
    transposed through registers;
  * each iteration has one barrier: after it, every wave's copies of the
    stage to be read are complete and every wave is done reading the stage
    about to be overwritten.

Only the plain pattern is pipelined; anything else falls back to synchronous
staging with identical semantics:

    for k in range(lo, hi, step):          # step a positive constant
        <assignments: masks, loads ...>    # a = nl.load(...), b = nl.load(...)
        acc = nl.dot(a, b, acc)
        <pointer advances: p += ...>

The loaded names, the temporaries and the advanced pointers must not be
read after the loop (the advances run S-1 iterations ahead), the
accumulator is read only by the dot, and the body has no stores, atomics or
nested control flow.
"""

import ast
import os

from . import layouts as lo
from . import types as tp
from .values import Affine, LazyLoad, PtrBlock, Scalar


def _is_call(node, names):
    if not isinstance(node, ast.Call):
        return False
    f = node.func
    name = f.attr if isinstance(f, ast.Attribute) else getattr(f, "id", None)
    return name in names


_SIDE_EFFECTS = {"store", "atomic_add", "atomic_max", "atomic_min", "static_print", "dot"}


class DotPipeline:
    # ------------------------------------------------------------ detection
    def pipeline_plan(self, node):
        if self.num_stages < 2 or os.environ.get("NEWT_PIPELINE_DOT", "1") == "0":
            return None
        if self.hints.get(("nopipe", node.lineno)):
            return None
        body = node.body
        dots = [i for i, s in enumerate(body)
                if isinstance(s, ast.Assign) and _is_call(s.value, {"dot"})]
        if len(dots) != 1:
            return None
        di = dots[0]
        dstmt = body[di]
        if len(dstmt.targets) != 1 or not isinstance(dstmt.targets[0], ast.Name):
            return None
        accn = dstmt.targets[0].id
        call = dstmt.value
        args = list(call.args)
        kw = {k.arg: k.value for k in call.keywords}
        if len(args) == 2 and "acc" in kw:
            args.append(kw.pop("acc"))
        if len(args) != 3 or kw or not all(isinstance(x, ast.Name) for x in args):
            return None
        an, bn, cn = (x.id for x in args)
        if cn != accn or len({an, bn, accn}) != 3:
            return None
        pre, post = body[:di], body[di + 1:]
        temps = set()
        loads = set()
        for s in pre:
            if not (isinstance(s, ast.Assign) and len(s.targets) == 1
                    and isinstance(s.targets[0], ast.Name)):
                return None
            if any(_is_call(n, _SIDE_EFFECTS) for n in ast.walk(s)):
                return None
            temps.add(s.targets[0].id)
            if _is_call(s.value, {"load"}):
                loads.add(s.targets[0].id)
        if an not in loads or bn not in loads:
            return None
        carried = set()
        for s in post:
            if isinstance(s, ast.AugAssign) and isinstance(s.target, ast.Name):
                carried.add(s.target.id)
            elif (isinstance(s, ast.Assign) and len(s.targets) == 1
                  and isinstance(s.targets[0], ast.Name)):
                carried.add(s.targets[0].id)
            else:
                return None
            if any(_is_call(n, _SIDE_EFFECTS) for n in ast.walk(s)):
                return None
        reads_post = {n.id for s in post for n in ast.walk(s) if isinstance(n, ast.Name)
                      and isinstance(n.ctx, ast.Load)}
        if reads_post & (temps | {accn}):
            return None
        reads_pre = {n.id for s in pre for n in ast.walk(s) if isinstance(n, ast.Name)
                     and isinstance(n.ctx, ast.Load)}
        if accn in reads_pre or (temps & carried) or accn in temps | carried:
            return None
        # a and b are read by the dot only
        uses = [n.id for s in pre for n in ast.walk(s) if isinstance(n, ast.Name)
                and isinstance(n.ctx, ast.Load)]
        if an in uses or bn in uses:
            return None
        kname = node.target.id
        if any(t in self.locals or t in self.storages for t in temps | {kname}):
            return None
        if not all(c in self.locals or c in self.storages for c in carried):
            return None
        if (temps | carried | {kname}) & self._read_after():
            return None
        return pre, dstmt, post, an, bn, accn, temps

    # ----------------------------------------------------------- emission
    def pipelined_for(self, node, plan, lo_, hi, st, idt):
        pre, dstmt, post, an, bn, accn, temps = plan
        S = int(self.hints.get(("pipe_stages", node.lineno), self.num_stages))
        kname = node.target.id
        stv = int(st.pyval)
        lo_e = self.scalar_expr(lo_, idt)
        hi_e = self.scalar_expr(hi, idt)
        n = self.new_scalar(idt, f"((({hi_e}) > ({lo_e})) ? ((({hi_e}) - ({lo_e}) + {stv - 1}) "
                                 f"/ {stv}) : 0)")
        state = {"node": node, "S": S, "dot": dstmt.value}
        self.pipe_records.append(state)
        for s in range(S - 1):
            self.locals[kname] = self.new_scalar(idt, f"({lo_e} + {s * stv})")
            self.visit_body(pre)
            self.pipe_issue(state, an, bn, s, f"({s} < {n.expr})")
            self.visit_body(post)
            for t in temps | {kname}:
                self.locals.pop(t, None)
        rec = self._enter_compound(node)
        self.drain_dots_for_loop(node)
        it0 = self.fresh("it")
        self.emit(f"for ({idt.ctype} {it0} = 0; {it0} < {n.expr}; {it0} += {S}) {{")
        self.indent += 1
        self.loop_depth += 1
        ops = state["ops"]
        for s in range(S):
            it = f"({it0} + {s})"
            if s:
                self.emit(f"if ({it} >= {n.expr}) break;")
            deep = (S - 2) * ops
            if deep:
                self.emit(f"if ({it} + {S - 2} < {n.expr}) newt::wait_vmcnt<{deep}>(); "
                          f"else newt::wait_vmcnt<0>();")
            else:
                self.emit("newt::wait_vmcnt<0>();")
            self.emit("__syncthreads();")
            self.emit("__builtin_amdgcn_sched_barrier(0);")
            self.locals[kname] = self.new_scalar(idt, f"({lo_e} + ({it} + {S - 1}) * {stv})")
            self.visit_body(pre)
            self.pipe_issue(state, an, bn, (s + S - 1) % S, f"({it} + {S - 1} < {n.expr})")
            self.visit_body(post)
            for t in temps | {kname}:
                self.locals.pop(t, None)
            acc = self.lookup(dstmt, accn)
            self.bind(dstmt, accn, self.pipe_mma(dstmt, state, acc, s))
        self.flush_loads()
        self.loop_backedge(node)
        self.loop_depth -= 1
        self.indent -= 1
        self.emit("}")
        self._exit_compound(rec)
        self.after_loop(node)

    def _no_pipe(self, state):
        self.new_hints[("nopipe", state["node"].lineno)] = True
        from .codegen import _Retry
        raise _Retry()

    def _tile_format(self, X, R, K):
        """'k' (K contiguous, ds_read_b128) or 'r' (rows contiguous, tr16 reads)."""
        off = X.ptr.offset
        if isinstance(off, Affine):
            ck, cr = off.coefs.get(1), off.coefs.get(0)
            if ck is not None and ck.is_const and ck.const == 1 and K % 8 == 0:
                return "k"
            if cr is not None and cr.is_const and cr.const == 1 and R % 32 == 0:
                return "r"
        return "k"

    def _dma_ok(self, X, fmt, R, K, dt):
        """Compile-time conditions for global_load_lds of whole 16-byte chunks."""
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
        chunks = R * K // epc
        return chunks % self.T == 0

    def pipe_geometry(self, state, a, b):
        dnode = state["dot"]
        M, N, K, dt, instr, wm, wn, rep = self.dot_geometry(dnode, a, b)
        MI, NI, KI, kpl, nacc = lo.INSTR[instr]
        if rep > 1 or dt not in (tp.float16, tp.bfloat16) or kpl != 8:
            self._no_pipe(state)
        Bt = self.permute(b, (1, 0))
        fa = self._tile_format(a, M, K)
        fb = self._tile_format(Bt, N, K)
        ba = self.tile_bytes(M, K, dt)
        bb = self.tile_bytes(N, K, dt)
        stage = (ba + bb + 15) // 16 * 16
        names = []
        for j in range(state["S"]):
            nm = f"_ldsP{len(self.lds_arrays)}"
            self.lds_arrays.append((nm, stage))
            names.append(nm)
        dma_a = self._dma_ok(a, fa, M, K, dt)
        dma_b = self._dma_ok(Bt, fb, N, K, dt)
        epc = 16 // dt.itemsize
        ops = (M * K // epc // self.T if dma_a else 0) + (N * K // epc // self.T if dma_b else 0)
        state.update(M=M, N=N, K=K, dt=dt, instr=instr, wm=wm, wn=wn, fmt=(fa, fb),
                     off=(0, ba), names=names, dma=(dma_a, dma_b), ops=ops)
        return Bt

    def pipe_issue(self, state, an, bn, slot, valid):
        a, b = self.locals.get(an), self.locals.get(bn)
        if not isinstance(a, LazyLoad) or not isinstance(b, LazyLoad) or a.result is not None \
                or b.result is not None:
            self._no_pipe(state)
        if "M" not in state:
            Bt = self.pipe_geometry(state, a, b)
        else:
            if (a.shape, b.shape, a.dtype) != ((state["M"], state["K"]), (state["K"], state["N"]),
                                              state["dt"]):
                self._no_pipe(state)
            Bt = self.permute(b, (1, 0))
        dt = state["dt"]
        T = dt.ctype
        ops = [(a, state["M"], state["fmt"][0], state["off"][0], state["dma"][0], a),
               (Bt, state["N"], state["fmt"][1], state["off"][1], state["dma"][1], b)]
        # register-path operands first: their (synchronous) loads must not
        # drain the asynchronous copies issued for this stage
        ops.sort(key=lambda o: o[4])
        K = state["K"]
        base = state["names"][slot]
        self.emit("{")
        self.indent += 1
        for X, R, fmt, boff, dma, src in ops:
            tile = f"(({T}*)({base} + {boff}))"
            if dma:
                full = self.mask_all_true(src.mask, src.shape)
                cond = valid if full in (None, "true") else f"{valid} && ({full})"
                if full is None:
                    self.emit(f"if ({valid}) {{")
                    self.indent += 1
                    self._reg_stage(X, tile, fmt, R, K, dt)
                    self.indent -= 1
                    self.emit("}")
                    continue
                # the in-bounds copy is the hot path; the hint moves the masked
                # register path out of the loop body's straight-line code
                self.emit(f"if (__builtin_expect({cond}, 1)) {{")
                self.indent += 1
                self._dma_stage(X, base, boff, fmt, R, K, dt)
                self.indent -= 1
                if full != "true":
                    self.emit(f"}} else if ({valid}) {{")
                    self.indent += 1
                    self._reg_stage(X, tile, fmt, R, K, dt)
                    self.indent -= 1
                self.emit("}")
            else:
                self.emit(f"if ({valid}) {{")
                self.indent += 1
                self._reg_stage(X, tile, fmt, R, K, dt)
                self.indent -= 1
                self.emit("}")
        self.indent -= 1
        self.emit("}")
        for ld in (a, b, Bt):
            ld.consumed = True
            if ld in self.pending_loads:
                self.pending_loads.remove(ld)

    def _dma_stage(self, X, base, boff, fmt, R, K, dt):
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
            else:
                self.emit(f"newt::LdsTileR<{T}, {R}>::slot(_s, _k, _r);")
            terms = [] if (off.base.is_const and off.base.const == 0) else [off.base.expr]
            for c, v in ((c0, "_r"), (c1, "_k")):
                if c is None:
                    continue
                terms.append(v if c.is_const and c.const == 1 else f"{c.expr} * {v}")
            gaddr = f"({gb} + {' + '.join(terms) if terms else '0'})"
            dst = f"(void*)({base} + {boff} + {16 * i * self.T} + _wave * 1024)"
            self.emit(f"newt::lds_dma16({gaddr}, {dst});")
            self.indent -= 1
            self.emit("}")

    def _reg_stage(self, X, tile, fmt, R, K, dt):
        if fmt == "k":
            L = self.staging_layout(X)
        else:
            v = 16 // dt.itemsize
            L = lo.blocked((K, R), self.W, min(v, R)).permute((1, 0))
        r = self.emit_load(X, L)
        if r.dtype != dt:
            r = self.to_reg(r, r.layout, dt)
        self.write_tile_to(r, tile, dt, fmt)

    def write_tile_to(self, r, tile, dt, fmt):
        """Write register block r ([R, K] view) into an LDS tile of format fmt."""
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
                 else f"newt::LdsTileR<{T}, {R}>::off({kk}, {rr})")
            if chunk > 1:
                self.emit(f"newt::store_vec<{T}, {chunk}>({tile} + {o}, {r.var} + {s});")
            else:
                self.emit(f"{tile}[{o}] = {r.at(s)};")
        if canon:
            self.indent -= 1
            self.emit("}")

    def _frag(self, state, which, r0, kk):
        M, N, K, dt, instr = state["M"], state["N"], state["K"], state["dt"], state["instr"]
        MI = lo.INSTR[instr][0]
        T = dt.ctype
        fmt = state["fmt"][which]
        tile, rows = ("_pa", M) if which == 0 else ("_pb", N)
        if fmt == "k":
            return f"newt::lds_frag_k<{T}, {K}, {MI}>({tile}, {r0}, {kk}, _lane)"
        return f"newt::lds_frag_r<{T}, {rows}, {MI}>({tile}, {r0}, {kk}, _lane)"

    def pipe_frags_first(self, state, slot):
        """Declare the fragment double buffer of a stage and read k-step 0."""
        M, N, dt, instr = state["M"], state["N"], state["dt"], state["instr"]
        wm, wn = state["wm"], state["wn"]
        MI, NI = lo.INSTR[instr][:2]
        RM, RN = M // wm // MI, N // wn // NI
        T = dt.ctype
        base = state["names"][slot]
        self.emit(f"const {T}* _pa = (const {T}*)({base} + {state['off'][0]});")
        self.emit(f"const {T}* _pb = (const {T}*)({base} + {state['off'][1]});")
        self.emit(f"const int _ra = (_wave & {wm - 1}) * {M // wm};")
        self.emit(f"const int _rb = ((_wave >> {lo.log2i(wm)}) & {wn - 1}) * {N // wn};")
        self.emit(f"i16x8 _fa[2][{RM}], _fb[2][{RN}];")
        self.emit("#pragma unroll")
        self.emit(f"for (int _i = 0; _i < {RM}; ++_i) _fa[0][_i] = "
                  f"{self._frag(state, 0, f'_ra + _i * {MI}', '0')};")
        self.emit("#pragma unroll")
        self.emit(f"for (int _j = 0; _j < {RN}; ++_j) _fb[0][_j] = "
                  f"{self._frag(state, 1, f'_rb + _j * {NI}', '0')};")

    def pipe_mma(self, dstmt, state, acc, slot):
        """MFMAs of one stage, double-buffering fragments across k-steps."""
        M, N, K, dt, instr = state["M"], state["N"], state["K"], state["dt"], state["instr"]
        wm, wn = state["wm"], state["wn"]
        MI, NI, KI, kpl, nacc = lo.INSTR[instr]
        Lc = self.mfma_layout(M, N, instr, wm, wn, 1)
        accv = self.init_acc(dstmt, acc, Lc, M, N)
        RM, RN = M // wm // MI, N // wn // NI
        T = dt.ctype
        nks = K // KI
        self.emit("{")
        self.indent += 1
        self.pipe_frags_first(state, slot)
        self.emit("#pragma unroll")
        self.emit(f"for (int _ks = 0; _ks < {nks}; ++_ks) {{")
        self.indent += 1
        self.emit(f"if (_ks + 1 < {nks}) {{")
        self.indent += 1
        self.emit("#pragma unroll")
        self.emit(f"for (int _i = 0; _i < {RM}; ++_i) _fa[(_ks + 1) & 1][_i] = "
                  f"{self._frag(state, 0, f'_ra + _i * {MI}', f'(_ks + 1) * {KI}')};")
        self.emit("#pragma unroll")
        self.emit(f"for (int _j = 0; _j < {RN}; ++_j) _fb[(_ks + 1) & 1][_j] = "
                  f"{self._frag(state, 1, f'_rb + _j * {NI}', f'(_ks + 1) * {KI}')};")
        self.indent -= 1
        self.emit("}")
        self.emit("#pragma unroll")
        self.emit(f"for (int _i = 0; _i < {RM}; ++_i)")
        self.emit("#pragma unroll")
        fa_, fb_ = f"newt::as_frag<{T}>(_fa[_ks & 1][_i])", f"newt::as_frag<{T}>(_fb[_ks & 1][_j])"
        x, y = (fb_, fa_) if self.dot_orient() == "row" else (fa_, fb_)
        self.emit(f"for (int _j = 0; _j < {RN}; ++_j) {accv.var}[_j + {RN} * _i] = "
                  f"newt::mfma_{instr}({x}, {y}, {accv.var}[_j + {RN} * _i]);")
        self.indent -= 1
        self.emit("}")
        self.indent -= 1
        self.emit("}")
        return accv
