"""nl.dot lowering onto the CDNA4 matrix cores.

Contract (reference newt/compiler/codegen.py:2174-2201, newt/language.py:161-168):
a[M,K] @ b[K,N] with fp32 accumulation; fp16/bf16/fp32 operands of one dtype;
M, N multiples of 16; K a multiple of 16 (fp16/bf16) or 8 (fp32); `acc`
accumulates; a dot-consumed load used again after a flush point is an error.

Lowering (this backend's own):
  * instruction: v_mfma_f32_16x16x32_{f16,bf16} or 32x32x16 by the kernel's
    shape (DotOps.pick_instr: 16x16x32 for kernels of at most 4 waves and for
    chained row-oriented dots), 16x16x16 when K % 32 != 0 and the tiles are
    not 32-wide; fp32 uses v_mfma_f32_32x32x2f32 / 16x16x4f32 (full fp32, no
    tf32 truncation);
  * orientation: in kernels that reduce rows (softmax-style statistics of a
    dot result) the MFMA computes C^T = B^T A^T so each lane owns one ROW of
    the result and row statistics stay in-lane; elsewhere it computes C = A B
    directly (layouts.mfma_c);
  * operands are staged into LDS as [rows][K] tiles with K contiguous and
    16-byte chunks XOR-swizzled by row (newt::LdsTile), read back as one
    ds_read_b128 (8 halfs) per lane per MFMA;
  * outside a pipelined loop, B ([K,N], usually N-contiguous in memory) is
    staged transposed: global loads stay 16-byte vectors along N and the
    transpose happens on the way into LDS;
  * k-loops of the plain load/load/dot form are software-pipelined across
    iterations with direct-to-LDS copies and transposed LDS reads instead
    (DotPipeline in ops_pipeline.py).
"""

import os

from . import layouts as lo
from . import types as tp
from .values import Block, Const, Fill, LazyLoad, Reg, Scalar, Staged


def _choose_instr(M, N, K, dt, small_first=False):
    """The MFMA instruction for an [M,K] @ [K,N] dot. Both 16-bit shapes run at
    the same rate on gfx950; 16x16x32 (half the latency, twice the
    instructions) is used when small_first says so (see DotOps.dot_geometry)."""
    if dt in (tp.float16, tp.bfloat16):
        mode = os.environ.get("NEWT_MFMA", "")
        if ((mode == "16" or (small_first and mode != "32")) and M % 16 == 0
                and N % 16 == 0 and K % 32 == 0):
            return "16x16x32"
        if M % 32 == 0 and N % 32 == 0 and K % 16 == 0:
            return "32x32x16"
        if K % 32 == 0:
            return "16x16x32"
        return "16x16x16"
    if M % 32 == 0 and N % 32 == 0 and K % 2 == 0:
        return "32x32x2"
    return "16x16x4"


class DotOps:
    prefer_rows = False
    chained_dots = False

    def wave_grid(self, M, N, instr):
        MI = lo.INSTR[instr][0]
        tm, tn = M // MI, N // MI
        best = None
        wm = 1
        while wm <= min(self.W, tm):
            wn = 1
            while wn <= min(self.W // wm, tn):
                used = wm * wn
                sq = -abs((M // wm).bit_length() - (N // wn).bit_length())
                score = (used, wm if self.prefer_rows else sq, sq)
                if best is None or score > best[0]:
                    best = (score, wm, wn)
                wn *= 2
            wm *= 2
        _, wm, wn = best
        return wm, wn, self.W // (wm * wn)

    def dot_geometry(self, node, a, b):
        if not (isinstance(a, Block) and isinstance(b, Block)) or len(a.shape) != 2 or len(b.shape) != 2:
            self.err(node, "dot expects 2D blocks")
        M, K = a.shape
        K2, N = b.shape
        if K != K2:
            self.err(node, f"dot shape mismatch: {a.shape} @ {b.shape}")
        if a.dtype != b.dtype:
            self.err(node, f"dot operands must share a dtype ({a.dtype} vs {b.dtype})")
        dt = a.dtype
        if dt not in (tp.float16, tp.bfloat16, tp.float32):
            self.err(node, f"dot supports fp16/bf16/fp32 inputs, got {dt}")
        KF = 16 if dt != tp.float32 else 8
        if M < 16 or N < 16 or K < KF or M % 16 or N % 16 or K % KF:
            self.err(node, f"dot requires M,N multiples of 16 and K multiple of {KF} "
                           f"(got {M}x{K} @ {K}x{N})")
        instr = self.pick_instr(M, N, K, dt)
        wm, wn, rep = self.wave_grid(M, N, instr)
        return M, N, K, dt, instr, wm, wn, rep

    def pick_instr(self, M, N, K, dt):
        """32x32x16, except for 16x16x32 (same rate, half the latency, half the
        accumulator registers read and written per flop)
        - for a column-oriented dot in a kernel of at most 4 waves (one wave
          per SIMD per workgroup), whose MFMA latency no second wave of the
          workgroup hides. Measured against 32x32x16, one box, back-to-back
          windows: the 4-wave 256x256x32 matmul tile +3.5%; 2048^3 on the
          128x128x64 4-stage tile +1.2% fp16 and +5-7.5% bf16, other 4-wave
          2048^3 tiles +0.6-1.2%; 1024^3 on 64x64x64 +4-5% with 4 stages, -3%
          with 3 (the autotuner chooses between them). Not for 128x128 wave
          tiles over k-steps deeper than 32, whose 16x16x32 fragments spill;
        - for a column-oriented dot of more waves whose waves each hold a tile
          of at least 128x128 over a single 32-deep k-step (8-wave tiles
          below that ran 2.5-27% slower on 16x16x32: 256x128x32, 256x256x32,
          256x256x64 at 4096^3);
        - for every dot of a row-oriented kernel that feeds one dot's result
          into another (flash attention): 16x16x32, whose accumulator feeds
          the next MFMA from registers as 32x32x16's does. At the package
          power limit it ran at an ~11% higher clock for the same power and
          1-3.5% faster on seven of eight attention shapes (2% slower at 1024
          causal keys). Other row-oriented kernels keep 32x32x16.
        NEWT_MFMA=16 / 32 forces the shape wherever it fits."""
        instr = _choose_instr(M, N, K, dt)
        mode = os.environ.get("NEWT_MFMA", "")
        if self.prefer_rows or instr != "32x32x16":
            small = mode == "16" or (self.prefer_rows and self.chained_dots and mode != "32")
            return _choose_instr(M, N, K, dt, small_first=small)
        if mode:
            return _choose_instr(M, N, K, dt, small_first=mode == "16")
        wm, wn, _ = self.wave_grid(M, N, instr)
        big = M // wm >= 128 and N // wn >= 128
        if self.W <= 4:
            # except 128x128 wave tiles over a deeper k-step: their 16x16x32
            # fragments spill (256x256x64 on 4 waves: 292 bytes of scratch)
            return instr if big and K > 32 else _choose_instr(M, N, K, dt, small_first=True)
        if K != 32:
            return instr
        return _choose_instr(M, N, K, dt, small_first=big)

    def dot_orient(self):
        """Row-per-lane accumulators when the kernel reduces rows (their row
        statistics then stay in-lane); plain C = A B orientation otherwise."""
        return "row" if self.prefer_rows else "col"

    def mfma_layout(self, M, N, instr, wm, wn, rep):
        L = lo.mfma_c(M, N, instr, wm, wn, self.dot_orient())
        if rep > 1:
            L = lo.Layout(L.shape, L.reg, L.lane, list(L.wave) + [None] * lo.log2i(rep), L.tag)
        return L

    def init_acc(self, node, acc, Lc, M, N):
        nacc = lo.INSTR[lo.mfma_tag_instr(Lc.tag)[0]][4]
        vt = "f32x16" if nacc == 16 else "f32x4"
        out = self.new_reg(tp.float32, (M, N), Lc, vec=nacc)
        nv = Lc.nslots // nacc
        if acc is None or (isinstance(acc, Fill) and isinstance(acc.value, Const) and acc.value.pyval == 0):
            for i in range(nv):
                self.emit(f"{out.var}[{i}] = ({vt})(0.0f);")
            return out
        if isinstance(acc, (Const, Scalar)):
            acc = Fill(tp.float32, (M, N), acc)
        if acc.shape != (M, N) or acc.dtype != tp.float32:
            self.err(node, f"dot accumulator must be a float32 [{M},{N}] block, got "
                           f"{acc.dtype} {acc.shape}")
        if isinstance(acc, Fill):
            e = self.scalar_expr(acc.value, tp.float32)
            for i in range(nv):
                self.emit(f"{out.var}[{i}] = ({vt})({e});")
            return out
        if isinstance(acc, Reg) and acc.layout == Lc and acc.vec == nacc:
            for i in range(nv):
                self.emit(f"{out.var}[{i}] = {acc.var}[{i}];")
            return out
        if isinstance(acc, LazyLoad):
            acc = self.materialize_load(acc, Lc)
        acc = self.prepare(acc, Lc)
        for s in range(Lc.nslots):
            self.emit(f"{out.at(s)} = {self.ev(acc, Lc, s)};")
        return out

    # ------------------------------------------------------------------ staging
    def staging_layout(self, X):
        """Register layout in which to fetch an operand tile X [R, K] from
        global memory: 16-byte vectors along whichever dim is contiguous."""
        R, K = X.shape
        esz = X.dtype.itemsize
        v = max(1, 16 // esz)
        if isinstance(X, LazyLoad):
            from .values import Affine
            off = X.ptr.offset
            if isinstance(off, Affine):
                ck = off.coefs.get(1)
                cr = off.coefs.get(0)
                if ck is not None and ck.is_const and ck.const == 1:
                    return lo.blocked((R, K), self.W, min(v, K))
                if cr is not None and cr.is_const and cr.const == 1:
                    return lo.blocked((K, R), self.W, min(v, R)).permute((1, 0))
        return lo.blocked((R, K), self.W, min(v, K))

    def stage_tile(self, X, area, dt):
        """Write operand X [R, K] into the LDS tile at `area` (byte offset)."""
        R, K = X.shape
        if isinstance(X, LazyLoad) and X.result is None and not X.poisoned:
            L = self.staging_layout(X)
            r = self.emit_load(X, L)
            X.consumed = True
            if getattr(X, "src", None) is not None:
                X.src.consumed = True
        elif isinstance(X, LazyLoad):
            r = self.materialize_load(X)
        elif isinstance(X, Reg) and not X.vec:
            r = X
        else:
            r = self.to_reg(X, self.default_layout(X.shape))
        if r.dtype != dt:
            r = self.to_reg(r, r.layout, dt)
        self.write_tile(r, area, dt)

    def write_tile(self, r, area, dt):
        L = r.layout
        R, K = L.shape
        T = dt.ctype
        tile = f"newt::LdsTile<{T}, {K}>"
        epc = 16 // dt.itemsize
        kb = 0
        while kb < len(L.reg) and L.reg[kb] == (1, kb):
            kb += 1
        chunk = max(1, min(1 << kb, epc))
        base = self.fresh("lt")
        self.emit(f"{T}* {base} = ({T}*)(_lds + {area});")
        canon = self.canon_cond(L)
        if canon:
            self.emit(f"if ({canon}) {{")
            self.indent += 1
        for s in range(0, L.nslots, chunk):
            if not L.slot_is_canonical(s):
                continue
            rr = self.coord(L, 0, s)
            kk = self.coord(L, 1, s)
            if chunk > 1:
                self.emit(f"newt::store_vec<{T}, {chunk}>({base} + {tile}::off({rr}, {kk}), {r.var} + {s});")
            else:
                self.emit(f"{base}[{tile}::off({rr}, {kk})] = {r.at(s)};")
        if canon:
            self.indent -= 1
            self.emit("}")

    @staticmethod
    def tile_bytes(rows, K, dt):
        epc = 16 // dt.itemsize
        cpr = (K + epc - 1) // epc
        return rows * cpr * 16

    def frag_type(self, dt, kpl):
        if kpl == 1:
            return "float"
        p = "f16" if dt == tp.float16 else "bf16"
        return f"{p}x{kpl}"

    def emit_mma(self, accv, instr, M, N, K, wm, wn, areaA, areaB, dt, ks_lo=0, ks_hi=None):
        MI, NI, KI, kpl, nacc = lo.INSTR[instr]
        RM = M // wm // MI
        RN = N // wn // NI
        T = dt.ctype
        ft = self.frag_type(dt, kpl)
        wmb = lo.log2i(wm)
        rbits = lo.log2i(MI)
        nks = K // KI
        ks_hi = nks if ks_hi is None else ks_hi
        self.emit("{")
        self.indent += 1
        self.emit(f"const {T}* _pa = (const {T}*)(_lds + {areaA});")
        self.emit(f"const {T}* _pb = (const {T}*)(_lds + {areaB});")
        self.emit(f"const int _ra = (_wave & {wm - 1}) * {M // wm} + (_lane & {MI - 1});")
        self.emit(f"const int _rb = ((_wave >> {wmb}) & {wn - 1}) * {N // wn} + (_lane & {NI - 1});")
        self.emit(f"const int _kl = {kpl} * (_lane >> {rbits});")
        self.emit("#pragma unroll")
        self.emit(f"for (int _ks = {ks_lo}; _ks < {ks_hi}; ++_ks) {{")
        self.indent += 1
        self.emit(f"{ft} _fa[{RM}];")
        self.emit(f"{ft} _fb[{RN}];")
        ta = f"newt::LdsTile<{T}, {K}>"
        self.emit("#pragma unroll")
        self.emit(f"for (int _i = 0; _i < {RM}; ++_i) _fa[_i] = "
                  f"*(const {ft}*)(_pa + {ta}::off(_ra + _i * {MI}, _ks * {KI} + _kl));")
        self.emit("#pragma unroll")
        self.emit(f"for (int _j = 0; _j < {RN}; ++_j) _fb[_j] = "
                  f"*(const {ft}*)(_pb + {ta}::off(_rb + _j * {NI}, _ks * {KI} + _kl));")
        self.emit("#pragma unroll")
        self.emit(f"for (int _i = 0; _i < {RM}; ++_i)")
        self.emit("#pragma unroll")
        x, y = ("_fb[_j]", "_fa[_i]") if self.dot_orient() == "row" else ("_fa[_i]", "_fb[_j]")
        self.emit(f"for (int _j = 0; _j < {RN}; ++_j) {accv.var}[_j + {RN} * _i] = "
                  f"newt::mfma_{instr}({x}, {y}, {accv.var}[_j + {RN} * _i]);")
        self.indent -= 1
        self.emit("}")
        self.indent -= 1
        self.emit("}")

    def op_dot(self, node, a, b, acc=None, out_dtype=None, allow_tf32=None):
        if isinstance(a, Staged) or isinstance(b, Staged):
            return self.staged_dot(node, a, b, acc)
        M, N, K, dt, instr, wm, wn, rep = self.dot_geometry(node, a, b)
        Lc = self.mfma_layout(M, N, instr, wm, wn, rep)
        accv = self.init_acc(node, acc, Lc, M, N)
        bA = self.tile_bytes(M, K, dt)
        bB = self.tile_bytes(N, K, dt)
        area = self.lds_arena(bA + bB)
        Bt = self.permute(b, (1, 0))
        self.barrier()
        self.stage_tile(a, area, dt)
        self.stage_tile(Bt, f"({area} + {bA})", dt)
        self.barrier()
        self.emit_mma(accv, instr, M, N, K, wm, wn, area, f"({area} + {bA})", dt)
        return accv

