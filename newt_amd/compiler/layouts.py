"""Register layouts of block values on a wave64 workgroup.

A block of power-of-two shape is spread over the workgroup's hardware index
bits: the register slot index of a thread (`reg` bits), the lane within its
wave64 (`lane`, 6 bits) and the wave within the workgroup (`wave`). A layout
maps every hardware bit to one logical coordinate bit `(dim, bit)` or to None
(the value is replicated along that hardware bit). Each logical bit of the
shape is produced by exactly one hardware bit.

This one representation covers:
  * the coalesced elementwise layout (groups of VEC consecutive elements per
    thread, groups strided over the workgroup) - the reference's group-cyclic
    layout (newt/compiler/codegen.py:250-288), re-derived for wave64;
  * MFMA accumulator and operand fragments (fixed lane maps of the matrix
    instructions);
  * slices left by reductions (reduced hardware bits become replicated).

Reshape, expand_dims and transposition only relabel logical bits (no data
moves); reductions classify the reduced dimension's bits by hardware source
(register -> in-thread, lane -> DPP/swizzle butterfly, wave -> LDS);
broadcasts are free when the source is already replicated along the new bits,
otherwise values go through LDS.
"""

import math

LANE_BITS = 6
WAVE = 64


def log2i(n):
    n = int(n)
    if n <= 0 or n & (n - 1):
        raise ValueError(f"{n} is not a power of two")
    return n.bit_length() - 1


def dim_bits(shape):
    return [log2i(d) for d in shape]


def flat_to_dimbit(shape):
    """List: flat row-major bit k -> (dim, bit)."""
    out = []
    for d in range(len(shape) - 1, -1, -1):
        for b in range(log2i(shape[d])):
            out.append((d, b))
    return out


def dimbit_to_flat(shape):
    return {db: k for k, db in enumerate(flat_to_dimbit(shape))}


class Layout:
    __slots__ = ("shape", "reg", "lane", "wave", "tag", "_key")

    def __init__(self, shape, reg, lane, wave, tag="blocked"):
        self.shape = tuple(int(s) for s in shape)
        self.reg = tuple(reg)
        self.lane = tuple(lane)
        self.wave = tuple(wave)
        self.tag = tag
        assert len(self.lane) == LANE_BITS, self.lane
        seen = [b for b in self.reg + self.lane + self.wave if b is not None]
        want = set((d, b) for d, n in enumerate(self.shape) for b in range(log2i(n)))
        if len(seen) != len(set(seen)) or set(seen) != want:
            raise AssertionError(f"bad layout for {self.shape}: {self.reg} {self.lane} {self.wave}")
        self._key = (self.shape, self.reg, self.lane, self.wave)

    # -- basic properties ----------------------------------------------------
    @property
    def nslots(self):
        return 1 << len(self.reg)

    @property
    def num_waves(self):
        return 1 << len(self.wave)

    @property
    def numel(self):
        return math.prod(self.shape) if self.shape else 1

    def key(self):
        return self._key

    def __eq__(self, other):
        return isinstance(other, Layout) and self._key == other._key

    def __hash__(self):
        return hash(self._key)

    def __repr__(self):
        return f"Layout[{self.tag}]{self.shape} reg={self.reg} lane={self.lane} wave={self.wave}"

    def lane_rep_mask(self):
        return sum(1 << i for i, b in enumerate(self.lane) if b is None)

    def wave_rep_mask(self):
        return sum(1 << i for i, b in enumerate(self.wave) if b is None)

    def reg_rep_mask(self):
        return sum(1 << i for i, b in enumerate(self.reg) if b is None)

    def slot_is_canonical(self, s):
        return (s & self.reg_rep_mask()) == 0

    # -- coordinates ---------------------------------------------------------
    def reg_coord(self, s, d):
        """Compile-time contribution of slot s's register bits to dim d."""
        v = 0
        for i, b in enumerate(self.reg):
            if b is not None and b[0] == d and (s >> i) & 1:
                v |= 1 << b[1]
        return v

    def hw_coord_terms(self, d, lane="_lane", wave="_wave"):
        """C expression terms of the lane/wave contribution to dim d."""
        terms = []
        for src, bits in ((lane, self.lane), (wave, self.wave)):
            for i, b in enumerate(bits):
                if b is not None and b[0] == d:
                    if b[1] >= i:
                        terms.append(f"(({src} & {1 << i}) << {b[1] - i})")
                    else:
                        terms.append(f"(({src} & {1 << i}) >> {i - b[1]})")
        return terms

    def reg_bits_of_dim(self, d):
        return [(i, b[1]) for i, b in enumerate(self.reg) if b is not None and b[0] == d]

    # -- relabelings (free) --------------------------------------------------
    def _relabel(self, fn, shape, tag=None):
        m = lambda b: None if b is None else fn(b)
        return Layout(shape, [m(b) for b in self.reg], [m(b) for b in self.lane],
                      [m(b) for b in self.wave], tag or self.tag)

    def expand_dims(self, axis):
        shape = list(self.shape)
        shape.insert(axis, 1)
        return self._relabel(lambda b: (b[0] + (b[0] >= axis), b[1]), shape)

    def squeeze(self, axis):
        assert self.shape[axis] == 1
        shape = list(self.shape)
        del shape[axis]
        return self._relabel(lambda b: (b[0] - (b[0] > axis), b[1]), shape)

    def permute(self, perm):
        """New dim i is old dim perm[i]."""
        inv = {old: new for new, old in enumerate(perm)}
        shape = [self.shape[p] for p in perm]
        return self._relabel(lambda b: (inv[b[0]], b[1]), shape)

    def reshape(self, shape):
        f_old = dimbit_to_flat(self.shape)
        f_new = flat_to_dimbit(tuple(shape))
        return self._relabel(lambda b: f_new[f_old[b]], shape)

    def reduce(self, axis):
        """Layout after reducing `axis` away; reduced lane/wave bits become
        replicated, reduced register bits disappear."""
        keep_reg = [b for b in self.reg if b is None or b[0] != axis]
        shape = list(self.shape)
        del shape[axis]

        def m(b):
            if b is None or b[0] == axis:
                return None
            return (b[0] - (b[0] > axis), b[1])

        return Layout(shape, [m(b) for b in keep_reg], [m(b) for b in self.lane],
                      [m(b) for b in self.wave], self.tag + "/slice")

    def broadcast_into(self, shape):
        """If values in this layout (shape broadcastable to `shape`, same rank)
        can serve every element of `shape` without moving data, return the
        target layout that results; else None. New bits go to replicated
        hardware bits (lane/wave first, then new register bits)."""
        if len(shape) != len(self.shape):
            return None
        need = []
        for d, (a, b) in enumerate(zip(self.shape, shape)):
            if a == b:
                continue
            if a != 1:
                return None
            need += [(d, k) for k in range(log2i(b))]
        lane = list(self.lane)
        wave = list(self.wave)
        for i in range(len(lane)):
            if lane[i] is None and need:
                lane[i] = need.pop(0)
        for i in range(len(wave)):
            if wave[i] is None and need:
                wave[i] = need.pop(0)
        reg = list(self.reg) + need
        return Layout(shape, reg, lane, wave, self.tag)


def slot_map(src, dst):
    """If every element that layout `dst` places at (slot s, lane, wave) is held
    by the same thread under layout `src` (whose shape is dst.shape with some
    dims possibly 1 = broadcast), return a function s -> src slot. Else None."""
    if len(src.shape) != len(dst.shape) or len(src.wave) != len(dst.wave):
        return None
    bcast = set()
    for d, (a, b) in enumerate(zip(src.shape, dst.shape)):
        if a != b:
            if a != 1:
                return None
            bcast.add(d)

    def proj(b):
        if b is None or b[0] in bcast:
            return None
        return b

    for hs, hd in ((src.lane, dst.lane), (src.wave, dst.wave)):
        for bs, bd in zip(hs, hd):
            if bs != proj(bd):
                return None
    # every src register bit must be produced by a dst register bit
    where = {}
    for i, b in enumerate(dst.reg):
        pb = proj(b)
        if pb is not None:
            where[pb] = i
    mapping = []
    for j, b in enumerate(src.reg):
        if b is None:
            mapping.append(None)  # replicated slot: use copy 0
            continue
        if b not in where:
            return None
        mapping.append(where[b])

    def f(s):
        t = 0
        for j, i in enumerate(mapping):
            if i is not None and (s >> i) & 1:
                t |= 1 << j
        return t

    return f


def blocked(shape, num_waves, vec):
    """Coalesced elementwise layout: VEC consecutive row-major elements per
    register group, groups spread over lanes, then waves, then more groups."""
    flat = flat_to_dimbit(shape)
    nb = len(flat)
    wb = log2i(num_waves)
    vb = log2i(vec)
    k = 0
    reg = []
    for _ in range(vb):
        reg.append(flat[k] if k < nb else None)
        k += 1 if k < nb else 0
    lane = []
    for _ in range(LANE_BITS):
        if k < nb:
            lane.append(flat[k])
            k += 1
        else:
            lane.append(None)
    wave = []
    for _ in range(wb):
        if k < nb:
            wave.append(flat[k])
            k += 1
        else:
            wave.append(None)
    while k < nb:
        reg.append(flat[k])
        k += 1
    return Layout(shape, reg, lane, wave, "blocked")


# ---------------------------------------------------------------------------
# MFMA layouts. Instructions are named (MI, NI, KI, elems-per-lane).
#
# Every dot is issued in "row-per-lane" orientation: the MFMA computes
# C^T = B^T A^T, so the lane index carries the ROW of the newt-level result and
# the accumulator registers carry columns. Row vectors produced by reducing a
# dot result along axis 1 then live one row per lane, and broadcasting them
# back over any other dot result with the same row tiling is free.
# ---------------------------------------------------------------------------

INSTR = {
    # name: (MI, NI, KI, kpl (k elems per lane per step), accum regs)
    "32x32x16": (32, 32, 16, 8, 16),
    "16x16x32": (16, 16, 32, 8, 4),
    "32x32x8": (32, 32, 8, 4, 16),
    "16x16x16": (16, 16, 16, 4, 4),
    "32x32x2": (32, 32, 2, 1, 16),
    "16x16x4": (16, 16, 4, 1, 4),
}


def mfma_c(M, N, instr, wm, wn, orient="row"):
    """Accumulator layout of an [M, N] dot result computed by a wm x wn grid of
    waves, each owning an (M/wm) x (N/wn) sub-tile of instr tiles.

    orient="row": the MFMA computes C^T = B^T A^T, so a lane holds (part of)
    one ROW of C and registers walk columns - row reductions stay in-lane.
    orient="col": the MFMA computes C = A B directly, a lane holds part of one
    COLUMN and registers walk rows (tag suffix "c")."""
    MI, NI, KI, kpl, nacc = INSTR[instr]
    assert MI == NI
    rb = log2i(MI)  # bits covered by one instruction tile along the lane dim (5 or 4)
    ld, rd = (0, 1) if orient == "row" else (1, 0)
    lane = [None] * LANE_BITS
    reg = []
    for i in range(rb):
        lane[i] = (ld, i)
    if MI == 32:
        # lane bit 5 -> bit 2 of the register dim; regs 0,1 -> bits 0,1; regs 2,3 -> bits 3,4
        lane[5] = (rd, 2)
        reg += [(rd, 0), (rd, 1), (rd, 3), (rd, 4)]
    else:
        # lane bits 4,5 -> bits 2,3 of the register dim; regs 0,1 -> bits 0,1
        lane[4] = (rd, 2)
        lane[5] = (rd, 3)
        reg += [(rd, 0), (rd, 1)]
    mb, nb = log2i(M), log2i(N)
    wmb, wnb = log2i(wm), log2i(wn)
    # per-wave repetitions: cols first (adjacent tiles along N), then rows
    rep_n = list(range(rb, nb - wnb))
    rep_m = list(range(rb, mb - wmb))
    reg += [(1, b) for b in rep_n] + [(0, b) for b in rep_m]
    wave = [(0, b) for b in range(mb - wmb, mb)] + [(1, b) for b in range(nb - wnb, nb)]
    return Layout((M, N), reg, lane, wave, f"mfma{instr}" + ("" if orient == "row" else "c"))


def mfma_tag_instr(tag):
    """(instruction, orientation) of an MFMA accumulator layout tag, or None for
    any other layout (operand fragments, reduction slices, blocked layouts)."""
    if not tag.startswith("mfma") or tag.startswith("mfmaop") or "/" in tag:
        return None
    body = tag[4:]
    orient = "row"
    if body.endswith("c"):
        body, orient = body[:-1], "col"
    return (body, orient) if body in INSTR else None


def mfma_operand(R, K, instr, wr, nwaves_other=1, other_first=False):
    """Register layout of a dot operand [R, K] (R = M for A, N for B): the
    per-lane fragment of the MFMA, for a grid where `wr` waves split R and
    `nwaves_other` waves (the other result dim) hold replicated copies."""
    MI, NI, KI, kpl, nacc = INSTR[instr]
    rb = log2i(MI)
    lane = [None] * LANE_BITS
    for i in range(rb):
        lane[i] = (0, i)
    kb = log2i(kpl)
    reg = [(1, b) for b in range(kb)]
    # remaining lane bits carry k bits kb..
    k = kb
    for i in range(rb, LANE_BITS):
        lane[i] = (1, k)
        k += 1
    kbits_total = log2i(K)
    rbits_total = log2i(R)
    wrb = log2i(wr)
    reg += [(1, b) for b in range(k, kbits_total)]
    reg += [(0, b) for b in range(rb, rbits_total - wrb)]
    ob = log2i(nwaves_other)
    rwave = [(0, b) for b in range(rbits_total - wrb, rbits_total)]
    if other_first:
        wave = [None] * ob + rwave
    else:
        wave = rwave + [None] * ob
    return Layout((R, K), reg, lane, wave, f"mfmaop{instr}")
