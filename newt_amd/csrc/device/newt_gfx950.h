// newt_gfx950.h - hand-written device templates for newt kernels on MI355X (gfx950).
//
// Every kernel the newt compiler emits includes this header (hipRTC receives it
// as an in-memory include). Generated code keeps the per-element arithmetic; the
// hardware-specific pieces live here:
//   * 16-byte vector global loads/stores (global_load_dwordx4 / store_dwordx4)
//   * wave64 cross-lane butterflies on the VALU: DPP (quad_perm, row mirrors)
//     and v_permlane16/32_swap; ds_swizzle / ds_bpermute only for partial
//     lane masks
//   * MFMA wrappers for the fp16/bf16/fp32 matrix-core instructions of CDNA4
//   * XOR-swizzled LDS tile addressing for MFMA operand staging
//   * float atomic max as a CAS loop on vector memory
// Nothing here writes through the scalar data cache: every store is a vector
// (global_/ds_) store.
#pragma once

typedef _Float16 f16;
typedef __bf16 bf16;
typedef unsigned int u32;
typedef unsigned long long u64;

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef u32 u32x2 __attribute__((ext_vector_type(2)));
typedef u32 u32x4 __attribute__((ext_vector_type(4)));

namespace newt {

// ---------------------------------------------------------------------------
// Conversions. Round-to-nearest-even both ways, matching torch's casts.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(f16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
__device__ __forceinline__ f16 to_f16(float x) { return (f16)x; }
__device__ __forceinline__ bf16 to_bf16(float x) { return (bf16)x; }

// ---------------------------------------------------------------------------
// exp on the transcendental unit: exp(x) = exp2(x * log2 e) with one rounding
// of the product, then v_exp_f32 (1 ulp). Relative error <= |x| * 1.5 * 2^-24
// + 2^-23, under 8e-6 for every x whose result is a normal float (|x| < 88),
// against ~13 instructions for the library's range-reduced form. +-inf and
// NaN propagate. Two deviations from expf: results below 2^-126 (x < -87.34)
// flush to zero where expf returns a subnormal, and an x within an ulp below
// ln(FLT_MAX) whose product with log2 e rounds to 128.0 gives inf where expf
// gives ~3.4e38.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float exp_f32(float x) {
  return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}

__device__ __forceinline__ float bits_f32(u32 b) { return __builtin_bit_cast(float, b); }
__device__ __forceinline__ u32 f32_bits(float f) { return __builtin_bit_cast(u32, f); }

// ---------------------------------------------------------------------------
// Vector memory access: N elements of T as one global transaction of
// N*sizeof(T) bytes (<= 16). The caller guarantees alignment.
// ---------------------------------------------------------------------------
template <int BYTES> struct raw_vec;
template <> struct raw_vec<1> { typedef unsigned char type; };
template <> struct raw_vec<2> { typedef unsigned short type; };
template <> struct raw_vec<4> { typedef u32 type; };
template <> struct raw_vec<8> { typedef u32x2 type; };
template <> struct raw_vec<16> { typedef u32x4 type; };

template <typename T, int N>
struct vec_t {
  T d[N];
};

template <typename T, int N>
__device__ __forceinline__ void load_vec(const T* __restrict__ p, T* out) {
  typedef typename raw_vec<sizeof(T) * N>::type R;
  R r = *reinterpret_cast<const R*>(p);
  vec_t<T, N> v = __builtin_bit_cast(vec_t<T, N>, r);
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = v.d[i];
}

// load_vec with the non-temporal hint (global_load ... nt): for data that
// no other program reads, so its lines need not stay in the caches.
template <typename T, int N>
__device__ __forceinline__ void load_vec_nt(const T* __restrict__ p, T* out) {
  typedef typename raw_vec<sizeof(T) * N>::type R;
  R r = __builtin_nontemporal_load(reinterpret_cast<const R*>(p));
  vec_t<T, N> v = __builtin_bit_cast(vec_t<T, N>, r);
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = v.d[i];
}

template <typename T, int N>
__device__ __forceinline__ void store_vec(T* __restrict__ p, const T* in) {
  typedef typename raw_vec<sizeof(T) * N>::type R;
  vec_t<T, N> v;
#pragma unroll
  for (int i = 0; i < N; ++i) v.d[i] = in[i];
  *reinterpret_cast<R*>(p) = __builtin_bit_cast(R, v);
}

// store_vec with the non-temporal hint (global_store ... nt): for tiles written
// once at the end of a long compute phase, whose lines should not displace the
// operands other workgroups are still reading through L2.
template <typename T, int N>
__device__ __forceinline__ void store_vec_nt(T* __restrict__ p, const T* in) {
  typedef typename raw_vec<sizeof(T) * N>::type R;
  vec_t<T, N> v;
#pragma unroll
  for (int i = 0; i < N; ++i) v.d[i] = in[i];
  __builtin_nontemporal_store(__builtin_bit_cast(R, v), reinterpret_cast<R*>(p));
}

__device__ __forceinline__ bool aligned(const void* p, int bytes) {
  return (reinterpret_cast<u64>(p) & (u64)(bytes - 1)) == 0;
}

// ---------------------------------------------------------------------------
// Wave64 butterflies. xor_lane<M>(v) returns v from lane (lane ^ M).
//   M = 1, 2  : DPP quad_perm (no LDS traffic)
//   M = 4..16 : ds_swizzle in bitmask mode (and=0x1f, xor=M) inside 32-lane halves
//   M = 32    : ds_bpermute across the two halves
// ---------------------------------------------------------------------------
template <int M>
__device__ __forceinline__ int xor_lane_i32(int v) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "xor mask");
  if constexpr (M == 1) {
    return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);  // quad_perm [1,0,3,2]
  } else if constexpr (M == 2) {
    return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);  // quad_perm [2,3,0,1]
  } else if constexpr (M < 32) {
    return __builtin_amdgcn_ds_swizzle(v, 0x1F | (M << 10));
  } else {
    int lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    return __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, v);
  }
}

template <int M, typename T>
__device__ __forceinline__ T xor_lane(T v) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, xor_lane_i32<M>(__builtin_bit_cast(int, v)));
  } else if constexpr (sizeof(T) == 8) {
    u32x2 w = __builtin_bit_cast(u32x2, v);
    w.x = (u32)xor_lane_i32<M>((int)w.x);
    w.y = (u32)xor_lane_i32<M>((int)w.y);
    return __builtin_bit_cast(T, w);
  } else {
    int w = (int)v;
    return (T)xor_lane_i32<M>(w);
  }
}

template <typename T>
__device__ __forceinline__ T xor_lane_dyn(T v, int m) {
  switch (m) {
    case 1: return xor_lane<1>(v);
    case 2: return xor_lane<2>(v);
    case 4: return xor_lane<4>(v);
    case 8: return xor_lane<8>(v);
    case 16: return xor_lane<16>(v);
    default: return xor_lane<32>(v);
  }
}

// ---------------------------------------------------------------------------
// Reduction combiners. Float max/min follow fmaxf/fminf (NaN-ignoring), as the
// reference's reductions do.
// ---------------------------------------------------------------------------
struct Sum {
  template <typename T> __device__ __forceinline__ static T op(T a, T b) { return a + b; }
};
struct Max {
  __device__ __forceinline__ static float op(float a, float b) { return __builtin_fmaxf(a, b); }
  __device__ __forceinline__ static double op(double a, double b) { return __builtin_fmax(a, b); }
  template <typename T> __device__ __forceinline__ static T op(T a, T b) { return a > b ? a : b; }
};
struct Min {
  __device__ __forceinline__ static float op(float a, float b) { return __builtin_fminf(a, b); }
  __device__ __forceinline__ static double op(double a, double b) { return __builtin_fmin(a, b); }
  template <typename T> __device__ __forceinline__ static T op(T a, T b) { return a < b ? a : b; }
};

// DPP row mirrors: lane i of each 8-lane half row takes lane 7 - i
// (row_half_mirror), of each 16-lane row lane 15 - i (row_mirror).
template <int W>
__device__ __forceinline__ int mirror_lane_i32(int v) {
  static_assert(W == 8 || W == 16, "mirror width");
  return __builtin_amdgcn_mov_dpp(v, W == 8 ? 0x141 : 0x140, 0xF, 0xF, true);
}

// Both members of the lane pair {l & ~M, l | M} (M = 16 or 32) in every lane,
// from one v_permlane{16,32}_swap: swapping the odd rows (M = 16) or the upper
// half (M = 32) of one copy of v with the even rows / lower half of another
// leaves v[l & ~M] in the first copy and v[l | M] in the second.
// With two different values a and b, the same swap leaves x = a[l] where bit
// M of l is clear and b[l & ~M] where it is set, and y = a[l | M] / b[l].
template <int M>
__device__ __forceinline__ void swap_lanes_i32(int a, int b, int& x, int& y) {
  static_assert(M == 16 || M == 32, "pair mask");
  if constexpr (M == 16) {
    auto r = __builtin_amdgcn_permlane16_swap((u32)a, (u32)b, false, false);
    u32 p = r[0], q = r[1];
    x = (int)p;
    y = (int)q;
  } else {
    auto r = __builtin_amdgcn_permlane32_swap((u32)a, (u32)b, false, false);
    u32 p = r[0], q = r[1];
    x = (int)p;
    y = (int)q;
  }
}

template <int M>
__device__ __forceinline__ void pair_lanes_i32(int v, int& lo, int& hi) {
  swap_lanes_i32<M>(v, v, lo, hi);
}

template <int W, typename T>
__device__ __forceinline__ T mirror_lane(T v) {
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, mirror_lane_i32<W>(__builtin_bit_cast(int, v)));
  } else if constexpr (sizeof(T) == 8) {
    u32x2 w = __builtin_bit_cast(u32x2, v);
    w.x = (u32)mirror_lane_i32<W>((int)w.x);
    w.y = (u32)mirror_lane_i32<W>((int)w.y);
    return __builtin_bit_cast(T, w);
  } else {
    return (T)mirror_lane_i32<W>((int)v);
  }
}

template <int M, typename T>
__device__ __forceinline__ void pair_lanes(T v, T& lo, T& hi) {
  if constexpr (sizeof(T) == 4) {
    int a, b;
    pair_lanes_i32<M>(__builtin_bit_cast(int, v), a, b);
    lo = __builtin_bit_cast(T, a);
    hi = __builtin_bit_cast(T, b);
  } else if constexpr (sizeof(T) == 8) {
    u32x2 w = __builtin_bit_cast(u32x2, v), l2, h2;
    int a, b;
    pair_lanes_i32<M>((int)w.x, a, b);
    l2.x = (u32)a;
    h2.x = (u32)b;
    pair_lanes_i32<M>((int)w.y, a, b);
    l2.y = (u32)a;
    h2.y = (u32)b;
    lo = __builtin_bit_cast(T, l2);
    hi = __builtin_bit_cast(T, h2);
  } else {
    int a, b;
    pair_lanes_i32<M>((int)v, a, b);
    lo = (T)a;
    hi = (T)b;
  }
}

template <int M, typename T>
__device__ __forceinline__ void swap_lanes(T a, T b, T& x, T& y) {
  if constexpr (sizeof(T) == 4) {
    int p, q;
    swap_lanes_i32<M>(__builtin_bit_cast(int, a), __builtin_bit_cast(int, b), p, q);
    x = __builtin_bit_cast(T, p);
    y = __builtin_bit_cast(T, q);
  } else if constexpr (sizeof(T) == 8) {
    u32x2 wa = __builtin_bit_cast(u32x2, a), wb = __builtin_bit_cast(u32x2, b), x2, y2;
    int p, q;
    swap_lanes_i32<M>((int)wa.x, (int)wb.x, p, q);
    x2.x = (u32)p;
    y2.x = (u32)q;
    swap_lanes_i32<M>((int)wa.y, (int)wb.y, p, q);
    x2.y = (u32)p;
    y2.y = (u32)q;
    x = __builtin_bit_cast(T, x2);
    y = __builtin_bit_cast(T, y2);
  } else {
    int p, q;
    swap_lanes_i32<M>((int)a, (int)b, p, q);
    x = (T)p;
    y = (T)q;
  }
}

// Butterfly over the lane bits set in MASK (compile-time), combining with Op,
// every step on the VALU (no LDS-pipe swizzle or bpermute) where it can be:
//   bits 0, 1: DPP quad_perm (the xor partner);
//   bit 2 (3): once bits 0-1 (0-2) are reduced, all lanes of a 4- (8-) lane
//     group hold the same value, so the half-row (row) mirror partner, which
//     lies in the other group, gives exactly what the xor partner would;
//     otherwise ds_swizzle's xor;
//   bits 4, 5: the permlane swaps, combining op(v[l & ~M], v[l | M]) in every
//     lane (the xor pair, in one operand order for all lanes).
template <typename Op, int MASK, typename T>
__device__ __forceinline__ T lane_reduce(T v) {
  if constexpr (MASK & 1) v = Op::op(v, xor_lane<1>(v));
  if constexpr (MASK & 2) v = Op::op(v, xor_lane<2>(v));
  if constexpr ((MASK & 7) == 7) v = Op::op(v, mirror_lane<8>(v));
  else if constexpr (MASK & 4) v = Op::op(v, xor_lane<4>(v));
  if constexpr ((MASK & 15) == 15) v = Op::op(v, mirror_lane<16>(v));
  else if constexpr (MASK & 8) v = Op::op(v, xor_lane<8>(v));
  if constexpr (MASK & 16) {
    T lo, hi;
    pair_lanes<16>(v, lo, hi);
    v = Op::op(lo, hi);
  }
  if constexpr (MASK & 32) {
    T lo, hi;
    pair_lanes<32>(v, lo, hi);
    v = Op::op(lo, hi);
  }
  return v;
}

// Two values reduced over the same lane bits, as two lane_reduce calls would,
// with the permlane steps shared (MASK has bit 4 or 5; M1 is 16 when it has
// bit 4, else 32). After the bits below 16 are reduced in each value, one
// swap between a and b combines a's lane pairs where bit M1 of the lane is
// clear and b's where it is set; with both bits, a second step reduces bit 5
// of that mix; one more swap hands every lane both results. Every combine
// takes the lower lane's value first, as lane_reduce does, so the results are
// bit-identical to two lane_reduce calls. Over bits 4 and 5 it issues 3 swaps
// and 2 combines where the two calls issue 4 and 4.
template <typename Op, int MASK, typename T>
__device__ __forceinline__ void lane_reduce2(T& a, T& b) {
  static_assert((MASK & 48) != 0, "lane_reduce2 shares the steps of lane bits 4 and 5");
  constexpr int LOW = MASK & 15;
  constexpr int M1 = (MASK & 16) ? 16 : 32;
  if constexpr (LOW != 0) {
    a = lane_reduce<Op, LOW>(a);
    b = lane_reduce<Op, LOW>(b);
  }
  T x, y;
  swap_lanes<M1>(a, b, x, y);
  T c = Op::op(x, y);
  if constexpr (M1 == 16 && (MASK & 32)) {
    T lo, hi;
    pair_lanes<32>(c, lo, hi);
    c = Op::op(lo, hi);
  }
  pair_lanes<M1>(c, a, b);
}

// ---------------------------------------------------------------------------
// Atomics (vector memory). atomic_max on float is a CAS loop.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void atomic_max_f32(float* p, float v) {
  u32* up = reinterpret_cast<u32*>(p);
  u32 old = __hip_atomic_load(up, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  while (!(bits_f32(old) >= v)) {
    u32 assumed = old;
    old = atomicCAS(up, assumed, f32_bits(v));
    if (old == assumed) break;
  }
}

template <typename T>
__device__ __forceinline__ void atomic_add(T* p, T v) { atomicAdd(p, v); }
template <typename T>
__device__ __forceinline__ void atomic_max(T* p, T v) { atomicMax(p, v); }
__device__ __forceinline__ void atomic_max(float* p, float v) { atomic_max_f32(p, v); }

// ---------------------------------------------------------------------------
// MFMA wrappers (CDNA4). Names spell M x N x K; operands are the per-lane
// fragments, C is the accumulator fragment. Lane layouts (per instruction, for
// lane l, A is the MFMA's left operand [M x K], B its right operand [K x N]):
//   32x32xK (K=16 fp16/bf16, 8 elems/lane): A[l%32][8*(l/32)+e], B[8*(l/32)+e][l%32]
//   16x16xK (K=32 fp16/bf16, 8 elems/lane): A[l%16][8*(l/16)+e], B[8*(l/16)+e][l%16]
//   32x32x8 / 16x16x16 (4 elems/lane):      k = 4*(l/32 or l/16) + e
//   32x32x2 / 16x16x4 f32 (1 elem/lane):    k = l/32 or l/16
//   C 32x32: C[8*(v/4) + 4*(l/32) + v%4][l%32];  C 16x16: C[4*(l/16) + v][l%16]
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x16 mfma_32x32x16(f16x8 a, f16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_16x16x32(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_32x32x8(f16x4 a, f16x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x8f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_32x32x8(bf16x4 a, bf16x4 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(__builtin_bit_cast(i16x4, a),
                                                  __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_16x16x16(f16x4 a, f16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_16x16x16(bf16x4 a, bf16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4, a),
                                                   __builtin_bit_cast(i16x4, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma_32x32x2(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_16x16x4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// LDS operand tiles. An MFMA operand tile of ROWS x KD elements of T is stored
// row-major with the reduction dim contiguous (so direct-to-LDS loads keep
// each row's bytes in consecutive lanes); its 16-byte chunks are XOR swizzled
// by row so the per-lane 16-byte fragment reads spread over the LDS banks.
// gfx950 has 64 banks x 4 B; measured with SQ_LDS_BANK_CONFLICT, a
// ds_read_b128 is served 16 lanes per cycle, lane l in cycle
// (parity(l & 0b011100), bit 5 of l), so two lanes conflict when they read
// the same 16-byte bank slot (address mod 256) in the same cycle. The key of
// row r is a function of the row bits above those that place it inside a
// 256-byte bank line (SHIFT) and is chosen so that neither fragment pattern
// (16x16x32: lane -> row l % 16, chunk l / 16; 32x32x16: row l % 32, chunk
// l / 32) puts two lanes of one cycle on one slot:
//   64-byte rows:  q ^ ((q & 1) << 1), q = (r >> 2) & 3;
//   128-byte rows: (r >> 1) & 7;
//   256-byte rows: r & 15 (every key of fewer bits leaves a conflict: the
//   key's null space must avoid the lane offsets that share a cycle).
// All three are conflict-free for both patterns.
// ---------------------------------------------------------------------------
template <typename T, int KD>
struct LdsTile {
  static constexpr int EPC = 16 / (int)sizeof(T);          // elements per chunk
  static constexpr int CPR = (KD + EPC - 1) / EPC;          // chunks per row
  static constexpr int ROW_BYTES = CPR * 16;
  static constexpr int SWZ = CPR >= 8 ? 7 : (CPR >= 4 ? 3 : (CPR >= 2 ? 1 : 0));
  static constexpr int SHIFT = ROW_BYTES >= 256 ? 0 : (ROW_BYTES == 128 ? 1 : (ROW_BYTES == 64 ? 2 : 3));
  __host__ __device__ __forceinline__ static int key(int r) {
    const int q = (r >> SHIFT) & SWZ;
    if constexpr (CPR == 4) return q ^ ((q & 1) << 1);
    else if constexpr (CPR == 16) return r & 15;
    else return q;
  }
  // element offset of (row r, reduction index k)
  __host__ __device__ __forceinline__ static int off(int r, int k) {
    int c = k / EPC;
    int pc = c ^ key(r);
    return r * (CPR * EPC) + pc * EPC + (k % EPC);
  }
  static constexpr int elems(int rows) { return rows * CPR * EPC; }
};

template <typename T, int N>
__device__ __forceinline__ void lds_read(const T* base, int off, T* out) {
  load_vec<T, N>(base + off, out);
}

// Inverse of LdsTile::off at 16-byte granularity: the (row, first k) whose
// chunk sits in physical chunk `slot` of the tile (used to aim direct-to-LDS
// loads, whose destination is fixed by the lane index).
template <typename T, int KD>
__host__ __device__ __forceinline__ void lds_tile_slot(int slot, int& r, int& k) {
  typedef LdsTile<T, KD> L;
  r = slot / L::CPR;
  k = ((slot % L::CPR) ^ L::key(r)) * L::EPC;
}

// ---------------------------------------------------------------------------
// LDS operand tiles stored with the ROW index contiguous: a [KD][RD] array of
// 16-bit elements (RD = rows of the [R, K] operand view, RD >= 32). This is how
// an operand whose rows are contiguous in global memory (B of a row-major
// A @ B) lands in LDS with plain 16-byte writes; fragments are read back
// transposed with ds_read_b64_tr_b16, 32 lanes (256 bytes) per LDS cycle.
// The 32-byte units (16 rows) of each k-row are XOR swizzled so that the
// k-rows one such cycle touches fall in distinct units of the 64 banks:
//   32-row instructions: 4 consecutive k-rows x 32 rows (two units each);
//   16-row instructions: k-rows kk..kk+3 and kk+8..kk+11 x 16 rows.
// k % 4 picks the 64-byte quarter (rows of >= 256 bytes; shorter rows already
// place consecutive k-rows in different quarters) and bit SB of k the 32-byte
// half of the quarter. SB = 3 serves the 16-row fragments above; SB = 2 serves
// the 16-row fragments in the permuted accumulator order (lds_frag_r_perm16),
// whose 32 lanes read k-rows kk..kk+7. 32-row fragments are conflict-free
// under either.
// ---------------------------------------------------------------------------
template <typename T, int RD, int SB = 3>
struct LdsTileR {
  static_assert(sizeof(T) == 2 && RD >= 32 && RD % 32 == 0, "R-major tiles hold >= 32 16-bit rows");
  static_assert(SB == 2 || SB == 3, "swizzle bit is 2 or 3");
  static constexpr int ROW_BYTES = RD * 2;
  static constexpr int LOG_ROWS_PER_256 = ROW_BYTES >= 256 ? 0 : (ROW_BYTES == 128 ? 1 : 2);
  __host__ __device__ __forceinline__ static int swz(int k) {
    return (((k & 3) >> LOG_ROWS_PER_256) << 1) | ((k >> SB) & 1);
  }
  __host__ __device__ __forceinline__ static int off(int k, int r) {
    return k * RD + (((r >> 4) ^ swz(k)) << 4) + (r & 15);
  }
  // (k, first r) of the 8-element chunk at physical chunk index `slot`
  __host__ __device__ __forceinline__ static void slot(int s, int& k, int& r) {
    k = s / (RD / 8);
    const int pe = (s % (RD / 8)) * 8;
    r = (((pe >> 4) ^ swz(k)) << 4) | (pe & 15);
  }
};

// fp32 operand tiles stored with the row index contiguous: a [KD][RD] array of
// floats (RD >= 64). Fragments of the fp32 MFMA are read one float per lane
// (ds_read_b32), lanes 0-31 from k-row kk+t and lanes 32-63 from k-row
// kk+4+t of the same 32 rows; the 128-byte halves of a k-row are swapped by
// bit 2 of k so those two k-rows fall in different halves of the 64 banks.
template <int RD>
struct LdsTileR32 {
  static_assert(RD >= 64 && RD % 64 == 0, "fp32 R-major tiles hold >= 64 rows");
  __host__ __device__ __forceinline__ static int off(int k, int r) {
    return k * RD + (r ^ (((k >> 2) & 1) << 5));
  }
  // (k, first r) of the 4-float chunk at physical chunk index `slot`
  __host__ __device__ __forceinline__ static void slot(int s, int& k, int& r) {
    k = s / (RD / 4);
    r = ((s % (RD / 4)) * 4) ^ (((k >> 2) & 1) << 5);
  }
};

typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// One MFMA operand fragment (8 consecutive k of one operand row per lane) from
// an R-major tile. MI is the instruction's row tile (32 or 16): lane l gets
// row r0 + (l % MI) and k = kk + 8 * (l / MI) + 0..7. Each ds_read_b64_tr_b16
// lets a group of 16 lanes read a 4(k) x 16(r) sub-block and hands lane i the
// four k values of row (group base + i).
template <int MI>
__host__ __device__ __forceinline__ void frag_r_coords(int r0, int kk, int lane, int& kr, int& cb) {
  const int i = lane & 15;
  cb = r0 + ((lane & (MI - 1)) & ~15) + 4 * (i & 3);
  kr = kk + 8 * (lane / MI) + (i >> 2);
}

template <typename T, int RD, int MI, int SB = 3>
__device__ __forceinline__ i16x8 lds_frag_r(const T* tile, int r0, int kk, int lane) {
  typedef LdsTileR<T, RD, SB> L;
  int kr, cb;
  frag_r_coords<MI>(r0, kk, lane, kr, cb);
  const __attribute__((address_space(3))) char* b =
      (const __attribute__((address_space(3))) char*)tile;
  i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(b + 2 * L::off(kr, cb)));
  i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(b + 2 * L::off(kr + 4, cb)));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Same fragment with the k order permuted the way a 32x32 MFMA accumulator
// holds its columns (lane half h owns columns 4h..4h+3 and 8+4h..8+4h+3 of
// each 16): element e of lane half h is k = kk + 8*(e/4) + 4h + e%4. A
// probability tile produced by one MFMA can then feed the next one straight
// from registers, with the other operand read in the matching order.
__host__ __device__ __forceinline__ void frag_r_perm32_coords(int r0, int kk, int lane, int& kr,
                                                              int& cb) {
  const int i = lane & 15;
  cb = r0 + (lane & 16) + 4 * (i & 3);
  kr = kk + 4 * (lane >> 5) + (i >> 2);
}

template <typename T, int RD, int SB = 3>
__device__ __forceinline__ i16x8 lds_frag_r_perm32(const T* tile, int r0, int kk, int lane) {
  typedef LdsTileR<T, RD, SB> L;
  int kr, cb;
  frag_r_perm32_coords(r0, kk, lane, kr, cb);
  const __attribute__((address_space(3))) char* b =
      (const __attribute__((address_space(3))) char*)tile;
  i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(b + 2 * L::off(kr, cb)));
  i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(b + 2 * L::off(kr + 8, cb)));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// The same for a 16x16 MFMA accumulator, whose lane group g = l / 16 holds
// columns 4g..4g+3 of each 16: element e of lane group g is
// k = kk + 16*(e/4) + 4g + e%4, so one 16x16x32 MFMA contracts the columns of
// two adjacent accumulator tiles.
__host__ __device__ __forceinline__ void frag_r_perm16_coords(int r0, int kk, int lane, int& kr,
                                                              int& cb) {
  const int i = lane & 15;
  cb = r0 + 4 * (i & 3);
  kr = kk + 4 * (lane >> 4) + (i >> 2);
}

template <typename T, int RD, int SB = 2>
__device__ __forceinline__ i16x8 lds_frag_r_perm16(const T* tile, int r0, int kk, int lane) {
  typedef LdsTileR<T, RD, SB> L;
  int kr, cb;
  frag_r_perm16_coords(r0, kk, lane, kr, cb);
  const __attribute__((address_space(3))) char* b =
      (const __attribute__((address_space(3))) char*)tile;
  i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(b + 2 * L::off(kr, cb)));
  i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(b + 2 * L::off(kr + 16, cb)));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Fragment of a K-major tile (LdsTile): lane l gets row r0 + (l % MI) and
// k = kk + 8 * (l / MI) + 0..7 as one ds_read_b128.
template <int MI>
__host__ __device__ __forceinline__ void frag_k_coords(int r0, int kk, int lane, int& r, int& k) {
  r = r0 + (lane & (MI - 1));
  k = kk + 8 * (lane / MI);
}

__host__ __device__ __forceinline__ void frag_k32f_coords(int r0, int kk, int lane, int& r,
                                                          int& k) {
  r = r0 + (lane & 31);
  k = kk + 4 * (lane >> 5);
}

template <typename T, int KD, int MI>
__device__ __forceinline__ i16x8 lds_frag_k(const T* tile, int r0, int kk, int lane) {
  int r, k;
  frag_k_coords<MI>(r0, kk, lane, r, k);
  return *(const i16x8*)(tile + LdsTile<T, KD>::off(r, k));
}

// fp32 fragment group of a K-major tile for the 32x32x2 MFMA in the permuted
// k order: lane l gets row r0 + (l % 32) and k = kk + 4 * (l / 32) + 0..3, one
// float for each of four MFMAs (MFMA t contracts k = kk + t and kk + 4 + t).
template <int KD>
__device__ __forceinline__ f32x4 lds_frag_k32f(const float* tile, int r0, int kk, int lane) {
  int r, k;
  frag_k32f_coords(r0, kk, lane, r, k);
  return *(const f32x4*)(tile + LdsTile<float, KD>::off(r, k));
}

// Direct global -> LDS copy of 16 bytes per lane (global_load_lds_dwordx4):
// lane l's 16 bytes land at wave_dst + 16 * l. wave_dst must be the same for
// every lane of the wave.
__device__ __forceinline__ void lds_dma16(const void* g, void* wave_dst) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)g,
                                   (__attribute__((address_space(3))) void*)wave_dst, 16, 0, 0);
}

// The same copy from base + lane_bytes through a raw buffer descriptor
// (buffer_load_dwordx4 ... offen lds). base must be the same for every lane
// (it lives in scalar registers); lane_bytes is each lane's own 32-bit byte
// offset, which stays in one VGPR across a loop where the 64-bit form needs a
// VGPR pair and a 64-bit add per copy. Descriptor: stride 0, num_records
// 0xFFFFFFFF (callers keep lane_bytes below 2^31, so the range check never
// drops a lane), word 3 = 0x00020000 (32-bit data format, the raw-buffer word
// of gfx9-family CDNA parts).
__device__ __forceinline__ void lds_dma16_buf(const void* base, unsigned lane_bytes, void* wave_dst) {
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, -1, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)wave_dst, 16,
                                           lane_bytes, 0, 0, 0);
}

// Wait until at most N vector-memory operations of this wave are outstanding
// (s_waitcnt vmcnt(N); expcnt and lgkmcnt left unconstrained).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Workgroup barrier without the fence __syncthreads() carries. That fence
// waits for all of this wave's LDS reads (lgkmcnt(0)) before the wave
// arrives, including a fragment prefetch of a pipeline stage that the
// barrier does not release. Callers wait for the copies the barrier publishes
// (wait_vmcnt) first; reads of the stage the barrier releases have all been
// consumed by then. The "memory" clobber keeps the compiler from moving
// memory accesses across it.
__device__ __forceinline__ void barrier_nofence() { asm volatile("s_barrier" ::: "memory"); }

template <typename T> struct frag8;
template <> struct frag8<f16> { typedef f16x8 type; };
template <> struct frag8<bf16> { typedef bf16x8 type; };

template <typename T>
__device__ __forceinline__ typename frag8<T>::type as_frag(i16x8 v) {
  return __builtin_bit_cast(typename frag8<T>::type, v);
}

// K-major tile fragment in the permuted 32x32 accumulator k order (see
// lds_frag_r_perm32): two 8-byte reads per lane.
template <typename T, int KD>
__device__ __forceinline__ i16x8 lds_frag_k_perm32(const T* tile, int r0, int kk, int lane) {
  typedef LdsTile<T, KD> L;
  const int r = r0 + (lane & 31);
  const int k = kk + 4 * (lane >> 5);
  i16x4 lo = *(const i16x4*)(tile + L::off(r, k));
  i16x4 hi = *(const i16x4*)(tile + L::off(r, k + 8));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// K-major tile fragment in the permuted 16x16 accumulator k order (see
// lds_frag_r_perm16): two 8-byte reads per lane.
template <typename T, int KD>
__device__ __forceinline__ i16x8 lds_frag_k_perm16(const T* tile, int r0, int kk, int lane) {
  typedef LdsTile<T, KD> L;
  const int r = r0 + (lane & 15);
  const int k = kk + 4 * (lane >> 4);
  i16x4 lo = *(const i16x4*)(tile + L::off(r, k));
  i16x4 hi = *(const i16x4*)(tile + L::off(r, k + 16));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Eight 16-bit register values as one MFMA operand fragment.
template <typename T>
__device__ __forceinline__ i16x8 pack8(T a0, T a1, T a2, T a3, T a4, T a5, T a6, T a7) {
  typename frag8<T>::type v = {a0, a1, a2, a3, a4, a5, a6, a7};
  return __builtin_bit_cast(i16x8, v);
}

}  // namespace newt
