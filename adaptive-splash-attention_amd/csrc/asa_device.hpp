// Device-side building blocks shared by the gfx950 kernels of libadasplash.
//
// MFMA conventions (v_mfma_f32_16x16x32_bf16 and v_mfma_f32_16x16x4_f32):
//   A operand: lane L supplies row (L % 16) of A, B operand: column (L % 16)
//   of B; lane group g = L / 16 supplies a fixed set of k slots, the same set
//   for A and B.  A product is therefore correct for any assignment of
//   reduction indices to (g, slot) as long as A and B use the same one; the
//   kernels exploit this to feed an accumulator straight back in as the next
//   product's operand.
//   D (accumulator, 4 floats per lane): element r of lane L is
//   D[4 * (L / 16) + r][L % 16].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace asa {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16;  // bf16 storage (raw bits)
typedef _Float16 h16;  // fp16 storage

constexpr int kWave = 64;
constexpr int kBlock = 64;          // query rows per block == key columns per block
constexpr float kEps = 1e-8f;       // reference EPS (adasplashattention.cu:21)
constexpr float kSentinel = -1e6f;  // empty top-k slot score (adasplashattention.cu:170)

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Rank of the calling lane among the set lanes of m below it.
__device__ __forceinline__ int lane_rank(uint64_t m) {
  return int(__builtin_amdgcn_mbcnt_hi(uint32_t(m >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(m), 0u)));
}

// A packed bf16 pair with the given bits, held in a scalar register that
// the compiler cannot fold into an inline constant.  The empty asm is not
// volatile, so it is no scheduling barrier and can be hoisted out of loops.
__device__ __forceinline__ bf16x2 opaque_bf16x2(uint32_t bits) {
  asm("" : "+s"(bits));
  return __builtin_bit_cast(bf16x2, bits);
}
template <typename V2> __device__ __forceinline__ V2 opaque_pair(uint32_t bits) {
  asm("" : "+s"(bits));
  return __builtin_bit_cast(V2, bits);
}

__device__ __forceinline__ float bf16_to_f32(u16 h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
// Round-to-nearest-even float -> bf16 bits (NaN stays NaN).
__device__ __forceinline__ u16 f32_to_bf16(float f) {
  __bf16 b = static_cast<__bf16>(f);
  return __builtin_bit_cast(u16, b);
}

// ---------------------------------------------------------------------------
// Element access for the two storage types.
// ---------------------------------------------------------------------------
template <typename T> struct Elem;
template <> struct Elem<float> {
  static __device__ __forceinline__ float load(const float* p) { return *p; }
  static __device__ __forceinline__ void store(float* p, float v) { *p = v; }
};
template <> struct Elem<u16> {
  static __device__ __forceinline__ float load(const u16* p) { return bf16_to_f32(*p); }
  static __device__ __forceinline__ void store(u16* p, float v) { *p = f32_to_bf16(v); }
};
template <> struct Elem<h16> {
  static __device__ __forceinline__ float load(const h16* p) { return static_cast<float>(*p); }
  static __device__ __forceinline__ void store(h16* p, float v) { *p = static_cast<h16>(v); }
};

// The two 16-bit storage formats (bf16 as raw bits, fp16): MFMA operand
// vectors, float -> format rounding (nearest even), and the packed-pair dot
// product with fp32 accumulation (v_dot2_f32_bf16 / v_dot2_f32_f16).
template <typename T> struct Half;
template <> struct Half<u16> {
  using v8 = bf16x8;
  using v4 = bf16x4;
  using v2 = bf16x2;
  using scalar = __bf16;
  static __device__ __forceinline__ float dot2(v2 a, v2 b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false);
  }
  // bits of the packed pairs (-1, 0) and (0, -1)
  static constexpr uint32_t kNegLoBits = 0x0000bf80u, kNegHiBits = 0xbf800000u;
};
template <> struct Half<h16> {
  using v8 = f16x8;
  using v4 = f16x4;
  using v2 = f16x2;
  using scalar = _Float16;
  static __device__ __forceinline__ float dot2(v2 a, v2 b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
  }
  static constexpr uint32_t kNegLoBits = 0x0000bc00u, kNegHiBits = 0xbc000000u;
};
template <typename T> constexpr bool is_half = sizeof(T) == 2;

// ---------------------------------------------------------------------------
// Powers.  x^e for x > 0 with the exponent known at compile time by class:
//   kE2 (alpha 1.5 weights), kE1, kE0, kE3, kE4 (alpha 1.25 weights),
//   kEM1 (alpha 2 f'' terms), kEGen (anything else, passed at run time).
// pow_exact rounds once to float (double product chain / double pow), the
// convention the CPU oracle uses too, so the tau recurrence agrees bit-for-bit
// when both see the same top-k values.  pow_fast is used per score in the
// attention passes: identical to pow_exact for kE0/kE1/kE2, within an ulp for
// kE3/kE4, exp2(e log2 x) in hardware for kEGen.
// ---------------------------------------------------------------------------
enum PowClass : int { kE0 = 0, kE1 = 1, kE2 = 2, kE3 = 3, kE4 = 4, kEM1 = 5, kEGen = 6 };

__host__ __device__ inline int pow_class_of(float e) {
  if (e == 0.0f) return kE0;
  if (e == 1.0f) return kE1;
  if (e == 2.0f) return kE2;
  if (e == 3.0f) return kE3;
  if (e == 4.0f) return kE4;
  if (e == -1.0f) return kEM1;
  return kEGen;
}

__device__ __forceinline__ float pow_exact(float x, float e) {
  const double xd = static_cast<double>(x);
  if (e == 2.0f) return static_cast<float>(xd * xd);
  if (e == 1.0f) return x;
  if (e == 0.0f) return 1.0f;
  if (e == 3.0f) return static_cast<float>(xd * xd * xd);
  if (e == 4.0f) { const double x2 = xd * xd; return static_cast<float>(x2 * x2); }
  if (e == -1.0f) return static_cast<float>(1.0 / xd);
  return static_cast<float>(pow(xd, static_cast<double>(e)));
}

// pow_exact with the exponent class fixed at compile time.  For kE2 the
// float product is correctly rounded, hence equal to the double product
// rounded once.
template <int PC>
__device__ __forceinline__ float pow_exact_c(float x, float e) {
  if constexpr (PC == kE2) return x * x;
  else if constexpr (PC == kE1) return x;
  else if constexpr (PC == kE0) return 1.0f;
  else if constexpr (PC == kE3) { const double xd = x; return static_cast<float>(xd * xd * xd); }
  else if constexpr (PC == kE4) { const double x2 = static_cast<double>(x) * x; return static_cast<float>(x2 * x2); }
  else if constexpr (PC == kEM1) return static_cast<float>(1.0 / static_cast<double>(x));
  else return static_cast<float>(pow(static_cast<double>(x), static_cast<double>(e)));
}

template <int PC>
__device__ __forceinline__ float pow_fast(float x, float e) {
  if constexpr (PC == kE2) return x * x;
  else if constexpr (PC == kE1) return x;
  else if constexpr (PC == kE0) return 1.0f;
  else if constexpr (PC == kE3) return static_cast<float>(static_cast<double>(x) * x * x);
  else if constexpr (PC == kE4) { const double x2 = static_cast<double>(x) * x; return static_cast<float>(x2 * x2); }
  else if constexpr (PC == kEM1) return static_cast<float>(1.0 / static_cast<double>(x));
  else return __builtin_amdgcn_exp2f(e * __builtin_amdgcn_logf(x));
}

__device__ __forceinline__ bool finite(float x) { return __builtin_isfinite(x); }

// Score clamp of the reference (adasplashattention.cu:195-197): one
// v_med3_f32, which returns the lower bound for a NaN input, as
// fmaxf(NaN, -10) does (NaN -> -10).
__device__ __forceinline__ float clamp_score(float s) {
  return __builtin_amdgcn_fmed3f(s, -10.0f, 10.0f);
}

// max(u, 0) for u = (alpha - 1) clamp_score(scale s) - tau, the argument of
// every per-score power (adasplashattention.cu:307-312), in two
// instructions per score: v = med3(c s - tau, lo, hi) with
// c = (alpha - 1) scale, lo = max(-10 (alpha - 1) - tau, 0) and
// hi = max(10 (alpha - 1) - tau, 0).  It equals max(u, 0) up to the rounding
// of the fused product (c s - tau is rounded once); a NaN score gives lo,
// which is what the clamp's NaN -> -10 gives.  Rows that get no weight use
// c = lo = hi = 0, so v = 0 for every score.
struct ClippedU {
  float c, nt, lo, hi;
  __device__ __forceinline__ ClippedU(float am1, float scale, float tau, bool valid) {
    c = valid ? am1 * scale : 0.0f;
    nt = valid ? -tau : 0.0f;
    lo = valid ? fmaxf(fmaf(-10.0f, am1, nt), 0.0f) : 0.0f;
    hi = valid ? fmaxf(fmaf(10.0f, am1, nt), 0.0f) : 0.0f;
  }
  __device__ __forceinline__ float operator()(float s) const {
    return __builtin_amdgcn_fmed3f(fmaf(c, s, nt), lo, hi);
  }
};

// ClippedU whose floor is -0 instead of +0 where u can reach it: v is u
// where u > 0 and a zero with the sign bit set elsewhere (u = 0 itself may
// give either zero), so the sign bit tells u <= 0 apart without a compare:
// one v_alignbit per score shifts it into a mask.  Rows that get no weight
// give -0 for every score.  Every power below maps -0 to a zero weight.
struct SignedClip {
  float c, nt, lo, hi;
  __device__ __forceinline__ SignedClip(float am1, float scale, float tau, bool valid) {
    const float l = fmaf(-10.0f, am1, -tau), h = fmaf(10.0f, am1, -tau);
    c = valid ? am1 * scale : 0.0f;
    nt = valid ? -tau : 0.0f;
    lo = valid && l > 0.0f ? l : -0.0f;
    hi = valid && h > 0.0f ? h : -0.0f;
  }
  __device__ __forceinline__ float operator()(float s) const {
    return __builtin_amdgcn_fmed3f(fmaf(c, s, nt), lo, hi);
  }
};

// v^e for v = max(u, 0) from ClippedU: 0 where v = 0, like the reference's
// (u > 0) ? max(u, EPS)^e : 0.  The positive integer classes give 0 at v = 0
// by themselves; they drop the EPS floor, which changes a weight by at most
// EPS = 1e-8.  Other classes keep the floor and zero non-finite results.
template <int PC>
__device__ __forceinline__ float pow_clipped(float v, float e) {
  if constexpr (PC == kE1 || PC == kE2 || PC == kE3 || PC == kE4) {
    return pow_fast<PC>(v, e);
  } else {
    const float r = v > 0.0f ? pow_fast<PC>(fmaxf(v, kEps), e) : 0.0f;
    return finite(r) ? r : 0.0f;
  }
}

// ---------------------------------------------------------------------------
// 64-bit selection keys: larger key == better entry under the order
// (score descending, key index ascending).  High word: order-preserving map
// of the float score (-0 folded onto +0 so that it ties with +0 as a float
// comparison does); low word: ~index.  The empty slot (score -1e6, index -1)
// has low word 0.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t ord_of(float s) {
  const uint32_t u = __float_as_uint(s + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float score_of_ord(uint32_t o) {
  const uint32_t u = (o & 0x80000000u) ? (o & 0x7fffffffu) : ~o;
  return __uint_as_float(u);
}
__device__ __forceinline__ uint64_t make_key(float s, int idx) {
  return (static_cast<uint64_t>(ord_of(s)) << 32) | static_cast<uint32_t>(~static_cast<uint32_t>(idx));
}
__device__ __forceinline__ float key_score(uint64_t k) { return score_of_ord(static_cast<uint32_t>(k >> 32)); }
__device__ __forceinline__ int key_index(uint64_t k) { return static_cast<int>(~static_cast<uint32_t>(k)); }

// XCD-aware block order.  MI355X places block i of a launch on XCD i % 8,
// and each XCD has its own L2.  A 1-D launch of `total` blocks is mapped so
// that the blocks of each XCD cover one contiguous range of tasks (a task
// index is (batch*head) * blocks_per_head + block), which keeps the K/V (or
// Q/dO) tiles of a head in the L2 of the XCD that reads them.
//
// Under the causal mask a block's work grows with its query block (and
// shrinks with its key block), so the query-major kernels walk each head's
// query blocks from the last to the first: the heaviest blocks of a head
// start first and the short ones fill in behind them, which shortens the
// tail of the launch.  The key-major kernels keep ascending key blocks,
// which is already heaviest first.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_task(int i, int total) {
  const int x = i % kXcds, j = i / kXcds;
  const int base = total / kXcds, rem = total % kXcds;
  return x * base + (x < rem ? x : rem) + j;
}

// Heaviest-first order across the heads an XCD serves.  Walking the XCD's
// heads one after another (xcd_task) starts the heavy blocks of its last
// heads near the end, and they set the launch's tail (under the causal
// mask a head's blocks differ several-fold in work).  Here an XCD still
// serves a contiguous range of heads, but its blocks go by weight rank
// (rank 0, the heaviest block of each head, first), heads innermost:
// forward 237 -> 186 us at the headline shape.  Needs BH % 8 == 0, else
// xcd_task's order.  `nblk` blocks per head; returns the block's weight
// rank and its head.
__device__ __forceinline__ void xcd_rank_order(int i, int nblk, int BH, int& rank, int& bh) {
  if (BH % kXcds == 0) {
    const int x = i % kXcds, jj = i / kXcds, hpx = BH / kXcds;
    rank = jj / hpx;
    bh = x * hpx + jj % hpx;
  } else {
    const int task = xcd_task(i, nblk * BH);
    rank = task % nblk;
    bh = task / nblk;
  }
}

// Transposing LDS read (ds_read_b64_tr_b16): in each 16-lane group, lane l
// supplies the address of 4 consecutive bf16 values; lane i receives value
// i % 4 of the rows supplied by lanes 4m + i / 4, m = 0..3.
typedef short short4_lds __attribute__((vector_size(8)));
template <typename T>
__device__ __forceinline__ typename Half<T>::v4 read_tr16(const T* p) {
  typedef __attribute__((address_space(3))) short4_lds lds_v4;
  const short4_lds v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4*)((__attribute__((address_space(3))) T*)(p)));
  return __builtin_bit_cast(typename Half<T>::v4, v);
}

// ---------------------------------------------------------------------------
// Cross-lane moves on the VALU (DPP), no trip through the LDS crossbar.
//   quad_perm 0xB1 / 0x4E / 0x1B: lane i <- lane i^1 / i^2 / i^3 (in quads)
//   row_half_mirror 0x141: lane i <- lane i^7 (in 8-lane half rows)
//   row_mirror 0x140: lane i <- lane i^15 (in 16-lane rows)
//   row_shr:n 0x110+n, row_bcast:15 0x142, row_bcast:31 0x143
// dpp_mov sets bound_ctrl (a lane whose source is out of range reads 0):
// the compiler then folds a move into the VALU operation that consumes it
// (v_add_f32_dpp and the like) instead of issuing both.  The patterns above
// other than row_shr never read out of range.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), CTRL, 0xf, 0xf, true));
}
// lane i <- lane i ^ M
template <int M>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
  if constexpr (M == 1) return dpp_mov<0xB1>(v);
  else if constexpr (M == 2) return dpp_mov<0x4E>(v);
  else if constexpr (M == 3) return dpp_mov<0x1B>(v);
  else if constexpr (M == 4) return dpp_mov<0x1B>(dpp_mov<0x141>(v));  // (i^7)^3
  else if constexpr (M == 7) return dpp_mov<0x141>(v);
  else if constexpr (M == 8) return dpp_mov<0x141>(dpp_mov<0x140>(v)); // (i^15)^7
  else if constexpr (M == 15) return dpp_mov<0x140>(v);
  else return static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), M, 64));
}
template <int M>
__device__ __forceinline__ uint64_t lane_xor64(uint64_t v) {
  const uint32_t lo = lane_xor<M>(static_cast<uint32_t>(v));
  const uint32_t hi = lane_xor<M>(static_cast<uint32_t>(v >> 32));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}
// Whole-wave min / max, result in every lane: DPP partial reductions inside
// 16-lane rows, row broadcasts into lane 63, then readlane.
template <bool kMax>
__device__ __forceinline__ int wave_reduce_minmax(int v) {
  const int id = kMax ? INT32_MIN : INT32_MAX;
  auto op = [](int a, int b) { return kMax ? (a > b ? a : b) : (a < b ? a : b); };
  v = op(v, __builtin_amdgcn_update_dpp(id, v, 0x111, 0xf, 0xf, false));
  v = op(v, __builtin_amdgcn_update_dpp(id, v, 0x112, 0xf, 0xf, false));
  v = op(v, __builtin_amdgcn_update_dpp(id, v, 0x114, 0xf, 0xf, false));
  v = op(v, __builtin_amdgcn_update_dpp(id, v, 0x118, 0xf, 0xf, false));
  v = op(v, __builtin_amdgcn_update_dpp(id, v, 0x142, 0xa, 0xf, false));
  v = op(v, __builtin_amdgcn_update_dpp(id, v, 0x143, 0xc, 0xf, false));
  return __builtin_amdgcn_readlane(v, 63);
}

// Reductions across the four lane groups that share a column of a 16x16
// accumulator (lanes L, L^16, L^32, L^48), on the VALU: v_permlane16_swap
// (v_permlane32_swap) applied to a value and itself leaves, in its two
// results, the lane's value and its partner's at distance 16 (32), in an
// order that depends on the lane.  The operation is applied to that pair,
// so for a commutative operation every lane gets a bit-identical result.
template <typename F>
__device__ __forceinline__ uint32_t group_reduce_bits(uint32_t v, F op) {
  const auto a = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = op(a[0], a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return op(b[0], b[1]);
}
__device__ __forceinline__ float sum_groups(float v) {
  return __uint_as_float(group_reduce_bits(__float_as_uint(v), [](uint32_t x, uint32_t y) {
    return __float_as_uint(__uint_as_float(x) + __uint_as_float(y));
  }));
}

}  // namespace asa
