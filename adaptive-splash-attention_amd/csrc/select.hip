// Score pass: scores, exact per-row top-k and block mask (tau follows in
// tau_kernel, from the sorted top-k values this pass writes, or in
// tau_compact_kernel, which builds the CSR lists in the same launch).
//
// Reference: build_mask_kernel + insert_topk + entmax_threshold
// (adasplashattention.cu:35-217), one thread per query that scans every key
// and keeps a sorted top-k by insertion.  Here one 256-thread block owns one
// 64-row query block of one (batch, head).  During the sweeps the waves
// split the keys, not the rows: wave w loads keys 16w..16w+15 of each
// visible key tile straight from L2 into MFMA operand registers (KQuarter,
// two tiles in flight, no barrier per tile; with 16-bit inputs sweep 1
// reads them through a per-wave LDS ring filled by global_load_lds) and
// scores them against all 64 rows.  The top-k is found in two sweeps over the
// visible key blocks instead of by insertion:
//
//   sweep 1  every score updates one of 64*R running "class maxima" of its
//            row (one v_med3 per score; class = key offset in the tile x
//            tile ordinal mod R).  Distinct classes hold distinct keys, so
//            if at least k class maxima are >= x, at least k keys score
//            >= x, and every top-k key scores >= x.  The class maxima meet
//            in LDS and an 8-step bisection per row (wave w: rows
//            16w..16w+15) finds such an x close to the k-th largest.
//   sweep 2  the scores are recomputed and every key scoring >= x is
//            appended, as (index, score bits), to the row's list in LDS
//            (about 1.05-1.15 k keys per row on random data).  If a row
//            overflows its list, the k-th best stored key becomes an exact
//            key threshold and the block sweeps again for those rows; each
//            round drops at least cap - k keys, so the rounds are bounded
//            (select_round_bound) and the status word reports them.
//   select   each row's candidates are sorted (segmented bitonic sort across
//            lanes, descending key order = score desc, index asc) when the
//            caller asked for top-k indices; otherwise only the values are
//            sorted and the top-k key set is the candidates above the k-th
//            value plus its lowest-index ties.  The first k values go to the
//            workspace for tau_kernel, padded with the empty slot (-1e6).
//   finish   the rows' top-k key blocks are OR-ed into a bitmap per 32-row
//            half of the block: the 64-row mask is their union, and with
//            32-row mask blocks each half's row is written as well.
//
// Sweep filters compare raw dot products (scale > 0) against a threshold
// widened by a relative margin, so that no key whose clamped, scaled score
// reaches the bound is missed; the exact score is only formed for the keys
// that pass.  With caller-given scores (asa_select_from_scores) or a
// non-positive scale the sweeps work on the exact scores directly.
#include <climits>
#include <type_traits>

#include "asa_compact.hpp"
#include "asa_device.hpp"
#include "asa_launch.hpp"
#include "asa_stage.hpp"
#include "asa_tiles.hpp"

namespace asa {
namespace {

constexpr int kThreads = 256;  // four waves of 16 query rows

__device__ __forceinline__ int wave_min(int v) { return wave_reduce_minmax<false>(v); }
__device__ __forceinline__ int wave_max(int v) { return wave_reduce_minmax<true>(v); }
// Reductions over the 4 lanes (L, L^16, L^32, L^48) that share a row.
__device__ __forceinline__ int group_sum(int v) {
  return int(group_reduce_bits(uint32_t(v), [](uint32_t x, uint32_t y) { return x + y; }));
}
__device__ __forceinline__ float group_min(float v) {
  return __uint_as_float(group_reduce_bits(__float_as_uint(v), [](uint32_t x, uint32_t y) {
    return __float_as_uint(fminf(__uint_as_float(x), __uint_as_float(y)));
  }));
}
__device__ __forceinline__ float group_max(float v) {
  return __uint_as_float(group_reduce_bits(__float_as_uint(v), [](uint32_t x, uint32_t y) {
    return __float_as_uint(fmaxf(__uint_as_float(x), __uint_as_float(y)));
  }));
}
// max(m, x) for a running maximum m (never NaN) and an MFMA result x, in
// one v_med3_f32: med3(x, m, +inf) is the larger of x and m, and m when x
// is NaN (NaN loses).  `pinf` is +inf held in a register the compiler
// cannot see into (with a constant +inf it rewrites the med3 as fmaxf(),
// which canonicalises both operands first).  The MFMA results are only
// ever read by compiler-visible instructions, never by inline asm, so the
// compiler keeps the MFMA-to-VALU wait states it owes those reads.
__device__ __forceinline__ float vmax(float m, float x, float pinf) {
  return __builtin_amdgcn_fmed3f(x, m, pinf);
}
__device__ __forceinline__ float opaque_inf() {
  float v = __builtin_inff();
  asm("" : "+v"(v));
  return v;
}
// c + (x >= t).
__device__ __forceinline__ uint32_t count_ge(uint32_t c, float x, float t) {
  return c + (x >= t ? 1u : 0u);
}
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

constexpr int ilog2(int x) { return x <= 1 ? 0 : 1 + ilog2(x / 2); }

// Descending bitonic sort of independent segments of 8*LS keys: lanes
// [s*LS, (s+1)*LS) hold segment s, element e = (lane % LS) * 8 + p in v[p].
// Keys are distinct except for the padding value 0.  Exchanges between
// lanes use DPP moves for lane distances below 16.
template <int LS>
__device__ __forceinline__ void segment_sort_desc(uint64_t (&v)[8], int lane) {
  const int i = lane & (LS - 1);
  static_for<1, ilog2(8 * LS) + 1>([&](auto sc) {
    constexpr int size = 1 << decltype(sc)::value;
    static_for<0, decltype(sc)::value>([&](auto jc) {
      constexpr int j = (size >> 1) >> decltype(jc)::value;
      if constexpr (j >= 8) {
        const bool lower = (i & (j >> 3)) == 0;  // e & j depends on the lane only
        for (int p = 0; p < 8; ++p) {
          const int e = i * 8 + p;
          const uint64_t o = lane_xor64<(j >> 3)>(v[p]);
          const bool keep_max = ((e & size) == 0) == lower;
          const bool gt = v[p] > o;
          v[p] = (keep_max == gt) ? v[p] : o;
        }
      } else {
        for (int p = 0; p < 8; ++p) {
          const int pp = p ^ j;
          if (pp > p) {
            const bool desc = ((i * 8 + p) & size) == 0;
            const uint64_t a = v[p], b = v[pp];
            const bool sw = desc ? (a < b) : (a > b);
            v[p] = sw ? b : a;
            v[pp] = sw ? a : b;
          }
        }
      }
    });
  });
}

// Descending sort of independent segments of 8*LS 32-bit values, no
// payload: lanes [s*LS, (s+1)*LS) hold segment s, element e = (lane % LS) * 8
// + p in v[p].  Bitonic network in the form where every comparator puts the
// larger value first: the first step of each merge compares e with its
// mirror e ^ (size - 1), the later steps e with e ^ j.  One max and one min
// per in-lane pair; a lane move, max or min and a select per element across
// lanes.
template <int LS>
__device__ __forceinline__ void segment_sort_desc32(uint32_t (&v)[8], int lane) {
  const int i = lane & (LS - 1);
  static_for<1, ilog2(8 * LS) + 1>([&](auto sc) {
    constexpr int size = 1 << decltype(sc)::value;
    static_for<0, decltype(sc)::value>([&](auto jc) {
      constexpr int j = (size >> 1) >> decltype(jc)::value;
      constexpr bool mirror = j == (size >> 1);
      if constexpr (j >= 8) {
        // partner lane i ^ M, element 7 - p (mirror) or p
        constexpr int M = mirror ? (size - 1) >> 3 : j >> 3;
        const bool lower = (i & (mirror ? (size >> 4) : (j >> 3))) == 0;
        uint32_t o[8];
        for (int p = 0; p < 8; ++p) o[p] = lane_xor<M>(v[mirror ? 7 - p : p]);
        for (int p = 0; p < 8; ++p) v[p] = lower ? max(v[p], o[p]) : min(v[p], o[p]);
      } else {
        for (int p = 0; p < 8; ++p) {
          const int pp = mirror ? (p ^ (size - 1)) : (p ^ j);
          if (pp > p) {
            const uint32_t a = v[p], b = v[pp];
            v[p] = max(a, b);
            v[pp] = min(a, b);
          }
        }
      }
    });
  });
}

// tau from the sorted top-k values of one row (best first), s(j) for
// j < k, following the reference recurrence step by step
// (adasplashattention.cu:51-125): bracket from the extreme kept values,
// midpoint start, up to five rounds of {f, f', f'' over the leading positive
// terms; exit when |f| < 1e-4; Halley step with the reference's f''
// coefficient a(a + 1 - alpha); bracket midpoint when the step leaves the
// bracket; bracket update from f at the new point; clamp}.  No contraction,
// powers in the exponent classes of alpha (pow_exact_c): bit-identical to
// the CPU oracle on equal inputs.  KMAX > 0: the caller guarantees k <= KMAX
// and s(j) is a compile-time-indexed register, so the loops are unrolled.
template <int AC, int KMAX, typename S>
__device__ float entmax_tau(S s, int k, float alpha_in) {
#pragma clang fp contract(off)
  constexpr int PA = AlphaPow<AC>::P, P1 = AlphaPow<AC>::W, P2 = AlphaPow<AC>::V;
  // register-resident values and closed-form powers: evaluate every slot
  constexpr bool kFlat = KMAX > 0 && AC != kAGen;
  const float alpha = fmaxf(1.05f, fminf(alpha_in, 3.0f));
  const float am1 = alpha - 1.0f;
  const float a = 1.0f / am1;
  const float e1 = (2.0f - alpha) * a;
  const float e2 = (3.0f - 2.0f * alpha) * a;
  const float c2 = a * ((a + 1.0f) - alpha);
  const float top = s(0);
  const float bottom = s(k - 1);
  float lo = am1 * bottom - 2.0f;
  float hi = am1 * top + 2.0f;
  float tau = 0.5f * (lo + hi);
  for (int it = 0; it < 5; ++it) {
    float f = -1.0f, df = 0.0f, d2f = 0.0f;
    // one term of f, f', f''; false once the terms end
    auto term = [&](int j) {
      if (j >= k) return false;
      const float u = am1 * s(j) - tau;
      if (u <= 0.0f) return false;
      const float ue = fmaxf(u, kEps);
      float t = pow_exact_c<PA>(ue, a);
      if (!finite(t)) t = 0.0f;
      f = f + t;
      const float t1 = -a * pow_exact_c<P1>(ue, e1);
      if (finite(t1)) df = df + t1;
      const float t2 = c2 * pow_exact_c<P2>(ue, e2);
      if (finite(t2)) d2f = d2f + t2;
      return true;
    };
    if constexpr (kFlat) {
      // Branch-free over all KMAX slots: the values are sorted, so u is
      // non-increasing in j and the terms the recurrence stops before are
      // exactly the ones with u <= 0 (or j >= k).  Those add +0.0f, which
      // leaves every sum unchanged (none of them can be -0.0f), so the
      // result is bit-identical to the early-exit loop.  The closed-form
      // powers cannot overflow here (u <= (alpha-1)(10 + 1e6) + 10 with
      // u^e, e in {-1, 0, ..., 4}, and u >= EPS), so the finiteness tests
      // of the general loop always pass and are left out.
#pragma unroll
      for (int j = 0; j < KMAX; ++j) {
        const float u = am1 * s(j) - tau;
        const bool on = j < k && !(u <= 0.0f);
        const float ue = fmaxf(u, kEps);
        f = f + (on ? pow_exact_c<PA>(ue, a) : 0.0f);
        df = df + (on ? -a * pow_exact_c<P1>(ue, e1) : 0.0f);
        d2f = d2f + (on ? c2 * pow_exact_c<P2>(ue, e2) : 0.0f);
      }
    } else if constexpr (KMAX > 0) {
#pragma unroll
      for (int j = 0; j < KMAX; ++j)
        if (!term(j)) break;
    } else {
      for (int j = 0; term(j); ++j) {
      }
    }
    if (fabsf(f) < 1e-4f) break;
    float next = tau;
    if (fabsf(df) > kEps) {
      const float den = 2.0f * df * df - f * d2f;
      if (fabsf(den) > kEps) next = tau - 2.0f * f * df / den;
    }
    if (!(next >= lo && next <= hi)) next = 0.5f * (lo + hi);
    float gsum = -1.0f;
    auto gterm = [&](int j) {
      if (j >= k) return false;
      const float u = am1 * s(j) - next;
      if (u <= 0.0f) return false;
      const float t = pow_exact_c<PA>(fmaxf(u, kEps), a);
      if (finite(t)) gsum = gsum + t;
      return true;
    };
    if constexpr (kFlat) {
#pragma unroll
      for (int j = 0; j < KMAX; ++j) {
        const float u = am1 * s(j) - next;
        gsum = gsum + (j < k && !(u <= 0.0f) ? pow_exact_c<PA>(fmaxf(u, kEps), a) : 0.0f);
      }
    } else if constexpr (KMAX > 0) {
#pragma unroll
      for (int j = 0; j < KMAX; ++j)
        if (!gterm(j)) break;
    } else {
      for (int j = 0; gterm(j); ++j) {
      }
    }
    if (gsum > 0.0f) lo = next;
    else hi = next;
    tau = next;
    tau = fmaxf(tau, bottom * am1 - 10.0f);
    tau = fminf(tau, top * am1 + 10.0f);
  }
  return tau;
}

// Lowest sweep value that a key scoring >= `th` can have.  `exact`: the
// sweep sees exact scores.  Otherwise it sees raw dot products r with
// score = clamp(fl(r * scale)), scale > 0, and the bound is widened by a
// relative margin far above the rounding error of that product.
__device__ __forceinline__ float sweep_floor(float th, bool exact, float scale) {
  if (exact) return th;
  if (!(th > -10.0f)) return -__builtin_inff();
  const double x = (static_cast<double>(th) - fabs(static_cast<double>(th)) * 0x1p-18 - 1e-30) /
                   static_cast<double>(scale);
  float f = static_cast<float>(x);
  if (static_cast<double>(f) > x) f = nextafterf(f, -__builtin_inff());
  return f;
}


enum SweepMode : int {
  kRawDots = 0,     // MFMA dot products, scale > 0: filters on raw dots
  kExactScores = 1, // MFMA dot products converted to exact scores (scale <= 0)
  kGivenScores = 2  // caller-given scores
};

// How the score pass addresses K: rows of exactly D elements at hd = D
// (compile-time strides), rows at a run-time stride with hd = D, or any
// stride and hd (column tests).
enum KLayout : int { kKDense = 0, kKRows = 1, kKGeneral = 2 };

// One wave's quarter of a 64-key tile (keys 16 w .. 16 w + 15) as MFMA A
// operands, loaded straight from global memory (L2) into registers: lane
// (c, g) holds key 16 w + c at the head-dimension slots that rows_x_frag
// gives lane group g.  product() forms, for each of the four 16-row groups
// cb of the query block, the scores of the quarter's keys against rows
// 16 cb + c with the same operands in the same accumulation order as the
// attention passes' rows_x_frag, so every score is bit-identical to theirs.
// acc[cb][r] is the score of key 16 w + 4 g + r and row 16 cb + c.
template <typename T, int D> struct KQuarter;
template <typename T, int D> struct KQuarter16 {
  using V8 = typename Half<T>::v8;
  V8 a[D / 32];
  // Keys >= NK read key 0 instead: they lie in partially visible tiles,
  // where the visibility test discards their scores, so no zeroing (and no
  // wait for the load where it is issued) is needed.  (This register path
  // loads 16 half rows per instruction, a third of the L2 rate of whole-row
  // loads; a whole-row load with the operands rebuilt by two DPP row
  // rotations per register measured the same sweep time, which the
  // candidate appends, not the loads, set.)
  // KL (KLayout): rows of exactly D elements (kKDense), or rows snb bytes
  // apart (32-bit offsets from the head's first row, which the C ABI
  // bounds below 2^31) with hd = D (kKRows) or with columns >= hd read as
  // zero (kKGeneral).
  template <int KL>
  __device__ __forceinline__ void load(const T* Kb, int key, int NK, uint32_t snb, int hd, int g) {
    const int kk = key < NK ? key : 0;
    if constexpr (KL != kKDense) {
      const unsigned char* src = reinterpret_cast<const unsigned char*>(Kb) + (uint32_t(kk) * snb + 16u * g);
      for (int s = 0; s < D / 32; ++s)
        a[s] = KL == kKRows || 32 * s + 8 * g < hd ? *reinterpret_cast<const V8*>(src + 64 * s) : V8{};
    } else {
      const T* src = Kb + size_t(kk) * D + 8 * g;
      for (int s = 0; s < D / 32; ++s) a[s] = *reinterpret_cast<const V8*>(src + 32 * s);
    }
  }
  __device__ __forceinline__ void product(f32x4 (&acc)[4], const RowFrag<T, D> (&qf)[4]) const {
    for (int cb = 0; cb < 4; ++cb) acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < D / 32; ++s)
      for (int cb = 0; cb < 4; ++cb) acc[cb] = mfma(a[s], qf[cb].v[s], acc[cb]);
  }
};
template <int D> struct KQuarter<u16, D> : KQuarter16<u16, D> {};
template <int D> struct KQuarter<h16, D> : KQuarter16<h16, D> {};
template <int D> struct KQuarter<float, D> {
  f32x4 a[D / 16];
  template <int KL>
  __device__ __forceinline__ void load(const float* Kb, int key, int NK, uint32_t snb, int hd, int g) {
    const int kk = key < NK ? key : 0;
    if constexpr (KL != kKDense) {
      const unsigned char* src = reinterpret_cast<const unsigned char*>(Kb) + (uint32_t(kk) * snb + 16u * g);
      for (int j = 0; j < D / 16; ++j)
        a[j] = KL == kKRows || 16 * j + 4 * g < hd ? *reinterpret_cast<const f32x4*>(src + 64 * j) : f32x4{};
    } else {
      const float* src = Kb + size_t(kk) * D + 4 * g;
      for (int j = 0; j < D / 16; ++j) a[j] = *reinterpret_cast<const f32x4*>(src + 16 * j);
    }
  }
  __device__ __forceinline__ void product(f32x4 (&acc)[4], const RowFrag<float, D> (&qf)[4]) const {
    for (int cb = 0; cb < 4; ++cb) acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < D / 16; ++j)
      for (int cb = 0; cb < 4; ++cb)
        for (int r = 0; r < 4; ++r) acc[cb] = mfma(a[j][r], qf[cb].v[j][r], acc[cb]);
  }
};

// LDS layout, shared by the kernel and the host-side size query.  The class
// maxima exchanged between the sweeps share their bytes with the candidate
// lists (they are read before the first candidate is written).
struct SelLayout {
  int cand, cm, scm, scr, tk, tkey, fl, cnt, ctl, bits, vlist, total;
};
__host__ __device__ inline int align_up(int x, int a) { return (x + a - 1) / a * a; }
// Class sets per (row, position) of sweep 1: 4 tighten the sweep-2 floor
// (fewer candidates) but double the class-maxima exchange in LDS; up to
// k = 64 the exchange at 2 sets keeps two select blocks per compute unit
// (at d = 128, k = 64: 68 KB of LDS and 199 VGPRs against 86 KB and 257
// for 4 sets, measured 11.8 against 17.4 ms at the c4 shape).
__host__ __device__ inline int classes_per_lane(int k) { return k <= 64 ? 2 : 4; }
// Sweep-2 value scratch: 16 floats per lane, the lane's 16-byte chunk j
// stored at chunk j ^ ((lane >> 1) & 3), so that the 8 lanes a 16-byte
// store serves per cycle hit distinct banks.
constexpr int kScrStride = 16;
__host__ __device__ inline SelLayout sel_layout(int k, int cap, int nKB) {
  SelLayout l;
  const int R = classes_per_lane(k);
  l.scm = 64 * R + 4;  // floats per row of the class-maxima exchange (+4: rows 4 banks apart)
  const int cand_bytes = kBlock * cap * 8;
  const int cm_bytes = kBlock * l.scm * 4;
  const int scr_bytes = kThreads * kScrStride * 4;
  const int tk_bytes = k * kBlock * 4;
  l.cand = 0;
  l.cm = 0;
  // the value scratch (sweeps) and the sorted top-k values (emission) share bytes
  l.scr = align_up(cand_bytes > cm_bytes ? cand_bytes : cm_bytes, 16);
  l.tk = l.scr;
  l.tkey = l.scr + align_up(scr_bytes > tk_bytes ? scr_bytes : tk_bytes, 16);
  l.fl = l.tkey + kBlock * 8;
  l.cnt = l.fl + kBlock * 4;
  l.ctl = l.cnt + kBlock * 4;
  l.bits = l.ctl + 16;
  l.vlist = l.bits + align_up(2 * ((nKB + 31) / 32) * 4, 16);  // one bitmap per 32-row half
  l.total = l.vlist + align_up(nKB * 4, 16);
  return l;
}

// Overflow rounds a row can need.  Round 0 stores the first `cap` of its c_0
// candidates; the k-th best stored key T_1 then excludes at least the cap - k
// stored keys below it, so round 1 finds c_1 <= c_0 - (cap - k) keys >= T_1,
// and so on: with c_0 <= NK, at most 2 + (NK - cap) / (cap - k) rounds end
// with every candidate stored.
__host__ __device__ inline int select_round_bound(int NK, int k, int cap) {
  return 2 + (NK > cap ? (NK - cap) / (cap - k) + 1 : 0);
}

// Score pass of one (batch, head) and 64-row query block; 4 waves.  Wave w
// multiplies its quarter of every visible key tile with all 64 rows (no LDS
// staging, no barrier inside a sweep); lane (c, g) sees rows 16 cb + c and
// keys 16 w + 4 g + r of each tile.  R class maxima per (lane, row, r)
// give 64 R classes per row.
// Waves per SIMD the headline variant (bf16, d = 64, two classes per lane)
// is held to: three blocks of its ~50 KB of LDS fit a CU, and 168 VGPRs
// let three waves share a SIMD (one more VGPR would drop it to two).
// Sweep 1's LDS ring (16-bit inputs): tiles in flight per wave, and its
// bytes (four waves x tiles x 16 keys x D x 2 bytes).  It fits below
// sel_layout's tkey for every k: the class-maxima exchange alone takes
// 64 (64 R + 4) floats, and the value scratch 16 KiB after it.
template <int D, int R>
constexpr int ring_tiles() { return (D == 128 && R == 2) ? 3 : 4; }
template <int D, int R>
constexpr int ring_bytes() { return 4 * ring_tiles<D, R>() * 32 * D; }

template <typename T, int D, int R>
constexpr int select_waves_per_simd() { return sizeof(T) == 2 && D == 64 && R == 2 ? 3 : 1; }

// KL: the K layout (KLayout).  With hd = D (kKDense, kKRows) there are no
// column tests, and with 16-bit inputs sweep 1 reads K through the LDS ring
// (whose loads read whole rows).
template <typename T, int D, int MODE, int R, int KL>
__global__ __launch_bounds__(kThreads, (select_waves_per_simd<T, D, R>())) void select_kernel(SelectParams p) {
  constexpr bool kExact = MODE != kRawDots;
  constexpr bool kTiles = MODE != kGivenScores;
  constexpr int UR = R > 2 ? R : 2;  // sweep-1 unroll: class of a tile = ordinal % R
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int k = p.d.k, NQ = p.d.NQ, NK = p.d.NK, nKB = p.d.nKB, nQB = p.d.nQB;
  const int cap = p.cap;
  const int nbw = (nKB + 31) >> 5;
  const SelLayout lay = sel_layout(k, cap, nKB);
  uint64_t* s_cand = reinterpret_cast<uint64_t*>(smem + lay.cand);
  float* s_cm = reinterpret_cast<float*>(smem + lay.cm);
  float* s_tk = reinterpret_cast<float*>(smem + lay.tk);
  uint64_t* s_tkey = reinterpret_cast<uint64_t*>(smem + lay.tkey);
  float* s_fl = reinterpret_cast<float*>(smem + lay.fl);
  uint32_t* s_cnt = reinterpret_cast<uint32_t*>(smem + lay.cnt);
  uint32_t* s_ctl = reinterpret_cast<uint32_t*>(smem + lay.ctl);
  uint32_t* s_bits = reinterpret_cast<uint32_t*>(smem + lay.bits);
  int32_t* s_vlist = reinterpret_cast<int32_t*>(smem + lay.vlist);
  // Slot of candidate e of row r: rows XOR-ed with bits 3-5 of e (moved to
  // row bits 1-3), so that the 8 lanes reading entries e = 8i + pp of one
  // row, and the lanes of two adjacent rows, fall in 16 distinct 8-byte banks.
  auto cslot = [](int e, int r) { return e * kBlock + (r ^ (((e >> 3) & 7) << 1)); };

  const int t = threadIdx.x, w = t >> 6, L = t & 63, g = L >> 4, c = L & 15;
  float* s_scr = reinterpret_cast<float*>(smem + lay.scr) + t * kScrStride;  // this lane's
  const int scr_sw = ((L >> 1) & 3) << 2;  // chunk swizzle, in floats
  int brank, bh;
  xcd_rank_order(blockIdx.x, nQB, p.d.BH, brank, bh);
  const int qb = nQB - 1 - brank, q0 = qb * kBlock;  // heaviest first
  const size_t grow0 = size_t(bh) * NQ + q0;  // global index of the block's row 0
  const float scale = p.d.scale;

  // The lane's rows 16 cb + c.
  bool rowok[4];
  int qpos[4];
  for (int cb = 0; cb < 4; ++cb) {
    rowok[cb] = q0 + 16 * cb + c < NQ;
    qpos[cb] = rowok[cb] ? p.q_idx[grow0 + 16 * cb + c] : 0;
  }
  // Position range of the valid rows of the whole block (lane L <-> row L).
  const bool lv = q0 + L < NQ;
  const int lpos = lv ? p.q_idx[grow0 + L] : 0;
  const int qmax_blk = wave_max(lv ? lpos : INT_MIN);
  const int qmin_blk = wave_min(lv ? lpos : INT_MAX);

  if (t < kBlock) s_cnt[t] = 0u;
  if (t < 4) s_ctl[t] = 0u;
  for (int i = t; i < 2 * nbw; i += kThreads) s_bits[i] = 0u;

  const int32_t* kidx = p.k_idx + size_t(bh) * NK;
  // Visible key blocks in ascending order, entry = block | class << 24, with
  // class 1 (partially visible: per-key tests needed) or 2 (every key
  // visible to every row), from the blocks' position bounds.
  if (w == 0) {
    const int2* kbnd = p.kbounds + size_t(bh) * nKB;
    int n = 0;
    for (int base = 0; base < nKB; base += kWave) {
      const int kt = base + L;
      int v = 0;
      if (kt < nKB) {
        const int2 kb = kbnd[kt];
        v = kb.x > qmax_blk ? 0 : ((kb.y > qmin_blk || (kt + 1) * kBlock > NK) ? 1 : 2);
      }
      const uint64_t m = __ballot(v != 0);
      const int before = __builtin_popcountll(m & ((uint64_t(1) << L) - 1));
      if (v != 0) s_vlist[n + before] = kt | (v << 24);
      n += __builtin_popcountll(m);
    }
    if (L == 0) s_ctl[1] = uint32_t(n);
  }
  __syncthreads();
  const int nvis = int(s_ctl[1]);

  RowFrag<T, D> qf[4];  // Q^T operands: row 16 cb + c in column c of the products
  const T* Kb = nullptr;
  if constexpr (kTiles) {
    const T* Qh = static_cast<const T*>(p.q) + head_at(p.lq, bh, p.d.H);
    for (int cb = 0; cb < 4; ++cb)
      qf[cb].load(Qh + size_t(rowok[cb] ? q0 + 16 * cb + c : 0) * p.lq.sn, rowok[cb], L, p.d.hd);
    Kb = static_cast<const T*>(p.k) + head_at(p.lk, bh, p.d.H);
  }
  const uint32_t ksnb = uint32_t(p.lk.sn) * uint32_t(sizeof(T));  // K row stride, bytes (GENERAL loads)
  const int kq0 = 16 * w + c;  // the lane's A-operand key within a tile

  // One pass over the visible key blocks: body(u, kt, visb, acc) for each,
  // u = (ordinal of the block) % U known at compile time.  The K quarters of
  // the next two tiles are in flight while a tile is used.  In partially
  // visible tiles bit 15 - (4 cb + r) of visb is cleared and acc set to
  // -inf where key 16 w + 4 g + r is not visible to row 16 cb + c (visb is
  // 0xffff for a whole tile); the body is called once, after the masking,
  // so its code is not repeated per case.  The first 64 list entries are
  // held one per lane.
  const int vl0 = L < nvis ? s_vlist[L] : 0;
  auto entry = [&](int i) {
    return i < kWave ? __builtin_amdgcn_readlane(vl0, i) : __builtin_amdgcn_readfirstlane(s_vlist[i]);
  };
  // Per tile, after its scores are formed: the visibility masking, then
  // body(u, kb0, visb, acc).  The padding of the last group of U tiles
  // (i >= nvis: no key visible, key limit INT_MIN) takes the partial
  // tiles' path: a separate path that set acc to constants made the
  // compiler copy acc between register sets on every whole tile.
  auto finish = [&](auto uc, int i, int e, f32x4(&acc)[4], auto&& body) __attribute__((always_inline)) {
    const int kb0 = (e & 0xffffff) * kBlock + 16 * w + 4 * g;  // the lane's first key
    if constexpr (MODE == kExactScores)
      for (int cb = 0; cb < 4; ++cb)
        for (int r = 0; r < 4; ++r) acc[cb][r] = clamp_score(acc[cb][r] * scale);
    uint32_t visb = 0xffffu;
    if (i >= nvis || (e >> 24) == 1) {  // wave-uniform
      const int klim = i < nvis ? NK : INT_MIN;
      for (int r = 0; r < 4; ++r) {
        const int key = kb0 + r;
        const int kp = key < klim ? kidx[key] : INT_MAX;
        for (int cb = 0; cb < 4; ++cb)
          if (!(key < klim && kp <= qpos[cb])) {
            visb &= ~(1u << (15 - (4 * cb + r)));
            acc[cb][r] = -__builtin_inff();
          }
      }
    }
    body(uc, kb0, visb, acc);
  };
  auto sweep = [&](auto u_tag, auto&& body) {
    constexpr int U = decltype(u_tag)::value;
    if (nvis == 0) return;  // block-uniform
    KQuarter<T, D> kq[2];
    auto fetch = [&](KQuarter<T, D>& f, int e) {
      f.template load<KL>(Kb, (e & 0xffffff) * kBlock + kq0, NK, ksnb, p.d.hd, g);
    };
    // The loads are unconditional (past the end of the list they repeat its
    // last tile), so the number in flight is the same on every path and the
    // waits before a tile's products cover that tile's loads only.
    int ent[2] = {entry(0), entry(nvis > 1 ? 1 : 0)};  // the tiles in kq[0], kq[1]
    if constexpr (kTiles) {
      // issued in the loop's order (kq[0]'s loads first), so that the
      // loop head's wait is the same from the prologue and the back edge
      fetch(kq[0], ent[0]);
      __builtin_amdgcn_sched_barrier(0);
      fetch(kq[1], ent[1]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (MODE == kGivenScores) {
      for (int i0 = 0; i0 < nvis; i0 += U) {
        static_for<0, U>([&](auto uc) {
          constexpr int u = decltype(uc)::value;
          const int i = i0 + u;
          const int e = ent[u & 1];
          f32x4 acc[4];
          const int kb0 = (e & 0xffffff) * kBlock + 16 * w + 4 * g;
          for (int cb = 0; cb < 4; ++cb)
            for (int r = 0; r < 4; ++r) {
              const int key = kb0 + r;
              acc[cb][r] = rowok[cb] && key < NK
                               ? clamp_score(p.scores[(grow0 + 16 * cb + c) * NK + key])
                               : 0.0f;
            }
          ent[u & 1] = entry(i + 2 < nvis ? i + 2 : nvis - 1);
          finish(uc, i, e, acc, body);
        });
      }
    } else {
      // Software-pipelined by one tile: the products of tile i + 1 are
      // issued before tile i's scores are used, so the matrix unit works
      // under tile i's filter and candidate appends (the appends wait on
      // LDS).  accs[i & 1] holds tile i's scores; kq[j & 1] holds tile j's
      // operands, fetched two steps before its products.  The last step's
      // products (tile nvis, a repeat of the list's last tile) are unused.
      f32x4 accs[2][4];
      kq[0].product(accs[0], qf);
      int ecur = ent[0];
      ent[0] = entry(2 < nvis ? 2 : nvis - 1);
      fetch(kq[0], ent[0]);
      for (int i0 = 0; i0 < nvis; i0 += U) {
        static_for<0, U>([&](auto uc) {
          constexpr int u = decltype(uc)::value;
          const int i = i0 + u;
          const int enext = ent[(u + 1) & 1];
          kq[(u + 1) & 1].product(accs[(u + 1) & 1], qf);
          ent[(u + 1) & 1] = entry(i + 3 < nvis ? i + 3 : nvis - 1);
          fetch(kq[(u + 1) & 1], ent[(u + 1) & 1]);
          finish(uc, i, ecur, accs[u & 1], body);
          ecur = enext;
        });
      }
    }
  };
  // Sweep 1 (16-bit inputs) reads its K quarters through a ring in LDS
  // filled by global_load_lds (the loads in flight hold no VGPRs, so each
  // wave keeps kRing tiles in flight instead of two).  The ring occupies
  // the candidate lists' and value scratch's bytes, which sweep 1 leaves
  // unused; each wave owns kRing slots of one wave quarter (16 keys x D
  // bytes of 2-byte elements, row-major).  The quarter's rows are
  // contiguous in memory, and each DMA instruction reads whole rows (8 rows
  // of 128 bytes at D = 64, 4 of 256 at D = 128): a load of 16 half rows,
  // the MFMA operand layout, streams from L2 at about a third of the rate
  // (measured at the headline shape: 8.5 against 28 TB/s).  global_load_lds
  // puts lane L's 16 bytes at the instruction's base + 16 L, so lane L
  // fetches the chunk that belongs at that place: row r's chunk x is stored
  // at chunk x ^ sw(r), which makes the operand reads (16 rows at one chunk
  // per 16 lanes) fall in distinct banks.  The compiler does not order LDS
  // reads after the DMA that fills them, so the waits are explicit: vmcnt
  // before a slot is read (the (kRing - 1) younger tiles' loads may stay in
  // flight), lgkmcnt(0) before a slot is refilled.
  constexpr int kCh = D / 32;              // DMA instructions (and MFMA k steps) per quarter
  constexpr int kSlot = kWave * 16 * kCh;  // bytes per wave and tile
  constexpr int kCpr = D / 8;              // 16-byte chunks per row
  constexpr int kRpi = kWave / kCpr;       // rows per DMA instruction
  auto qsw = [](int r) { return D == 64 ? (r >> 1) & 7 : r & 15; };
  constexpr int kRing = ring_tiles<D, R>();
  constexpr bool kRingSweep = kTiles && is_half<T> && KL != kKGeneral;
  auto sweep_ring = [&](auto u_tag, auto&& body) {
    constexpr int U = decltype(u_tag)::value;
    if (nvis == 0) return;  // block-uniform
    unsigned char* ringw = smem + w * kRing * kSlot;  // this wave's slots
    // lane L of instruction j: quarter row r = kRpi j + L / kCpr, stored
    // chunk L % kCpr, fetched chunk (L % kCpr) ^ sw(r)
    auto dma = [&](int slot, int e) __attribute__((always_inline)) {
      const int kq = (e & 0xffffff) * kBlock + 16 * w;  // the quarter's first key
      unsigned char* dst = ringw + slot * kSlot;
      for (int j = 0; j < kCh; ++j) {
        const int r = kRpi * j + L / kCpr, key = kq + r;
        const int kk = key < NK ? key : 0, ch = (L % kCpr) ^ qsw(r);
        const void* src;
        if constexpr (KL == kKDense)
          src = Kb + size_t(kk) * D + 8 * ch;
        else
          src = reinterpret_cast<const unsigned char*>(Kb) + (uint32_t(kk) * ksnb + 16u * ch);
        __builtin_amdgcn_global_load_lds(src,
                                         (__attribute__((address_space(3))) void*)(dst + j * kWave * 16),
                                         16, 0, 0);
      }
    };
    // The Q fragments' loads are waited for here, by an s_waitcnt the
    // compiler sees: otherwise its wait for them before the first product
    // stays in the loop as vmcnt(0) on every tile (encoding: vmcnt 0,
    // expcnt 7, lgkmcnt 15).
    __builtin_amdgcn_s_waitcnt(0x0f70);
    for (int j = 0; j < kRing; ++j) dma(j, entry(j < nvis ? j : nvis - 1));
    int slot = 0;  // slot of tile i
    for (int i0 = 0; i0 < nvis; i0 += U) {
      static_for<0, U>([&](auto uc) {
        const int i = i0 + decltype(uc)::value;
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((kRing - 1) * kCh) : "memory");
        KQuarter<T, D> kq;
        using A = std::remove_reference_t<decltype(kq.a[0])>;
        // operand s of lane (c, g): quarter row c, chunk 4 s + g
        for (int s = 0; s < kCh; ++s)
          kq.a[s] = *reinterpret_cast<const A*>(ringw + slot * kSlot + c * (16 * kCpr) +
                                                16 * ((4 * s + g) ^ qsw(c)));
        f32x4 acc[4];
        kq.product(acc, qf);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        dma(slot, entry(i + kRing < nvis ? i + kRing : nvis - 1));
        slot = slot + 1 == kRing ? 0 : slot + 1;
        finish(uc, i, entry(i < nvis ? i : nvis - 1), acc, body);
      });
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  };

  // ---------------- sweep 1: class maxima ----------------
  float cm[4][4 * R];
  const float pinf = opaque_inf();
  for (int cb = 0; cb < 4; ++cb)
    for (int j = 0; j < 4 * R; ++j) cm[cb][j] = -__builtin_inff();
  auto maxima = [&](auto uc, int, uint32_t, f32x4 (&acc)[4]) {
    constexpr int j = decltype(uc)::value % R;
    for (int cb = 0; cb < 4; ++cb)
      for (int r = 0; r < 4; ++r) cm[cb][r + 4 * j] = vmax(cm[cb][r + 4 * j], acc[cb][r], pinf);
  };
  if constexpr (kRingSweep) {
    sweep_ring(std::integral_constant<int, UR>{}, maxima);
    __syncthreads();  // every wave's ring reads are done before the exchange reuses the bytes
  } else {
    sweep(std::integral_constant<int, UR>{}, maxima);
  }

  // Exchange: row 16 cb + c's 64 R class maxima, 4 R from each of its 16
  // lanes (4 waves x 4 lane groups), then wave w finds the floors of rows
  // 16 w + c, lane group g holding classes [16 R g, 16 R (g + 1)).
  for (int cb = 0; cb < 4; ++cb)
    for (int r = 0; r < 4; ++r)
      for (int j = 0; j < R; ++j)
        s_cm[(16 * cb + c) * lay.scm + ((w * 4 + g) * 4 + r) * R + j] = cm[cb][r + 4 * j];
  __syncthreads();
  {
    const int row = 16 * w + c;
    float v[16 * R];
    for (int i = 0; i < 16 * R; i += 4) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(s_cm + row * lay.scm + 16 * R * g + i);
      for (int j = 0; j < 4; ++j) v[i + j] = x[j];
    }
    // a value x with at least k class maxima >= x (bisection between the
    // smallest and largest class maximum), then the sweep-2 floor
    float lo = __builtin_inff(), hi = -__builtin_inff();
    uint32_t nfin = 0;
    for (int i = 0; i < 16 * R; ++i) {
      nfin = count_ge(nfin, v[i], -3.0e38f);
      if (v[i] >= -3.0e38f) {
        lo = fminf(lo, v[i]);
        hi = fmaxf(hi, v[i]);
      }
    }
    const int nf = group_sum(int(nfin));
    lo = group_min(lo);
    hi = group_max(hi);
    float x = -__builtin_inff();
    if (nf >= k) {
      for (int it = 0; it < 8; ++it) {
        const float mid = 0.5f * (lo + hi);
        uint32_t cnt = 0;
        for (int i = 0; i < 16 * R; ++i) cnt = count_ge(cnt, v[i], mid);
        if (group_sum(int(cnt)) >= k) lo = mid;
        else hi = mid;
      }
      x = lo;
    }
    const float th = kExact ? x : (x == -__builtin_inff() ? x : clamp_score(x * scale));
    // NaN marks a row that collects nothing (past NQ)
    if (g == 0) s_fl[row] = q0 + row < NQ ? sweep_floor(th, kExact, scale) : __builtin_nanf("");
  }
  __syncthreads();

  // ---------------- sweep 2 (and overflow rounds): candidates ----------------
  // A key of row 16 cb + c is a candidate when visible and !(v < fl[cb]):
  // with fl[cb] = -inf (the row's threshold is <= -10) every visible key is
  // one.  NaN dots (score -10) always pass; where the threshold is above -10
  // they cannot reach the top-k and only take a slot.  In rounds > 0 the
  // candidate's key must also reach the row's exact threshold s_tkey.
  // selection key of a stored candidate
  auto raw_key = [&](uint64_t raw) {
    const float v = __uint_as_float(uint32_t(raw));
    return make_key(kExact ? v : clamp_score(v * scale), int(raw >> 32));
  };
  float fl[4];
  int max_round = 0;
  const int round_bound = select_round_bound(NK, k, cap);
  for (int round = 0;; ++round) {
    // fl = NaN marks a row that collects nothing this round
    // A zero floor is held as -0, so that v - fl is +0 for both signed
    // zeros v (with +0, -0 - +0 = -0 would read as v < fl).
    // Rows with fl = -inf take every visible key (amask), whatever the sign
    // of a NaN difference.
    uint32_t cmask = 0, amask = 0;
    for (int cb = 0; cb < 4; ++cb) {
      fl[cb] = s_fl[16 * cb + c];
      if (fl[cb] == 0.0f) fl[cb] = -0.0f;
      if (!__builtin_isnan(fl[cb])) cmask |= 0xfu << (12 - 4 * cb);  // bit order of collect's m
      if (fl[cb] == -__builtin_inff()) amask |= 0xfu << (12 - 4 * cb);
    }
    // Candidates are stored raw, (index << 32) | bits of the sweep value,
    // and turned into selection keys when they are sorted.  Per tile, the
    // lane's candidate bits m (bit 15 - (4 cb + r): key kb0 + r of row
    // 16 cb + c) come branch-free, two instructions per score, in the order
    // the MFMA results arrive (cb = 0 first); the few lanes with
    // candidates then park their 16 values in their LDS scratch and append
    // one candidate per round (LDS atomic on the row's count), so the wave
    // runs as many rounds as its busiest lane has candidates (about two at
    // the headline shape) instead of visiting every slot.  (Storing every
    // candidate straight from its register instead, one atomic per row and
    // 16 predicated stores, measured 1.5 times slower: the predicated
    // stores cost more VALU than the LDS round trips they remove.)
    auto collect = [&](int kb0, uint32_t visb, f32x4 (&acc)[4], auto later) {
      // bit 15 - (4 cb + r) <- sign of v - fl: set where v < fl, so that
      // the complement marks !(v < fl) (NaN differences have a clear sign
      // bit)
      uint32_t m = 0;
      for (int cb = 0; cb < 4; ++cb)
        for (int r = 0; r < 4; ++r)
          m = __builtin_amdgcn_alignbit(m, __float_as_uint(acc[cb][r] - fl[cb]), 31);
      m = (~m | amask) & cmask & visb;
      if (m != 0u) {
        for (int cb = 0; cb < 4; ++cb) *reinterpret_cast<f32x4*>(s_scr + ((4 * cb) ^ scr_sw)) = acc[cb];
      }
      while (m != 0u) {
        const int b = 15 - __builtin_ctz(m);  // 4 cb + r
        m &= m - 1u;
        const int row = 4 * (b & 12) + c, key = kb0 + (b & 3);
        const float v = s_scr[b ^ scr_sw];
        if constexpr (decltype(later)::value) {
          if (make_key(kExact ? v : clamp_score(v * scale), key) < s_tkey[row]) continue;
        }
        const uint32_t pos = atomicAdd(&s_cnt[row], 1u);
        if (pos < uint32_t(cap))
          s_cand[cslot(pos, row)] = (uint64_t(uint32_t(key)) << 32) | __float_as_uint(v);
      }
    };
    if (round == 0)
      sweep(std::integral_constant<int, 2>{}, [&](auto, int kb0, uint32_t visb, f32x4 (&acc)[4]) {
        collect(kb0, visb, acc, std::false_type{});
      });
    else
      sweep(std::integral_constant<int, 2>{}, [&](auto, int kb0, uint32_t visb, f32x4 (&acc)[4]) {
        collect(kb0, visb, acc, std::true_type{});
      });
    __syncthreads();
    max_round = round;
    // rows that overflowed: the k-th best stored key becomes the row's exact
    // threshold (every top-k key is >= it) and the row's list restarts
    if (t < kBlock && q0 + t < NQ && s_cnt[t] > uint32_t(cap)) s_ctl[0] = uint32_t(round + 1);
    __syncthreads();
    if (s_ctl[0] != uint32_t(round + 1)) break;  // block-uniform
    if (round + 1 >= round_bound) {
      // cannot happen (select_round_bound); reported, not looped on
      if (t == 0 && p.status) atomicOr(p.status, kStatusSelectRounds);
      break;
    }
    for (int j = 0; j < 16; ++j) {
      const int r = 16 * w + j;
      const bool over = q0 + r < NQ && s_cnt[r] > uint32_t(cap);  // wave-uniform
      if (!over) {
        if (L == 0) s_fl[r] = __builtin_nanf("");
        continue;
      }
      uint64_t v[8];
      for (int pp = 0; pp < 8; ++pp) {
        const int e = (L & 31) * 8 + pp;
        v[pp] = e < cap ? raw_key(s_cand[cslot(e, r)]) : 0ull;
      }
      segment_sort_desc<32>(v, L);
      // element k-1 lives in lane (k-1)/8, slot (k-1)%8 (both halves agree)
      const int src = (k - 1) >> 3, sp = (k - 1) & 7;
      uint64_t mine = v[0];
      for (int pp = 1; pp < 8; ++pp)
        if (pp == sp) mine = v[pp];
      const uint64_t th =
          (static_cast<uint64_t>(__shfl(static_cast<uint32_t>(mine >> 32), src, kWave)) << 32) |
          __shfl(static_cast<uint32_t>(mine), src, kWave);
      if (L == 0) {
        s_tkey[r] = th;
        s_fl[r] = sweep_floor(key_score(th), kExact, scale);
      }
    }
    __syncthreads();  // all overflow reads of the lists and counts are done
    if (t < kBlock && !__builtin_isnan(s_fl[t])) s_cnt[t] = 0u;
    __syncthreads();
  }
  if (max_round > 0 && t == 0 && p.status)
    atomicMax(p.status, (uint32_t(max_round > 255 ? 255 : max_round) << 8));

  // ---------------- select: sort each row's candidates ----------------
  // The top-k key blocks go into the mask bitmap of the row's 32-row half
  // (wave w sorts rows 16 w .. 16 w + 15, half w / 2): with at most 64 key
  // blocks as one register word per lane, OR-ed over the wave at the end
  // (the per-entry LDS atomics would all hit the same two words).
  const bool kb_word = nKB <= 64;
  uint32_t* s_hbits = s_bits + (w >> 1) * nbw;
  uint64_t kbm = 0;
  auto emit = [&](int r, int e, uint64_t key) {
    if (e >= k || q0 + r >= NQ) return;
    const bool real = key != 0ull;
    const float sv = real ? key_score(key) : kSentinel;
    const int idx = real ? key_index(key) : -1;
    s_tk[e * kWave + r] = sv;
    const size_t gr = size_t(bh) * NQ + q0 + r;
    if (p.topk_idx) {
      p.topk_idx[gr * k + e] = idx;
      p.topk_val[gr * k + e] = sv;
    }
    if (idx >= 0) {
      const int kb = idx / kBlock;
      if (kb_word) kbm |= uint64_t(1) << kb;
      else atomicOr(&s_hbits[kb >> 5], 1u << (kb & 31));
    }
  };
  auto ncand = [&](int r) -> int { return (q0 + r < NQ) ? min(int(s_cnt[r]), cap) : 0; };
  // With top-k outputs requested: segments of LS lanes x 8 keys sort one
  // row's (score, index) keys each; a group of 8 rows runs as one LS=8 pass
  // (<= 64 keys per row), two LS=16 or four LS=32 passes.
  auto sort_rows = [&](auto ls_tag, int row0) {
    constexpr int LS = decltype(ls_tag)::value;
    const int r = row0 + L / LS, i = L & (LS - 1), n = ncand(r);
    uint64_t v[8];
    for (int pp = 0; pp < 8; ++pp) {
      const int e = i * 8 + pp;
      v[pp] = e < n ? raw_key(s_cand[cslot(e, r)]) : 0ull;
    }
    segment_sort_desc<LS>(v, L);
    for (int pp = 0; pp < 8; ++pp) emit(r, i * 8 + pp, v[pp]);
  };
  // Otherwise only the values are sorted (32-bit order codes, no payload):
  // tau needs the top-k values in order, and the block mask needs the set of
  // top-k keys, which is every candidate scoring above the k-th value v_k
  // plus, of those scoring v_k, the ones with the lowest indices.  The
  // candidates are then read once more, unsorted, for the mask bits.
  auto select_rows = [&](auto ls_tag, int row0) {
    constexpr int LS = decltype(ls_tag)::value;
    const int r = row0 + L / LS, i = L & (LS - 1), n = ncand(r);
    const bool rok = q0 + r < NQ;
    auto ord_raw = [&](uint64_t raw) {
      const float x = __uint_as_float(uint32_t(raw));
      return ord_of(kExact ? x : clamp_score(x * scale));
    };
    uint32_t v[8], o8[8];  // o8: the lane's unsorted order codes, kept for the mask bits
    int x8[8];             //     and their key indices
    for (int pp = 0; pp < 8; ++pp) {
      const int e = i * 8 + pp;
      const uint64_t raw = e < n ? s_cand[cslot(e, r)] : 0ull;
      o8[pp] = e < n ? ord_raw(raw) : 0u;  // 0: empty slot
      x8[pp] = int(raw >> 32);
      v[pp] = o8[pp];
    }
    segment_sort_desc32<LS>(v, L);
    for (int pp = 0; pp < 8; ++pp) {
      const int e = i * 8 + pp;
      if (e < k && rok) s_tk[e * kWave + r] = v[pp] ? score_of_ord(v[pp]) : kSentinel;
    }
    // v_k and, over the row's sorted values, how many exceed / equal it
    const int src = (k - 1) >> 3, sp = (k - 1) & 7;
    uint32_t mine = v[0];
    for (int pp = 1; pp < 8; ++pp)
      if (pp == sp) mine = v[pp];
    const uint32_t vk = src < LS ? uint32_t(__shfl(int(mine), (L & ~(LS - 1)) + src, kWave)) : 0u;
    int gt = 0, eq = 0;
    for (int pp = 0; pp < 8; ++pp) {
      gt += v[pp] > vk ? 1 : 0;
      eq += v[pp] == vk ? 1 : 0;
    }
    for (int d = 1; d < LS; d <<= 1) {
      gt += __shfl_xor(gt, d, kWave);
      eq += __shfl_xor(eq, d, kWave);
    }
    // vk == 0: fewer than k candidates, all selected; else take the ties'
    // lowest indices when not all of them fit
    const int need = k - gt;
    const bool split = vk != 0u && eq > need;
    for (int pp = 0; pp < 8; ++pp) {
      const int e = i * 8 + pp;
      if (e >= n) continue;
      const uint32_t o = o8[pp];
      const int idx = x8[pp];
      bool sel = vk == 0u || o > vk || (o == vk && !split);
      if (split && o == vk) {
        int before = 0;  // ties with a lower index
        for (int f = 0; f < n; ++f) {
          const uint64_t q = s_cand[cslot(f, r)];
          before += (ord_raw(q) == vk && int(q >> 32) < idx) ? 1 : 0;
        }
        sel = before < need;
      }
      if (sel) {
        const int kb = idx / kBlock;
        if (kb_word) kbm |= uint64_t(1) << kb;
        else atomicOr(&s_hbits[kb >> 5], 1u << (kb & 31));
      }
    }
  };
  const bool want_topk = p.topk_idx != nullptr;
  for (int base = 16 * w; base < 16 * w + 16; base += 8) {
    int need = k;
    for (int j = 0; j < 8; ++j) need = max(need, ncand(base + j));
    if (want_topk) {
      if (need <= 64) {
        sort_rows(std::integral_constant<int, 8>{}, base);
      } else if (need <= 128) {
        sort_rows(std::integral_constant<int, 16>{}, base);
        sort_rows(std::integral_constant<int, 16>{}, base + 4);
      } else {
        for (int h = 0; h < 4; ++h) sort_rows(std::integral_constant<int, 32>{}, base + 2 * h);
      }
    } else {
      if (need <= 64) {
        select_rows(std::integral_constant<int, 8>{}, base);
      } else if (need <= 128) {
        select_rows(std::integral_constant<int, 16>{}, base);
        select_rows(std::integral_constant<int, 16>{}, base + 4);
      } else {
        for (int h = 0; h < 4; ++h) select_rows(std::integral_constant<int, 32>{}, base + 2 * h);
      }
    }
  }
  if (kb_word) {  // block-uniform
    kbm |= lane_xor64<1>(kbm);
    kbm |= lane_xor64<2>(kbm);
    kbm |= lane_xor64<4>(kbm);
    kbm |= lane_xor64<8>(kbm);
    auto bor = [](uint32_t x, uint32_t y) { return x | y; };
    const uint32_t lo = group_reduce_bits(uint32_t(kbm), bor);
    const uint32_t hi = group_reduce_bits(uint32_t(kbm >> 32), bor);
    if (L == 0) {
      if (lo) atomicOr(&s_hbits[0], lo);
      if (hi) atomicOr(&s_hbits[1], hi);  // nonzero only when nKB > 32 (nbw = 2)
    }
  }
  __syncthreads();

  // ---------------- mask row; sorted values for the tau kernel ----------------
  // the 64-row mask is the union of the halves; with 32-row blocks each
  // half's row is written too (the second only when the block has one)
  uint8_t* mrow = p.mask + (size_t(bh) * nQB + qb) * nKB;
  const int nQH = half_blocks(NQ);
  uint8_t* hrow = p.half ? p.half + (size_t(bh) * nQH + 2 * qb) * nKB : nullptr;
  const bool second = 2 * qb + 1 < nQH;
  for (int kb = t; kb < nKB; kb += kThreads) {
    const uint32_t b0 = (s_bits[kb >> 5] >> (kb & 31)) & 1u;
    const uint32_t b1 = (s_bits[nbw + (kb >> 5)] >> (kb & 31)) & 1u;
    mrow[kb] = uint8_t(b0 | b1);
    if (hrow) {
      hrow[kb] = uint8_t(b0);
      if (second) hrow[nKB + kb] = uint8_t(b1);
    }
  }
  const size_t rows = size_t(p.d.BH) * NQ;
  for (int i = t; i < k * kBlock; i += kThreads) {
    const int e = i >> 6, r = i & 63;
    if (q0 + r < NQ) p.tkv[size_t(e) * rows + size_t(bh) * NQ + q0 + r] = s_tk[e * kWave + r];
  }
}

// Smallest and largest position of every 64-key block of every (batch,
// head): kbounds[bh * nKB + kb] = (min, max) over the block's keys < NK.
// One wave per key block.  Also clears the per-call status word: this is the
// first kernel of a forward on the stream.
__global__ __launch_bounds__(kThreads) void bounds_kernel(SelectParams p) {
  const int nKB = p.d.nKB, NK = p.d.NK;
  if (blockIdx.x == 0 && threadIdx.x == 0 && p.status) *p.status = 0u;
  const int blk = blockIdx.x * (kThreads / kWave) + (threadIdx.x >> 6);
  if (blk >= p.d.BH * nKB) return;  // wave-uniform
  const int bh = blk / nKB, kb = blk % nKB, L = threadIdx.x & 63;
  const int key = kb * kBlock + L;
  const int pos = key < NK ? p.k_idx[size_t(bh) * NK + key] : 0;
  const int mn = wave_min(key < NK ? pos : INT_MAX);
  const int mx = wave_max(key < NK ? pos : INT_MIN);
  if (L == 0) p.kbounds[blk] = int2{mn, mx};
}

// tau of every row from its sorted top-k values (one thread per row):
// tkv[e * rows + row], e < k.
template <int AC, int KMAX>
__device__ __forceinline__ void tau_row(const SelectParams& p, int blk) {
  const size_t rows = size_t(p.d.BH) * p.d.NQ;
  const size_t r = size_t(blk) * kThreads + threadIdx.x;
  if (r >= rows) return;
  const int k = p.d.k;
  const float* v = p.tkv + r;
  if constexpr (KMAX > 0) {
    float reg[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) reg[j] = v[size_t(min(j, k - 1)) * rows];  // k >= 1
    p.taus[r] = entmax_tau<AC, KMAX>([&](int j) { return reg[j]; }, k, p.d.alpha);
  } else {
    p.taus[r] = entmax_tau<AC, 0>([&](int j) { return v[size_t(j) * rows]; }, k, p.d.alpha);
  }
}


template <int AC, int KMAX>
__global__ __launch_bounds__(kThreads) void tau_kernel(SelectParams p) {
  tau_row<AC, KMAX>(p, blockIdx.x);
}

// compact_kernel's blocks, then tau_kernel's (both read only what the
// score pass wrote): one launch, the compaction running beside the tau
// rows instead of after them.  The compaction's blocks come first: each
// runs longer than a block of tau rows, and on large masks they are many
// (compact_grid).
template <int AC, int KMAX>
__global__ __launch_bounds__(kThreads) void tau_compact_kernel(SelectParams p, CompactParams cp, int ncomp) {
  if (int(blockIdx.x) < ncomp) {  // block-uniform
    extern __shared__ int sm[];
    compact_detail::compact_block(cp, sm, blockIdx.x);
  } else {
    tau_row<AC, KMAX>(p, int(blockIdx.x) - ncomp);
  }
}

template <typename T, int D, int MODE, int R, int KL>
hipError_t launch_one(const SelectParams& p, hipStream_t s) {
  const SelLayout l = sel_layout(p.d.k, p.cap, p.d.nKB);
  auto kern = select_kernel<T, D, MODE, R, KL>;
  if (KL != kKGeneral && is_half<T> && MODE != kGivenScores && ring_bytes<D, R>() > l.tkey)
    return hipErrorInvalidValue;
  if (l.total > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, l.total);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3(p.d.nQB * p.d.BH), dim3(kThreads), l.total, s, p);
  return hipGetLastError();
}

// The hd = D variants (kKDense, kKRows) for the 16-bit MFMA sweeps with raw
// dots (the usual scale > 0); the others take the general loads (and
// sweep 1 on the register path).
template <typename T, int D, int MODE, int R>
hipError_t launch_ring(const SelectParams& p, hipStream_t s) {
  if constexpr (is_half<T> && MODE == kRawDots)
    if (p.d.hd == D) {
      if (p.lk.sn == D) return launch_one<T, D, MODE, R, kKDense>(p, s);
      return launch_one<T, D, MODE, R, kKRows>(p, s);
    }
  return launch_one<T, D, MODE, R, kKGeneral>(p, s);
}

// Class sets per (row, position): classes_per_lane.
template <typename T, int D, int MODE>
hipError_t launch_r(const SelectParams& p, hipStream_t s) {
  if (classes_per_lane(p.d.k) == 2) return launch_ring<T, D, MODE, 2>(p, s);
  return launch_ring<T, D, MODE, 4>(p, s);
}

template <typename T, int D>
hipError_t launch_mode(const SelectParams& p, hipStream_t s) {
  if (p.d.scale > 0.0f) return launch_r<T, D, kRawDots>(p, s);
  return launch_r<T, D, kExactScores>(p, s);
}


}  // namespace

hipError_t launch_bounds(const SelectParams& p, hipStream_t s) {
  const int blocks = p.d.BH * p.d.nKB;
  const int per = kThreads / kWave;
  hipLaunchKernelGGL(bounds_kernel, dim3(unsigned((blocks + per - 1) / per)), dim3(kThreads), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_tau(const SelectParams& p, hipStream_t s) {
  const size_t rows = size_t(p.d.BH) * p.d.NQ;
  const dim3 grid(unsigned((rows + kThreads - 1) / kThreads));
  const bool reg = p.d.k <= 32;  // the row's values fit in registers
  switch (alpha_class_of(p.d.alpha)) {
    case kA15:
      if (reg) hipLaunchKernelGGL((tau_kernel<kA15, 32>), grid, dim3(kThreads), 0, s, p);
      else hipLaunchKernelGGL((tau_kernel<kA15, 0>), grid, dim3(kThreads), 0, s, p);
      break;
    case kA20:
      if (reg) hipLaunchKernelGGL((tau_kernel<kA20, 32>), grid, dim3(kThreads), 0, s, p);
      else hipLaunchKernelGGL((tau_kernel<kA20, 0>), grid, dim3(kThreads), 0, s, p);
      break;
    case kA125:
      if (reg) hipLaunchKernelGGL((tau_kernel<kA125, 32>), grid, dim3(kThreads), 0, s, p);
      else hipLaunchKernelGGL((tau_kernel<kA125, 0>), grid, dim3(kThreads), 0, s, p);
      break;
    default:
      if (reg) hipLaunchKernelGGL((tau_kernel<kAGen, 32>), grid, dim3(kThreads), 0, s, p);
      else hipLaunchKernelGGL((tau_kernel<kAGen, 0>), grid, dim3(kThreads), 0, s, p);
      break;
  }
  return hipGetLastError();
}

hipError_t launch_tau_compact(const SelectParams& p, const CompactParams& cp, hipStream_t s) {
  const size_t rows = size_t(p.d.BH) * p.d.NQ;
  const int ntau = int((rows + kThreads - 1) / kThreads);
  const int ncomp = compact_detail::compact_grid(cp);
  const dim3 grid(unsigned(ntau + ncomp));
  const size_t lds = compact_detail::compact_lds_bytes(cp);
  const bool reg = p.d.k <= 32;  // the row's values fit in registers
  switch (alpha_class_of(p.d.alpha)) {
    case kA15:
      if (reg) hipLaunchKernelGGL((tau_compact_kernel<kA15, 32>), grid, dim3(kThreads), lds, s, p, cp, ncomp);
      else hipLaunchKernelGGL((tau_compact_kernel<kA15, 0>), grid, dim3(kThreads), lds, s, p, cp, ncomp);
      break;
    case kA20:
      if (reg) hipLaunchKernelGGL((tau_compact_kernel<kA20, 32>), grid, dim3(kThreads), lds, s, p, cp, ncomp);
      else hipLaunchKernelGGL((tau_compact_kernel<kA20, 0>), grid, dim3(kThreads), lds, s, p, cp, ncomp);
      break;
    case kA125:
      if (reg) hipLaunchKernelGGL((tau_compact_kernel<kA125, 32>), grid, dim3(kThreads), lds, s, p, cp, ncomp);
      else hipLaunchKernelGGL((tau_compact_kernel<kA125, 0>), grid, dim3(kThreads), lds, s, p, cp, ncomp);
      break;
    default:
      if (reg) hipLaunchKernelGGL((tau_compact_kernel<kAGen, 32>), grid, dim3(kThreads), lds, s, p, cp, ncomp);
      else hipLaunchKernelGGL((tau_compact_kernel<kAGen, 0>), grid, dim3(kThreads), lds, s, p, cp, ncomp);
      break;
  }
  return hipGetLastError();
}

size_t select_lds_bytes(const Dims& d, int dtype, bool from_scores, int cap) {
  (void)dtype;
  (void)from_scores;
  return size_t(sel_layout(d.k, cap, d.nKB).total);
}

int select_capacity(const Dims& d, int dtype, bool from_scores, size_t max_lds) {
  // k + 32 keys per row holds the candidates of random rows with room to
  // spare; less still works (overflow rounds), as long as it exceeds k.
  int cap = d.k + 32;
  if (cap > 256) cap = 256;
  while (cap > d.k && select_lds_bytes(d, dtype, from_scores, cap) > max_lds) cap -= 8;
  return cap > d.k ? cap : -1;
}

hipError_t launch_select(const SelectParams& p, int dtype, bool from_scores, hipStream_t s) {
  if (from_scores) return launch_r<float, 64, kGivenScores>(p, s);
  if (dtype == kElemBF16) {
    if (p.d.D == 64) return launch_mode<u16, 64>(p, s);
    if (p.d.D == 128) return launch_mode<u16, 128>(p, s);
  } else if (dtype == kElemF16) {
    if (p.d.D == 64) return launch_mode<h16, 64>(p, s);
    if (p.d.D == 128) return launch_mode<h16, 128>(p, s);
  } else {
    if (p.d.D == 64) return launch_mode<float, 64>(p, s);
    if (p.d.D == 128) return launch_mode<float, 128>(p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace asa
