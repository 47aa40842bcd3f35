// Score pass: scores, exact per-row top-k, tau and block mask.
//
// Reference: build_mask_kernel + insert_topk + entmax_threshold
// (adasplashattention.cu:35-217), one thread per query that scans every key
// and keeps a sorted top-k by insertion.  Here one block owns one 64-row
// query block of one (batch, head); each wave owns 16*QF of its rows and
// forms S^T = K Q^T tiles on MFMA (K fragments straight from global memory,
// Q^T fragments in registers).  The top-k is found in two sweeps over the
// visible key blocks instead of by insertion:
//
//   sweep 1  every score updates one of 64*R running "class maxima" of its
//            row (one v_max per score).  Distinct classes hold distinct keys,
//            so if at least k class maxima are >= x, at least k keys score
//            >= x, and every top-k key scores >= x.  A short bisection per
//            row finds such an x close to the k-th largest class maximum.
//   sweep 2  the scores are recomputed and every key scoring >= x is
//            appended, as a 64-bit (score, ~index) key, to the row's slice of
//            a candidate buffer in the workspace (about 1.2-1.4 k keys per row
//            on random data).  If a row overflows its slice, the k-th best
//            stored key becomes an exact key threshold and the sweep repeats
//            for that row; the threshold rises strictly, so this ends.
//   select   each row's candidates are sorted (segmented bitonic sort across
//            lanes, descending key order = score desc, index asc); the first
//            k are the reference's top-k, padded with the empty slot
//            (score -1e6, index -1).
//   finish   the tau recurrence runs per row on the sorted values, the row's
//            top-k key blocks are OR-ed into the block's mask bitmap.
//
// Sweep filters compare raw dot products (scale > 0) against a threshold
// widened by a relative margin, so that no key whose clamped, scaled score
// reaches the bound is missed; the exact score is only formed for the keys
// that pass.  With caller-given scores (asa_select_from_scores) or a
// non-positive scale the sweeps work on the exact scores directly.
#include <climits>
#include <type_traits>

#include "asa_device.hpp"
#include "asa_launch.hpp"

namespace asa {
namespace {

constexpr int kStride = 68;  // floats per staged row (16-byte aligned)

__device__ __forceinline__ int wave_min(int v) {
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ int wave_max(int v) {
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, kWave));
  return v;
}
// Reductions over the 4 lanes (L, L^16, L^32, L^48) that share a row.
__device__ __forceinline__ int group_sum(int v) {
  v += __shfl_xor(v, 16, kWave);
  v += __shfl_xor(v, 32, kWave);
  return v;
}
__device__ __forceinline__ float group_min(float v) {
  v = fminf(v, __shfl_xor(v, 16, kWave));
  return fminf(v, __shfl_xor(v, 32, kWave));
}
__device__ __forceinline__ float group_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  return fmaxf(v, __shfl_xor(v, 32, kWave));
}
// v_max_f32 without the operand canonicalisation that fmaxf() carries (the
// inputs are MFMA results or -inf, never signalling NaNs); NaN loses.
__device__ __forceinline__ float vmax(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
// m = 2 m + (x >= t || isnan(x)): one compare and one add-with-carry.
__device__ __forceinline__ uint32_t shift_in_nlt(uint32_t m, float x, float t) {
  asm("v_cmp_nlt_f32 vcc, %1, %2\n\tv_addc_co_u32 %0, vcc, %0, %0, vcc"
      : "+v"(m)
      : "v"(x), "v"(t)
      : "vcc");
  return m;
}
// c + (x >= t): counts with the same two instructions.
__device__ __forceinline__ uint32_t count_ge(uint32_t c, float x, float t) {
  asm("v_cmp_ge_f32 vcc, %1, %2\n\tv_addc_co_u32 %0, vcc, 0, %0, vcc"
      : "+v"(c)
      : "v"(x), "v"(t)
      : "vcc");
  return c;
}
__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), m, kWave);
  const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), m, kWave);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// Descending bitonic sort of independent segments of 8*LS keys: lanes
// [s*LS, (s+1)*LS) hold segment s, element e = (lane % LS) * 8 + p in v[p].
// Keys are distinct except for the padding value 0.
template <int LS>
__device__ __forceinline__ void segment_sort_desc(uint64_t (&v)[8], int lane) {
  const int i = lane & (LS - 1);
  for (int size = 2; size <= 8 * LS; size <<= 1) {
    for (int j = size >> 1; j > 0; j >>= 1) {
      if (j >= 8) {
        const bool lower = (i & (j >> 3)) == 0;  // e & j depends on the lane only
        for (int p = 0; p < 8; ++p) {
          const int e = i * 8 + p;
          const uint64_t o = shfl_xor64(v[p], j >> 3);
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
    }
  }
}

// tau from the sorted top-k values of one row, tk[j * 64 + lq] (best first),
// following the reference recurrence step by step
// (adasplashattention.cu:51-125): bracket from the extreme kept values,
// midpoint start, up to five rounds of {f, f', f'' over the leading positive
// terms; exit when |f| < 1e-4; Halley step with the reference's f''
// coefficient a(a + 1 - alpha); bracket midpoint when the step leaves the
// bracket; bracket update from f at the new point; clamp}.  No contraction,
// powers via pow_exact: bit-identical to the CPU oracle on equal inputs.
// The sorted values are read four at a time so that one LDS round trip
// serves four terms.
__device__ float entmax_tau(const float* tk, int lq, int k, float alpha_in) {
#pragma clang fp contract(off)
  const float alpha = fmaxf(1.05f, fminf(alpha_in, 3.0f));
  const float am1 = alpha - 1.0f;
  const float a = 1.0f / am1;
  const float e1 = (2.0f - alpha) * a;
  const float e2 = (3.0f - 2.0f * alpha) * a;
  const float c2 = a * ((a + 1.0f) - alpha);
  const float top = tk[lq];
  const float bottom = tk[(k - 1) * kWave + lq];
  float lo = am1 * bottom - 2.0f;
  float hi = am1 * top + 2.0f;
  float tau = 0.5f * (lo + hi);
  for (int it = 0; it < 5; ++it) {
    float f = -1.0f, df = 0.0f, d2f = 0.0f;
    float buf[4];
    for (int j = 0; j < k; ++j) {
      if ((j & 3) == 0)
        for (int i = 0; i < 4; ++i) buf[i] = tk[min(j + i, k - 1) * kWave + lq];
      float sj = buf[0];
      for (int i = 1; i < 4; ++i)
        if (i == (j & 3)) sj = buf[i];
      const float u = am1 * sj - tau;
      if (u <= 0.0f) break;
      const float ue = fmaxf(u, kEps);
      float t = pow_exact(ue, a);
      if (!finite(t)) t = 0.0f;
      f = f + t;
      const float t1 = -a * pow_exact(ue, e1);
      if (finite(t1)) df = df + t1;
      const float t2 = c2 * pow_exact(ue, e2);
      if (finite(t2)) d2f = d2f + t2;
    }
    if (fabsf(f) < 1e-4f) break;
    float next = tau;
    if (fabsf(df) > kEps) {
      const float den = 2.0f * df * df - f * d2f;
      if (fabsf(den) > kEps) next = tau - 2.0f * f * df / den;
    }
    if (!(next >= lo && next <= hi)) next = 0.5f * (lo + hi);
    float gsum = -1.0f;
    for (int j = 0; j < k; ++j) {
      if ((j & 3) == 0)
        for (int i = 0; i < 4; ++i) buf[i] = tk[min(j + i, k - 1) * kWave + lq];
      float sj = buf[0];
      for (int i = 1; i < 4; ++i)
        if (i == (j & 3)) sj = buf[i];
      const float u = am1 * sj - next;
      if (u <= 0.0f) break;
      const float t = pow_exact(fmaxf(u, kEps), a);
      if (finite(t)) gsum = gsum + t;
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

// Q^T operand fragments of QF 16-row groups.
template <typename T, int D, int QF> struct QFrags;
template <int D, int QF> struct QFrags<u16, D, QF> {
  bf16x8 v[QF][D / 32];
  __device__ void load(const u16* Q, int row0, int NQ, int lane) {
    const int g = lane >> 4, c = lane & 15;
    for (int m = 0; m < QF; ++m) {
      const int row = row0 + 16 * m + c;
      for (int s = 0; s < D / 32; ++s)
        v[m][s] = row < NQ ? *reinterpret_cast<const bf16x8*>(Q + size_t(row) * D + 32 * s + 8 * g)
                           : bf16x8{};
    }
  }
};
template <int D, int QF> struct QFrags<float, D, QF> {
  f32x4 v[QF][D / 16];
  __device__ void load(const float* Q, int row0, int NQ, int lane) {
    const int g = lane >> 4, c = lane & 15;
    for (int m = 0; m < QF; ++m) {
      const int row = row0 + 16 * m + c;
      for (int j = 0; j < D / 16; ++j)
        v[m][j] = row < NQ ? *reinterpret_cast<const f32x4*>(Q + size_t(row) * D + 16 * j + 4 * g)
                           : f32x4{};
    }
  }
};

// K^T operand fragments of one 64-key block (4 groups of 16 keys).
template <typename T, int D> struct KFrags;
template <int D> struct KFrags<u16, D> {
  bf16x8 v[4][D / 32];
  __device__ void load(const u16* K, int kbase, int NK, int lane) {
    const int g = lane >> 4, c = lane & 15;
    for (int f = 0; f < 4; ++f) {
      const int row = min(kbase + 16 * f + c, NK - 1);
      for (int s = 0; s < D / 32; ++s)
        v[f][s] = *reinterpret_cast<const bf16x8*>(K + size_t(row) * D + 32 * s + 8 * g);
    }
  }
};
template <int D> struct KFrags<float, D> {
  f32x4 v[4][D / 16];
  __device__ void load(const float* K, int kbase, int NK, int lane) {
    const int g = lane >> 4, c = lane & 15;
    for (int f = 0; f < 4; ++f) {
      const int row = min(kbase + 16 * f + c, NK - 1);
      for (int j = 0; j < D / 16; ++j)
        v[f][j] = *reinterpret_cast<const f32x4*>(K + size_t(row) * D + 16 * j + 4 * g);
    }
  }
};

template <int D, int QF>
__device__ __forceinline__ void mma(f32x4 (&acc)[4][QF], const KFrags<u16, D>& kf,
                                    const QFrags<u16, D, QF>& qf) {
  for (int f = 0; f < 4; ++f)
    for (int m = 0; m < QF; ++m) acc[f][m] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < D / 32; ++s)
    for (int f = 0; f < 4; ++f)
      for (int m = 0; m < QF; ++m) acc[f][m] = mfma(kf.v[f][s], qf.v[m][s], acc[f][m]);
}
template <int D, int QF>
__device__ __forceinline__ void mma(f32x4 (&acc)[4][QF], const KFrags<float, D>& kf,
                                    const QFrags<float, D, QF>& qf) {
  for (int f = 0; f < 4; ++f)
    for (int m = 0; m < QF; ++m) acc[f][m] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < D / 16; ++j)
    for (int r = 0; r < 4; ++r)
      for (int f = 0; f < 4; ++f)
        for (int m = 0; m < QF; ++m) acc[f][m] = mfma(kf.v[f][j][r], qf.v[m][j][r], acc[f][m]);
}

struct Lds {
  float* stage;    // [64][kStride]   staged sweep values, row = local query
  float* tk;       // [k][64]         sorted top-k scores, slot-major
  uint64_t* tkey;  // [64]            exact key threshold of an overflow round
  uint32_t* cnt;   // [64]            candidates appended per row
  uint32_t* bits;  // [ceil(nKB/32)]  block mask of the query block
  uint8_t* kvis;   // [nKB]           visibility class of every key block
};

enum SweepMode : int {
  kRawDots = 0,     // MFMA dot products, scale > 0: filters on raw dots
  kExactScores = 1, // MFMA dot products converted to exact scores (scale <= 0)
  kGivenScores = 2  // caller-given scores
};

template <typename T, int D, int QF, int MODE>
__global__ __launch_bounds__(kWave * (4 / QF)) void select_kernel(SelectParams p) {
  constexpr int NW = 4 / QF;   // waves per block
  constexpr int R = NW;        // class sets per (lane, row, slot): 64 R classes per row
  constexpr int QW = 16 * QF;  // rows per wave
  constexpr int NB = 16 * QF;  // sweep values per lane per key block
  constexpr bool kExact = MODE != kRawDots;
  static_assert(NB <= 32, "candidate masks are 32-bit");
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int k = p.d.k, NQ = p.d.NQ, NK = p.d.NK, nKB = p.d.nKB, nQB = p.d.nQB;
  const int cap = p.cap;
  const int nbw = (nKB + 31) >> 5;
  Lds s;
  s.stage = reinterpret_cast<float*>(smem);
  s.tk = s.stage + kBlock * kStride;
  s.tkey = reinterpret_cast<uint64_t*>(s.tk + size_t(k) * kWave);
  s.cnt = reinterpret_cast<uint32_t*>(s.tkey + kBlock);
  s.bits = s.cnt + kBlock;
  s.kvis = reinterpret_cast<uint8_t*>(s.bits + nbw);

  const int t = threadIdx.x, w = t >> 6, L = t & 63, g = L >> 4, c16 = L & 15;
  const int task = xcd_task(blockIdx.x, nQB * p.d.BH);
  const int qb = task % nQB, bh = task / nQB, q0 = qb * kBlock;
  const int qw0 = w * QW;  // first local row of this wave
  const float scale = p.d.scale;

  // Rows of this lane in the accumulator layout: local row qw0 + 16m + c16.
  int qid[QF];
  uint32_t rowbits = 0;  // bits of the sweep values that belong to valid rows
  for (int m = 0; m < QF; ++m) {
    const int qq = q0 + qw0 + 16 * m + c16;
    const bool ok = qq < NQ;
    qid[m] = ok ? p.q_idx[size_t(bh) * NQ + qq] : 0;
    if (ok) rowbits |= 0xffffu << (16 * m);
  }
  // Position range of the valid rows of the whole query block.
  const bool lv = q0 + L < NQ;
  const int lpos = lv ? p.q_idx[size_t(bh) * NQ + q0 + L] : 0;
  const int qmax_blk = wave_max(lv ? lpos : INT_MIN);
  const int qmin_blk = wave_min(lv ? lpos : INT_MAX);

  if (t < kBlock) s.cnt[t] = 0u;
  for (int i = t; i < nbw; i += kWave * NW) s.bits[i] = 0u;

  QFrags<T, D, QF> qf;
  const T* Kb = nullptr;
  if constexpr (MODE != kGivenScores) {
    qf.load(static_cast<const T*>(p.q) + size_t(bh) * NQ * D, q0 + qw0, NQ, L);
    Kb = static_cast<const T*>(p.k) + size_t(bh) * NK * D;
  }
  const int32_t* kidx = p.k_idx + size_t(bh) * NK;
  // Visibility class of every key block: 0 no key visible to any row of the
  // query block, 1 partially visible, 2 every key visible to every row.
  // Four blocks per wave per step keep four loads in flight.
  for (int kt0 = 4 * w; kt0 < nKB; kt0 += 4 * NW) {
    int kid[4];
    bool kin[4];
    for (int j = 0; j < 4; ++j) {
      const int kl = (kt0 + j) * kBlock + L;
      kin[j] = kt0 + j < nKB && kl < NK;
      kid[j] = kin[j] ? kidx[kl] : 0;
    }
    for (int j = 0; j < 4; ++j) {
      const int kt = kt0 + j;
      const int kmin = wave_min(kin[j] ? kid[j] : INT_MAX);
      const int kmax = wave_max(kin[j] ? kid[j] : INT_MIN);
      if (kt < nKB && L == 0)
        s.kvis[kt] = kmin > qmax_blk ? 0 : ((kmax > qmin_blk || (kt + 1) * kBlock > NK) ? 1 : 2);
    }
  }
  __syncthreads();

  // Sweep values of key block kt in the accumulator layout (bit 16m+4f+r of
  // the returned mask set where the value is visible to its valid row;
  // invisible values are set to -inf).
  KFrags<T, D> kf;
  auto sweep_values = [&](int kt, int vis, f32x4 (&acc)[4][QF]) -> uint32_t {
    const int kbase = kt * kBlock;
    if constexpr (MODE == kGivenScores) {
      for (int f = 0; f < 4; ++f)
        for (int m = 0; m < QF; ++m)
          for (int r = 0; r < 4; ++r) {
            const int key = kbase + 16 * f + 4 * g + r;
            const size_t row = size_t(bh) * NQ + q0 + qw0 + 16 * m + c16;
            acc[f][m][r] = ((rowbits >> (16 * m)) & 1u) && key < NK
                               ? clamp_score(p.scores[row * NK + key]) : 0.0f;
          }
    } else {
      mma<D, QF>(acc, kf, qf);
      if constexpr (MODE == kExactScores)
        for (int f = 0; f < 4; ++f)
          for (int m = 0; m < QF; ++m)
            for (int r = 0; r < 4; ++r) acc[f][m][r] = clamp_score(acc[f][m][r] * scale);
    }
    uint32_t vb = rowbits;
    if (vis == 1) {
      for (int f = 0; f < 4; ++f)
        for (int r = 0; r < 4; ++r) {
          const int key = kbase + 16 * f + 4 * g + r;
          const int kp = key < NK ? kidx[key] : INT_MAX;
          for (int m = 0; m < QF; ++m)
            if (!(key < NK && kp <= qid[m])) {
              vb &= ~(1u << (16 * m + 4 * f + r));
              acc[f][m][r] = -__builtin_inff();
            }
        }
    }
    return vb;
  };

  // ---------------- sweep 1: class maxima ----------------
  float cm[QF][16][R];
  for (int m = 0; m < QF; ++m)
    for (int i = 0; i < 16; ++i)
      for (int c = 0; c < R; ++c) cm[m][i][c] = -__builtin_inff();
  if constexpr (MODE != kGivenScores) kf.load(Kb, 0, NK, L);
  for (int kt0 = 0; kt0 < nKB; kt0 += R) {
    for (int c = 0; c < R; ++c) {
      const int kt = kt0 + c;
      if (kt >= nKB) break;
      const int vis = s.kvis[kt];
      if (vis == 0) {
        if constexpr (MODE != kGivenScores) kf.load(Kb, (kt + 1) * kBlock, NK, L);
        continue;
      }
      f32x4 acc[4][QF];
      sweep_values(kt, vis, acc);
      if constexpr (MODE != kGivenScores) kf.load(Kb, (kt + 1) * kBlock, NK, L);
      for (int m = 0; m < QF; ++m)
        for (int f = 0; f < 4; ++f)
          for (int r = 0; r < 4; ++r) cm[m][4 * f + r][c] = vmax(cm[m][4 * f + r][c], acc[f][m][r]);
    }
  }

  // Per row: a value x with at least k class maxima >= x (bisection between
  // the smallest and largest class maximum), then the sweep-2 floor.
  float floor_m[QF];
  for (int m = 0; m < QF; ++m) {
    float lo = __builtin_inff(), hi = -__builtin_inff();
    uint32_t nfin = 0;
    for (int i = 0; i < 16; ++i)
      for (int c = 0; c < R; ++c) {
        const float v = cm[m][i][c];
        nfin = count_ge(nfin, v, -3.0e38f);
        if (v >= -3.0e38f) {
          lo = fminf(lo, v);
          hi = fmaxf(hi, v);
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
        for (int i = 0; i < 16; ++i)
          for (int c = 0; c < R; ++c) cnt = count_ge(cnt, cm[m][i][c], mid);
        if (group_sum(int(cnt)) >= k) lo = mid;
        else hi = mid;
      }
      x = lo;
    }
    const float th = kExact ? x : (x == -__builtin_inff() ? x : clamp_score(x * scale));
    floor_m[m] = sweep_floor(th, kExact, scale);
  }

  // ---------------- sweep 2 (and overflow rounds): candidates ----------------
  float* wstage = s.stage + qw0 * kStride;
  const size_t cand_row0 = (size_t(bh) * NQ + q0) * cap;
  // Round 0 takes every key at or above the row's floor.  A row whose count
  // exceeds `cap` gets the k-th best of its stored keys as an exact key
  // threshold and is swept again; the other rows are final.
  for (int round = 0;; ++round) {
    uint32_t take = rowbits;
    uint64_t tkey[QF];
    for (int m = 0; m < QF; ++m) tkey[m] = 0;
    if (round > 0) {
      take = 0;
      for (int m = 0; m < QF; ++m)
        if (s.cnt[qw0 + 16 * m + c16] > uint32_t(cap)) take |= rowbits & (0xffffu << (16 * m));
      if (!__any(take != 0)) break;
      for (int lq = qw0; lq < qw0 + QW; ++lq) {
        if (!(s.cnt[lq] > uint32_t(cap)) || q0 + lq >= NQ) continue;  // uniform
        uint64_t v[8];
        for (int pp = 0; pp < 8; ++pp) {
          const int e = (L & 31) * 8 + pp;
          v[pp] = e < cap ? p.cand[cand_row0 + size_t(lq) * cap + e] : 0ull;
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
        if (L == 0) s.tkey[lq] = th;
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
      for (int m = 0; m < QF; ++m)
        if ((take >> (16 * m)) & 1u) {
          tkey[m] = s.tkey[qw0 + 16 * m + c16];
          floor_m[m] = sweep_floor(key_score(tkey[m]), kExact, scale);
        }
      __builtin_amdgcn_wave_barrier();
      for (int m = 0; m < QF; ++m)
        if (((take >> (16 * m)) & 1u) && g == 0) s.cnt[qw0 + 16 * m + c16] = 0u;
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }

    if constexpr (MODE != kGivenScores) kf.load(Kb, 0, NK, L);
    for (int kt = 0; kt < nKB; ++kt) {
      const int vis = s.kvis[kt];
      if (vis == 0) {
        if constexpr (MODE != kGivenScores) kf.load(Kb, (kt + 1) * kBlock, NK, L);
        continue;
      }
      f32x4 acc[4][QF];
      const uint32_t vb = sweep_values(kt, vis, acc);
      if constexpr (MODE != kGivenScores) kf.load(Kb, (kt + 1) * kBlock, NK, L);
      // bit 16m + 4f + r <- value >= floor (or NaN), highest bit first
      uint32_t cand = 0;
      for (int m = QF - 1; m >= 0; --m)
        for (int f = 3; f >= 0; --f)
          for (int r = 3; r >= 0; --r) cand = shift_in_nlt(cand, acc[f][m][r], floor_m[m]);
      cand &= vb & take;
      if (!__any(cand != 0)) continue;
      for (int f = 0; f < 4; ++f)
        for (int m = 0; m < QF; ++m)
          *reinterpret_cast<f32x4*>(wstage + (16 * m + c16) * kStride + 16 * f + 4 * g) = acc[f][m];
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
      const int kbase = kt * kBlock;
      if (round > 0) {
        // Exact key thresholds: drop the candidates below them first.
        uint32_t c2 = cand;
        while (c2) {
          const int b = __builtin_ctz(c2);
          c2 &= c2 - 1;
          const int m = b >> 4, f = (b >> 2) & 3, r = b & 3;
          const float v = wstage[(16 * m + c16) * kStride + 16 * f + 4 * g + r];
          const float sc = kExact ? v : clamp_score(v * scale);
          uint64_t th = tkey[0];
          for (int mm = 1; mm < QF; ++mm)
            if (mm == m) th = tkey[mm];
          if (make_key(sc, kbase + 16 * f + 4 * g + r) < th) cand &= ~(1u << b);
        }
      }
      // One slot reservation per (lane, row), then the stores.
      uint32_t pos[QF];
      for (int m = 0; m < QF; ++m) {
        const uint32_t mb = (cand >> (16 * m)) & 0xffffu;
        pos[m] = mb ? atomicAdd(&s.cnt[qw0 + 16 * m + c16], uint32_t(__builtin_popcount(mb))) : 0u;
      }
      while (cand) {
        const int b = __builtin_ctz(cand);
        cand &= cand - 1;
        const int m = b >> 4, f = (b >> 2) & 3, r = b & 3;
        const int lq = qw0 + 16 * m + c16;
        const float v = wstage[(16 * m + c16) * kStride + 16 * f + 4 * g + r];
        const float sc = kExact ? v : clamp_score(v * scale);
        uint32_t at = pos[0];
        for (int mm = 1; mm < QF; ++mm)
          if (mm == m) at = pos[mm];
        if (at < uint32_t(cap))
          p.cand[cand_row0 + size_t(lq) * cap + at] = make_key(sc, kbase + 16 * f + 4 * g + r);
        for (int mm = 0; mm < QF; ++mm)
          if (mm == m) ++pos[mm];
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    if (round > 64) break;  // the threshold rises every round; never reached
  }

  // ---------------- select: sort each row's candidates ----------------
  auto emit = [&](int lq, int e, uint64_t key) {
    if (e >= k || q0 + lq >= NQ) return;
    const bool real = key != 0ull;
    const float sv = real ? key_score(key) : kSentinel;
    const int idx = real ? key_index(key) : -1;
    s.tk[e * kWave + lq] = sv;
    const size_t r = size_t(bh) * NQ + q0 + lq;
    if (p.topk_idx) {
      p.topk_idx[r * k + e] = idx;
      p.topk_val[r * k + e] = sv;
    }
    if (idx >= 0) {
      const int kb = idx / kBlock;
      atomicOr(&s.bits[kb >> 5], 1u << (kb & 31));
    }
  };
  auto ncand = [&](int lq) -> int { return (q0 + lq < NQ) ? min(int(s.cnt[lq]), cap) : 0; };
  // Segments of LS lanes x 8 keys sort one row each; a group of 8 rows runs as
  // one LS=8 pass (<= 64 keys per row), two LS=16 or four LS=32 passes.
  auto sort_rows = [&](auto ls_tag, int row0) {
    constexpr int LS = decltype(ls_tag)::value;
    const int lq = row0 + L / LS, i = L & (LS - 1), n = ncand(lq);
    uint64_t v[8];
    for (int pp = 0; pp < 8; ++pp) {
      const int e = i * 8 + pp;
      v[pp] = e < n ? p.cand[cand_row0 + size_t(lq) * cap + e] : 0ull;
    }
    segment_sort_desc<LS>(v, L);
    for (int pp = 0; pp < 8; ++pp) emit(lq, i * 8 + pp, v[pp]);
  };
  for (int base = qw0; base < qw0 + QW; base += 8) {
    int need = k;
    for (int j = 0; j < 8; ++j) need = max(need, ncand(base + j));
    if (need <= 64) {
      sort_rows(std::integral_constant<int, 8>{}, base);
    } else if (need <= 128) {
      sort_rows(std::integral_constant<int, 16>{}, base);
      sort_rows(std::integral_constant<int, 16>{}, base + 4);
    } else {
      for (int h = 0; h < 4; ++h) sort_rows(std::integral_constant<int, 32>{}, base + 2 * h);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();

  // ---------------- tau per row ----------------
  if (L < QW) {
    const int lq = qw0 + L;
    if (q0 + lq < NQ) p.taus[size_t(bh) * NQ + q0 + lq] = entmax_tau(s.tk, lq, k, p.d.alpha);
  }
  __syncthreads();
  uint8_t* mrow = p.mask + (size_t(bh) * nQB + qb) * nKB;
  for (int kb = t; kb < nKB; kb += kWave * NW) mrow[kb] = uint8_t((s.bits[kb >> 5] >> (kb & 31)) & 1u);
}

template <typename T, int D, int QF, int MODE>
hipError_t launch_one(const SelectParams& p, hipStream_t s) {
  const size_t lds = select_lds_bytes(p.d);
  auto kern = select_kernel<T, D, QF, MODE>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3(p.d.nQB * p.d.BH), dim3(kWave * (4 / QF)), lds, s, p);
  return hipGetLastError();
}

template <typename T, int D, int MODE>
hipError_t launch_qf(const SelectParams& p, hipStream_t s) {
  if (p.d.k <= 64) return launch_one<T, D, 2, MODE>(p, s);
  return launch_one<T, D, 1, MODE>(p, s);
}

template <typename T, int D>
hipError_t launch_mode(const SelectParams& p, hipStream_t s) {
  if (p.d.scale > 0.0f) return launch_qf<T, D, kRawDots>(p, s);
  return launch_qf<T, D, kExactScores>(p, s);
}

}  // namespace

int select_capacity(int k) {
  const int c = k + (k > 64 ? k : 64);
  return c > 256 ? 256 : c;
}

size_t select_lds_bytes(const Dims& d) {
  const size_t nbw = size_t(d.nKB + 31) / 32;
  size_t b = size_t(kBlock) * kStride * sizeof(float)      // stage
             + size_t(d.k) * kWave * sizeof(float)         // sorted top-k scores
             + size_t(kBlock) * sizeof(uint64_t)           // key thresholds
             + size_t(kBlock) * sizeof(uint32_t)           // counters
             + nbw * sizeof(uint32_t)                      // mask bits
             + size_t(d.nKB);                              // key-block visibility
  return (b + 15) & ~size_t(15);
}

hipError_t launch_select(const SelectParams& p, bool bf16, bool from_scores, hipStream_t s) {
  if (from_scores) return launch_qf<float, 64, kGivenScores>(p, s);
  if (bf16) {
    if (p.d.D == 64) return launch_mode<u16, 64>(p, s);
    if (p.d.D == 128) return launch_mode<u16, 128>(p, s);
  } else {
    if (p.d.D == 64) return launch_mode<float, 64>(p, s);
    if (p.d.D == 128) return launch_mode<float, 128>(p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace asa
