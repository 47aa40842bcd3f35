// Score pass: scores, exact per-row top-k, tau and block mask.
//
// Reference: build_mask_kernel + insert_topk + entmax_threshold
// (adasplashattention.cu:35-217), one thread per query that scans every key
// and keeps a sorted top-k by insertion.  Here one 256-thread block owns one
// 64-row query block of one (batch, head); wave w owns rows 16w..16w+15 and
// forms S^T = K Q^T tiles on MFMA.  The K tiles of the visible key blocks
// stream through a double-buffered LDS stage shared by the four waves (each
// thread prefetches its share of the next tile into registers while the
// current one is multiplied).  The top-k is found in two sweeps over the
// visible key blocks instead of by insertion:
//
//   sweep 1  every score updates one of 64*R running "class maxima" of its
//            row (one v_max per score).  Distinct classes hold distinct keys,
//            so if at least k class maxima are >= x, at least k keys score
//            >= x, and every top-k key scores >= x.  A short bisection per
//            row finds such an x close to the k-th largest class maximum.
//   sweep 2  the scores are recomputed and every key scoring >= x is
//            appended, as a 64-bit (score, ~index) key, to the row's list in
//            LDS (about 1.05-1.15 k keys per row on random data).  If a row
//            overflows its list, the k-th best stored key becomes an exact
//            key threshold and the block sweeps again for those rows; the
//            threshold rises strictly, so this ends.
//   select   each row's candidates are sorted (segmented bitonic sort across
//            lanes, descending key order = score desc, index asc); the first
//            k are the reference's top-k, padded with the empty slot
//            (score -1e6, index -1).
//   finish   the rows' top-k key blocks are OR-ed into the block's mask
//            bitmap; one wave runs the tau recurrence, one lane per row.
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
// m = 2 m + (x >= t || isnan(x)).
__device__ __forceinline__ uint32_t shift_in_nlt(uint32_t m, float x, float t) {
  return m + m + (x < t ? 0u : 1u);
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


// acc[b >> 2][b & 3] for a per-lane index b in [0, 16): a select tree on
// the index bits instead of a dynamically indexed register array.
__device__ __forceinline__ float pick16(const f32x4 (&acc)[4], int b) {
  const bool b2 = (b & 4) != 0, b3 = (b & 8) != 0;
  f32x4 x;
  for (int r = 0; r < 4; ++r) {
    const float lo = b2 ? acc[1][r] : acc[0][r];
    const float hi = b2 ? acc[3][r] : acc[2][r];
    x[r] = b3 ? hi : lo;
  }
  const float y0 = (b & 1) ? x[1] : x[0];
  const float y1 = (b & 1) ? x[3] : x[2];
  return (b & 2) ? y1 : y0;
}

enum SweepMode : int {
  kRawDots = 0,     // MFMA dot products, scale > 0: filters on raw dots
  kExactScores = 1, // MFMA dot products converted to exact scores (scale <= 0)
  kGivenScores = 2  // caller-given scores
};

// LDS layout, shared by the kernel and the host-side size query.
struct SelLayout {
  int tiles, tk, cand, tkey, cnt, ctl, bits, vlist, total;
};
__host__ __device__ inline int align_up(int x, int a) { return (x + a - 1) / a * a; }
__host__ __device__ inline SelLayout sel_layout(int k, int cap, int nKB, int D, int tbytes,
                                                bool given_scores) {
  SelLayout l;
  const int rs = tbytes == 2 ? D + 8 : D + 4;
  const int tiles = given_scores ? 0 : 2 * kBlock * rs * tbytes;
  const int tk = k * kWave * 4;
  // the sorted top-k values reuse the tile buffers once the sweeps are over
  const int a = align_up(tiles > tk ? tiles : tk, 16);
  l.tiles = 0;
  l.tk = 0;
  l.cand = a;
  l.tkey = l.cand + kBlock * cap * 8;
  l.cnt = l.tkey + kBlock * 8;
  l.ctl = l.cnt + kBlock * 4;
  l.bits = l.ctl + 16;
  l.vlist = l.bits + align_up((nKB + 31) / 32 * 4, 16);
  l.total = l.vlist + align_up(nKB * 4, 16);
  return l;
}

template <typename T, int D, int MODE, int R>
__global__ __launch_bounds__(kThreads) void select_kernel(SelectParams p) {
  constexpr bool kExact = MODE != kRawDots;
  constexpr bool kTiles = MODE != kGivenScores;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int k = p.d.k, NQ = p.d.NQ, NK = p.d.NK, nKB = p.d.nKB, nQB = p.d.nQB;
  const int cap = p.cap;
  const int nbw = (nKB + 31) >> 5;
  const SelLayout lay = sel_layout(k, cap, nKB, D, int(sizeof(T)), !kTiles);
  T* s_tiles = reinterpret_cast<T*>(smem + lay.tiles);
  float* s_tk = reinterpret_cast<float*>(smem + lay.tk);
  uint64_t* s_cand = reinterpret_cast<uint64_t*>(smem + lay.cand);
  uint64_t* s_tkey = reinterpret_cast<uint64_t*>(smem + lay.tkey);
  uint32_t* s_cnt = reinterpret_cast<uint32_t*>(smem + lay.cnt);
  uint32_t* s_ctl = reinterpret_cast<uint32_t*>(smem + lay.ctl);
  uint32_t* s_bits = reinterpret_cast<uint32_t*>(smem + lay.bits);
  int32_t* s_vlist = reinterpret_cast<int32_t*>(smem + lay.vlist);
  constexpr int kTileElems = kBlock * KStage<T, D>::kRs;

  const int t = threadIdx.x, w = t >> 6, L = t & 63, g = L >> 4, c = L & 15;
  const int task = xcd_task(blockIdx.x, nQB * p.d.BH);
  const int qb = nQB - 1 - task % nQB, bh = task / nQB, q0 = qb * kBlock;
  const int lq = 16 * w + c;  // this lane's row within the block
  const bool rowok = q0 + lq < NQ;
  const size_t grow = size_t(bh) * NQ + q0 + lq;  // global row (valid if rowok)
  const int qpos = rowok ? p.q_idx[grow] : 0;
  const float scale = p.d.scale;

  // Position range of the valid rows of the whole block (lane L <-> row L).
  const bool lv = q0 + L < NQ;
  const int lpos = lv ? p.q_idx[size_t(bh) * NQ + q0 + L] : 0;
  const int qmax_blk = wave_max(lv ? lpos : INT_MIN);
  const int qmin_blk = wave_min(lv ? lpos : INT_MAX);

  if (t < kBlock) s_cnt[t] = 0u;
  if (t < 4) s_ctl[t] = 0u;
  for (int i = t; i < nbw; i += kThreads) s_bits[i] = 0u;

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

  RowFrag<T, D> qf;  // Q^T operand: the lane's query row (column c of the products)
  const T* Kb = nullptr;
  if constexpr (kTiles) {
    qf.load(static_cast<const T*>(p.q) + grow * D, rowok, L);
    Kb = static_cast<const T*>(p.k) + size_t(bh) * NK * D;
  }
  KStage<T, D> ks;

  // Sweep values of one key block for the lane's row: acc[f][r] is the value
  // of key 16f + 4g + r.  Bit 4f + r of the returned mask is set where that
  // key is visible to a valid row; invisible values are set to -inf.
  auto sweep_values = [&](const T* buf, int kt, int vis, f32x4 (&acc)[4]) -> uint32_t {
    const int kbase = kt * kBlock;
    if constexpr (MODE == kGivenScores) {
      for (int f = 0; f < 4; ++f)
        for (int r = 0; r < 4; ++r) {
          const int key = kbase + 16 * f + 4 * g + r;
          acc[f][r] = rowok && key < NK ? clamp_score(p.scores[grow * NK + key]) : 0.0f;
        }
    } else {
      rows_x_frag<D>(acc, buf, qf, L);
      if constexpr (MODE == kExactScores)
        for (int f = 0; f < 4; ++f)
          for (int r = 0; r < 4; ++r) acc[f][r] = clamp_score(acc[f][r] * scale);
    }
    uint32_t vb = rowok ? 0xffffu : 0u;
    if (vis == 1) {
      for (int f = 0; f < 4; ++f)
        for (int r = 0; r < 4; ++r) {
          const int key = kbase + 16 * f + 4 * g + r;
          const int kp = key < NK ? kidx[key] : INT_MAX;
          if (!(key < NK && kp <= qpos)) {
            vb &= ~(1u << (4 * f + r));
            acc[f][r] = -__builtin_inff();
          }
        }
    }
    return vb;
  };

  // One pass over the visible key blocks: body(u, kt, vb, acc) for each, with
  // u = (ordinal of the block) % U known at compile time.  The next tile is
  // stored to the other LDS buffer and the one after it fetched into
  // registers while the current tile is in use.
  auto sweep = [&](auto u_tag, auto&& body) {
    constexpr int U = decltype(u_tag)::value;
    if constexpr (kTiles) {
      if (nvis > 0) {
        ks.load(Kb, (s_vlist[0] & 0xffffff) * kBlock, NK, t);
        ks.store(s_tiles, t);
      }
      if (nvis > 1) ks.load(Kb, (s_vlist[1] & 0xffffff) * kBlock, NK, t);
      __syncthreads();
    }
    for (int i0 = 0; i0 < nvis; i0 += U) {
      static_for<0, U>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        const int i = i0 + u;
        if (i < nvis) {
          const int e = s_vlist[i];
          const int kt = e & 0xffffff, vis = e >> 24;
          const T* buf = s_tiles + (i & 1) * kTileElems;
          f32x4 acc[4];
          const uint32_t vb = sweep_values(buf, kt, vis, acc);
          body(uc, kt, vb, acc);
          if constexpr (kTiles) {
            if (i + 1 < nvis) {
              ks.store(s_tiles + ((i + 1) & 1) * kTileElems, t);
              if (i + 2 < nvis) ks.load(Kb, (s_vlist[i + 2] & 0xffffff) * kBlock, NK, t);
            }
            __syncthreads();
          }
        }
      });
    }
    __syncthreads();
  };

  // ---------------- sweep 1: class maxima ----------------
  float cm[16][R];
  const float pinf = opaque_inf();
  for (int i = 0; i < 16; ++i)
    for (int j = 0; j < R; ++j) cm[i][j] = -__builtin_inff();
  sweep(std::integral_constant<int, R>{}, [&](auto uc, int, uint32_t, f32x4 (&acc)[4]) {
    constexpr int u = decltype(uc)::value;
    for (int f = 0; f < 4; ++f)
      for (int r = 0; r < 4; ++r) cm[4 * f + r][u] = vmax(cm[4 * f + r][u], acc[f][r], pinf);
  });

  // Per row: a value x with at least k class maxima >= x (bisection between
  // the smallest and largest class maximum), then the sweep-2 floor.
  float floor_v;
  {
    float lo = __builtin_inff(), hi = -__builtin_inff();
    uint32_t nfin = 0;
    for (int i = 0; i < 16; ++i)
      for (int j = 0; j < R; ++j) {
        const float v = cm[i][j];
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
          for (int j = 0; j < R; ++j) cnt = count_ge(cnt, cm[i][j], mid);
        if (group_sum(int(cnt)) >= k) lo = mid;
        else hi = mid;
      }
      x = lo;
    }
    const float th = kExact ? x : (x == -__builtin_inff() ? x : clamp_score(x * scale));
    floor_v = sweep_floor(th, kExact, scale);
  }

  // ---------------- sweep 2 (and overflow rounds): candidates ----------------
  uint64_t* my_cand = s_cand + size_t(lq) * cap;
  bool take = rowok;  // this lane's row collects in the current round
  uint64_t tkey = 0;  // exact key threshold of the row (rounds > 0)
  for (int round = 0;; ++round) {
    sweep(std::integral_constant<int, 1>{}, [&](auto, int kt, uint32_t vb, f32x4 (&acc)[4]) {
      // bit 4f + r <- value >= floor (or NaN), highest bit first
      uint32_t cand = 0;
      for (int f = 3; f >= 0; --f)
        for (int r = 3; r >= 0; --r) cand = shift_in_nlt(cand, acc[f][r], floor_v);
      cand &= take ? vb : 0u;
      if (!__any(cand != 0)) return;
      const int kbase = kt * kBlock + 4 * g;
      // key of value b = 4f + r: score, index kbase + 16f + r
      auto key_of = [&](int b) {
        const float v = pick16(acc, b);
        const float sc = kExact ? v : clamp_score(v * scale);
        return make_key(sc, kbase + 16 * (b >> 2) + (b & 3));
      };
      if (round > 0) {
        // exact key threshold: drop the candidates below it first
        uint32_t c2 = cand;
        while (c2) {
          const int b = __builtin_ctz(c2);
          c2 &= c2 - 1;
          if (key_of(b) < tkey) cand &= ~(1u << b);
        }
      }
      uint32_t pos = cand ? atomicAdd(&s_cnt[lq], uint32_t(__builtin_popcount(cand))) : 0u;
      while (cand) {
        const int b = __builtin_ctz(cand);
        cand &= cand - 1;
        const uint64_t key = key_of(b);
        if (pos < uint32_t(cap)) my_cand[pos] = key;
        ++pos;
      }
    });
    // (the sweep ends with a block barrier: every count is final)
    const bool over = rowok && s_cnt[lq] > uint32_t(cap);
    if (__any(over) && L == 0) s_ctl[0] = uint32_t(round + 1);
    __syncthreads();
    if (s_ctl[0] != uint32_t(round + 1) || round >= 64) break;  // block-uniform
    // Rows that overflowed: the k-th best stored key becomes the row's exact
    // threshold (every top-k key is >= it), the row's list restarts.
    for (int j = 0; j < 16; ++j) {
      const int r = 16 * w + j;
      if (!(q0 + r < NQ && s_cnt[r] > uint32_t(cap))) continue;  // wave-uniform
      uint64_t v[8];
      for (int pp = 0; pp < 8; ++pp) {
        const int e = (L & 31) * 8 + pp;
        v[pp] = e < cap ? s_cand[size_t(r) * cap + e] : 0ull;
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
      if (c == j) {
        tkey = th;
        floor_v = sweep_floor(key_score(th), kExact, scale);
      }
    }
    __syncthreads();  // all overflow reads of the lists and counts are done
    take = rowok && s_cnt[lq] > uint32_t(cap);
    __syncthreads();
    if (take && g == 0) s_cnt[lq] = 0u;
    // (the next sweep's prologue barrier orders this reset before any append)
  }

  // ---------------- select: sort each row's candidates ----------------
  // The top-k key blocks go into the block's mask bitmap: with at most 64
  // key blocks as one register word per lane, OR-ed over the wave at the
  // end (the per-entry LDS atomics would all hit the same two words).
  const bool kb_word = nKB <= 64;
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
      else atomicOr(&s_bits[kb >> 5], 1u << (kb & 31));
    }
  };
  auto ncand = [&](int r) -> int { return (q0 + r < NQ) ? min(int(s_cnt[r]), cap) : 0; };
  // Segments of LS lanes x 8 keys sort one row each; a group of 8 rows runs as
  // one LS=8 pass (<= 64 keys per row), two LS=16 or four LS=32 passes.
  auto sort_rows = [&](auto ls_tag, int row0) {
    constexpr int LS = decltype(ls_tag)::value;
    const int r = row0 + L / LS, i = L & (LS - 1), n = ncand(r);
    uint64_t v[8];
    for (int pp = 0; pp < 8; ++pp) {
      const int e = i * 8 + pp;
      v[pp] = e < n ? s_cand[size_t(r) * cap + e] : 0ull;
    }
    segment_sort_desc<LS>(v, L);
    for (int pp = 0; pp < 8; ++pp) emit(r, i * 8 + pp, v[pp]);
  };
  for (int base = 16 * w; base < 16 * w + 16; base += 8) {
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
  if (kb_word) {  // block-uniform
    kbm |= lane_xor64<1>(kbm);
    kbm |= lane_xor64<2>(kbm);
    kbm |= lane_xor64<4>(kbm);
    kbm |= lane_xor64<8>(kbm);
    auto bor = [](uint32_t x, uint32_t y) { return x | y; };
    const uint32_t lo = group_reduce_bits(uint32_t(kbm), bor);
    const uint32_t hi = group_reduce_bits(uint32_t(kbm >> 32), bor);
    if (L == 0) {
      if (lo) atomicOr(&s_bits[0], lo);
      if (hi) atomicOr(&s_bits[1], hi);
    }
  }
  __syncthreads();

  // ---------------- mask row; sorted values for the tau kernel ----------------
  uint8_t* mrow = p.mask + (size_t(bh) * nQB + qb) * nKB;
  for (int kb = t; kb < nKB; kb += kThreads) mrow[kb] = uint8_t((s_bits[kb >> 5] >> (kb & 31)) & 1u);
  const size_t rows = size_t(p.d.BH) * NQ;
  for (int i = t; i < k * kBlock; i += kThreads) {
    const int e = i >> 6, r = i & 63;
    if (q0 + r < NQ) p.tkv[size_t(e) * rows + size_t(bh) * NQ + q0 + r] = s_tk[e * kWave + r];
  }
}

// Smallest and largest position of every 64-key block of every (batch,
// head): kbounds[bh * nKB + kb] = (min, max) over the block's keys < NK.
// One wave per key block.
__global__ __launch_bounds__(kThreads) void bounds_kernel(SelectParams p) {
  const int nKB = p.d.nKB, NK = p.d.NK;
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
__global__ __launch_bounds__(kThreads) void tau_kernel(SelectParams p) {
  const size_t rows = size_t(p.d.BH) * p.d.NQ;
  const size_t r = size_t(blockIdx.x) * kThreads + threadIdx.x;
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

template <typename T, int D, int MODE, int R>
hipError_t launch_one(const SelectParams& p, hipStream_t s) {
  const SelLayout l = sel_layout(p.d.k, p.cap, p.d.nKB, D, int(sizeof(T)), MODE == kGivenScores);
  auto kern = select_kernel<T, D, MODE, R>;
  if (l.total > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, l.total);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3(p.d.nQB * p.d.BH), dim3(kThreads), l.total, s, p);
  return hipGetLastError();
}

// Class sets per (row, position): more sets tighten the sweep-2 floor; the
// larger k, the more candidates a loose floor admits.
template <typename T, int D, int MODE>
hipError_t launch_r(const SelectParams& p, hipStream_t s) {
  if (p.d.k <= 32) return launch_one<T, D, MODE, 2>(p, s);
  if (p.d.k <= 64) return launch_one<T, D, MODE, 4>(p, s);
  return launch_one<T, D, MODE, 8>(p, s);
}

template <typename T, int D>
hipError_t launch_mode(const SelectParams& p, hipStream_t s) {
  if (p.d.scale > 0.0f) return launch_r<T, D, kRawDots>(p, s);
  return launch_r<T, D, kExactScores>(p, s);
}

int tbytes_of(bool bf16) { return bf16 ? 2 : 4; }
int dim_of(const Dims& d, bool from_scores) { return from_scores ? 64 : d.D; }

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

size_t select_lds_bytes(const Dims& d, bool bf16, bool from_scores, int cap) {
  return size_t(sel_layout(d.k, cap, d.nKB, dim_of(d, from_scores),
                           from_scores ? 4 : tbytes_of(bf16), from_scores).total);
}

int select_capacity(const Dims& d, bool bf16, bool from_scores, size_t max_lds) {
  // k + 32 keys per row holds the candidates of random rows with room to
  // spare; less still works (overflow rounds), as long as it exceeds k.
  int cap = d.k + 32;
  if (cap > 256) cap = 256;
  while (cap > d.k && select_lds_bytes(d, bf16, from_scores, cap) > max_lds) cap -= 8;
  return cap > d.k ? cap : -1;
}

hipError_t launch_select(const SelectParams& p, bool bf16, bool from_scores, hipStream_t s) {
  if (from_scores) return launch_r<float, 64, kGivenScores>(p, s);
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
