// Exact threshold over every visible key of a row ("exact" tau mode).
//
// The reference solves tau on the row's top-k scores only, with a fixed
// five-step recurrence (entmax_threshold, adasplashattention.cu:51-125), so
// rows whose alpha-entmax support is larger than k, or whose recurrence has
// not converged, get a threshold that is not the alpha-entmax one.  This
// kernel, run after the score pass and before CSR compaction, replaces tau
// by the root of
//
//   f(tau) = sum_{j visible} [(alpha - 1) s_j - tau]_+^a - 1,  a = 1/(alpha-1),
//
// over the whole visible row (the dense alpha-entmax threshold), and marks
// every key block that holds a key with u = (alpha - 1) s - tau > 0 at that
// threshold as active, so that the block-sparse forward weights exactly the
// dense alpha-entmax support.
//
// f is decreasing in tau, and f over the whole row is at least f over any
// subset of it.  Per row:
//   1. Newton on the sorted top-k values (the score pass's workspace),
//      safeguarded by the bracket [z1 - 1, z1], z1 = (alpha - 1) s_max, where
//      f >= 0 at the left end and f = -1 at the right.  Its root tau_k is at
//      most the exact one.  If the k-th value satisfies z_k <= tau_k, no key
//      outside the top-k can have u > 0 at tau_k (its score is at most s_k),
//      so tau_k is already the exact threshold (every row with fewer than k
//      visible keys, and every row whose support is smaller than k).
//   2. Otherwise the row needs the whole row.  A sweep recomputes the row's
//      scores (S^T = K Q^T on MFMA from K tiles staged through LDS, as in
//      the forward) and sums v^a and v^(a-1) over v = max(u, 0).  The
//      first sweep, at tau_k, also lists in LDS every key with u > 0 (its
//      raw dot product and key block): the exact support lies inside that
//      list, since tau_exact >= tau_k (lists for up to kListRows rows per
//      block).  A row whose list fits (lcap entries) finishes there: safeguarded Newton steps over
//      the listed keys, then its support's key blocks are marked from the
//      list.  A row whose list overflowed takes one safeguarded Newton
//      step per further sweep instead (bracket: left end from step 1,
//      right end z1), until |f| <= 1e-6, a step leaves tau unchanged, or
//      kMaxSweeps sweeps.  The block sweeps until all its rows have
//      stopped; in that last sweep every row uses its final tau, and the
//      key blocks where some row had u > 0 in it join the mask.
//
// One 256-thread block per (batch*head, 64-query block).  In step 1 wave w
// owns rows 16w..16w+15; for step 2 the rows that need sweeps are packed
// into the first waves (about 5 of 64 rows at the headline shape, so
// usually one wave computes while the others only stage K tiles).  Lane L
// holds keys 16f + 4g + r (g = L / 16) of its row L % 16: the four lanes of
// a row hold identical per-row state, and their partial sums are combined
// with sum_groups (bit-identical in all four).
#include <climits>

#include "asa_device.hpp"
#include "asa_launch.hpp"
#include "asa_stage.hpp"
#include "asa_tiles.hpp"

namespace asa {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxTopkSteps = 64;  // Newton / bisection steps on the top-k values
constexpr int kMaxSweeps = 32;     // full-row sweeps per query block
constexpr float kTol = 1e-6f;      // |sum p - 1| at which a row's tau is final
// Packed rows with a key list (the first 16: one wave's rows).  More rows
// than this per block are rare (about 5 of 64 need sweeps at the headline
// shape); the others sweep.  Fewer lists keep the LDS per block small, so
// that more blocks share a compute unit.
constexpr int kListRows = 16;

// v^a and v^(a-1) for v = max(u, 0); both zero at v = 0.
template <int PC>
__device__ __forceinline__ void pow_pair(float v, float a, float& pa, float& pa1) {
  if constexpr (PC == kE2) {  // alpha 1.5
    pa = v * v;
    pa1 = v;
  } else if constexpr (PC == kE1) {  // alpha 2
    pa = v;
    pa1 = v > 0.0f ? 1.0f : 0.0f;
  } else if constexpr (PC == kE4) {  // alpha 1.25
    const float v2 = v * v;
    pa1 = v2 * v;
    pa = v2 * v2;
  } else {
    const float l = __builtin_amdgcn_logf(v);  // log2
    const float x = __builtin_amdgcn_exp2f(a * l);
    const float y = __builtin_amdgcn_exp2f((a - 1.0f) * l);
    pa = v > 0.0f && finite(x) ? x : 0.0f;
    pa1 = v > 0.0f && finite(y) ? y : 0.0f;
  }
}

// One safeguarded Newton step from tau, where f(tau) = f and
// f'(tau) = -a F1: the bracket end on tau's side of the root moves to tau;
// a step that leaves the open bracket (or F1 = 0) is replaced by bisection.
__device__ __forceinline__ float newton_step(float tau, float f, float F1, float a, float& lo,
                                             float& hi) {
  if (f >= 0.0f) lo = tau;
  else hi = tau;
  const float nt = tau + f / (a * F1);
  return (nt > lo && nt < hi) ? nt : 0.5f * (lo + hi);
}

struct ExactLayout {
  int kid, busy, cnt, rowst, ldot, lkb, vlist, bits, total;
};
__host__ __device__ inline int align16(int x) { return (x + 15) & ~15; }
// lcap: listed keys per row (0: no lists)
__host__ __device__ inline ExactLayout exact_layout(int D, int tbytes, int nKB, int lcap) {
  const int rs = tbytes == 2 ? D + 8 : D + 4;  // Tile<T, D>::kRs
  ExactLayout l;
  l.kid = align16(2 * kBlock * rs * tbytes);
  l.busy = l.kid + 2 * kBlock * 4;
  l.cnt = l.busy + 16 * 4;
  l.rowst = l.cnt + kBlock * 4;  // tau, lo, z1 and packed row of each row
  l.ldot = l.rowst + 4 * kBlock * 4;
  l.lkb = l.ldot + kListRows * lcap * 4;
  l.vlist = l.lkb + kListRows * lcap * 4;
  l.bits = l.vlist + align16(nKB * 4);
  l.total = l.bits + align16((nKB + 31) / 32 * 4);
  return l;
}

template <typename T, int D, int PC>
__global__ __launch_bounds__(kThreads) void refine_kernel(SelectParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  using Ks = KStage<T, D, kThreads>;
  static_assert(Tile<T, D>::kRs == (sizeof(T) == 2 ? D + 8 : D + 4), "layout row stride");
  const int NQ = p.d.NQ, NK = p.d.NK, nQB = p.d.nQB, nKB = p.d.nKB, k = p.d.k;
  const int lcap = p.lcap;
  const ExactLayout lay = exact_layout(D, int(sizeof(T)), nKB, lcap);
  T* s_k = reinterpret_cast<T*>(smem);
  int* s_kid = reinterpret_cast<int*>(smem + lay.kid);
  int* s_busy = reinterpret_cast<int*>(smem + lay.busy);
  uint32_t* s_cnt = reinterpret_cast<uint32_t*>(smem + lay.cnt);
  float* s_tau = reinterpret_cast<float*>(smem + lay.rowst);
  float* s_lo = s_tau + kBlock;
  float* s_z1 = s_lo + kBlock;
  int* s_rows = reinterpret_cast<int*>(s_z1 + kBlock);
  float* s_ldot = reinterpret_cast<float*>(smem + lay.ldot);
  int* s_lkb = reinterpret_cast<int*>(smem + lay.lkb);
  int* s_vlist = reinterpret_cast<int*>(smem + lay.vlist);
  uint32_t* s_bits = reinterpret_cast<uint32_t*>(smem + lay.bits);
  constexpr int kTileElems = kBlock * Tile<T, D>::kRs;

  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int task = xcd_task(blockIdx.x, nQB * p.d.BH);
  const int qb = nQB - 1 - task % nQB, bh = task / nQB;
  const int q = qb * kBlock + 16 * w + c16;
  const bool rowok = q < NQ;
  const size_t rows = size_t(p.d.BH) * NQ;
  const size_t grow = size_t(bh) * NQ + (rowok ? q : 0);
  const float am1 = p.d.alpha - 1.0f;
  const float a = 1.0f / am1;

  // ---- 1. Newton on the row's sorted top-k values ----
  const float* tk = p.tkv + grow;  // slot e at tk[e * rows], best first
  const float s1 = rowok ? tk[0] : kSentinel;
  const bool seen = rowok && s1 > kSentinel;  // the row sees at least one key
  const float z1 = am1 * s1;
  float lo = z1 - 1.0f, hi = z1;
  // start from the reference recurrence's tau when it lies in the bracket
  float tau = rowok ? p.taus[grow] : lo;
  if (!(tau > lo && tau < hi)) tau = lo;
  bool busy = seen;
  for (int it = 0; it < kMaxTopkSteps; ++it) {
    if (__ballot(busy) == 0) break;  // wave-uniform
    float F = 0.0f, F1 = 0.0f;
    for (int e = g; e < k; e += 4) {
      float pa, pa1;
      pow_pair<PC>(fmaxf(am1 * tk[size_t(e) * rows] - tau, 0.0f), a, pa, pa1);
      F += pa;
      F1 += pa1;
    }
    F = sum_groups(F);
    F1 = sum_groups(F1);
    const float f = F - 1.0f;
    if (busy) {
      if (fabsf(f) <= kTol) {
        busy = false;
      } else {
        const float nt = newton_step(tau, f, F1, a, lo, hi);
        busy = nt != tau;
        tau = nt;
      }
    }
  }
  // rows whose k-th value is inside the support need the full row
  const bool need = seen && am1 * tk[size_t(k - 1) * rows] > tau;

  // ---- 2. full-row sweeps, for the rows that need them ----
  if (seen && !need && g == 0) p.taus[grow] = tau;  // final
  // The rows that need sweeps are packed into the first waves (slot j of
  // the packed list goes to wave j / 16, column j % 16), so that waves with
  // no such row only help stage the K tiles.
  const int lrow = 16 * w + c16;  // the lane's row within the block
  const uint32_t wneed = uint32_t(__ballot(need)) & 0xffffu;  // lanes 0-15: one per row
  if (lane == 0) s_busy[8 + w] = __builtin_popcount(wneed);
  if (need && g == 0) {
    s_tau[lrow] = tau;
    s_lo[lrow] = lo;
    s_z1[lrow] = z1;
  }
  if (t < kBlock) s_cnt[t] = 0u;
  // visible key blocks (block | class << 24; class 2: every key visible to
  // every row of the block)
  const bool lv = qb * kBlock + lane < NQ;
  const int lpos = lv ? p.q_idx[size_t(bh) * NQ + qb * kBlock + lane] : 0;
  const int qmax = wave_reduce_minmax<true>(lv ? lpos : INT_MIN);
  const int qmin = wave_reduce_minmax<false>(lv ? lpos : INT_MAX);
  if (w == 0) {
    const int2* kbnd = p.kbounds + size_t(bh) * nKB;
    int n = 0;
    for (int base = 0; base < nKB; base += kWave) {
      const int kt = base + lane;
      int v = 0;
      if (kt < nKB) {
        const int2 kb = kbnd[kt];
        v = kb.x > qmax ? 0 : ((kb.y > qmin || (kt + 1) * kBlock > NK) ? 1 : 2);
      }
      const uint64_t m = __ballot(v != 0);
      if (v != 0) s_vlist[n + lane_rank(m)] = kt | (v << 24);
      n += __builtin_popcountll(m);
    }
    if (lane == 0) s_busy[12] = n;
  }
  __syncthreads();
  const int nneed = s_busy[8] + s_busy[9] + s_busy[10] + s_busy[11];
  if (need && g == 0) {
    int before = 0;
    for (int i = 0; i < w; ++i) before += s_busy[8 + i];
    s_rows[before + __builtin_popcount(wneed & ((1u << c16) - 1u))] = lrow;
  }
  const int nvis = s_busy[12];
  __syncthreads();

  if (nneed > 0) {  // block-uniform
    // this lane's packed row
    const int slot = 16 * w + c16;
    const bool pk = slot < nneed;
    const int prow = pk ? s_rows[slot] : 0;
    const int pq = qb * kBlock + prow;
    const size_t pgrow = size_t(bh) * NQ + pq;
    tau = pk ? s_tau[prow] : 0.0f;
    lo = pk ? s_lo[prow] : 0.0f;
    const float pz1 = pk ? s_z1[prow] : 0.0f;
    hi = pz1;  // f over the whole row is -1 there; lo keeps f >= 0

    const T* Kb = static_cast<const T*>(p.k) + size_t(bh) * NK * D;
    const int32_t* kidx = p.k_idx + size_t(bh) * NK;
    RowFrag<T, D> qf;
    qf.load(static_cast<const T*>(p.q) + pgrow * D, pk, lane);
    const int qpos = pk ? p.q_idx[pgrow] : 0;
    const bool wsweep = 16 * w < nneed;  // wave-uniform
    const int nbw = (nKB + 31) >> 5;
    const bool lslot = slot < kListRows;  // this row has a key list
    float* ldot = s_ldot + (lslot ? slot : 0) * lcap;
    int* lkb = s_lkb + (lslot ? slot : 0) * lcap;
    bool done = !pk;
    bool listed = false;  // the row finished on its list
    Ks ks;
    PosStager ps;
    for (int sw = 0;; ++sw) {
      for (int i = t; i < nbw; i += kThreads) s_bits[i] = 0u;
      // rows that stopped keep their final tau and still mark their blocks
      const ClippedU clip(am1, p.d.scale, tau, pk);
      // first sweep (at tau_k): the keys with u > 0 go to the row's list
      const bool collect = sw == 0 && lcap > 0;  // block-uniform
      double F = 0.0, F1 = 0.0;
      auto fetch = [&](int e) {
        const int kbase = (s_vlist[e] & 0xffffff) * kBlock;
        ks.load(Kb, kbase, NK, t);
        ps.load(kidx, kbase, NK, INT32_MAX, t);
      };
      auto put = [&](int b) {
        ks.store(s_k + b * kTileElems, t);
        ps.store(s_kid + b * kBlock, t);
      };
      __syncthreads();  // bitmap cleared; the previous sweep's tiles consumed
      if (nvis > 0) {
        fetch(0);
        put(0);
        if (nvis > 1) fetch(1);
      }
      __syncthreads();
      for (int e = 0; e < nvis; ++e) {
        const int b = e & 1;
        const int ent = s_vlist[e];
        if (wsweep) {
          f32x4 acc[4];
          rows_x_frag<D>(acc, s_k + b * kTileElems, qf, lane);
          const bool full = (ent >> 24) == 2;
          float tF = 0.0f, tF1 = 0.0f, vmax = 0.0f;
          uint32_t m = 0;  // bit 4f + r: key 16f + 4g + r has u > 0
          for (int f = 3; f >= 0; --f)
            for (int r = 3; r >= 0; --r) {
              float v = clip(acc[f][r]);
              if (!full) v = s_kid[b * kBlock + 16 * f + 4 * g + r] <= qpos ? v : 0.0f;
              float pa, pa1;
              pow_pair<PC>(v, a, pa, pa1);
              tF += pa;
              tF1 += pa1;
              if (collect) m = 2u * m + (v > 0.0f ? 1u : 0u);
              else vmax = fmaxf(vmax, v);
            }
          F += double(tF);
          F1 += double(tF1);
          const int kb = ent & 0xffffff;
          if (__ballot(collect ? m != 0u : vmax > 0.0f) != 0 && lane == 0)
            atomicOr(&s_bits[kb >> 5], 1u << (kb & 31));
          if (collect && lslot && m) {
            int j = int(atomicAdd(&s_cnt[slot], uint32_t(__builtin_popcount(m))));
            for (int f = 0; f < 4; ++f)
              for (int r = 0; r < 4; ++r)
                if ((m >> (4 * f + r)) & 1u) {
                  if (j < lcap) {
                    ldot[j] = acc[f][r];
                    lkb[j] = kb;
                  }
                  ++j;
                }
          }
        }
        if (e + 1 < nvis) {
          put(b ^ 1);
          if (e + 2 < nvis) fetch(e + 2);
        }
        __syncthreads();
      }
      const float Fs = sum_groups(float(F));
      const float F1s = sum_groups(float(F1));
      const float f = Fs - 1.0f;
      if (collect) {
        // a row whose list holds every key with u > 0 at tau_k finishes on
        // it: f over the list is exact for tau >= tau_k (the fused u is
        // monotone in tau), and tau_exact >= tau_k
        listed = lslot && !done && s_cnt[slot] <= uint32_t(lcap);
        const int n = listed ? int(s_cnt[slot]) : 0;
        float llo = tau, lhi = pz1;
        bool lbusy = listed;
        for (int it = 0; it < kMaxTopkSteps; ++it) {
          if (__ballot(lbusy) == 0) break;  // wave-uniform
          const ClippedU cl(am1, p.d.scale, tau, true);
          float LF = 0.0f, LF1 = 0.0f;
          for (int j = g; j < n; j += 4) {
            float pa, pa1;
            pow_pair<PC>(cl(ldot[j]), a, pa, pa1);
            LF += pa;
            LF1 += pa1;
          }
          LF = sum_groups(LF);
          LF1 = sum_groups(LF1);
          if (lbusy) {
            const float lf = LF - 1.0f;
            if (fabsf(lf) <= kTol) {
              lbusy = false;
            } else {
              const float nt = newton_step(tau, lf, LF1, a, llo, lhi);
              lbusy = nt != tau;
              tau = nt;
            }
          }
        }
        if (listed) done = true;
      }
      if (!done) {
        if (fabsf(f) <= kTol || sw + 1 == kMaxSweeps) {
          done = true;
        } else {
          const float nt = newton_step(tau, f, F1s, a, lo, hi);
          done = nt == tau;
          tau = nt;
        }
      }
      // After the first sweep a block with an overflowed list sweeps again
      // even if every row stopped: its marks must come from a sweep at the
      // rows' final tau.
      const uint64_t wbusy = __ballot(!done || (collect && pk && !listed));
      if (lane == 0) s_busy[4 * (sw & 1) + w] = wbusy != 0;
      __syncthreads();
      const int* bz = s_busy + 4 * (sw & 1);
      if ((bz[0] | bz[1] | bz[2] | bz[3]) == 0) {  // block-uniform
        if (collect) {
          // every row that swept finished on its list, but the sweep ran at
          // tau_k: mark the blocks of the listed keys with u > 0 at the
          // final tau instead
          for (int i = t; i < nbw; i += kThreads) s_bits[i] = 0u;
          __syncthreads();
          const ClippedU cl(am1, p.d.scale, tau, listed);
          const int n = listed ? int(s_cnt[slot]) : 0;
          for (int j = g; j < n; j += 4)
            if (cl(ldot[j]) > 0.0f) atomicOr(&s_bits[lkb[j] >> 5], 1u << (lkb[j] & 31));
          __syncthreads();
        }
        break;
      }
    }
    // the marks are those of the rows' final tau: their blocks join the mask
    uint8_t* mrow = p.mask + (size_t(bh) * nQB + qb) * nKB;
    for (int kb = t; kb < nKB; kb += kThreads)
      if ((s_bits[kb >> 5] >> (kb & 31)) & 1u) mrow[kb] = 1;
    if (pk && g == 0) p.taus[pgrow] = tau;
  }
}

template <typename T, int D, int PC>
hipError_t launch_one(const SelectParams& p, size_t lds, hipStream_t s) {
  auto kern = refine_kernel<T, D, PC>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(kern, dim3(p.d.nQB * p.d.BH), dim3(kThreads), lds, s, p);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_td(const SelectParams& p, size_t lds, hipStream_t s) {
  switch (alpha_class_of(p.d.alpha)) {
    case kA15: return launch_one<T, D, kE2>(p, lds, s);
    case kA20: return launch_one<T, D, kE1>(p, lds, s);
    case kA125: return launch_one<T, D, kE4>(p, lds, s);
    default: return launch_one<T, D, kEGen>(p, lds, s);
  }
}

}  // namespace

size_t refine_lds_bytes(const Dims& d, bool bf16, int lcap) {
  return size_t(exact_layout(d.D, bf16 ? 2 : 4, d.nKB, lcap).total);
}

int refine_list_capacity(const Dims& d, bool bf16, size_t max_lds) {
  // k + 32 listed keys hold the u > 0 keys of random rows at tau_k with
  // room to spare (at most ~1.7 k at k = 32); rows that overflow sweep on
  int lcap = d.k + 32 > 64 ? d.k + 32 : 64;
  while (lcap > 0 && refine_lds_bytes(d, bf16, lcap) > max_lds) lcap -= 16;
  if (lcap < 0) lcap = 0;
  return refine_lds_bytes(d, bf16, lcap) <= max_lds ? lcap : -1;
}

hipError_t launch_refine(const SelectParams& p, bool bf16, hipStream_t s) {
  const size_t lds = refine_lds_bytes(p.d, bf16, p.lcap);
  if (bf16) {
    if (p.d.D == 64) return launch_td<u16, 64>(p, lds, s);
    if (p.d.D == 128) return launch_td<u16, 128>(p, lds, s);
  } else {
    if (p.d.D == 64) return launch_td<float, 64>(p, lds, s);
    if (p.d.D == 128) return launch_td<float, 128>(p, lds, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace asa
