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
//      scores (S^T = K Q^T on MFMA, the forward's operands and order, so
//      the same bits) and sums v^a and v^(a-1) over v = max(u, 0).  The
//      first sweep, at tau_k, also lists in LDS every key with u > 0 (its
//      raw dot product and key block): the exact support lies inside that
//      list, since tau_exact >= tau_k.  A row whose lists fit finishes
//      there: safeguarded Newton steps over the listed keys, then its
//      support's key blocks are marked from them.  A row whose lists
//      overflowed (or beyond the first kListRows of a block) takes one
//      safeguarded Newton step per further sweep instead (bracket: left
//      end from step 1, right end z1), until |f| <= 1e-6, a step leaves tau
//      unchanged, or kMaxSweeps sweeps.  The block sweeps until all its rows
//      have stopped; in that last sweep every row uses its final tau, and
//      the key blocks where some row had u > 0 in it join the mask.
//
// One 256-thread block per (batch*head, 64-query block).  In step 1 wave w
// owns rows 16w..16w+15, starting from the reference recurrence's tau when
// it lies in the bracket.  The rows that need sweeps (about 5 of 64 at the
// headline shape) are packed into groups of 16, their Q rows staged in LDS.
// In a sweep every wave takes every fourth visible key tile, loads the
// tile's K fragments once straight from global memory (a head's K stays in
// L2) and multiplies them by every group's Q rows, so no barrier separates
// the tiles, all four waves compute and K is read once per sweep.  The
// waves' partial sums and key lists (one per wave and row) meet in LDS and
// are combined in a fixed order, so results do not depend on timing.  Lane L holds keys 16f + 4g + r (g = L / 16) of its
// row L % 16: the four lanes of a row hold identical per-row state, and
// their partial sums are combined with sum_groups (bit-identical in all
// four).
#include <climits>

#include "asa_device.hpp"
#include "asa_launch.hpp"
#include "asa_tiles.hpp"

namespace asa {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxTopkSteps = 64;  // Newton / bisection steps on the top-k values
constexpr int kMaxSweeps = 32;     // full-row sweeps per query block
constexpr float kTol = 1e-6f;      // |sum p - 1| at which a row's tau is final
// Packed rows with key lists (the first 16 of a block).  More rows than
// this per block are rare (about 5 of 64 need sweeps at the headline
// shape); the others sweep.
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
// For a >= 1 (alpha <= 2) the terms of F1 are bounded, so a step below
// half an ulp of tau means tau is the root to float precision: it is
// returned unchanged (the caller stops) instead of being taken for a step
// out of the bracket, which would restart a bisection from the bracket's
// width.  For a < 1 a key with u -> 0+ makes F1 unbounded while f may
// still be far from 0, so the bisection safeguard stays.
__device__ __forceinline__ float newton_step(float tau, float f, float F1, float a, float& lo,
                                             float& hi) {
  if (f >= 0.0f) lo = tau;
  else hi = tau;
  const float nt = tau + f / (a * F1);
  if (nt == tau && a >= 1.0f) return tau;
  return (nt > lo && nt < hi) ? nt : 0.5f * (lo + hi);
}

struct ExactLayout {
  int busy, cnt, rowst, part, qrows, ldot, lkb, vlist, bits, total;
};
__host__ __device__ inline int align16(int x) { return (x + 15) & ~15; }
// lcap: listed keys per packed row and wave (0: no lists); qbytes: one
// query row (D elements)
__host__ __device__ inline ExactLayout exact_layout(int nKB, int lcap, int qbytes) {
  ExactLayout l;
  l.busy = 0;
  l.cnt = l.busy + 16 * 4;          // list lengths [wave][packed row < kListRows]
  l.rowst = l.cnt + kBlock * 4;     // per row: tau, lo, z1, packed row; per slot: tau
  l.part = l.rowst + 5 * kBlock * 4;  // per wave and slot: partial F and F1
  l.qrows = l.part + 2 * 4 * kBlock * 4;  // the packed rows' Q, [slot][D]
  l.ldot = l.qrows + kBlock * qbytes;
  l.lkb = l.ldot + 4 * kListRows * lcap * 4;
  l.vlist = l.lkb + 4 * kListRows * lcap * 4;
  l.bits = l.vlist + align16(nKB * 4);
  l.total = l.bits + align16((nKB + 31) / 32 * 4);
  return l;
}

template <typename T, int D, int PC>
__global__ __launch_bounds__(kThreads) void refine_kernel(SelectParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int NQ = p.d.NQ, NK = p.d.NK, nQB = p.d.nQB, nKB = p.d.nKB, k = p.d.k;
  const int lcap = p.lcap;
  const ExactLayout lay = exact_layout(nKB, lcap, D * int(sizeof(T)));
  int* s_busy = reinterpret_cast<int*>(smem + lay.busy);
  uint32_t* s_cnt = reinterpret_cast<uint32_t*>(smem + lay.cnt);
  float* s_tau = reinterpret_cast<float*>(smem + lay.rowst);
  float* s_lo = s_tau + kBlock;
  float* s_z1 = s_lo + kBlock;
  int* s_rows = reinterpret_cast<int*>(s_z1 + kBlock);
  float* s_ptau = reinterpret_cast<float*>(s_rows + kBlock);
  float* s_pF = reinterpret_cast<float*>(smem + lay.part);
  float* s_pF1 = s_pF + 4 * kBlock;
  T* s_q = reinterpret_cast<T*>(smem + lay.qrows);
  float* s_ldot = reinterpret_cast<float*>(smem + lay.ldot);
  int* s_lkb = reinterpret_cast<int*>(smem + lay.lkb);
  int* s_vlist = reinterpret_cast<int*>(smem + lay.vlist);
  uint32_t* s_bits = reinterpret_cast<uint32_t*>(smem + lay.bits);

  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int g = lane >> 4, c16 = lane & 15;
  int brank, bh;
  xcd_rank_order(blockIdx.x, nQB, p.d.BH, brank, bh);
  const int qb = nQB - 1 - brank;  // heaviest first
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
  // a row still stepping after kMaxTopkSteps keeps its last iterate; the
  // caller can see that in the status word
  if (__ballot(busy) != 0 && lane == 0 && p.status) atomicOr(p.status, kStatusRefineSweeps);
  // rows whose k-th value is inside the support need the full row
  const bool need = seen && am1 * tk[size_t(k - 1) * rows] > tau;

  // ---- 2. full-row sweeps, for the rows that need them ----
  if (seen && !need && g == 0) p.taus[grow] = tau;  // final
  // The rows that need sweeps are packed in row order: slot j of the
  // packed list is row s_rows[j]; its state is read by wave j / 16, column
  // j % 16 in the update phase, and by every wave in the sweeps.
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
    // Update-phase identity: wave w, column c16 owns packed slot 16w + c16
    // (its per-row state lives in registers of the row's four lanes).
    const int slot = 16 * w + c16;
    const bool pk = slot < nneed;
    const int prow = pk ? s_rows[slot] : 0;
    const size_t pgrow = size_t(bh) * NQ + qb * kBlock + prow;
    tau = pk ? s_tau[prow] : 0.0f;
    lo = pk ? s_lo[prow] : 0.0f;
    const float pz1 = pk ? s_z1[prow] : 0.0f;
    hi = pz1;  // f over the whole row is -1 there; lo keeps f >= 0
    if (pk && g == 0) s_ptau[slot] = tau;
    {  // the packed rows' Q, 16 bytes per thread and step (columns >= hd: zero)
      constexpr int kEpc = 16 / int(sizeof(T)), kCpr = D / kEpc;
      const T* Qh = static_cast<const T*>(p.q) + head_at(p.lq, bh, p.d.H) + size_t(qb * kBlock) * p.lq.sn;
      for (int i = t; i < nneed * kCpr; i += kThreads) {
        const int sl = i / kCpr, cc = i % kCpr;
        *reinterpret_cast<uint4*>(s_q + sl * D + cc * kEpc) =
            cc * kEpc < p.d.hd
                ? *reinterpret_cast<const uint4*>(Qh + size_t(s_rows[sl]) * p.lq.sn + cc * kEpc)
                : uint4{0u, 0u, 0u, 0u};
      }
    }

    // Sweep phase: every wave takes every fourth visible key tile and
    // multiplies its K fragments by all packed row groups (below).  Partial
    // sums meet in LDS in a fixed order.
    const int ngroups = (nneed + 15) >> 4;
    const T* Kb = static_cast<const T*>(p.k) + head_at(p.lk, bh, p.d.H);
    const int32_t* kidx = p.k_idx + size_t(bh) * NK;
    const int nbw = (nKB + 31) >> 5;
    bool done = !pk;
    bool listed = false;  // the row finished on its key lists
    for (int sw = 0;; ++sw) {
      for (int i = t; i < nbw; i += kThreads) s_bits[i] = 0u;
      // first sweep (at tau_k): every key with u > 0 goes to a list of its
      // (wave, row), for the first kListRows packed rows
      const bool collect = sw == 0 && lcap > 0;  // block-uniform
      __syncthreads();  // bitmap cleared; s_ptau published
      // per packed row group (at most 4), the lane's row state
      int sqpos[4];
      ClippedU clips[4] = {ClippedU(am1, p.d.scale, 0.0f, false), ClippedU(am1, p.d.scale, 0.0f, false),
                           ClippedU(am1, p.d.scale, 0.0f, false), ClippedU(am1, p.d.scale, 0.0f, false)};
      double F[4] = {0.0, 0.0, 0.0, 0.0}, F1[4] = {0.0, 0.0, 0.0, 0.0};
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int sl = 16 * rg + c16;
        const bool spk = sl < nneed;
        sqpos[rg] = spk ? p.q_idx[size_t(bh) * NQ + qb * kBlock + s_rows[sl]] : 0;
        // rows that stopped keep their final tau and still mark their blocks
        clips[rg] = ClippedU(am1, p.d.scale, spk ? s_ptau[sl] : 0.0f, spk);
      }
      const bool scol = collect && c16 < nneed;  // group 0 rows have lists
      float* ldot = s_ldot + (w * kListRows + c16) * lcap;
      int* lkb = s_lkb + (w * kListRows + c16) * lcap;
      // Tiles outermost: a tile's K fragments are loaded once and multiplied
      // by every group's Q rows (staged in LDS), so K is read once per sweep
      // whatever the number of groups.
      for (int e = w; e < nvis; e += 4) {
        const int ent = s_vlist[e];
        const int kb = ent & 0xffffff, kbase = kb * kBlock;
        const bool full = (ent >> 24) == 2;
        KFrags<T, D> kf;
        kf.load(Kb + size_t(kbase) * p.lk.sn, NK - kbase, size_t(p.lk.sn), p.d.hd, lane);
        float vany = 0.0f;  // > 0: some row of the wave has u > 0 in the tile
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          if (rg < ngroups) {  // block-uniform
            RowFrag<T, D> qf;
            qf.load(s_q + (16 * rg + c16) * D, 16 * rg + c16 < nneed, lane);
            f32x4 acc[4];
            kf.product(acc, qf);
            float tF = 0.0f, tF1 = 0.0f;
            uint32_t m = 0;  // bit 4f + r: key 16f + 4g + r has u > 0 (group 0)
            for (int f = 3; f >= 0; --f)
              for (int r = 3; r >= 0; --r) {
                float v = clips[rg](acc[f][r]);
                if (!full) {
                  const int key = kbase + 16 * f + 4 * g + r;
                  v = key < NK && kidx[key] <= sqpos[rg] ? v : 0.0f;
                }
                float pa, pa1;
                pow_pair<PC>(v, a, pa, pa1);
                tF += pa;
                tF1 += pa1;
                vany = fmaxf(vany, v);
                if (rg == 0 && collect) m = 2u * m + (v > 0.0f ? 1u : 0u);
              }
            F[rg] += double(tF);
            F1[rg] += double(tF1);
            if (rg == 0 && scol && m) {
              int j = int(atomicAdd(&s_cnt[w * kListRows + c16], uint32_t(__builtin_popcount(m))));
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
        }
        if (__ballot(vany > 0.0f) != 0 && lane == 0) atomicOr(&s_bits[kb >> 5], 1u << (kb & 31));
      }
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        if (rg < ngroups) {
          const int sl = 16 * rg + c16;
          const float Fs = sum_groups(float(F[rg]));
          const float F1s = sum_groups(float(F1[rg]));
          if (sl < nneed && g == 0) {
            s_pF[w * kBlock + sl] = Fs;
            s_pF1[w * kBlock + sl] = F1s;
          }
        }
      }
      __syncthreads();  // partial sums and lists complete

      // ---- update phase ----
      float f = 0.0f, F1s = 0.0f;
      if (pk) {
        f = ((s_pF[slot] + s_pF[kBlock + slot]) + (s_pF[2 * kBlock + slot] + s_pF[3 * kBlock + slot])) - 1.0f;
        F1s = (s_pF1[slot] + s_pF1[kBlock + slot]) + (s_pF1[2 * kBlock + slot] + s_pF1[3 * kBlock + slot]);
      }
      if (collect) {
        // a row whose lists hold every key with u > 0 at tau_k finishes on
        // them: f over the lists is exact for tau >= tau_k (the fused u is
        // monotone in tau), and tau_exact >= tau_k
        listed = pk && !done && slot < kListRows;
        for (int ww = 0; ww < 4; ++ww)
          listed = listed && s_cnt[ww * kListRows + (slot < kListRows ? slot : 0)] <= uint32_t(lcap);
        float llo = tau, lhi = pz1;
        bool lbusy = listed;
        for (int it = 0; it < kMaxTopkSteps; ++it) {
          if (__ballot(lbusy) == 0) break;  // wave-uniform
          const ClippedU cl(am1, p.d.scale, tau, true);
          float LF = 0.0f, LF1 = 0.0f;
          if (listed)
            for (int ww = 0; ww < 4; ++ww) {
              const float* ld = s_ldot + (ww * kListRows + slot) * lcap;
              const int n = int(s_cnt[ww * kListRows + slot]);
              for (int j = g; j < n; j += 4) {
                float pa, pa1;
                pow_pair<PC>(cl(ld[j]), a, pa, pa1);
                LF += pa;
                LF1 += pa1;
              }
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
        if (__ballot(lbusy) != 0 && lane == 0 && p.status) atomicOr(p.status, kStatusRefineSweeps);
        if (listed) done = true;
      }
      if (!done) {
        if (fabsf(f) <= kTol || sw + 1 == kMaxSweeps) {
          if (!(fabsf(f) <= kTol) && p.status) atomicOr(p.status, kStatusRefineSweeps);
          done = true;
        } else {
          const float nt = newton_step(tau, f, F1s, a, lo, hi);
          done = nt == tau;
          tau = nt;
        }
      }
      if (pk && g == 0) s_ptau[slot] = tau;
      // After the first sweep a block with a row that did not finish on its
      // lists sweeps again even if every row stopped: its marks must come
      // from a sweep at the rows' final tau.
      const uint64_t wbusy = __ballot(!done || (collect && pk && !listed));
      if (lane == 0) s_busy[4 * (sw & 1) + w] = wbusy != 0;
      __syncthreads();
      const int* bz = s_busy + 4 * (sw & 1);
      if ((bz[0] | bz[1] | bz[2] | bz[3]) == 0) {  // block-uniform
        if (collect) {
          // every row finished on its lists, but the sweep ran at tau_k:
          // mark the blocks of the listed keys with u > 0 at the final tau
          for (int i = t; i < nbw; i += kThreads) s_bits[i] = 0u;
          __syncthreads();
          const ClippedU cl(am1, p.d.scale, tau, listed);
          if (listed)
            for (int ww = 0; ww < 4; ++ww) {
              const float* ld = s_ldot + (ww * kListRows + slot) * lcap;
              const int* lk = s_lkb + (ww * kListRows + slot) * lcap;
              const int n = int(s_cnt[ww * kListRows + slot]);
              for (int j = g; j < n; j += 4)
                if (cl(ld[j]) > 0.0f) atomicOr(&s_bits[lk[j] >> 5], 1u << (lk[j] & 31));
            }
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

size_t refine_lds_bytes(const Dims& d, int dtype, int lcap) {
  return size_t(exact_layout(d.nKB, lcap, d.D * elem_bytes(dtype)).total);
}

int refine_list_capacity(const Dims& d, int dtype, size_t max_lds) {
  // Per wave and row: the u > 0 keys of random rows at tau_k number at
  // most ~1.7 k at k = 32, a quarter of them per wave on average; (k + 32)
  // / 2 per wave leaves room for uneven splits.  Rows that overflow sweep.
  int lcap = (d.k + 32) / 2 > 32 ? (d.k + 32) / 2 : 32;
  while (lcap > 0 && refine_lds_bytes(d, dtype, lcap) > max_lds) lcap -= 16;
  if (lcap < 0) lcap = 0;
  return refine_lds_bytes(d, dtype, lcap) <= max_lds ? lcap : -1;
}

hipError_t launch_refine(const SelectParams& p, int dtype, hipStream_t s) {
  const size_t lds = refine_lds_bytes(p.d, dtype, p.lcap);
  if (dtype == kElemBF16) {
    if (p.d.D == 64) return launch_td<u16, 64>(p, lds, s);
    if (p.d.D == 128) return launch_td<u16, 128>(p, lds, s);
  } else if (dtype == kElemF16) {
    if (p.d.D == 64) return launch_td<h16, 64>(p, lds, s);
    if (p.d.D == 128) return launch_td<h16, 128>(p, lds, s);
  } else {
    if (p.d.D == 64) return launch_td<float, 64>(p, lds, s);
    if (p.d.D == 128) return launch_td<float, 128>(p, lds, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace asa
