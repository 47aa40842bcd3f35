// Block-sparse forward: out = sum_j p_j v_j / (sum_j p_j + EPS) over the
// visible keys of the active key blocks of each query block.
//
// Reference: splash_forward_sparse (adasplashattention.cu:244-341), which
// recomputes each score with one thread per query and accumulates p*v in
// registers.  Here one 256-thread block (4 waves x 16 query rows) walks the
// query block's CSR list.  The K and V tiles of each active key block
// stream through double-buffered LDS (asa_stage.hpp); S^T = K Q^T is formed
// on MFMA,
// p = max(u, EPS)^(1/(alpha-1)) with u = (alpha-1) s - tau is applied in
// registers (clamp, scale and tau folded into one fma and one median whose
// zero bounds are -0.0, SignedClip, so the sign bit of max(u, 0) is the
// support-mask bit), and O^T += V^T P^T runs on MFMA with P^T taken
// directly from the score accumulators.  Row sums of p are kept per lane
// and reduced across the four lane groups at the end.  With 32-row mask
// blocks the list is the union of the block's two halves' key blocks, and
// a wave skips the tiles its half's mask row lacks.
#include <type_traits>

#include "asa_device.hpp"
#include "asa_launch.hpp"
#include "asa_stage.hpp"
#include "asa_tiles.hpp"

namespace asa {
namespace {

constexpr int kThreads = 256;

template <typename T, int D> struct alignas(16) FwdSmem {
  T K[2][kBlock * Tile<T, D>::kRs];
  T V[2][kBlock * Tile<T, D>::kRs];
  int kid[2][kBlock];
};

template <typename T, int D, int PC, bool EMIT, bool HALF>
__global__ __launch_bounds__(kThreads) void forward_kernel(ForwardParams p) {
  __shared__ FwdSmem<T, D> sm;
  using St = Stager<T, D>;
  const int NQ = p.d.NQ, NK = p.d.NK, nQB = p.d.nQB, nKB = p.d.nKB;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int g = lane >> 4, c16 = lane & 15;
  int brank, bh;
  xcd_rank_order(blockIdx.x, nQB, p.d.BH, brank, bh);
  const int qb = nQB - 1 - brank;  // heaviest first
  const int q = qb * kBlock + 16 * w + c16;  // this lane's query row
  const bool qok = q < NQ;
  const size_t row = size_t(bh) * NQ + (qok ? q : 0);
  const int H = p.d.H, hd = p.d.hd;

  const T* Kb = static_cast<const T*>(p.k) + head_at(p.lk, bh, H);
  const T* Vb = static_cast<const T*>(p.v) + head_at(p.lv, bh, H);
  const int32_t* kidx = p.k_idx + size_t(bh) * NK;

  RowFrag<T, D> qf;
  qf.load(static_cast<const T*>(p.q) + head_at(p.lq, bh, H) + size_t(qok ? q : 0) * p.lq.sn, qok,
          lane, hd);
  const int qpos = qok ? p.q_idx[row] : 0;
  const float am1 = p.d.alpha - 1.0f;
  const float a = 1.0f / am1;
  const SignedClip clip(am1, p.d.scale, qok ? p.taus[row] : 0.0f, qok);  // invalid rows: p = 0
  // fp16 P operands: the weights are scaled by 2^-e, e the exponent of the
  // row's largest weight (that of its best key), so that they fit fp16's
  // range (rows with fewer visible keys than k carry the -1e6 sentinel
  // into tau and can have weights far above 65504); the output divides the
  // scale out again.  bf16 and fp32 have fp32's range and use 1.
  float pscale = 1.0f;
  if constexpr (std::is_same<T, h16>::value) {
    if (qok) {
      const float s1 = p.top1[row];
      const float u1 = fmaxf(fminf(fmaf(am1, s1, -p.taus[row]), fmaf(10.0f, am1, -p.taus[row])), 0.0f);
      const float p1 = pow_clipped<PC>(u1, a);
      int e = 0;
      (void)frexpf(p1, &e);
      pscale = p1 > 0.0f ? (finite(p1) ? ldexpf(1.0f, -e) : 0.0f) : 1.0f;
    }
  }
  // smallest position of the block's valid rows: a key block whose largest
  // position (from the score pass's bounds) is at most this, and that lies
  // wholly below NK, is visible to every row of the block
  int qmin;
  {
    const int qq = qb * kBlock + lane;
    qmin = wave_reduce_minmax<false>(qq < NQ ? p.q_idx[size_t(bh) * NQ + qq] : INT32_MAX);
  }
  const int2* kbnd = p.kbounds + size_t(bh) * nKB;

  f32x4 o[D / 16];
  for (int db = 0; db < D / 16; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float rowsum = 0.0f;

  // Support masks: this wave's 64 lanes x 16 bits for each tile.
  uint16_t* smask = nullptr;
  if constexpr (EMIT) smask = p.sup.mask + size_t(bh) * nQB * nKB * 256 + w * 64 + 4 * c16 + g;

  // 32-row mask blocks: the mask row of this wave's half (rows 32 (w / 2)
  // of the block); a tile that row lacks contributes nothing to the wave
  const uint8_t* hrow = nullptr;
  bool hvalid = true;
  if constexpr (HALF) {
    const int h = 2 * qb + (w >> 1), nQH = half_blocks(NQ);
    hvalid = h < nQH;  // else every row of the half is past NQ
    hrow = p.half + (size_t(bh) * nQH + (hvalid ? h : 0)) * nKB;
  }

  const int32_t* qp = p.q_ptr + size_t(bh) * (nQB + 1);
  const int32_t* ql = p.q_list + size_t(bh) * nQB * nKB;
  const int e0 = qp[qb], e1 = qp[qb + 1];
  St st;
  PosStager ps;
  auto fetch = [&](int e) {
    const int kbase = ql[e] * kBlock;
    st.template load<kRowsStrided>(Kb, p.lk.sn, Vb, p.lv.sn, kbase, NK, hd, t);
    ps.load(kidx, kbase, NK, INT32_MAX, t);
  };
  auto put = [&](int b) {
    st.store(sm.K[b], sm.V[b], t);
    ps.store(sm.kid[b], t);
  };
  if (e0 < e1) {
    fetch(e0);
    put(0);
    if (e0 + 1 < e1) fetch(e0 + 1);
  }
  __syncthreads();
  for (int e = e0; e < e1; ++e) {
    const int b = (e - e0) & 1;
    const int kb = ql[e];
    bool act = true;  // wave-uniform
    if constexpr (HALF) act = hvalid && hrow[kb] != 0;
    f32x4 acc[4];
    if (act) rows_x_frag<D>(acc, sm.K[b], qf, lane);
    // p for every score, then masked: no per-score branches.  v = max(u, 0)
    // carries its sign bit where u <= 0 (SignedClip); with support masks the
    // lane's 16 bits of u > 0 are those sign bits, complemented.  The row
    // sums are of the float32 weights (the bf16 copies the P^T V product
    // takes would bias sums of many equal weights by up to 2^-9).
    auto weights = [&](auto partial) {
      uint32_t nm = 0;  // bit 4f + r <- u <= 0, highest bit first
      for (int f = 3; f >= 0; --f)
        for (int r = 3; r >= 0; --r) {
          float v = clip(acc[f][r]);  // max(u, 0)
          if constexpr (decltype(partial)::value)
            v = sm.kid[b][16 * f + 4 * g + r] <= qpos ? v : -0.0f;
          acc[f][r] = v;
          if constexpr (EMIT) nm = __builtin_amdgcn_alignbit(nm, __float_as_uint(v), 31);
        }
      if constexpr (EMIT) smask[size_t(e) * 256] = uint16_t(~nm);
      for (int f = 0; f < 4; ++f)
        for (int r = 0; r < 4; ++r) {
          const float pv = pow_clipped<PC>(acc[f][r], a);
          if constexpr (std::is_same<T, h16>::value) acc[f][r] = pv * pscale;
          else acc[f][r] = pv;
          rowsum += pv;
        }
    };
    if (act) {
      if (kb * kBlock + kBlock <= NK && kbnd[kb].y <= qmin) weights(std::false_type{});
      else weights(std::true_type{});
      tile_t_x_acc<D>(o, sm.V[b], acc, lane);
    } else if constexpr (EMIT) {
      smask[size_t(e) * 256] = 0;
    }
    if (e + 1 < e1) {
      put(b ^ 1);
      if (e + 2 < e1) fetch(e + 2);
    }
    __syncthreads();
  }

  const float norm = sum_groups(rowsum);
  const float inv = 1.0f / ((norm + kEps) * pscale);  // pscale 0: non-finite weights, output 0
  if (qok) {
    T* orow = static_cast<T*>(p.out) + head_at(p.lo, bh, H) + size_t(q) * p.lo.sn;
    for (int db = 0; db < D / 16; ++db)
      if (16 * db + 4 * g < hd)
        for (int r = 0; r < 4; ++r) {
          float v = o[db][r] * inv;
          if (!finite(v)) v = 0.0f;
          Elem<T>::store(orow + 16 * db + 4 * g + r, v);
        }
    if (g == 0) p.norms[row] = norm;
  }
}

// Two query blocks per workgroup (16-bit inputs): wave w holds rows
// 16w..16w+15 of both query blocks 2m and 2m+1, as two B fragments, and the
// workgroup walks the union of the two blocks' key-block lists (merged on
// the fly from the CSR).  Each K and V tile read from LDS then feeds two
// fragments' products (rows_x_frag2, tile_t_x_acc2): half the LDS reads
// per row of the one-block kernel, whose waves were half-bound by them.
//
// The clip is folded into the products (launch_tde checks that it applies,
// pair_fold_ok: an integer power class and c = (alpha - 1) scale in
// [2^-8, 2^8]): the score products start from -tau / c instead of 0, so
// that x = s - tau / c comes out of the MFMA and one v_med3 per score gives
// v' = med3(x, lo / c, hi / c) = max(u, 0) / c, with SignedClip's sign-bit
// rule.  The weights p' = v'^e are p / c^e, a per-launch constant that the
// output's ratio cancels; the row sums are scaled back by c^e.  This saves
// forward_kernel's fma per score (the kernel is VALU-bound); u is rounded
// as c (s - tau / c) instead of once, an ulp-level difference from
// forward_kernel.
// DENSE: Q, K, V and Out contiguous [B, H, N, D] (hd = D), compile-time
// strides; else any strides and hd.  Three waves per SIMD at d = 64; at
// d = 128 its 70 KB of LDS allow two blocks per compute unit, and the
// accumulators of both blocks' rows take up to 255 VGPRs.
template <typename T, int D, int PC, bool EMIT, bool HALF, bool DENSE>
__global__ __launch_bounds__(kThreads, (D == 64 ? 3 : 2)) void forward_pair_kernel(ForwardParams p) {
  static_assert(is_half<T>, "16-bit inputs only");
  __shared__ FwdSmem<T, D> sm;
  using St = Stager<T, D>;
  const int NQ = p.d.NQ, NK = p.d.NK, nQB = p.d.nQB, nKB = p.d.nKB;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int nP = (nQB + 1) / 2;
  int brank, bh;
  xcd_rank_order(blockIdx.x, nP, p.d.BH, brank, bh);
  const int qp2 = nP - 1 - brank;  // heaviest first
  const int H = p.d.H, hd = DENSE ? D : p.d.hd;

  const T* Kb = row_at<DENSE, D>(static_cast<const T*>(p.k), p.lk, bh, H, NK, 0);
  const T* Vb = row_at<DENSE, D>(static_cast<const T*>(p.v), p.lv, bh, H, NK, 0);
  const int32_t* kidx = p.k_idx + size_t(bh) * NK;
  const int2* kbnd = p.kbounds + size_t(bh) * nKB;
  const float am1 = p.d.alpha - 1.0f;
  const float a = 1.0f / am1;
  const int32_t* qp = p.q_ptr + size_t(bh) * (nQB + 1);
  const int32_t* ql = p.q_list + size_t(bh) * nQB * nKB;

  // per block h of the pair: rows, fragments, clipping, list, masks
  int qb[2], qpos[2], qmin[2], lb[2], le[2];
  bool qok[2], hvalid[2];
  size_t row[2];
  RowFrag<T, D> qf[2];
  const float cs = am1 * p.d.scale;  // c > 0 (pair_fold_ok)
  float x0[2] = {0.0f, 0.0f}, lo[2] = {-0.0f, -0.0f}, hi[2] = {-0.0f, -0.0f};  // folded clip
  float pscale[2] = {1.0f, 1.0f}, rowsum[2] = {0.0f, 0.0f};
  const uint8_t* hrow[2] = {nullptr, nullptr};
  uint16_t* smask = nullptr;
  if constexpr (EMIT) smask = p.sup.mask + size_t(bh) * nQB * nKB * 256 + w * 64 + 4 * c16 + g;
  for (int h = 0; h < 2; ++h) {
    qb[h] = 2 * qp2 + h;
    const bool bok = qb[h] < nQB;  // block-uniform
    const int q = qb[h] * kBlock + 16 * w + c16;
    qok[h] = bok && q < NQ;
    row[h] = size_t(bh) * NQ + (qok[h] ? q : 0);
    qf[h].load(row_at<DENSE, D>(static_cast<const T*>(p.q), p.lq, bh, H, NQ, qok[h] ? q : 0), qok[h],
               lane, hd);
    qpos[h] = qok[h] ? p.q_idx[row[h]] : 0;
    if (qok[h]) {
      // SignedClip's bounds, divided by c (rows that get no weight keep
      // x0 = 0 and lo = hi = -0: v' = -0 for every score)
      const float tau = p.taus[row[h]];
      const float l = fmaf(-10.0f, am1, -tau), u = fmaf(10.0f, am1, -tau);
      x0[h] = -tau / cs;
      lo[h] = l > 0.0f ? l / cs : -0.0f;
      hi[h] = u > 0.0f ? u / cs : -0.0f;
    }
    if constexpr (std::is_same<T, h16>::value) {
      // fp16 P operands scaled by 2^-e, e the exponent of the row's
      // largest weight p' (as in forward_kernel, for p)
      if (qok[h]) {
        const float s1 = p.top1[row[h]];
        const float u1 = fmaxf(fminf(fmaf(am1, s1, -p.taus[row[h]]), fmaf(10.0f, am1, -p.taus[row[h]])), 0.0f);
        const float p1 = pow_clipped<PC>(u1 / cs, a);
        int e = 0;
        (void)frexpf(p1, &e);
        pscale[h] = p1 > 0.0f ? (finite(p1) ? ldexpf(1.0f, -e) : 0.0f) : 1.0f;
      }
    }
    {
      const int qq = qb[h] * kBlock + lane;
      qmin[h] = wave_reduce_minmax<false>(bok && qq < NQ ? p.q_idx[size_t(bh) * NQ + qq] : INT32_MAX);
    }
    lb[h] = bok ? qp[qb[h]] : 0;
    le[h] = bok ? qp[qb[h] + 1] : 0;
    hvalid[h] = bok;
    if constexpr (HALF) {
      const int hh = 2 * qb[h] + (w >> 1), nQH = half_blocks(NQ);
      hvalid[h] = bok && hh < nQH;
      hrow[h] = p.half + (size_t(bh) * nQH + (hvalid[h] ? hh : 0)) * nKB;
    }
  }

  f32x4 o[2][D / 16];
  for (int h = 0; h < 2; ++h)
    for (int db = 0; db < D / 16; ++db) o[h][db] = f32x4{0.f, 0.f, 0.f, 0.f};

  // The merged list: entry = key block | bit 30 (in block 0's list) | bit
  // 31 (in block 1's), or -1 past the end.  Two cursors run ahead of the
  // tile being multiplied (its successor is in LDS, the next one loading).
  int c0 = lb[0], c1 = lb[1];
  auto advance = [&]() -> int {
    const int k0 = c0 < le[0] ? ql[c0] : INT32_MAX;
    const int k1 = c1 < le[1] ? ql[c1] : INT32_MAX;
    const int kb = min(k0, k1);
    if (kb == INT32_MAX) return -1;
    const bool a0 = k0 == kb, a1 = k1 == kb;
    c0 += a0 ? 1 : 0;
    c1 += a1 ? 1 : 0;
    return kb | (a0 ? 1 << 30 : 0) | (a1 ? int(1u << 31) : 0);
  };
  St st;
  PosStager ps;
  auto fetch = [&](int ent) {
    const int kbase = (ent & 0x3fffffff) * kBlock;
    st.template load<DENSE ? kRowsDense : kRowsStrided>(Kb, p.lk.sn, Vb, p.lv.sn, kbase, NK, hd, t);
    ps.load(kidx, kbase, NK, INT32_MAX, t);
  };
  auto put = [&](int b) {
    st.store(sm.K[b], sm.V[b], t);
    ps.store(sm.kid[b], t);
  };
  int cur = advance(), nxt = -1;
  if (cur != -1) {
    fetch(cur);
    put(0);
    nxt = advance();
    if (nxt != -1) fetch(nxt);
  }
  __syncthreads();
  int e[2] = {lb[0], lb[1]};  // list positions of the blocks' current tiles (their mask slots)
  // One straight-line body for every tile: both blocks' halves always run.
  // A tile outside block h's list (or skipped by its 32-row half) runs h's
  // half with the clip bounds set to -0.0, which makes every weight of it
  // 0: O and the row sums gain exact zeros (finite V), no mask is written
  // for a tile not in the list, and an in-list tile skipped by its half
  // writes the all-zero mask.  Branching per case instead made the
  // compiler move the accumulators between register sets on every tile
  // (66 register copies per tile, a third of the VALU overhead beyond the
  // weights).  The cost is the idle half's products on tiles in only one
  // of the two lists (one tile per pair in a causal pattern).
  for (int i = 0; cur != -1; ++i) {
    const int b = i & 1;
    const int kb = cur & 0x3fffffff;
    const bool in[2] = {(cur & (1 << 30)) != 0, cur < 0};
    const bool whole_keys = kb * kBlock + kBlock <= NK;
    const int kmax = kbnd[kb].y;
    f32x4 acc[2][4];
    rows_x_frag2<D>(acc[0], acc[1], sm.K[b], qf[0], qf[1], lane, f32x4{x0[0], x0[0], x0[0], x0[0]},
                    f32x4{x0[1], x0[1], x0[1], x0[1]});
    for (int h = 0; h < 2; ++h) {
      bool act = in[h];  // wave-uniform
      if constexpr (HALF) act = act && hvalid[h] && hrow[h][kb] != 0;
      const float l = act ? lo[h] : -0.0f, u = act ? hi[h] : -0.0f;  // med3(x, -0, -0) = -0: no weight
      // forward_kernel's weights, over c: v' = max(u, 0) / c, then keys past
      // the row's position set to -0.0 on tiles not wholly visible
      for (int f = 0; f < 4; ++f)
        for (int r = 0; r < 4; ++r) acc[h][f][r] = __builtin_amdgcn_fmed3f(acc[h][f][r], l, u);
      if (act && !(whole_keys && kmax <= qmin[h]))
        for (int f = 0; f < 4; ++f)
          for (int r = 0; r < 4; ++r)
            acc[h][f][r] = sm.kid[b][16 * f + 4 * g + r] <= qpos[h] ? acc[h][f][r] : -0.0f;
      if constexpr (EMIT) {
        uint32_t nm = 0;  // bit 4f + r <- u <= 0, highest bit first
        for (int f = 3; f >= 0; --f)
          for (int r = 3; r >= 0; --r) nm = __builtin_amdgcn_alignbit(nm, __float_as_uint(acc[h][f][r]), 31);
        if (in[h]) smask[size_t(e[h]) * 256] = uint16_t(~nm);
      }
      for (int f = 0; f < 4; ++f)
        for (int r = 0; r < 4; ++r) {
          const float pv = pow_clipped<PC>(acc[h][f][r], a);
          if constexpr (std::is_same<T, h16>::value) acc[h][f][r] = pv * pscale[h];
          else acc[h][f][r] = pv;
          rowsum[h] += pv;
        }
    }
    tile_t_x_acc2<D>(o[0], o[1], sm.V[b], acc[0], acc[1], lane);
    for (int h = 0; h < 2; ++h) e[h] += in[h] ? 1 : 0;
    cur = nxt;
    if (cur != -1) {
      put(b ^ 1);
      nxt = advance();
      if (nxt != -1) fetch(nxt);
    }
    __syncthreads();
  }

  const float ce = pow_fast<PC>(cs, a);  // p = c^e p'
  for (int h = 0; h < 2; ++h) {
    const float norm = ce * sum_groups(rowsum[h]);
    const float inv = ce / ((norm + kEps) * pscale[h]);  // pscale 0: non-finite weights, output 0
    if (qok[h]) {
      T* orow = row_at<DENSE, D>(static_cast<T*>(p.out), p.lo, bh, H, NQ, int(row[h] - size_t(bh) * NQ));
      for (int db = 0; db < D / 16; ++db)
        if (DENSE || 16 * db + 4 * g < hd)
          for (int r = 0; r < 4; ++r) {
            float v = o[h][db][r] * inv;
            if (!finite(v)) v = 0.0f;
            Elem<T>::store(orow + 16 * db + 4 * g + r, v);
          }
      if (g == 0) p.norms[row[h]] = norm;
    }
  }
}

template <typename T, int D, bool EMIT, bool HALF, bool DENSE>
hipError_t launch_pair_rows(const ForwardParams& p, hipStream_t s) {
  dim3 grid(((p.d.nQB + 1) / 2) * p.d.BH);
  switch (alpha_class_of(p.d.alpha)) {
    case kA15: hipLaunchKernelGGL((forward_pair_kernel<T, D, kE2, EMIT, HALF, DENSE>), grid, dim3(kThreads), 0, s, p); break;
    case kA20: hipLaunchKernelGGL((forward_pair_kernel<T, D, kE1, EMIT, HALF, DENSE>), grid, dim3(kThreads), 0, s, p); break;
    case kA125: hipLaunchKernelGGL((forward_pair_kernel<T, D, kE4, EMIT, HALF, DENSE>), grid, dim3(kThreads), 0, s, p); break;
    default: return hipErrorInvalidValue;  // excluded by pair_fold_ok
  }
  return hipGetLastError();
}
// Q, K, V and Out contiguous [B, H, N, D] (hd = D).
inline bool fwd_dense(const ForwardParams& p) {
  const int H = p.d.H, D = p.d.D;
  return p.d.hd == D && lay_dense(p.lq, H, p.d.NQ, D) && lay_dense(p.lk, H, p.d.NK, D) &&
         lay_dense(p.lv, H, p.d.NK, D) && lay_dense(p.lo, H, p.d.NQ, D);
}

template <typename T, int D, bool EMIT, bool HALF>
hipError_t launch_pair(const ForwardParams& p, hipStream_t s) {
  if (fwd_dense(p)) return launch_pair_rows<T, D, EMIT, HALF, true>(p, s);
  return launch_pair_rows<T, D, EMIT, HALF, false>(p, s);
}

// forward_pair_kernel's folded clip applies: an integer power class (the
// general power keeps an EPS floor on u) and c = (alpha - 1) scale in
// [2^-8, 2^8], so that p / c^e is within 2^32 of p either way.
inline bool pair_fold_ok(const ForwardParams& p) {
  const float c = (p.d.alpha - 1.0f) * p.d.scale;
  return alpha_class_of(p.d.alpha) != kAGen && c >= 0x1p-8f && c <= 0x1p8f;
}

// The paired kernel pays where its workgroups fill the GPU: it runs half as
// many as the one-block kernel, and with fewer pairs than one wave of
// resident ones (three per compute unit at d = 64, two at 128) the
// one-block kernel's twice as many workgroups finish first (measured,
// bf16 fwd: 2x8x4096x64, 512 pairs: 107 against 87 us; 1x1x32768x64: 620
// against 352 us; 1024 pairs: 112 against 134 us).
inline bool pair_pays(const ForwardParams& p) {
  if (p.pairing != 0) return p.pairing == 1;
  const size_t pairs = size_t((p.d.nQB + 1) / 2) * size_t(p.d.BH);
  return pairs >= size_t(p.cus > 0 ? p.cus : 1) * (p.d.D == 64 ? 3 : 2);
}

template <typename T, int D, bool EMIT, bool HALF>
hipError_t launch_tde(const ForwardParams& p, hipStream_t s) {
  if constexpr (is_half<T>)
    if (pair_fold_ok(p) && pair_pays(p)) return launch_pair<T, D, EMIT, HALF>(p, s);
  dim3 grid(p.d.nQB * p.d.BH);
  switch (alpha_class_of(p.d.alpha)) {
    case kA15: hipLaunchKernelGGL((forward_kernel<T, D, kE2, EMIT, HALF>), grid, dim3(kThreads), 0, s, p); break;
    case kA20: hipLaunchKernelGGL((forward_kernel<T, D, kE1, EMIT, HALF>), grid, dim3(kThreads), 0, s, p); break;
    case kA125: hipLaunchKernelGGL((forward_kernel<T, D, kE4, EMIT, HALF>), grid, dim3(kThreads), 0, s, p); break;
    default: hipLaunchKernelGGL((forward_kernel<T, D, kEGen, EMIT, HALF>), grid, dim3(kThreads), 0, s, p); break;
  }
  return hipGetLastError();
}
template <typename T, int D>
hipError_t launch_td(const ForwardParams& p, hipStream_t s) {
  // 32-row mask blocks: the per-half tile test is compiled in only there
  if (p.half)
    return p.sup.mask ? launch_tde<T, D, true, true>(p, s) : launch_tde<T, D, false, true>(p, s);
  return p.sup.mask ? launch_tde<T, D, true, false>(p, s) : launch_tde<T, D, false, false>(p, s);
}

}  // namespace

hipError_t launch_forward(const ForwardParams& p, int dtype, hipStream_t s) {
  if (dtype == kElemBF16) {
    if (p.d.D == 64) return launch_td<u16, 64>(p, s);
    if (p.d.D == 128) return launch_td<u16, 128>(p, s);
  } else if (dtype == kElemF16) {
    if (p.d.D == 64) return launch_td<h16, 64>(p, s);
    if (p.d.D == 128) return launch_td<h16, 128>(p, s);
  } else {
    if (p.d.D == 64) return launch_td<float, 64>(p, s);
    if (p.d.D == 128) return launch_td<float, 128>(p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace asa
