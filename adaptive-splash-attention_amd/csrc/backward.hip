// Backward: dQ, dK, dV without atomics.
//
// Reference: splash_backward_sparse (adasplashattention.cu:343-535), one
// thread per query, dQ in registers, dK and dV by fp32 atomicAdd.  Here:
//
//   delta kernel   (reference-gradient mode only) per row:
//                  shift = out . dO, c = 1 / (sum p + EPS).
//   dQ kernel      query-major, one 256-thread block per query block,
//                  walking the query-major CSR list.  Per key block: S^T =
//                  K Q^T and dP^T = V dO^T on MFMA, weights w = u^((2-a)/(a-1))
//                  (= p^(2-alpha)) in registers, and the dQ^T products on
//                  MFMA.  Entmax mode keeps two accumulators,
//                  A = K^T (w dp) and B = K^T w, with row sums sum(w) and
//                  sum(w dp), and finishes dQ = scale c (A - shift B) with
//                  shift = sum(w dp)/sum(w) and c = (sum p + EPS)^(alpha-2),
//                  so that one sweep suffices; it stores shift and c for
//                  the dK/dV kernel.
//   dK/dV kernel   key-major, one block per key block, walking the key-major
//                  CSR list; each key block's gradients are reduced in
//                  registers of the block that owns it, so the result is
//                  deterministic.  Per query block: S = Q K^T and dP = dO V^T
//                  on MFMA, P = p / (sum p + EPS), ds = c w (dp - shift),
//                  dV^T += dO^T P and dK^T += Q^T ds on MFMA.
//
// bf16 inputs: the per-score operands of the dQ products (w dp, w) enter
// the MFMA as hi + lo bf16 pairs.  A row's ds sums to zero, so with keys
// that share a common component the dQ sum cancels heavily; a single bf16
// rounding of its operands would leave an error relative to
// sum |ds| |k| rather than to the (much smaller) result (measured: 3.7e-2
// relative on clustered keys with alpha = 2, against 2.5e-3 with the
// split).  The dK sum runs over queries, whose ds do not sum to zero; its
// single-rounding error measured the same as the split's (<= 3.1e-3), so
// ds enters the dK product once.
//
// In both modes ds = c * w * (dp - shift); the modes differ in (c, shift):
//   entmax (ASA_GRAD_ENTMAX):     c = (sum p + EPS)^(alpha-2),
//                                 shift = sum(w dp) / sum(w)
//   reference (ASA_GRAD_REFERENCE): c = 1 / (sum p + EPS), shift = out . dO,
//                                 and w = 0 unless u > EPS (:494).
#include <type_traits>

#include "asa_device.hpp"
#include "asa_launch.hpp"
#include "asa_stage.hpp"
#include "asa_tiles.hpp"

namespace asa {
namespace {

constexpr int kThreads = 256;

// ---------------------------------------------------------------------------
// Row constants for the reference-gradient mode.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(kThreads) void delta_kernel(BackwardParams p) {
  const size_t rows = size_t(p.d.BH) * p.d.NQ;
  const size_t r = size_t(blockIdx.x) * kThreads + threadIdx.x;
  if (r >= rows) return;
  const int bh = int(r / p.d.NQ), n = int(r % p.d.NQ);
  const T* o = static_cast<const T*>(p.out) + head_at(p.lo, bh, p.d.H) + size_t(n) * p.lo.sn;
  const T* go = static_cast<const T*>(p.dout) + head_at(p.ldo, bh, p.d.H) + size_t(n) * p.ldo.sn;
  float acc = 0.0f;
  for (int t = 0; t < p.d.hd; ++t) acc += Elem<T>::load(o + t) * Elem<T>::load(go + t);
  float* shift = p.delta;
  float* cfac = p.delta + rows;
  shift[r] = acc;
  cfac[r] = 1.0f / (p.norms[r] + kEps);
}

// ---------------------------------------------------------------------------
// dQ (query-major)
// ---------------------------------------------------------------------------
template <typename T, int D> struct alignas(16) DqSmem {
  T K[2][kBlock * Tile<T, D>::kRs];
  T V[2][kBlock * Tile<T, D>::kRs];
  int kid[2][kBlock];
  int full[2];
};

// Three waves per SIMD for bf16 at d = 64 (dQ and dK/dV): the third wave
// hides part of the LDS and MFMA latency.
template <typename T, int D>
constexpr int dq_waves_per_simd() { return sizeof(T) == 2 && D == 64 ? 3 : 1; }

template <typename T, int D, int AC, bool REF>
__global__ __launch_bounds__(kThreads, (dq_waves_per_simd<T, D>())) void dq_kernel(BackwardParams p) {
  constexpr bool kOpScaled = std::is_same<T, h16>::value;  // see the weights below
  __shared__ DqSmem<T, D> sm;
  using St = Stager<T, D>;
  constexpr int PW = AlphaPow<AC>::W;
  const int NQ = p.d.NQ, NK = p.d.NK, nQB = p.d.nQB, nKB = p.d.nKB;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int g = lane >> 4, c16 = lane & 15;
  int brank, bh;
  xcd_rank_order(blockIdx.x, nQB, p.d.BH, brank, bh);
  const int qb = nQB - 1 - brank;  // heaviest first
  const int q = qb * kBlock + 16 * w + c16;
  const bool qok = q < NQ;
  const size_t rows = size_t(p.d.BH) * NQ;
  const size_t row = size_t(bh) * NQ + (qok ? q : 0);
  const int H = p.d.H, hd = p.d.hd;

  const T* Kb = static_cast<const T*>(p.k) + head_at(p.lk, bh, H);
  const T* Vb = static_cast<const T*>(p.v) + head_at(p.lv, bh, H);
  const int32_t* kidx = p.k_idx + size_t(bh) * NK;

  RowFrag<T, D> qf, df;
  qf.load(static_cast<const T*>(p.q) + head_at(p.lq, bh, H) + size_t(qok ? q : 0) * p.lq.sn, qok, lane, hd);
  df.load(static_cast<const T*>(p.dout) + head_at(p.ldo, bh, H) + size_t(qok ? q : 0) * p.ldo.sn, qok, lane,
          hd);
  const int qpos = qok ? p.q_idx[row] : 0;
  const float alpha = p.d.alpha;
  const float am1 = alpha - 1.0f;
  const float ew = (2.0f - alpha) / am1;
  const ClippedU clip(am1, p.d.scale, qok ? p.taus[row] : 0.0f, qok);  // invalid rows: w = 0
  const float norm = qok ? p.norms[row] : 0.0f;
  float cfac, shift;
  if constexpr (REF) {
    cfac = qok ? p.delta[rows + row] : 0.0f;
    shift = qok ? p.delta[row] : 0.0f;
  } else {
    cfac = static_cast<float>(pow(static_cast<double>(norm + kEps), static_cast<double>(alpha) - 2.0));
    shift = 0.0f;
  }
  const float scale = p.d.scale;
  int qmin = 0;
  if (w == 0) {
    const int qq = qb * kBlock + lane;
    qmin = wave_reduce_minmax<false>(qq < NQ ? p.q_idx[size_t(bh) * NQ + qq] : INT32_MAX);
  }

  f32x4 a1[D / 16], a2[D / 16];
  for (int db = 0; db < D / 16; ++db) a1[db] = a2[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float sw = 0.0f, swdp = 0.0f;
  // 32-row mask blocks: the mask row of this wave's half; a tile that row
  // lacks contributes nothing to the wave
  const uint8_t* hrow = nullptr;
  bool hvalid = true;
  if (p.half) {
    const int h = 2 * qb + (w >> 1), nQH = half_blocks(NQ);
    hvalid = h < nQH;
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
    ps.store<true>(sm.kid[b], &sm.full[b], qmin, t);
  };
  if (e0 < e1) {
    fetch(e0);
    put(0);
    if (e0 + 1 < e1) fetch(e0 + 1);
  }
  __syncthreads();
  for (int e = e0; e < e1; ++e) {
    const int b = (e - e0) & 1;
    const bool act = !hrow || (hvalid && hrow[ql[e]] != 0);  // wave-uniform
    f32x4 sacc[4], dacc[4];
    auto weights = [&](auto partial) {
      for (int f = 0; f < 4; ++f)
        for (int r = 0; r < 4; ++r) {
          const float v = clip(sacc[f][r]);  // max(u, 0)
          float wv = pow_clipped<PW>(v, ew);
          if constexpr (REF) wv = v > kEps ? wv : 0.0f;  // the reference's u > EPS
          if constexpr (decltype(partial)::value)
            wv = sm.kid[b][16 * f + 4 * g + r] <= qpos ? wv : 0.0f;
          const float dp = dacc[f][r];
          if constexpr (REF) {
            const float ds = cfac * wv * (dp - shift);
            sacc[f][r] = finite(ds) ? ds : 0.0f;
          } else {
            sw += wv;
            swdp += wv * dp;
            // fp16 operands carry c w (c = (sum p + EPS)^(alpha-2) <= 1 per
            // unit of w's scale): w alone can exceed fp16's range
            const float wq = kOpScaled ? wv * cfac : wv;
            sacc[f][r] = wq * dp;
            dacc[f][r] = wq;
          }
        }
    };
    if (act) {
      rows_x_frag<D>(sacc, sm.K[b], qf, lane);
      rows_x_frag<D>(dacc, sm.V[b], df, lane);
      if (sm.full[b] != 0) weights(std::false_type{});
      else weights(std::true_type{});
      tile_t_x_acc<D, true>(a1, sm.K[b], sacc, lane);
      if constexpr (!REF) tile_t_x_acc<D, true>(a2, sm.K[b], dacc, lane);
    }
    if (e + 1 < e1) {
      put(b ^ 1);
      if (e + 2 < e1) fetch(e + 2);
    }
    __syncthreads();
  }

  if constexpr (!REF) {
    sw = sum_groups(sw);
    swdp = sum_groups(swdp);
    shift = sw > 0.0f ? swdp / sw : 0.0f;
    if (!finite(shift)) shift = 0.0f;
    if (qok && g == 0) {
      p.delta[row] = shift;
      p.delta[rows + row] = cfac;
    }
  }
  if (qok) {
    T* out = static_cast<T*>(p.dq) + head_at(p.ldq, bh, H) + size_t(q) * p.ldq.sn;
    const float cs = (REF || kOpScaled) ? scale : scale * cfac;
    for (int db = 0; db < D / 16; ++db)
      if (16 * db + 4 * g < hd)
        for (int r = 0; r < 4; ++r) {
          const float acc = REF ? a1[db][r] : (a1[db][r] - shift * a2[db][r]);
          float v = cs * acc;
          if (!finite(v)) v = 0.0f;
          Elem<T>::store(out + 16 * db + 4 * g + r, v);
        }
  }
}

// ---------------------------------------------------------------------------
// dK, dV (key-major)
// ---------------------------------------------------------------------------
template <typename T, int D> struct alignas(16) DkvSmem {
  T Q[2][kBlock * Tile<T, D>::kRs];
  T dO[2][kBlock * Tile<T, D>::kRs];
};

// Per-query constants of a query tile: the ClippedU terms -tau, lo, hi;
// 1/(sum p + EPS); the gradient factor c and -c * shift, so that
// c (dp - shift) is one fma.
struct alignas(16) QConst {
  float nt[kBlock], lo[kBlock], hi[kBlock], invn[kBlock], c[kBlock], cs[kBlock];
  int pos[kBlock];
};
struct QConstStager {
  float nt, lo, hi, invn, c, cs;
  // Row qbase + t of head bh against key block kb: rows past NQ, and with
  // 32-row mask blocks rows whose half's mask row lacks kb, get p = w = 0.
  __device__ __forceinline__ void load(const BackwardParams& p, size_t rows, int bh, int qbase,
                                       int kb, int NQ, float am1, int t) {
    if (t < kWave) {
      const size_t rbase = size_t(bh) * NQ;
      bool ok = qbase + t < NQ;
      if (p.half && ok)
        ok = p.half[(size_t(bh) * half_blocks(NQ) + (qbase + t) / 32) * p.d.nKB + kb] != 0;
      const size_t r = rbase + (ok ? qbase + t : 0);
      const ClippedU u(am1, p.d.scale, ok ? p.taus[r] : 0.0f, ok);  // invalid rows: p = w = 0
      nt = u.nt;
      lo = u.lo;
      hi = u.hi;
      invn = ok ? 1.0f / (p.norms[r] + kEps) : 0.0f;
      c = ok ? p.delta[rows + r] : 0.0f;
      cs = ok ? -c * p.delta[r] : 0.0f;
    }
  }
  __device__ __forceinline__ void store(QConst& qc, int t) const {
    if (t < kWave) {
      qc.nt[t] = nt;
      qc.lo[t] = lo;
      qc.hi[t] = hi;
      qc.invn[t] = invn;
      qc.c[t] = c;
      qc.cs[t] = cs;
    }
  }
};

template <typename T, int D, int AC, bool REF>
__global__ __launch_bounds__(kThreads, (dq_waves_per_simd<T, D>())) void dkdv_kernel(BackwardParams p) {
  __shared__ DkvSmem<T, D> sm;
  __shared__ QConst qcs[2];
  __shared__ int full[2];
  using St = Stager<T, D>;
  constexpr int PP = AlphaPow<AC>::P, PW = AlphaPow<AC>::W;
  const int NQ = p.d.NQ, NK = p.d.NK, nQB = p.d.nQB, nKB = p.d.nKB;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int g = lane >> 4, c16 = lane & 15;
  int kb, bh;
  xcd_rank_order(blockIdx.x, nKB, p.d.BH, kb, bh);  // ascending key blocks: heaviest first
  const int j = kb * kBlock + 16 * w + c16;  // this lane's key row
  const bool jok = j < NK;
  const size_t krow = size_t(bh) * NK + (jok ? j : 0);
  const size_t rows = size_t(p.d.BH) * NQ;
  const int H = p.d.H, hd = p.d.hd;

  const T* Qb = static_cast<const T*>(p.q) + head_at(p.lq, bh, H);
  const T* dOb = static_cast<const T*>(p.dout) + head_at(p.ldo, bh, H);
  const int32_t* qidx = p.q_idx + size_t(bh) * NQ;

  RowFrag<T, D> kf, vf;
  kf.load(static_cast<const T*>(p.k) + head_at(p.lk, bh, H) + size_t(jok ? j : 0) * p.lk.sn, jok, lane, hd);
  vf.load(static_cast<const T*>(p.v) + head_at(p.lv, bh, H) + size_t(jok ? j : 0) * p.lv.sn, jok, lane, hd);
  const int kpos = jok ? p.k_idx[krow] : 0;
  const float alpha = p.d.alpha;
  const float am1 = alpha - 1.0f;
  const float a = 1.0f / am1;
  const float ew = (2.0f - alpha) / am1;
  const float scale = p.d.scale;
  const float cu = am1 * scale;  // ClippedU's c (uniform)
  // largest position of the block's valid keys (wave 0 tests tiles with it)
  int kmax = 0;
  if (w == 0) {
    const int kk = kb * kBlock + lane;
    kmax = wave_reduce_minmax<true>(kk < NK ? p.k_idx[size_t(bh) * NK + kk] : INT32_MIN);
  }

  f32x4 ak[D / 16], av[D / 16];
  for (int db = 0; db < D / 16; ++db) ak[db] = av[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int32_t* kp = p.k_ptr + size_t(bh) * (nKB + 1);
  const int32_t* kl = p.k_list + size_t(bh) * nKB * nQB;
  const int e0 = kp[kb], e1 = kp[kb + 1];
  St st;
  PosStager ps;
  QConstStager qs;
  auto fetch = [&](int e) {
    const int qbase = kl[e] * kBlock;
    st.template load<kRowsStrided>(Qb, p.lq.sn, dOb, p.ldo.sn, qbase, NQ, hd, t);
    ps.load(qidx, qbase, NQ, INT32_MAX, t);
    qs.load(p, rows, bh, qbase, kb, NQ, am1, t);
  };
  auto put = [&](int b) {
    st.store(sm.Q[b], sm.dO[b], t);
    ps.store<false>(qcs[b].pos, &full[b], kmax, t);
    qs.store(qcs[b], t);
  };
  if (e0 < e1) {
    fetch(e0);
    put(0);
    if (e0 + 1 < e1) fetch(e0 + 1);
  }
  __syncthreads();
  for (int e = e0; e < e1; ++e) {
    const int b = (e - e0) & 1;
    const QConst& qc = qcs[b];
    f32x4 sacc[4], dacc[4];
    auto grads = [&](auto partial, int fb) {
      for (int f = fb; f < fb + 2; ++f) {
        // constants of queries 16f + 4g + 0..3
        const int q4 = 16 * f + 4 * g;
        const f32x4 nt4 = *reinterpret_cast<const f32x4*>(&qc.nt[q4]);
        const f32x4 lo4 = *reinterpret_cast<const f32x4*>(&qc.lo[q4]);
        const f32x4 hi4 = *reinterpret_cast<const f32x4*>(&qc.hi[q4]);
        const f32x4 invn4 = *reinterpret_cast<const f32x4*>(&qc.invn[q4]);
        const f32x4 c4 = *reinterpret_cast<const f32x4*>(&qc.c[q4]);
        const f32x4 cs4 = *reinterpret_cast<const f32x4*>(&qc.cs[q4]);
        for (int r = 0; r < 4; ++r) {
          // max(u, 0) of ClippedU with the query's terms
          const float v = __builtin_amdgcn_fmed3f(fmaf(cu, sacc[f][r], nt4[r]), lo4[r], hi4[r]);
          float pn = pow_clipped<PP>(v, a) * invn4[r];
          float wv = pow_clipped<PW>(v, ew);
          if constexpr (REF) wv = v > kEps ? wv : 0.0f;  // the reference's u > EPS
          float ds = wv * fmaf(c4[r], dacc[f][r], cs4[r]);
          ds = finite(ds) ? ds : 0.0f;
          if constexpr (decltype(partial)::value) {
            const bool vis = kpos <= qc.pos[q4 + r];
            pn = vis ? pn : 0.0f;
            ds = vis ? ds : 0.0f;
          }
          sacc[f][r] = ds;
          dacc[f][r] = pn;
        }
      }
    };
    const bool tile_full = full[b] != 0;
    // two halves (score rows 16f.., f = 0,1 then 2,3): each half's scores,
    // P and ds are formed and fed to their products before the next half
    // is started, which keeps the register footprint within three waves
    // per SIMD
    rows_x_frag<D, 0, 2>(sacc, sm.Q[b], kf, lane);
    rows_x_frag<D, 0, 2>(dacc, sm.dO[b], vf, lane);
    if (tile_full) grads(std::false_type{}, 0);
    else grads(std::true_type{}, 0);
    tile_t_x_acc<D, false, 0, 1>(av, sm.dO[b], dacc, lane);
    tile_t_x_acc<D, false, 0, 1>(ak, sm.Q[b], sacc, lane);
    rows_x_frag<D, 2, 4>(sacc, sm.Q[b], kf, lane);
    rows_x_frag<D, 2, 4>(dacc, sm.dO[b], vf, lane);
    if (tile_full) grads(std::false_type{}, 2);
    else grads(std::true_type{}, 2);
    tile_t_x_acc<D, false, 1, 2>(av, sm.dO[b], dacc, lane);
    tile_t_x_acc<D, false, 1, 2>(ak, sm.Q[b], sacc, lane);
    if (e + 1 < e1) {
      put(b ^ 1);
      if (e + 2 < e1) fetch(e + 2);
    }
    __syncthreads();
  }

  if (jok) {
    T* dk = static_cast<T*>(p.dk) + head_at(p.ldk, bh, H) + size_t(j) * p.ldk.sn;
    T* dv = static_cast<T*>(p.dv) + head_at(p.ldv, bh, H) + size_t(j) * p.ldv.sn;
    for (int db = 0; db < D / 16; ++db)
      if (16 * db + 4 * g < hd)
        for (int r = 0; r < 4; ++r) {
          // NaN -> 0; an overflowed sum stays +-inf (reference atomics, cu:684-697)
          float vk = scale * ak[db][r], vv = av[db][r];
          if (__builtin_isnan(vk)) vk = 0.0f;
          if (__builtin_isnan(vv)) vv = 0.0f;
          Elem<T>::store(dk + 16 * db + 4 * g + r, vk);
          Elem<T>::store(dv + 16 * db + 4 * g + r, vv);
        }
  }
}

template <typename T, int D, bool REF>
hipError_t launch_dq_m(const BackwardParams& p, hipStream_t s) {
  dim3 grid(p.d.nQB * p.d.BH);
  switch (alpha_class_of(p.d.alpha)) {
    case kA15: hipLaunchKernelGGL((dq_kernel<T, D, kA15, REF>), grid, dim3(kThreads), 0, s, p); break;
    case kA20: hipLaunchKernelGGL((dq_kernel<T, D, kA20, REF>), grid, dim3(kThreads), 0, s, p); break;
    case kA125: hipLaunchKernelGGL((dq_kernel<T, D, kA125, REF>), grid, dim3(kThreads), 0, s, p); break;
    default: hipLaunchKernelGGL((dq_kernel<T, D, kAGen, REF>), grid, dim3(kThreads), 0, s, p); break;
  }
  return hipGetLastError();
}
template <typename T, int D>
hipError_t launch_dq_td(const BackwardParams& p, hipStream_t s) {
  return p.mode == 1 ? launch_dq_m<T, D, true>(p, s) : launch_dq_m<T, D, false>(p, s);
}

template <typename T, int D, bool REF>
hipError_t launch_dkdv_m(const BackwardParams& p, hipStream_t s) {
  dim3 grid(p.d.nKB * p.d.BH);
  switch (alpha_class_of(p.d.alpha)) {
    case kA15: hipLaunchKernelGGL((dkdv_kernel<T, D, kA15, REF>), grid, dim3(kThreads), 0, s, p); break;
    case kA20: hipLaunchKernelGGL((dkdv_kernel<T, D, kA20, REF>), grid, dim3(kThreads), 0, s, p); break;
    case kA125: hipLaunchKernelGGL((dkdv_kernel<T, D, kA125, REF>), grid, dim3(kThreads), 0, s, p); break;
    default: hipLaunchKernelGGL((dkdv_kernel<T, D, kAGen, REF>), grid, dim3(kThreads), 0, s, p); break;
  }
  return hipGetLastError();
}
template <typename T, int D>
hipError_t launch_dkdv_td(const BackwardParams& p, hipStream_t s) {
  return p.mode == 1 ? launch_dkdv_m<T, D, true>(p, s) : launch_dkdv_m<T, D, false>(p, s);
}

template <typename T, int D>
hipError_t launch_delta_td(const BackwardParams& p, hipStream_t s) {
  const size_t rows = size_t(p.d.BH) * p.d.NQ;
  const unsigned blocks = unsigned((rows + kThreads - 1) / kThreads);
  hipLaunchKernelGGL((delta_kernel<T, D>), dim3(blocks), dim3(kThreads), 0, s, p);
  return hipGetLastError();
}

}  // namespace

#define ASA_DISPATCH_TD(fn)                                \
  if (dtype == kElemBF16) {                                \
    if (p.d.D == 64) return fn<u16, 64>(p, s);             \
    if (p.d.D == 128) return fn<u16, 128>(p, s);           \
  } else if (dtype == kElemF16) {                          \
    if (p.d.D == 64) return fn<h16, 64>(p, s);             \
    if (p.d.D == 128) return fn<h16, 128>(p, s);           \
  } else {                                                 \
    if (p.d.D == 64) return fn<float, 64>(p, s);           \
    if (p.d.D == 128) return fn<float, 128>(p, s);         \
  }                                                        \
  return hipErrorInvalidValue;

hipError_t launch_bwd_delta(const BackwardParams& p, int dtype, hipStream_t s) { ASA_DISPATCH_TD(launch_delta_td) }
hipError_t launch_bwd_dq(const BackwardParams& p, int dtype, hipStream_t s) { ASA_DISPATCH_TD(launch_dq_td) }
hipError_t launch_bwd_dkdv(const BackwardParams& p, int dtype, hipStream_t s) { ASA_DISPATCH_TD(launch_dkdv_td) }

#undef ASA_DISPATCH_TD

}  // namespace asa
