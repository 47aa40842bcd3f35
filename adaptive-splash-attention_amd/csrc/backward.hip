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
// bf16 inputs: the per-score operands of the dQ and dK products (w dp, w,
// ds) enter the MFMA as hi + lo bf16 pairs.  A row's ds sums to zero, so
// with keys (or queries) that share a common component the products cancel
// heavily; a single bf16 rounding of ds would leave an error relative to
// sum |ds| |k| rather than to the (much smaller) result.
//
// In both modes ds = c * w * (dp - shift); the modes differ in (c, shift):
//   entmax (ASA_GRAD_ENTMAX):     c = (sum p + EPS)^(alpha-2),
//                                 shift = sum(w dp) / sum(w)
//   reference (ASA_GRAD_REFERENCE): c = 1 / (sum p + EPS), shift = out . dO,
//                                 and w = 0 unless u > EPS (:494).
#include "asa_device.hpp"
#include "asa_launch.hpp"
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
  const T* o = static_cast<const T*>(p.out) + r * D;
  const T* go = static_cast<const T*>(p.dout) + r * D;
  float acc = 0.0f;
  for (int t = 0; t < D; ++t) acc += Elem<T>::load(o + t) * Elem<T>::load(go + t);
  float* shift = p.delta;
  float* cfac = p.delta + rows;
  shift[r] = acc;
  cfac[r] = 1.0f / (p.norms[r] + kEps);
}

// ---------------------------------------------------------------------------
// dQ (query-major)
// ---------------------------------------------------------------------------
template <typename T, int D> struct DqSmem;
template <int D> struct alignas(16) DqSmem<u16, D> {
  u16 K[kBlock * Tile<u16, D>::kRs];
  u16 Kt[D * Tile<u16, D>::kTs];
  u16 V[kBlock * Tile<u16, D>::kRs];
  int kid[kBlock];
  __device__ const u16* k_operand() const { return Kt; }
  __device__ u16* k_transposed() { return Kt; }
};
template <int D> struct alignas(16) DqSmem<float, D> {
  float K[kBlock * Tile<float, D>::kRs];
  float V[kBlock * Tile<float, D>::kRs];
  int kid[kBlock];
  __device__ const float* k_operand() const { return K; }
  __device__ float* k_transposed() { return nullptr; }
};

template <typename T, int D, int AC>
__global__ __launch_bounds__(kThreads) void dq_kernel(BackwardParams p) {
  __shared__ DqSmem<T, D> sm;
  constexpr int PP = AlphaPow<AC>::P, PW = AlphaPow<AC>::W;
  (void)PP;
  const bool ref = p.mode == 1;
  const int NQ = p.d.NQ, NK = p.d.NK, nQB = p.d.nQB, nKB = p.d.nKB;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int task = xcd_task(blockIdx.x, nQB * p.d.BH);
  const int qb = task % nQB, bh = task / nQB;
  const int q = qb * kBlock + 16 * w + c16;
  const bool qok = q < NQ;
  const size_t rows = size_t(p.d.BH) * NQ;
  const size_t row = size_t(bh) * NQ + (qok ? q : 0);

  const T* Kb = static_cast<const T*>(p.k) + size_t(bh) * NK * D;
  const T* Vb = static_cast<const T*>(p.v) + size_t(bh) * NK * D;
  const int32_t* kidx = p.k_idx + size_t(bh) * NK;

  RowFrag<T, D> qf, df;
  qf.load(static_cast<const T*>(p.q) + row * D, qok, lane);
  df.load(static_cast<const T*>(p.dout) + row * D, qok, lane);
  const int qpos = qok ? p.q_idx[row] : 0;
  const float tau = qok ? p.taus[row] : 0.0f;
  const float alpha = p.d.alpha;
  const float am1 = alpha - 1.0f;
  const float ew = (2.0f - alpha) / am1;
  const float thr = ref ? kEps : 0.0f;
  const float norm = qok ? p.norms[row] : 0.0f;
  float cfac, shift;
  if (ref) {
    cfac = qok ? p.delta[rows + row] : 0.0f;
    shift = qok ? p.delta[row] : 0.0f;
  } else {
    cfac = static_cast<float>(pow(static_cast<double>(norm + kEps), static_cast<double>(alpha) - 2.0));
    shift = 0.0f;
  }
  const float scale = p.d.scale;

  f32x4 a1[D / 16], a2[D / 16];
  for (int db = 0; db < D / 16; ++db) a1[db] = a2[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float sw = 0.0f, swdp = 0.0f;

  const int32_t* qp = p.q_ptr + size_t(bh) * (nQB + 1);
  const int32_t* ql = p.q_list + size_t(bh) * nQB * nKB;
  const int e0 = qp[qb], e1 = qp[qb + 1];
  for (int e = e0; e < e1; ++e) {
    const int kbase = ql[e] * kBlock;
    __syncthreads();
    stage_tile<D>(sm.K, sm.k_transposed(), Kb, kbase, NK, t, kThreads);
    stage_tile<D>(sm.V, static_cast<T*>(nullptr), Vb, kbase, NK, t, kThreads);
    if (t < kBlock) sm.kid[t] = (kbase + t < NK) ? kidx[kbase + t] : 0;
    __syncthreads();

    f32x4 sacc[4], dacc[4];
    rows_x_frag<D>(sacc, sm.K, qf, lane);
    rows_x_frag<D>(dacc, sm.V, df, lane);
    for (int f = 0; f < 4; ++f)
      for (int r = 0; r < 4; ++r) {
        const int kl = 16 * f + 4 * g + r;
        const bool vis = qok && (kbase + kl) < NK && sm.kid[kl] <= qpos;
        float wv = 0.0f;
        if (vis) {
          const float u = am1 * clamp_score(sacc[f][r] * scale) - tau;
          if (u > thr) {
            wv = pow_fast<PW>(fmaxf(u, kEps), ew);
            if (!finite(wv)) wv = 0.0f;
          }
        }
        const float dp = dacc[f][r];
        if (ref) {
          float ds = cfac * wv * (dp - shift);
          if (!finite(ds)) ds = 0.0f;
          sacc[f][r] = ds;
        } else {
          sw += wv;
          swdp += wv * dp;
          sacc[f][r] = wv * dp;
          dacc[f][r] = wv;
        }
      }
    tile_t_x_acc<D, true>(a1, sm.k_operand(), sacc, lane);
    if (!ref) tile_t_x_acc<D, true>(a2, sm.k_operand(), dacc, lane);
  }

  if (!ref) {
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
    T* out = static_cast<T*>(p.dq) + row * D;
    const float cs = ref ? scale : scale * cfac;
    for (int db = 0; db < D / 16; ++db)
      for (int r = 0; r < 4; ++r) {
        const float acc = ref ? a1[db][r] : (a1[db][r] - shift * a2[db][r]);
        float v = cs * acc;
        if (!finite(v)) v = 0.0f;
        Elem<T>::store(out + 16 * db + 4 * g + r, v);
      }
  }
}

// ---------------------------------------------------------------------------
// dK, dV (key-major)
// ---------------------------------------------------------------------------
template <typename T, int D> struct DkvSmem;
template <int D> struct alignas(16) DkvSmem<u16, D> {
  u16 Q[kBlock * Tile<u16, D>::kRs];
  u16 Qt[D * Tile<u16, D>::kTs];
  u16 dO[kBlock * Tile<u16, D>::kRs];
  u16 dOt[D * Tile<u16, D>::kTs];
  __device__ const u16* q_operand() const { return Qt; }
  __device__ const u16* do_operand() const { return dOt; }
  __device__ u16* q_transposed() { return Qt; }
  __device__ u16* do_transposed() { return dOt; }
};
template <int D> struct alignas(16) DkvSmem<float, D> {
  float Q[kBlock * Tile<float, D>::kRs];
  float dO[kBlock * Tile<float, D>::kRs];
  __device__ const float* q_operand() const { return Q; }
  __device__ const float* do_operand() const { return dO; }
  __device__ float* q_transposed() { return nullptr; }
  __device__ float* do_transposed() { return nullptr; }
};

template <typename T, int D, int AC>
__global__ __launch_bounds__(kThreads) void dkdv_kernel(BackwardParams p) {
  __shared__ DkvSmem<T, D> sm;
  __shared__ float s_tau[kBlock], s_c[kBlock], s_shift[kBlock], s_invn[kBlock];
  __shared__ int s_pos[kBlock], s_ok[kBlock];
  constexpr int PP = AlphaPow<AC>::P, PW = AlphaPow<AC>::W;
  const bool ref = p.mode == 1;
  const int NQ = p.d.NQ, NK = p.d.NK, nQB = p.d.nQB, nKB = p.d.nKB;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int task = xcd_task(blockIdx.x, nKB * p.d.BH);
  const int kb = task % nKB, bh = task / nKB;
  const int j = kb * kBlock + 16 * w + c16;  // this lane's key row
  const bool jok = j < NK;
  const size_t krow = size_t(bh) * NK + (jok ? j : 0);
  const size_t rows = size_t(p.d.BH) * NQ;

  const T* Qb = static_cast<const T*>(p.q) + size_t(bh) * NQ * D;
  const T* dOb = static_cast<const T*>(p.dout) + size_t(bh) * NQ * D;

  RowFrag<T, D> kf, vf;
  kf.load(static_cast<const T*>(p.k) + krow * D, jok, lane);
  vf.load(static_cast<const T*>(p.v) + krow * D, jok, lane);
  const int kpos = jok ? p.k_idx[krow] : 0;
  const float alpha = p.d.alpha;
  const float am1 = alpha - 1.0f;
  const float a = 1.0f / am1;
  const float ew = (2.0f - alpha) / am1;
  const float thr = ref ? kEps : 0.0f;
  const float scale = p.d.scale;

  f32x4 ak[D / 16], av[D / 16];
  for (int db = 0; db < D / 16; ++db) ak[db] = av[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int32_t* kp = p.k_ptr + size_t(bh) * (nKB + 1);
  const int32_t* kl = p.k_list + size_t(bh) * nKB * nQB;
  const int e0 = kp[kb], e1 = kp[kb + 1];
  for (int e = e0; e < e1; ++e) {
    const int qbase = kl[e] * kBlock;
    __syncthreads();
    stage_tile<D>(sm.Q, sm.q_transposed(), Qb, qbase, NQ, t, kThreads);
    stage_tile<D>(sm.dO, sm.do_transposed(), dOb, qbase, NQ, t, kThreads);
    if (t < kBlock) {
      const int qi = qbase + t;
      const bool ok = qi < NQ;
      const size_t r = size_t(bh) * NQ + (ok ? qi : 0);
      s_ok[t] = ok;
      s_pos[t] = ok ? p.q_idx[r] : 0;
      s_tau[t] = ok ? p.taus[r] : 0.0f;
      s_invn[t] = ok ? 1.0f / (p.norms[r] + kEps) : 0.0f;
      s_shift[t] = ok ? p.delta[r] : 0.0f;
      s_c[t] = ok ? p.delta[rows + r] : 0.0f;
    }
    __syncthreads();

    f32x4 sacc[4], dacc[4];
    rows_x_frag<D>(sacc, sm.Q, kf, lane);
    rows_x_frag<D>(dacc, sm.dO, vf, lane);
    for (int f = 0; f < 4; ++f)
      for (int r = 0; r < 4; ++r) {
        const int qi = 16 * f + 4 * g + r;
        const bool vis = jok && s_ok[qi] && kpos <= s_pos[qi];
        float pn = 0.0f, ds = 0.0f;
        if (vis) {
          const float u = am1 * clamp_score(sacc[f][r] * scale) - s_tau[qi];
          if (u > 0.0f) {
            float pv = pow_fast<PP>(fmaxf(u, kEps), a);
            if (!finite(pv)) pv = 0.0f;
            pn = pv * s_invn[qi];
          }
          if (u > thr) {
            float wv = pow_fast<PW>(fmaxf(u, kEps), ew);
            if (!finite(wv)) wv = 0.0f;
            ds = s_c[qi] * wv * (dacc[f][r] - s_shift[qi]);
            if (!finite(ds)) ds = 0.0f;
          }
        }
        sacc[f][r] = ds;
        dacc[f][r] = pn;
      }
    tile_t_x_acc<D>(av, sm.do_operand(), dacc, lane);
    tile_t_x_acc<D, true>(ak, sm.q_operand(), sacc, lane);
  }

  if (jok) {
    T* dk = static_cast<T*>(p.dk) + krow * D;
    T* dv = static_cast<T*>(p.dv) + krow * D;
    for (int db = 0; db < D / 16; ++db)
      for (int r = 0; r < 4; ++r) {
        float vk = scale * ak[db][r], vv = av[db][r];
        if (!finite(vk)) vk = 0.0f;
        if (!finite(vv)) vv = 0.0f;
        Elem<T>::store(dk + 16 * db + 4 * g + r, vk);
        Elem<T>::store(dv + 16 * db + 4 * g + r, vv);
      }
  }
}

template <typename T, int D>
hipError_t launch_dq_td(const BackwardParams& p, hipStream_t s) {
  dim3 grid(p.d.nQB * p.d.BH);
  switch (alpha_class_of(p.d.alpha)) {
    case kA15: hipLaunchKernelGGL((dq_kernel<T, D, kA15>), grid, dim3(kThreads), 0, s, p); break;
    case kA20: hipLaunchKernelGGL((dq_kernel<T, D, kA20>), grid, dim3(kThreads), 0, s, p); break;
    case kA125: hipLaunchKernelGGL((dq_kernel<T, D, kA125>), grid, dim3(kThreads), 0, s, p); break;
    default: hipLaunchKernelGGL((dq_kernel<T, D, kAGen>), grid, dim3(kThreads), 0, s, p); break;
  }
  return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_dkdv_td(const BackwardParams& p, hipStream_t s) {
  dim3 grid(p.d.nKB * p.d.BH);
  switch (alpha_class_of(p.d.alpha)) {
    case kA15: hipLaunchKernelGGL((dkdv_kernel<T, D, kA15>), grid, dim3(kThreads), 0, s, p); break;
    case kA20: hipLaunchKernelGGL((dkdv_kernel<T, D, kA20>), grid, dim3(kThreads), 0, s, p); break;
    case kA125: hipLaunchKernelGGL((dkdv_kernel<T, D, kA125>), grid, dim3(kThreads), 0, s, p); break;
    default: hipLaunchKernelGGL((dkdv_kernel<T, D, kAGen>), grid, dim3(kThreads), 0, s, p); break;
  }
  return hipGetLastError();
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
  if (bf16) {                                              \
    if (p.d.D == 64) return fn<u16, 64>(p, s);             \
    if (p.d.D == 128) return fn<u16, 128>(p, s);           \
  } else {                                                 \
    if (p.d.D == 64) return fn<float, 64>(p, s);           \
    if (p.d.D == 128) return fn<float, 128>(p, s);         \
  }                                                        \
  return hipErrorInvalidValue;

hipError_t launch_bwd_delta(const BackwardParams& p, bool bf16, hipStream_t s) { ASA_DISPATCH_TD(launch_delta_td) }
hipError_t launch_bwd_dq(const BackwardParams& p, bool bf16, hipStream_t s) { ASA_DISPATCH_TD(launch_dq_td) }
hipError_t launch_bwd_dkdv(const BackwardParams& p, bool bf16, hipStream_t s) { ASA_DISPATCH_TD(launch_dkdv_td) }

#undef ASA_DISPATCH_TD

}  // namespace asa
