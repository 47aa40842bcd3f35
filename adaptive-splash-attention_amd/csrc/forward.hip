// Block-sparse forward: out = sum_j p_j v_j / (sum_j p_j + EPS) over the
// visible keys of the active key blocks of each query block.
//
// Reference: splash_forward_sparse (adasplashattention.cu:244-341), which
// recomputes each score with one thread per query and accumulates p*v in
// registers.  Here one 256-thread block (4 waves x 16 query rows) walks the
// query block's CSR list; per active key block the K tile (row-major) and
// the V tile (transposed, bf16) are staged in LDS, S^T = K Q^T is formed on
// MFMA, p = max(u, EPS)^(1/(alpha-1)) with u = (alpha-1) s - tau is applied
// in registers, and O^T += V^T P^T runs on MFMA with P^T taken directly
// from the score accumulators.  Row sums of p are kept per lane and reduced
// across the four lane groups at the end.
#include "asa_device.hpp"
#include "asa_launch.hpp"
#include "asa_tiles.hpp"

namespace asa {
namespace {

constexpr int kThreads = 256;

template <typename T, int D> struct FwdSmem;
template <int D> struct alignas(16) FwdSmem<u16, D> {
  u16 K[kBlock * Tile<u16, D>::kRs];
  u16 Vt[D * Tile<u16, D>::kTs];
  __device__ const u16* v_operand() const { return Vt; }
  int kid[kBlock];
};
template <int D> struct alignas(16) FwdSmem<float, D> {
  float K[kBlock * Tile<float, D>::kRs];
  float V[kBlock * Tile<float, D>::kRs];
  __device__ const float* v_operand() const { return V; }
  int kid[kBlock];
};

template <typename T, int D>
__device__ __forceinline__ void stage_kv(FwdSmem<T, D>& sm, const T* K, const T* V,
                                         const int32_t* kidx, int kbase, int NK, int t) {
  stage_tile<D>(sm.K, static_cast<T*>(nullptr), K, kbase, NK, t, kThreads);
  if constexpr (sizeof(T) == 2) stage_tile<D>(static_cast<u16*>(nullptr), sm.Vt, V, kbase, NK, t, kThreads);
  else stage_tile<D>(sm.V, static_cast<T*>(nullptr), V, kbase, NK, t, kThreads);
  if (t < kBlock) sm.kid[t] = (kbase + t < NK) ? kidx[kbase + t] : 0;
}

template <typename T, int D, int PC>
__global__ __launch_bounds__(kThreads) void forward_kernel(ForwardParams p) {
  __shared__ FwdSmem<T, D> sm;
  const int NQ = p.d.NQ, NK = p.d.NK, nQB = p.d.nQB, nKB = p.d.nKB;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int g = lane >> 4, c16 = lane & 15;
  const int task = xcd_task(blockIdx.x, nQB * p.d.BH);
  const int qb = task % nQB, bh = task / nQB;
  const int q = qb * kBlock + 16 * w + c16;  // this lane's query row
  const bool qok = q < NQ;
  const size_t row = size_t(bh) * NQ + (qok ? q : 0);

  const T* Kb = static_cast<const T*>(p.k) + size_t(bh) * NK * D;
  const T* Vb = static_cast<const T*>(p.v) + size_t(bh) * NK * D;
  const int32_t* kidx = p.k_idx + size_t(bh) * NK;

  RowFrag<T, D> qf;
  qf.load(static_cast<const T*>(p.q) + row * D, qok, lane);
  const int qpos = qok ? p.q_idx[row] : 0;
  const float tau = qok ? p.taus[row] : 0.0f;
  const float am1 = p.d.alpha - 1.0f;
  const float a = 1.0f / am1;
  const float scale = p.d.scale;

  f32x4 o[D / 16];
  for (int db = 0; db < D / 16; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float rowsum = 0.0f;

  const int32_t* qp = p.q_ptr + size_t(bh) * (nQB + 1);
  const int32_t* ql = p.q_list + size_t(bh) * nQB * nKB;
  const int e0 = qp[qb], e1 = qp[qb + 1];
  for (int e = e0; e < e1; ++e) {
    const int kbase = ql[e] * kBlock;
    __syncthreads();
    stage_kv<T, D>(sm, Kb, Vb, kidx, kbase, NK, t);
    __syncthreads();

    f32x4 acc[4];
    rows_x_frag<D>(acc, sm.K, qf, lane);
    for (int f = 0; f < 4; ++f)
      for (int r = 0; r < 4; ++r) {
        const int kl = 16 * f + 4 * g + r;
        const bool vis = qok && (kbase + kl) < NK && sm.kid[kl] <= qpos;
        float pv = 0.0f;
        if (vis) {
          const float s = clamp_score(acc[f][r] * scale);
          const float u = am1 * s - tau;
          if (u > 0.0f) {
            pv = pow_fast<PC>(fmaxf(u, kEps), a);
            if (!finite(pv)) pv = 0.0f;
          }
        }
        acc[f][r] = pv;
        rowsum += pv;
      }
    tile_t_x_acc<D>(o, sm.v_operand(), acc, lane);
  }

  const float norm = sum_groups(rowsum);
  const float inv = 1.0f / (norm + kEps);
  if (qok) {
    T* orow = static_cast<T*>(p.out) + row * D;
    for (int db = 0; db < D / 16; ++db)
      for (int r = 0; r < 4; ++r) {
        float v = o[db][r] * inv;
        if (!finite(v)) v = 0.0f;
        Elem<T>::store(orow + 16 * db + 4 * g + r, v);
      }
    if (g == 0) p.norms[row] = norm;
  }
}

template <typename T, int D>
hipError_t launch_td(const ForwardParams& p, hipStream_t s) {
  dim3 grid(p.d.nQB * p.d.BH);
  switch (alpha_class_of(p.d.alpha)) {
    case kA15: hipLaunchKernelGGL((forward_kernel<T, D, kE2>), grid, dim3(kThreads), 0, s, p); break;
    case kA20: hipLaunchKernelGGL((forward_kernel<T, D, kE1>), grid, dim3(kThreads), 0, s, p); break;
    case kA125: hipLaunchKernelGGL((forward_kernel<T, D, kE4>), grid, dim3(kThreads), 0, s, p); break;
    default: hipLaunchKernelGGL((forward_kernel<T, D, kEGen>), grid, dim3(kThreads), 0, s, p); break;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_forward(const ForwardParams& p, bool bf16, hipStream_t s) {
  if (bf16) {
    if (p.d.D == 64) return launch_td<u16, 64>(p, s);
    if (p.d.D == 128) return launch_td<u16, 128>(p, s);
  } else {
    if (p.d.D == 64) return launch_td<float, 64>(p, s);
    if (p.d.D == 128) return launch_td<float, 128>(p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace asa
