// Block mask -> CSR lists.
//
// Reference: build_lookup_kernel (adasplashattention.cu:219-242), which
// builds the query-major list (Qi_ptr / Qi_idx) with one serial thread per
// (batch, head).  Here 256-thread blocks (two per (batch, head), or one
// per 32 mask lines for masks too large for LDS) build
//   query-major:  q_ptr[nQB+1], q_list[nQB*nKB]  (same layout as Qi_ptr/Qi_idx)
//   key-major:    k_ptr[nKB+1], k_list[nKB*nQB]  (feeds the atomic-free dK/dV)
// with lists in ascending block order and zero-filled tails.  A wave takes
// one row (column) of the mask at a time, 64 entries per step: one load per
// lane, a ballot, and the set lanes write their block index at their rank.
#include "asa_compact.hpp"
#include "asa_device.hpp"
#include "asa_launch.hpp"

namespace asa {
namespace {

using compact_detail::kThreads;

__global__ __launch_bounds__(kThreads) void compact_kernel(CompactParams p) {
  extern __shared__ int sm[];
  compact_detail::compact_block(p, sm, blockIdx.x);
}

// 64-row mask from a 32-row one (grid-stride over the 64-row mask's bytes).
__global__ __launch_bounds__(kThreads) void fold_halves_kernel(const uint8_t* half, uint8_t* mask,
                                                               int NQ, int nQB, int nKB,
                                                               size_t n) {
  const int nQH = half_blocks(NQ);
  for (size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += size_t(gridDim.x) * kThreads) {
    const int kb = int(i % size_t(nKB));
    const size_t r = i / size_t(nKB);  // bh * nQB + qb
    const int qb = int(r % size_t(nQB));
    const size_t bh = r / size_t(nQB);
    const uint8_t* h = half + (bh * nQH + 2 * size_t(qb)) * nKB + kb;
    const bool on = h[0] != 0 || (2 * qb + 1 < nQH && h[nKB] != 0);
    mask[i] = on ? 1 : 0;
  }
}

}  // namespace

hipError_t launch_fold_halves(const uint8_t* half, uint8_t* mask, int BH, int NQ, int nQB,
                              int nKB, hipStream_t s) {
  const size_t n = size_t(BH) * nQB * nKB;
  size_t blocks = (n + kThreads - 1) / kThreads;
  if (blocks > (size_t(1) << 20)) blocks = size_t(1) << 20;
  hipLaunchKernelGGL(fold_halves_kernel, dim3(unsigned(blocks)), dim3(kThreads), 0, s, half, mask,
                     NQ, nQB, nKB, n);
  return hipGetLastError();
}

hipError_t launch_compact(const CompactParams& p, hipStream_t s) {
  hipLaunchKernelGGL(compact_kernel, dim3(compact_detail::compact_grid(p)), dim3(kThreads),
                     compact_detail::compact_lds_bytes(p), s, p);
  return hipGetLastError();
}

}  // namespace asa
