// Block mask -> CSR lists.
//
// Reference: build_lookup_kernel (adasplashattention.cu:219-242), which
// builds the query-major list (Qi_ptr / Qi_idx) with one serial thread per
// (batch, head).  Here one 256-thread block per (batch, head) builds both
//   query-major:  q_ptr[nQB+1], q_list[nQB*nKB]  (same layout as Qi_ptr/Qi_idx)
//   key-major:    k_ptr[nKB+1], k_list[nKB*nQB]  (feeds the atomic-free dK/dV)
// with lists in ascending block order and zero-filled tails.  Row / column
// counts are computed in parallel, offsets by a block-wide scan, and each
// row / column is then written by one thread.
#include "asa_device.hpp"
#include "asa_launch.hpp"

namespace asa {
namespace {

constexpr int kThreads = 256;

// Exclusive scan of cnt[0..n) into ptr[0..n] (ptr[n] = total), in LDS.
__device__ void block_scan(const int* cnt, int* ptr_lds, int n) {
  __shared__ int partial[kThreads + 1];
  const int t = threadIdx.x;
  const int per = (n + kThreads - 1) / kThreads;
  const int b = min(n, t * per), e = min(n, b + per);
  int s = 0;
  for (int i = b; i < e; ++i) s += cnt[i];
  partial[t] = s;
  __syncthreads();
  if (t == 0) {
    int run = 0;
    for (int i = 0; i < kThreads; ++i) {
      const int v = partial[i];
      partial[i] = run;
      run += v;
    }
    partial[kThreads] = run;
  }
  __syncthreads();
  int run = partial[t];
  for (int i = b; i < e; ++i) {
    ptr_lds[i] = run;
    run += cnt[i];
  }
  if (t == 0) ptr_lds[n] = partial[kThreads];
  __syncthreads();
}

__global__ __launch_bounds__(kThreads) void compact_kernel(CompactParams p) {
  extern __shared__ int sm[];
  const int nQB = p.nQB, nKB = p.nKB, bh = blockIdx.x, t = threadIdx.x;
  const uint8_t* m = p.mask + size_t(bh) * nQB * nKB;
  int* cnt = sm;                  // max(nQB, nKB)
  int* ptr = sm + max(nQB, nKB);  // max(nQB, nKB) + 1

  // ---- query-major ----
  for (int i = t; i < nQB; i += kThreads) {
    int c = 0;
    for (int j = 0; j < nKB; ++j) c += m[size_t(i) * nKB + j];
    cnt[i] = c;
  }
  __syncthreads();
  block_scan(cnt, ptr, nQB);
  int32_t* qp = p.q_ptr + size_t(bh) * (nQB + 1);
  int32_t* ql = p.q_list + size_t(bh) * nQB * nKB;
  for (int i = t; i <= nQB; i += kThreads) qp[i] = ptr[i];
  for (int i = t; i < nQB; i += kThreads) {
    int w = ptr[i];
    for (int j = 0; j < nKB; ++j)
      if (m[size_t(i) * nKB + j]) ql[w++] = j;
  }
  for (int e = ptr[nQB] + t; e < nQB * nKB; e += kThreads) ql[e] = 0;
  __syncthreads();

  // ---- key-major ----
  for (int j = t; j < nKB; j += kThreads) {
    int c = 0;
    for (int i = 0; i < nQB; ++i) c += m[size_t(i) * nKB + j];
    cnt[j] = c;
  }
  __syncthreads();
  block_scan(cnt, ptr, nKB);
  int32_t* kp = p.k_ptr + size_t(bh) * (nKB + 1);
  int32_t* kl = p.k_list + size_t(bh) * nKB * nQB;
  for (int j = t; j <= nKB; j += kThreads) kp[j] = ptr[j];
  for (int j = t; j < nKB; j += kThreads) {
    int w = ptr[j];
    for (int i = 0; i < nQB; ++i)
      if (m[size_t(i) * nKB + j]) kl[w++] = i;
  }
  for (int e = ptr[nKB] + t; e < nQB * nKB; e += kThreads) kl[e] = 0;
}

}  // namespace

hipError_t launch_compact(const CompactParams& p, hipStream_t s) {
  const int n = p.nQB > p.nKB ? p.nQB : p.nKB;
  const size_t lds = sizeof(int) * size_t(2 * n + 1);
  hipLaunchKernelGGL(compact_kernel, dim3(p.BH), dim3(kThreads), lds, s, p);
  return hipGetLastError();
}

}  // namespace asa
