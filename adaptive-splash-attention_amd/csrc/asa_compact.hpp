// Block mask -> CSR lists: the per-head device code of compact_kernel
// (compact.hip), shared with the launch that runs it beside the tau pass
// (select.hip).
#pragma once

#include "asa_device.hpp"
#include "asa_launch.hpp"

namespace asa {
namespace compact_detail {

constexpr int kThreads = 256;  // one block per (batch, head) and list kind
constexpr int kWaves = kThreads / kWave;

// Exclusive scan of cnt[0..n) into ptr[0..n] (ptr[n] = total), in LDS, by
// the first wave, 64 entries per step.
__device__ inline void block_scan(const int* cnt, int* ptr, int n) {
  const int t = threadIdx.x;
  if (t < kWave) {
    int run = 0;
    for (int base = 0; base < n; base += kWave) {
      const int i = base + t;
      const int v = i < n ? cnt[i] : 0;
      int x = v;  // inclusive scan over the wave
      for (int o = 1; o < kWave; o <<= 1) {
        const int y = __shfl_up(x, o, kWave);
        if (t >= o) x += y;
      }
      if (i < n) ptr[i] = run + x - v;
      run += __shfl(x, kWave - 1, kWave);
    }
    if (t == 0) ptr[n] = run;
  }
  __syncthreads();
}

// Row i of a row-major [rows, cols] byte mask (stride `rs`, element stride
// `es`): counts (pass 0) or writes the ascending indices of the set entries
// at out[0..) (pass 1).  One wave; returns the count.
__device__ __forceinline__ int scan_line(const uint8_t* m, size_t rs, size_t es, int i, int n,
                                         int32_t* out, int L) {
  int c = 0;
  for (int base = 0; base < n; base += kWave) {
    const int j = base + L;
    const bool set = j < n && m[size_t(i) * rs + size_t(j) * es] != 0;
    const uint64_t bits = __ballot(set);
    if (out && set) out[c + __builtin_popcountll(bits & ((uint64_t(1) << L) - 1))] = j;
    c += __builtin_popcountll(bits);
  }
  return c;
}

// Mask bytes of one head staged in LDS when they fit (the scans then read
// LDS instead of making dependent global loads, 4 per line of the mask).
constexpr int kStageMax = 32 * 1024;

// Block `blk` of the launch: (batch, head) blk / 2, list kind blk % 2.
template <bool STAGED>
__device__ __forceinline__ void compact_head(const CompactParams& p, int* sm, int blk) {
  const int nQB = p.nQB, nKB = p.nKB, bh = blk >> 1, t = threadIdx.x;
  const bool key_major = (blk & 1) != 0;  // the two lists in separate blocks
  const int w = t >> 6, L = t & 63;
  int* cnt = sm;                  // max(nQB, nKB)
  int* ptr = sm + max(nQB, nKB);  // max(nQB, nKB) + 1
  const uint8_t* m = p.mask + size_t(bh) * nQB * nKB;
  if constexpr (STAGED) {
    // 16-byte chunks, then the tail bytes; the staged copy starts 16-byte
    // aligned after the scan arrays
    uint8_t* sl = reinterpret_cast<uint8_t*>(sm + ((2 * max(nQB, nKB) + 1 + 3) & ~3));
    const int nb = nQB * nKB, n16 = (size_t(m) % 16 == 0) ? nb / 16 : 0;
    for (int i = t; i < n16; i += kThreads)
      reinterpret_cast<uint4*>(sl)[i] = reinterpret_cast<const uint4*>(m)[i];
    for (int i = n16 * 16 + t; i < nb; i += kThreads) sl[i] = m[i];
    __syncthreads();
    m = sl;
  }

  if (!key_major) {
    // ---- query-major: rows of the mask ----
    for (int i = w; i < nQB; i += kWaves) {
      const int c = scan_line(m, nKB, 1, i, nKB, nullptr, L);
      if (L == 0) cnt[i] = c;
    }
    __syncthreads();
    block_scan(cnt, ptr, nQB);
    int32_t* qp = p.q_ptr + size_t(bh) * (nQB + 1);
    int32_t* ql = p.q_list + size_t(bh) * nQB * nKB;
    for (int i = t; i <= nQB; i += kThreads) qp[i] = ptr[i];
    for (int i = w; i < nQB; i += kWaves) scan_line(m, nKB, 1, i, nKB, ql + ptr[i], L);
    for (int e = ptr[nQB] + t; e < nQB * nKB; e += kThreads) ql[e] = 0;
    return;
  }

  // ---- key-major: columns of the mask ----
  for (int j = w; j < nKB; j += kWaves) {
    const int c = scan_line(m, 1, nKB, j, nQB, nullptr, L);
    if (L == 0) cnt[j] = c;
  }
  __syncthreads();
  block_scan(cnt, ptr, nKB);
  int32_t* kp = p.k_ptr + size_t(bh) * (nKB + 1);
  int32_t* kl = p.k_list + size_t(bh) * nKB * nQB;
  for (int j = t; j <= nKB; j += kThreads) kp[j] = ptr[j];
  for (int j = w; j < nKB; j += kWaves) scan_line(m, 1, nKB, j, nQB, kl + ptr[j], L);
  for (int e = ptr[nKB] + t; e < nQB * nKB; e += kThreads) kl[e] = 0;
}

// The block's LDS bytes (dynamic shared memory of the launch).
inline size_t compact_lds_bytes(const CompactParams& p) {
  const int n = p.nQB > p.nKB ? p.nQB : p.nKB;
  size_t lds = sizeof(int) * size_t(2 * n + 1);
  if (p.nQB * p.nKB <= kStageMax) lds = ((lds + 15) & ~size_t(15)) + size_t(p.nQB) * p.nKB;
  return lds;
}

// Both lists of every head: blocks [0, 2 BH) of a launch, from `blk`.
__device__ __forceinline__ void compact_block(const CompactParams& p, int* sm, int blk) {
  if (p.nQB * p.nKB <= kStageMax) compact_head<true>(p, sm, blk);  // block-uniform
  else compact_head<false>(p, sm, blk);
}

}  // namespace compact_detail
}  // namespace asa
