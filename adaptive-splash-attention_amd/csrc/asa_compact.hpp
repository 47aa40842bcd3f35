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

// ---- Masks too large to stage: lines (mask rows for the query-major list,
// columns for the key-major one) dealt to blocks kChunkLines at a time, so
// that a head's lists are built by many blocks instead of two (one block
// per list scanned a 512 x 512 mask in ~0.4 ms).  Every block counts the
// set entries of the whole head mask (16-byte loads, L2-resident after the
// first block): those before its lines give its lines' list offsets, its
// own lines' counts their lengths, and the total the zero-filled tail, of
// which each block clears an equal share.  The lists come out exactly as
// compact_head writes them.
constexpr int kChunkLines = 32;

// The chunked path applies: a mask too large to stage, rows of whole
// 16-byte chunks (nKB % 16 == 0) at a 16-byte aligned base.
__host__ __device__ inline bool compact_chunked(const CompactParams& p) {
  return int64_t(p.nQB) * p.nKB > kStageMax && p.nKB % 16 == 0 &&
         reinterpret_cast<uintptr_t>(p.mask) % 16 == 0;
}
__host__ __device__ inline int compact_chunks(int n) { return (n + kChunkLines - 1) / kChunkLines; }

__device__ __forceinline__ int block_sum(int v, int* red) {
  for (int o = kWave / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, kWave);
  __syncthreads();  // red free from any earlier use
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  int s = 0;
  for (int i = 0; i < kWaves; ++i) s += red[i];
  return s;
}

// Bit q <- byte q of v is nonzero.
__device__ __forceinline__ uint32_t nonzero_bytes(const uint4 v) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  uint32_t m = 0;
  for (int j = 0; j < 4; ++j)
    for (int q = 0; q < 4; ++q) m |= ((w[j] >> (8 * q)) & 0xffu) != 0u ? 1u << (4 * j + q) : 0u;
  return m;
}

// Block `blk` of the chunked launch: (batch, head) blk / per, then the
// query-major chunks, then the key-major ones.
__device__ __forceinline__ void compact_chunk(const CompactParams& p, int* sm, int blk) {
  const int nQB = p.nQB, nKB = p.nKB, t = threadIdx.x, w = t >> 6, L = t & 63;
  const int ncq = compact_chunks(nQB), nck = compact_chunks(nKB);
  const int bh = blk / (ncq + nck), b = blk % (ncq + nck);
  const bool key_major = b >= ncq;  // block-uniform
  const int chunk = key_major ? b - ncq : b;
  const int n = key_major ? nKB : nQB;      // lines
  const int len = key_major ? nQB : nKB;    // entries per line
  const int l0 = chunk * kChunkLines, nl = min(n, l0 + kChunkLines) - l0;
  int* cnt = sm;                      // [kChunkLines]
  int* ptr = sm + kChunkLines;        // [kChunkLines + 1]
  int* red = ptr + kChunkLines + 1;   // [kWaves]
  if (t < kChunkLines) cnt[t] = 0;
  __syncthreads();
  const uint8_t* m = p.mask + size_t(bh) * nQB * nKB;
  const size_t n16 = size_t(nQB) * nKB / 16;
  const int cpr = nKB / 16;  // 16-byte chunks per mask row
  int before = 0, total = 0;
  for (size_t i = t; i < n16; i += kThreads) {
    const uint32_t nz = nonzero_bytes(reinterpret_cast<const uint4*>(m)[i]);
    const int c = __builtin_popcount(nz);
    total += c;
    if (!key_major) {
      const int row = int(i / size_t(cpr));
      if (row < l0) before += c;
      else if (row < l0 + nl && c) atomicAdd(&cnt[row - l0], c);
    } else {
      const int col0 = int(i % size_t(cpr)) * 16;
      if (col0 + 16 <= l0) {
        before += c;
      } else if (col0 < l0 + nl) {
        for (int q = 0; q < 16; ++q)
          if ((nz >> q) & 1u) {
            const int col = col0 + q;
            if (col < l0) ++before;
            else if (col < l0 + nl) atomicAdd(&cnt[col - l0], 1);
          }
      }
    }
  }
  before = block_sum(before, red);
  total = block_sum(total, red);
  block_scan(cnt, ptr, nl);  // ends with a barrier
  int32_t* lp = (key_major ? p.k_ptr : p.q_ptr) + size_t(bh) * (n + 1);
  int32_t* ll = (key_major ? p.k_list : p.q_list) + size_t(bh) * nQB * nKB;
  for (int i = t; i < nl; i += kThreads) lp[l0 + i] = before + ptr[i];
  if (t == 0 && l0 + nl == n) lp[n] = total;
  for (int i = w; i < nl; i += kWaves) {
    if (!key_major) scan_line(m, nKB, 1, l0 + i, len, ll + before + ptr[i], L);
    else scan_line(m, 1, nKB, l0 + i, len, ll + before + ptr[i], L);
  }
  // this block's share of the zero tail [total, nQB nKB)
  const size_t cap = size_t(nQB) * nKB, tail = cap - size_t(total);
  const int nch = key_major ? nck : ncq;
  const size_t share = (tail + nch - 1) / nch;
  const size_t z0 = size_t(total) + size_t(chunk) * share;
  const size_t z1 = min(cap, z0 + share);
  for (size_t e = z0 + t; e < z1; e += kThreads) ll[e] = 0;
}

// Blocks of a launch that builds every head's lists.
inline int compact_grid(const CompactParams& p) {
  return compact_chunked(p) ? p.BH * (compact_chunks(p.nQB) + compact_chunks(p.nKB)) : 2 * p.BH;
}

// The block's LDS bytes (dynamic shared memory of the launch).
inline size_t compact_lds_bytes(const CompactParams& p) {
  if (compact_chunked(p)) return sizeof(int) * size_t(2 * kChunkLines + 1 + kWaves);
  const int n = p.nQB > p.nKB ? p.nQB : p.nKB;
  size_t lds = sizeof(int) * size_t(2 * n + 1);
  if (p.nQB * p.nKB <= kStageMax) lds = ((lds + 15) & ~size_t(15)) + size_t(p.nQB) * p.nKB;
  return lds;
}

// Both lists of every head: blocks [0, compact_grid(p)) of a launch, from
// `blk`.
__device__ __forceinline__ void compact_block(const CompactParams& p, int* sm, int blk) {
  if (compact_chunked(p)) compact_chunk(p, sm, blk);  // block-uniform
  else if (p.nQB * p.nKB <= kStageMax) compact_head<true>(p, sm, blk);
  else compact_head<false>(p, sm, blk);
}

}  // namespace compact_detail
}  // namespace asa
