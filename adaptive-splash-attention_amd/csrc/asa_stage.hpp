// Pipelined staging of 64-row tiles into LDS.
//
// Every attention pass streams, per active block pair, two 64-row tiles
// (K and V, or Q and dO) of one (batch, head) through LDS.  A Stager holds
// one step's share of those tiles in registers: the kernels fetch tile i+2
// into registers while tile i is multiplied out of one LDS buffer and tile
// i+1 sits in the other, so global-load latency overlaps the MFMA work of a
// whole step.
//
// Work split: a tile is cut into "quads" of 4 consecutive rows x one
// 16-byte column chunk; the quads of both tiles are dealt to the 256
// threads (quad index = thread + 256 * i, tile 0's quads first, so that
// every wave works on one tile at a time) and stored in the tile layout
// (row stride Tile<T, D>::kRs, chunk swizzle Tile<T, D>::sw).  Products that need a tile transposed read it with the
// transposing LDS read, so no transposed copy is staged.
#pragma once

#include "asa_device.hpp"
#include "asa_tiles.hpp"

namespace asa {

template <typename T, int D, int NT = 256>
struct Stager {
  static constexpr int kEpc = 16 / int(sizeof(T));   // elements per 16-byte chunk
  static constexpr int kCpr = D / kEpc;              // chunks per row
  static constexpr int kQuads = (kBlock / 4) * kCpr; // quads per tile
  static constexpr int kPer = 2 * kQuads / NT;       // quads per thread
  static_assert(2 * kQuads % NT == 0, "quads must divide evenly");
  static constexpr int kRs = Tile<T, D>::kRs;

  uint4 r[kPer][4];

  // Rows [row0, row0 + 64) of src0 / src1 ([*, D] row-major); rows >= nrows
  // read as zero.  A tile wholly inside loads its quad's four rows from one
  // address (the row steps become immediate offsets), without tests.
  __device__ __forceinline__ void load(const T* src0, const T* src1, int row0, int nrows, int t) {
    const bool whole = row0 + kBlock <= nrows;  // block-uniform
    for (int i = 0; i < kPer; ++i) {
      const int qi = t + i * NT;
      const int job = qi / kQuads, q = qi % kQuads;
      const int rq = q / kCpr, cc = q % kCpr;
      const T* src = (job == 0 ? src0 : src1) + size_t(row0 + 4 * rq) * D + cc * kEpc;
      if (whole) {
        for (int j = 0; j < 4; ++j) r[i][j] = *reinterpret_cast<const uint4*>(src + j * D);
      } else {
        for (int j = 0; j < 4; ++j)
          r[i][j] = row0 + 4 * rq + j < nrows ? *reinterpret_cast<const uint4*>(src + j * D)
                                              : uint4{0u, 0u, 0u, 0u};
      }
    }
  }

  // Tile 0 to dst0, tile 1 to dst1.
  __device__ __forceinline__ void store(T* dst0, T* dst1, int t) const {
    for (int i = 0; i < kPer; ++i) {
      const int qi = t + i * NT;
      const int job = qi / kQuads, q = qi % kQuads;
      const int rq = q / kCpr, cc = q % kCpr;
      T* dst = job == 0 ? dst0 : dst1;
      // the chunk swizzle depends on row bits 2-3: constant over the quad
      T* d = dst + 4 * rq * kRs + ((cc * kEpc) ^ Tile<T, D>::sw(4 * rq));
      for (int j = 0; j < 4; ++j) *reinterpret_cast<uint4*>(d + j * kRs) = r[i][j];
    }
  }
};

// K tile of 64 keys in LDS, in the attention passes' tile layout (padded
// row stride, swizzled 16-byte chunks: Tile<T, D>), filled by all NT
// threads in 16-byte chunks (consecutive threads, consecutive chunks of a
// row: coalesced global reads).  The scores are formed by rows_x_frag, the
// attention passes' score product with the same operands and accumulation
// order, so every pass sees bit-identical scores.
template <typename T, int D, int NT = 256> struct KStage {
  static constexpr int kRs = Tile<T, D>::kRs;                   // elements per LDS row
  static constexpr int kRowChunks = D * int(sizeof(T)) / 16;    // 16-byte chunks per row
  static constexpr int kPerThread = kBlock * kRowChunks / NT;
  static_assert(kBlock * kRowChunks % NT == 0, "tile chunks must divide the block");
  uint4 r[kPerThread];
  // rows >= NK read as zero (such keys are never visible)
  __device__ __forceinline__ void load(const T* Kb, int kbase, int NK, int t) {
    for (int j = 0; j < kPerThread; ++j) {
      const int ch = t + j * NT, row = ch / kRowChunks;
      const int col = (ch % kRowChunks) * (16 / int(sizeof(T)));
      r[j] = kbase + row < NK
                 ? *reinterpret_cast<const uint4*>(Kb + size_t(kbase + row) * D + col)
                 : uint4{0u, 0u, 0u, 0u};
    }
  }
  __device__ __forceinline__ void store(T* buf, int t) const {
    for (int j = 0; j < kPerThread; ++j) {
      const int ch = t + j * NT, row = ch / kRowChunks;
      const int col = (ch % kRowChunks) * (16 / int(sizeof(T)));
      *reinterpret_cast<uint4*>(buf + row * kRs + (col ^ Tile<T, D>::sw(row))) = r[j];
    }
  }
};

// Positions of the 64 keys (or queries) of a tile, staged beside it by the
// first wave, with a flag telling whether the whole tile passes a block-wide
// visibility test (then the per-element checks can be skipped).
struct PosStager {
  int v;
  // entries past `n` read as `pad`
  __device__ __forceinline__ void load(const int32_t* pos, int base, int n, int pad, int t) {
    if (t < kWave) v = base + t < n ? pos[base + t] : pad;
  }
  // positions only (the caller knows the flag otherwise)
  __device__ __forceinline__ void store(int* dst, int t) const {
    if (t < kWave) dst[t] = v;
  }
  // kMax: flag = max over the tile <= bound; else flag = min over the tile >= bound
  template <bool kMax>
  __device__ __forceinline__ void store(int* dst, int* flag, int bound, int t) const {
    if (t < kWave) {
      dst[t] = v;
      const int m = wave_reduce_minmax<kMax>(v);
      if (t == 0) *flag = kMax ? (m <= bound) : (m >= bound);
    }
  }
};

}  // namespace asa
