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

enum StageRows : int { kRowsAny = 0, kRowsDense = 1, kRowsStrided = 2 };

template <typename T, int D, int NT = 256>
struct Stager {
  static constexpr int kEpc = 16 / int(sizeof(T));   // elements per 16-byte chunk
  static constexpr int kCpr = D / kEpc;              // chunks per row
  static constexpr int kQuads = (kBlock / 4) * kCpr; // quads per tile
  static constexpr int kPer = 2 * kQuads / NT;       // quads per thread
  static_assert(2 * kQuads % NT == 0, "quads must divide evenly");
  static_assert(kQuads % 64 == 0, "a wave's quads must lie in one tile");
  static constexpr int kRs = Tile<T, D>::kRs;

  uint4 r[kPer][4];

  // Rows [row0, row0 + 64) of src0 / src1, their rows sn0 / sn1 elements
  // apart; rows >= nrows and columns >= hd read as zero.  A tile wholly
  // inside rows of exactly D elements (sn = hd = D) loads its quad's four
  // rows from one address (the row steps become immediate offsets),
  // without tests.  ROWS: kRowsAny tests for that case at run time;
  // kRowsDense (the caller guarantees sn0 = sn1 = hd = D) and
  // kRowsStrided compile one case in, which keeps the other's registers
  // out of a kernel that is short of them.
  template <int ROWS = kRowsAny>
  __device__ __forceinline__ void load(const T* src0, size_t sn0, const T* src1, size_t sn1,
                                       int row0, int nrows, int hd, int t) {
    const bool whole = row0 + kBlock <= nrows;  // block-uniform
    const bool dense = ROWS == kRowsDense ||
                       (ROWS == kRowsAny && sn0 == D && sn1 == D && hd == D);  // uniform
    for (int i = 0; i < kPer; ++i) {
      const int qi = t + i * NT;
      const int job = qi / kQuads, q = qi % kQuads;
      const int rq = q / kCpr, cc = q % kCpr;
      if (whole && dense) {
        const T* src = (job == 0 ? src0 : src1) + size_t(row0 + 4 * rq) * D + cc * kEpc;
        for (int j = 0; j < 4; ++j) r[i][j] = *reinterpret_cast<const uint4*>(src + j * D);
      } else {
        // the tile's rows from a wave-uniform base (kQuads is a multiple of
        // the wave: one tile per wave and i) at 32-bit byte offsets (a
        // head's rows lie within 2^31 bytes of its first), so that the
        // strided path holds no 64-bit addresses
        const int jw = __builtin_amdgcn_readfirstlane(job);
        const size_t sn = jw == 0 ? sn0 : sn1;
        const unsigned char* base =
            reinterpret_cast<const unsigned char*>((jw == 0 ? src0 : src1) + size_t(row0) * sn);
        const uint32_t snb = uint32_t(sn) * uint32_t(sizeof(T));
        const uint32_t off = uint32_t(4 * rq) * snb + uint32_t(cc * kEpc) * uint32_t(sizeof(T));
        const bool col = cc * kEpc < hd;
        for (int j = 0; j < 4; ++j)
          r[i][j] = col && row0 + 4 * rq + j < nrows
                        ? *reinterpret_cast<const uint4*>(base + (off + uint32_t(j) * snb))
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
