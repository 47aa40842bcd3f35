// LDS tiles and the two MFMA tile products used by the attention passes.
//
// A "tile" is 64 rows x D columns of a [rows, D] tensor, staged row-major
// in LDS (stride D+8 with swizzled 16-byte chunks for bf16, D+4 for fp32).  Products that contract over
// the tile's rows read their bf16 operand with the gfx950 transposing LDS
// read; the fp32 MFMA takes one element per lane and k slot, which the
// row-major tile serves directly.
//
//   rows_x_frag:  acc[f] (16 tile rows 16f.. x 16 lanes' columns)
//                 = sum_d Tile[16f + i][d] * Bfrag[d][col]
//   tile_t_x_acc: o[db] (16 head dims 16db.. x 16 columns)
//                 += sum_r Tile[r][16db + i] * X[r][col]
//                 where X is given in the accumulator layout of rows_x_frag
//                 (the row index r plays the MFMA k role; lane group g holds
//                 rows 16f + 4g + 0..3 of each block f).  Template bounds
//                 [CC0, CC1) restrict it to the row halves 32cc..32cc+31
//                 (blocks f = 2cc, 2cc+1), so a caller can feed each half as
//                 soon as it is formed.
#pragma once

#include <type_traits>

#include "asa_device.hpp"

namespace asa {

template <typename T, int D> struct Tile;
// bf16: row stride D + 8 elements (a 16-byte pad per row), and the index of
// each 16-byte chunk of row r XORed with bit 2 ^ bit 3 of r.  Measured on
// gfx950 (64 x 64 tiles, 16 waves per CU), per wave instruction:
//   ds_read_b128, 16 lanes x one chunk of 16 consecutive rows (rows_x_frag):
//     2.05 ns with the swizzle, 3.55 ns without (a 2-way bank conflict);
//   ds_read_b64_tr_b16 (tile_t_x_acc): 2.37 ns either way (conflict-free);
//   ds_write_b128 of the staging quads: 5.6 ns either way (write-rate bound).
// A 32-byte pad removes the read conflict without the swizzle but costs
// 4 KiB of LDS per tile pair, one resident block per CU in the forward pass.
// The XOR mask (in elements, sw(row)) depends on row bits 2 and 3 only, so
// it is constant per lane in every access pattern here.
template <int D> struct Tile<u16, D> {
  static constexpr int kRs = D + 8;  // row stride (elements)
  __host__ __device__ static constexpr int sw(int row) { return 8 * (((row >> 2) ^ (row >> 3)) & 1); }
};
template <int D> struct Tile<h16, D> : Tile<u16, D> {};  // fp16: the bf16 layout
template <int D> struct Tile<float, D> {
  static constexpr int kRs = D + 4;
  __host__ __device__ static constexpr int sw(int) { return 0; }
};

// B-operand fragment of one row per lane (lane column c16 <- `row`),
// covering the whole head dimension; columns >= hd read as zero.
template <typename T, int D> struct RowFrag;
// 16-bit formats (bf16, fp16)
template <typename T, int D> struct RowFrag16 {
  using V8 = typename Half<T>::v8;
  V8 v[D / 32];
  __device__ void load(const T* row, bool ok, int lane, int hd = D) {
    const int g = lane >> 4;
    for (int s = 0; s < D / 32; ++s)
      v[s] = ok && 32 * s + 8 * g < hd ? *reinterpret_cast<const V8*>(row + 32 * s + 8 * g) : V8{};
  }
};
template <int D> struct RowFrag<u16, D> : RowFrag16<u16, D> {};
template <int D> struct RowFrag<h16, D> : RowFrag16<h16, D> {};
template <int D> struct RowFrag<float, D> {
  f32x4 v[D / 16];
  __device__ void load(const float* row, bool ok, int lane, int hd = D) {
    const int g = lane >> 4;
    for (int j = 0; j < D / 16; ++j)
      v[j] = ok && 16 * j + 4 * g < hd ? *reinterpret_cast<const f32x4*>(row + 16 * j + 4 * g) : f32x4{};
  }
};

// [F0, F1) restricts the product to row blocks f = F0..F1-1 (16 rows each);
// the other entries of acc are left alone.
template <int D, int F0 = 0, int F1 = 4, typename T,
          typename std::enable_if<is_half<T>, int>::type = 0>
__device__ __forceinline__ void rows_x_frag(f32x4 (&acc)[4], const T* rm,
                                            const RowFrag<T, D>& b, int lane) {
  using V8 = typename Half<T>::v8;
  const int g = lane >> 4, c = lane & 15;
  // row 16f + c, chunk 4s + g (swizzled by row bits 2-3, i.e. by c)
  const T* base = rm + c * Tile<T, D>::kRs + ((8 * g) ^ Tile<T, D>::sw(c));
  for (int f = F0; f < F1; ++f) acc[f] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < D / 32; ++s)
    for (int f = F0; f < F1; ++f) {
      const V8 a = *reinterpret_cast<const V8*>(base + 16 * f * Tile<T, D>::kRs + 32 * s);
      acc[f] = mfma(a, b.v[s], acc[f]);
    }
}
template <int D, int F0 = 0, int F1 = 4>
__device__ __forceinline__ void rows_x_frag(f32x4 (&acc)[4], const float* rm,
                                            const RowFrag<float, D>& b, int lane) {
  const int g = lane >> 4, c = lane & 15;
  for (int f = F0; f < F1; ++f) acc[f] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < D / 16; ++j)
    for (int f = F0; f < F1; ++f) {
      const f32x4 a =
          *reinterpret_cast<const f32x4*>(rm + (16 * f + c) * Tile<float, D>::kRs + 16 * j + 4 * g);
      for (int r = 0; r < 4; ++r) acc[f] = mfma(a[r], b.v[j][r], acc[f]);
    }
}

// rows_x_frag with the tile read straight from global memory: `rows` points
// at the tile's first row, rows `sn` elements apart; rows >= nrows and
// columns >= hd read as zero.  The same operands in the same MFMA order as the LDS versions above
// (the LDS tile holds the same values; its swizzle only moves them), so the
// results are bit-identical.
template <int D, typename T, typename std::enable_if<is_half<T>, int>::type = 0>
__device__ __forceinline__ void rows_x_frag_global(f32x4 (&acc)[4], const T* rows, int nrows,
                                                   size_t sn, int hd, const RowFrag<T, D>& b,
                                                   int lane) {
  using V8 = typename Half<T>::v8;
  const int g = lane >> 4, c = lane & 15;
  V8 a[D / 32][4];
  for (int s = 0; s < D / 32; ++s)
    for (int f = 0; f < 4; ++f)
      a[s][f] = 16 * f + c < nrows && 32 * s + 8 * g < hd
                    ? *reinterpret_cast<const V8*>(rows + (16 * f + c) * sn + 32 * s + 8 * g)
                    : V8{};
  for (int f = 0; f < 4; ++f) acc[f] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < D / 32; ++s)
    for (int f = 0; f < 4; ++f) acc[f] = mfma(a[s][f], b.v[s], acc[f]);
}
template <int D>
__device__ __forceinline__ void rows_x_frag_global(f32x4 (&acc)[4], const float* rows, int nrows,
                                                   size_t sn, int hd, const RowFrag<float, D>& b,
                                                   int lane) {
  const int g = lane >> 4, c = lane & 15;
  for (int f = 0; f < 4; ++f) acc[f] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < D / 16; ++j) {
    f32x4 a[4];
    for (int f = 0; f < 4; ++f)
      a[f] = 16 * f + c < nrows && 16 * j + 4 * g < hd
                 ? *reinterpret_cast<const f32x4*>(rows + (16 * f + c) * sn + 16 * j + 4 * g)
                 : f32x4{};
    for (int f = 0; f < 4; ++f)
      for (int r = 0; r < 4; ++r) acc[f] = mfma(a[f][r], b.v[j][r], acc[f]);
  }
}

// A key tile's A operands of rows_x_frag_global, loaded once and multiplied
// by several B fragments (bf16: held in registers; fp32: re-read per
// product, since D = 128 would take 128 registers).
template <typename T, int D> struct KFrags;
template <typename T, int D> struct KFrags16 {
  using V8 = typename Half<T>::v8;
  V8 a[D / 32][4];
  __device__ __forceinline__ void load(const T* rows, int nrows, size_t sn, int hd, int lane) {
    const int g = lane >> 4, c = lane & 15;
    for (int s = 0; s < D / 32; ++s)
      for (int f = 0; f < 4; ++f)
        a[s][f] = 16 * f + c < nrows && 32 * s + 8 * g < hd
                      ? *reinterpret_cast<const V8*>(rows + (16 * f + c) * sn + 32 * s + 8 * g)
                      : V8{};
  }
  __device__ __forceinline__ void product(f32x4 (&acc)[4], const RowFrag<T, D>& b) const {
    for (int f = 0; f < 4; ++f) acc[f] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < D / 32; ++s)
      for (int f = 0; f < 4; ++f) acc[f] = mfma(a[s][f], b.v[s], acc[f]);
  }
};
template <int D> struct KFrags<u16, D> : KFrags16<u16, D> {};
template <int D> struct KFrags<h16, D> : KFrags16<h16, D> {};
template <int D> struct KFrags<float, D> {
  const float* rows;
  size_t sn;
  int nrows, hd, lane;
  __device__ __forceinline__ void load(const float* r, int n, size_t s, int h, int l) {
    rows = r;
    nrows = n;
    sn = s;
    hd = h;
    lane = l;
  }
  __device__ __forceinline__ void product(f32x4 (&acc)[4], const RowFrag<float, D>& b) const {
    rows_x_frag_global<D>(acc, rows, nrows, sn, hd, b, lane);
  }
};

// bf16 / fp16: `rm` is the row-major tile.  The A operand (4 consecutive tile rows
// at one column per lane and half) is read with ds_read_b64_tr_b16: in each
// 16-lane group, lane l reads the 8 bytes at row key0 + l/4, columns
// col0 + 4 (l % 4) .. +3, and lane c receives rows key0 .. key0 + 3 of
// column col0 + c.  x is rounded to the tile's format; with Split, x is
// carried as the sum of two such terms (hi = r(x), lo = r(x - hi): 16
// significant bits with bf16, 22 with fp16 unless lo underflows
// bits), so that sums with heavy cancellation -- gradient rows whose
// weights sum to zero against keys that share a common component -- keep
// fp32-level accuracy at the cost of a second MFMA.
template <int D, bool Split = false, int CC0 = 0, int CC1 = 2, typename T,
          typename std::enable_if<is_half<T>, int>::type = 0>
__device__ __forceinline__ void tile_t_x_acc(f32x4 (&o)[D / 16], const T* rm,
                                             const f32x4 (&x)[4], int lane) {
  using H = Half<T>;
  using V8 = typename H::v8;
  using V4 = typename H::v4;
  using V2 = typename H::v2;
  using S = typename H::scalar;
  const int g = lane >> 4, l = lane & 15;
  constexpr int rs = Tile<T, D>::kRs;
  // x - hi is exact in fp32; it is formed from the packed hi pair by
  // v_dot2c_f32_bf16 / _f16 (x + hi.lo * -1 + hi.hi * 0), one instruction
  // per value.  The (-1, 0) and (0, -1) pairs are passed in scalar
  // registers: as an inline constant the compiler encodes (-1, 0) as the
  // float -1.0, whose bits the instruction reads as the pair (0, -1)
  // (measured on gfx950).
  const V2 kNegLo = opaque_pair<V2>(H::kNegLoBits);
  const V2 kNegHi = opaque_pair<V2>(H::kNegHiBits);
  for (int cc = CC0; cc < CC1; ++cc) {
    V8 b, bl;
    for (int h = 0; h < 2; ++h)
      for (int r = 0; r < 4; r += 2) {
        const float x0 = x[2 * cc + h][r], x1 = x[2 * cc + h][r + 1];
        const V2 hp = {static_cast<S>(x0), static_cast<S>(x1)};
        b[4 * h + r] = hp[0];
        b[4 * h + r + 1] = hp[1];
        if (Split) {
          bl[4 * h + r] = static_cast<S>(H::dot2(hp, kNegLo, x0));
          bl[4 * h + r + 1] = static_cast<S>(H::dot2(hp, kNegHi, x1));
        }
      }
    // rows 32cc + 4g + 0..3 (low half) and 32cc + 16 + 4g + 0..3 (high
    // half); the chunk swizzle depends on g only (row bits 2-3)
    const T* base = rm + (32 * cc + 4 * g + (l >> 2)) * rs + ((4 * (l & 3)) ^ Tile<T, D>::sw(4 * g));
    V8 a[D / 16];
    for (int db = 0; db < D / 16; ++db) {
      const V4 lo = read_tr16(base + 16 * db);
      const V4 hi = read_tr16(base + 16 * rs + 16 * db);
      a[db] = V8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      o[db] = mfma(a[db], b, o[db]);
    }
    // the lo terms after all hi terms: D/16 independent chains between
    // two products into the same accumulator
    if (Split)
      for (int db = 0; db < D / 16; ++db) o[db] = mfma(a[db], bl, o[db]);
  }
}
// rows_x_frag for two B fragments at once: each A operand is read from LDS
// once and feeds both products (the same operands and order per product as
// rows_x_frag, so each result is bit-identical to it).
// The products start from the accumulators c0, c1 (every block f), zero by
// default.
template <int D, typename T, typename std::enable_if<is_half<T>, int>::type = 0>
__device__ __forceinline__ void rows_x_frag2(f32x4 (&acc0)[4], f32x4 (&acc1)[4], const T* rm,
                                             const RowFrag<T, D>& b0, const RowFrag<T, D>& b1,
                                             int lane, const f32x4 c0 = f32x4{0.f, 0.f, 0.f, 0.f},
                                             const f32x4 c1 = f32x4{0.f, 0.f, 0.f, 0.f}) {
  using V8 = typename Half<T>::v8;
  const int g = lane >> 4, c = lane & 15;
  const T* base = rm + c * Tile<T, D>::kRs + ((8 * g) ^ Tile<T, D>::sw(c));
  for (int f = 0; f < 4; ++f) {
    acc0[f] = c0;
    acc1[f] = c1;
  }
  for (int s = 0; s < D / 32; ++s)
    for (int f = 0; f < 4; ++f) {
      const V8 a = *reinterpret_cast<const V8*>(base + 16 * f * Tile<T, D>::kRs + 32 * s);
      acc0[f] = mfma(a, b0.v[s], acc0[f]);
      acc1[f] = mfma(a, b1.v[s], acc1[f]);
    }
}

// tile_t_x_acc (no Split) for two X / accumulator pairs at once: each
// transposed A read feeds both products (per product, the operands and
// order of tile_t_x_acc).
template <int D, typename T, typename std::enable_if<is_half<T>, int>::type = 0>
__device__ __forceinline__ void tile_t_x_acc2(f32x4 (&o0)[D / 16], f32x4 (&o1)[D / 16], const T* rm,
                                              const f32x4 (&x0)[4], const f32x4 (&x1)[4], int lane) {
  using H = Half<T>;
  using V8 = typename H::v8;
  using V4 = typename H::v4;
  using S = typename H::scalar;
  const int g = lane >> 4, l = lane & 15;
  constexpr int rs = Tile<T, D>::kRs;
  for (int cc = 0; cc < 2; ++cc) {
    V8 b0, b1;
    for (int h = 0; h < 2; ++h)
      for (int r = 0; r < 4; ++r) {
        b0[4 * h + r] = static_cast<S>(x0[2 * cc + h][r]);
        b1[4 * h + r] = static_cast<S>(x1[2 * cc + h][r]);
      }
    const T* base = rm + (32 * cc + 4 * g + (l >> 2)) * rs + ((4 * (l & 3)) ^ Tile<T, D>::sw(4 * g));
    for (int db = 0; db < D / 16; ++db) {
      const V4 lo = read_tr16(base + 16 * db);
      const V4 hi = read_tr16(base + 16 * rs + 16 * db);
      const V8 a = V8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      o0[db] = mfma(a, b0, o0[db]);
      o1[db] = mfma(a, b1, o1[db]);
    }
  }
}

// fp32: `rm` is the row-major tile (exact operands; Split has no effect).
template <int D, bool Split = false, int CC0 = 0, int CC1 = 2>
__device__ __forceinline__ void tile_t_x_acc(f32x4 (&o)[D / 16], const float* rm,
                                             const f32x4 (&x)[4], int lane) {
  const int g = lane >> 4, c = lane & 15;
  for (int f = 2 * CC0; f < 2 * CC1; ++f)
    for (int r = 0; r < 4; ++r) {
      const float* p = rm + (16 * f + 4 * g + r) * Tile<float, D>::kRs + c;
      for (int db = 0; db < D / 16; ++db) o[db] = mfma(p[16 * db], x[f][r], o[db]);
    }
}

// Exponent classes of the per-score powers, chosen from alpha:
//   p = u^(1/(alpha-1)), w = u^((2-alpha)/(alpha-1)) = p^(2-alpha), and the
//   tau recurrence's f'' terms u^((3-2 alpha)/(alpha-1)) (class V).
enum AlphaClass : int { kA15 = 0, kA20 = 1, kA125 = 2, kAGen = 3 };
template <int AC> struct AlphaPow;
template <> struct AlphaPow<kA15> { static constexpr int P = kE2, W = kE1, V = kE0; };
template <> struct AlphaPow<kA20> { static constexpr int P = kE1, W = kE0, V = kEM1; };
template <> struct AlphaPow<kA125> { static constexpr int P = kE4, W = kE3, V = kE2; };
template <> struct AlphaPow<kAGen> { static constexpr int P = kEGen, W = kEGen, V = kEGen; };

__host__ __device__ inline int alpha_class_of(float alpha) {
  const float am1 = alpha - 1.0f;
  const float a = 1.0f / am1;
  const float ew = (2.0f - alpha) / am1;
  if (a == 2.0f && ew == 1.0f) return kA15;
  if (a == 1.0f && ew == 0.0f) return kA20;
  if (a == 4.0f && ew == 3.0f) return kA125;
  return kAGen;
}

}  // namespace asa
