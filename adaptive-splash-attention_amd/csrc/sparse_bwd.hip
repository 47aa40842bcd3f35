// Support-mask backward: dQ, dK, dV over the (row, key) pairs the forward
// weighted with u > 0 (its support masks, asa_state.sup_mask), instead of
// over whole 64 x 64 tiles.
//
// Every backward term lives on a row's support: the weights p,
// w = u^((2-a)/(a-1)) and both gradient modes' ds vanish where u <= 0 (the
// reference backward, adasplashattention.cu:343-535, visits every key and
// multiplies by those zeros).  With a few tens of supported keys per row
// against thousands of visible ones, the dense tile passes spend almost
// all their work on zeros.  These kernels visit only the listed pairs, in
// a fixed order (no atomics: the results are deterministic), and form
// every sum in fp32.  A listed pair's score is recomputed in fp32 from the
// gathered rows (the forward formed it on MFMA; the two differ by rounding
// only, and a pair whose recomputed u is not positive gets zero weight).
//
//   dQ pass    one 256-thread block per query block, one wave per 16 rows,
//              a group of lanes (16 bytes of the head dimension each) per
//              row.  Phase A walks the row's tile masks and lists its keys
//              in LDS; phase B gathers K_j and V_j for the listed keys in
//              lock-step batches: s = q.k_j, w, dp = dO.v_j, and the fp32
//              sums A = sum w dp k_j, B = sum w k_j, sum w, sum w dp give
//              dQ = scale c (A - shift B).  It also writes each row's
//              constants and the tiles' position map (tile (qb, kb) -> its
//              q_list position) for the dK/dV pass.  The lock step runs as
//              long as the longest list among the lane groups, so when the wave's
//              16 rows list at most kFlat keys in all, it counts them first,
//              lists every row whole, and gives lane group g the rows of
//              count ranks g, 15 - g, 16 + g, ... (a snake over the sorted
//              counts): at the headline this cuts the lock-step iterations
//              per wave from 35 to 23 (21 would be perfect balance).  Larger
//              waves list their rows in rounds and chunks of tiles.
//   dK/dV pass one block per slice of a key block, one lane group per key.
//              Phase A walks the key block's query tiles (key-major CSR):
//              the tile's masks give, by one ballot per key, the rows that
//              list the key, appended to the key's list in LDS in row
//              order; phase B gathers q_i and dO_i for the listed rows:
//              dK_j += ds q_i, dV_j += P dO_i.
#include <climits>
#include <type_traits>

#include "asa_device.hpp"
#include "asa_launch.hpp"
#include "asa_tiles.hpp"

namespace asa {
namespace {

constexpr int kThreads = 256;
constexpr int kRowList = 64;   // keys listed per row before a dQ phase B
// rows listed per key before a dK/dV phase B (KPW keys per wave)
template <int KPW> constexpr int key_list() { return KPW > 8 ? 96 : 128; }
// Entries per lane group whose gathers are in flight together: dK/dV and
// dQ.  Measured at the headline (alpha 1.5, bf16, d 64): dK/dV 2 -> 3 -> 4
// gave 204 -> 195 -> 191 us, dQ 3 -> 4 -> 5 gave 144 -> 137 -> 135 us.  The
// alpha 1.25 and general-alpha instantiations keep 2 and 3: at 4 and 5
// their weights' extra registers spill.
template <int AC> constexpr int batch_kv() { return AC == kA15 || AC == kA20 ? 4 : 2; }
template <int AC> constexpr int batch_q() { return AC == kA15 || AC == kA20 ? 5 : 3; }
constexpr int kChunk = 16;     // tiles whose masks are fetched together
constexpr int kFlat = 1024;    // keys a dQ wave lists at once on its balanced path

// 16 bytes of a row: raw (as loaded) and as floats.
template <typename T> struct Chunk;
template <> struct Chunk<u16> {
  static constexpr int E = 8;
  static __device__ __forceinline__ uint4 raw(const u16* p) { return *reinterpret_cast<const uint4*>(p); }
  static __device__ __forceinline__ void unpack(const uint4& v, float (&x)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  static __device__ __forceinline__ void load(const u16* p, float (&x)[8]) { unpack(raw(p), x); }
  // sum_i a_i b_i of two raw chunks: products exact, fp32 sums (v_dot2_f32_bf16)
  static __device__ __forceinline__ float dot(const uint4& a, const uint4& b, float s = 0.0f) {
    s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.x), __builtin_bit_cast(bf16x2, b.x), s, false);
    s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.y), __builtin_bit_cast(bf16x2, b.y), s, false);
    s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.z), __builtin_bit_cast(bf16x2, b.z), s, false);
    s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a.w), __builtin_bit_cast(bf16x2, b.w), s, false);
    return s;
  }
  static __device__ __forceinline__ void store(u16* p, const float (&x)[8]) {
    uint32_t w[4];
    for (int i = 0; i < 4; ++i)
      w[i] = uint32_t(f32_to_bf16(x[2 * i])) | (uint32_t(f32_to_bf16(x[2 * i + 1])) << 16);
    *reinterpret_cast<uint4*>(p) = uint4{w[0], w[1], w[2], w[3]};
  }
};
template <> struct Chunk<h16> {
  static constexpr int E = 8;
  static __device__ __forceinline__ uint4 raw(const h16* p) { return *reinterpret_cast<const uint4*>(p); }
  static __device__ __forceinline__ void unpack(const uint4& v, float (&x)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    for (int i = 0; i < 4; ++i) {
      const f16x2 h = __builtin_bit_cast(f16x2, w[i]);
      x[2 * i] = static_cast<float>(h[0]);
      x[2 * i + 1] = static_cast<float>(h[1]);
    }
  }
  static __device__ __forceinline__ void load(const h16* p, float (&x)[8]) { unpack(raw(p), x); }
  // sum_i a_i b_i of two raw chunks: products exact, fp32 sums (v_dot2_f32_f16)
  static __device__ __forceinline__ float dot(const uint4& a, const uint4& b, float s = 0.0f) {
    s = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a.x), __builtin_bit_cast(f16x2, b.x), s, false);
    s = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a.y), __builtin_bit_cast(f16x2, b.y), s, false);
    s = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a.z), __builtin_bit_cast(f16x2, b.z), s, false);
    s = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a.w), __builtin_bit_cast(f16x2, b.w), s, false);
    return s;
  }
  static __device__ __forceinline__ void store(h16* p, const float (&x)[8]) {
    f16x2 h[4];
    for (int i = 0; i < 4; ++i) h[i] = f16x2{static_cast<h16>(x[2 * i]), static_cast<h16>(x[2 * i + 1])};
    *reinterpret_cast<uint4*>(p) = uint4{__builtin_bit_cast(uint32_t, h[0]), __builtin_bit_cast(uint32_t, h[1]),
                                         __builtin_bit_cast(uint32_t, h[2]), __builtin_bit_cast(uint32_t, h[3])};
  }
};
template <> struct Chunk<float> {
  static constexpr int E = 4;
  static __device__ __forceinline__ uint4 raw(const float* p) { return *reinterpret_cast<const uint4*>(p); }
  static __device__ __forceinline__ void unpack(const uint4& v, float (&x)[4]) {
    x[0] = __uint_as_float(v.x);
    x[1] = __uint_as_float(v.y);
    x[2] = __uint_as_float(v.z);
    x[3] = __uint_as_float(v.w);
  }
  static __device__ __forceinline__ void load(const float* p, float (&x)[4]) { unpack(raw(p), x); }
  static __device__ __forceinline__ float dot(const uint4& a, const uint4& b, float s = 0.0f) {
    s = fmaf(__uint_as_float(a.x), __uint_as_float(b.x), s);
    s = fmaf(__uint_as_float(a.y), __uint_as_float(b.y), s);
    s = fmaf(__uint_as_float(a.z), __uint_as_float(b.z), s);
    return fmaf(__uint_as_float(a.w), __uint_as_float(b.w), s);
  }
  static __device__ __forceinline__ void store(float* p, const float (&x)[4]) {
    *reinterpret_cast<float4*>(p) = float4{x[0], x[1], x[2], x[3]};
  }
};

// 16 bytes at a byte offset from a wave-uniform base: the 32-bit offset
// lets the load take the base from scalar registers (global_load's saddr
// form), one VALU instruction per row address instead of the 64-bit
// multiply-add of an element index.  Offsets stay within one head's rows
// (NK or NQ rows of D elements: far below 2^32 bytes).
template <typename T>
__device__ __forceinline__ uint4 raw_at(const T* base, uint32_t byte_off) {
  return *reinterpret_cast<const uint4*>(reinterpret_cast<const unsigned char*>(base) + byte_off);
}

// Sum over aligned groups of G lanes (G a power of two <= 32) by lane
// exchanges: each step adds a lane's value and its partner's, so every lane
// of a group gets a bit-identical sum.  After the steps within a quad
// (partners i^1, i^2) every lane of a quad holds the quad's sum, so the
// next steps may pair lane i with any lane of the other quad (octet) of its
// octet (16 lanes): i^7 and i^15 are single DPP mirrors, which the compiler
// fuses into the adds.
template <int G>
__device__ __forceinline__ float group_lanes_sum(float v) {
  auto x = [](float a, auto ctrl) {
    return __uint_as_float(dpp_mov<decltype(ctrl)::value>(__float_as_uint(a)));
  };
  if constexpr (G >= 2) v += x(v, std::integral_constant<int, 0xB1>{});   // i^1
  if constexpr (G >= 4) v += x(v, std::integral_constant<int, 0x4E>{});   // i^2
  if constexpr (G >= 8) v += x(v, std::integral_constant<int, 0x141>{});  // i^7
  if constexpr (G >= 16) v += x(v, std::integral_constant<int, 0x140>{}); // i^15
  if constexpr (G >= 32) v += __uint_as_float(lane_xor<16>(__float_as_uint(v)));
  return v;
}

// Lane i <- lane 4 (i / 4) + J: word J of a quad to all its lanes.
template <int J>
__device__ __forceinline__ float quad_bcast(float v) {
  return __uint_as_float(dpp_mov<J | (J << 2) | (J << 4) | (J << 6)>(__float_as_uint(v)));
}

// Maximum of a lane-group-uniform value over the wave's groups of G lanes.
template <int G>
__device__ __forceinline__ int groups_max(int v) {
  for (int o = G; o < kWave; o <<= 1) v = max(v, __shfl_xor(v, o, kWave));
  return v;
}

// ---------------------------------------------------------------------------
// dQ
// ---------------------------------------------------------------------------
template <typename T, int D, int AC, bool REF, bool FULL>
__global__ __launch_bounds__(kThreads, 4) void dq_sparse_kernel(BackwardParams p) {
  constexpr int kBatchQ = batch_q<AC>();
  using C = Chunk<T>;
  constexpr int E = C::E;
  constexpr int LPR = D / E;          // lanes per row (16 bytes each)
  constexpr int RPR = kWave / LPR;    // rows per round of a wave (lane groups)
  constexpr int NR = 16 / RPR;        // rows per lane group
  constexpr int PW = AlphaPow<AC>::W;
  __shared__ int s_flat[4][kFlat];           // balanced path: the wave's rows' lists
  __shared__ int s_rn[4][16];                // listed keys per row of the wave
  __shared__ int s_off[4][16];               // start of each row's list in s_flat
  __shared__ int s_rank[4][16];              // rows in descending count order
  __shared__ float s_cfac[4][16];            // per row: c ((norm + eps)^(alpha - 2), or delta's)
  __shared__ float s_shift[4][16];           //   the reference mode's shift (delta)
  __shared__ float s_norm[4][16];            //   sum p
  __shared__ float s_tau[4][16];             //   tau
  __shared__ int s_list[4][RPR][kRowList];   // chunked path
  __shared__ uint64_t s_mw[4][kChunk][16];   // mask words of a chunk of tiles: [tile][row]
  __shared__ int s_kb[4][kChunk];            // first key of each tile
  const int NQ = p.d.NQ, nQB = p.d.nQB, nKB = p.d.nKB;
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  // head by head (xcd_task): the pass's work per block hardly depends on
  // the query block, and two heads' K/V rows at a time stay in the L2
  // (heaviest-first over all the XCD's heads measured the same time at
  // twice the HBM traffic)
  const int task = xcd_task(blockIdx.x, nQB * p.d.BH);
  const int qb = nQB - 1 - task % nQB, bh = task / nQB;
  const int sub = lane % LPR, grp = lane / LPR;
  // The lane's 16 bytes of a row: inside the head dimension (colok), or a
  // lane past hd, which gathers the row's first chunk instead (an address
  // inside the row) and drops its partial dot products; its own sums are
  // never stored.  FULL: hd = D and rows of D elements (compile-time
  // strides).
  const bool colok = FULL || sub * E < p.d.hd;
  const uint32_t lcol = uint32_t(colok ? sub * E : 0) * uint32_t(sizeof(T));  // bytes
  const uint32_t ksb = uint32_t(FULL ? D : p.lk.sn) * uint32_t(sizeof(T));   // row strides, bytes
  const uint32_t vsb = uint32_t(FULL ? D : p.lv.sn) * uint32_t(sizeof(T));

  const float alpha = p.d.alpha, am1 = alpha - 1.0f, ew = (2.0f - alpha) / am1;
  const float scale = p.d.scale;
  const size_t rows = size_t(p.d.BH) * NQ;
  const T* Kb = static_cast<const T*>(p.k) + head_at(p.lk, bh, p.d.H);
  const T* Vb = static_cast<const T*>(p.v) + head_at(p.lv, bh, p.d.H);
  const T* Qh = static_cast<const T*>(p.q) + head_at(p.lq, bh, p.d.H);
  const T* dOh = static_cast<const T*>(p.dout) + head_at(p.ldo, bh, p.d.H);
  const int32_t* qp = p.q_ptr + size_t(bh) * (nQB + 1);
  const int32_t* ql = p.q_list + size_t(bh) * nQB * nKB;
  const int e0 = qp[qb], e1 = qp[qb + 1];
  // Position map for the dK/dV pass (which runs after this one):
  // posmap[bh][qb * nKB + kb] = the head's q_list position of tile (qb, kb).
  {
    int32_t* pm = p.posmap + size_t(bh) * nQB * nKB + size_t(qb) * nKB;
    for (int e = e0 + t; e < e1; e += kThreads) pm[ql[e]] = e;
  }
  // the wave's masks of tile e: row c's word at + e * 256 + 4 c
  const uint16_t* wmask = p.sup.mask + size_t(bh) * nQB * nKB * 256 + w * 64;
  auto weight = [&](float v) {
    float wv = pow_clipped<PW>(v, ew);
    if constexpr (REF) wv = v > kEps ? wv : 0.0f;  // the reference's u > EPS
    return wv;
  };

  // The rows' constants, one lane per row of the wave, into LDS: the lane
  // groups start and finish their rows at different steps, so per-row
  // loads (and the double pow of (norm + eps)^(alpha - 2)) would run one
  // after another, each a full memory latency.
  if (lane < 16) {
    const int qrow = qb * kBlock + 16 * w + lane;
    float c = 0.0f, sh = 0.0f, nrm = 0.0f, ta = 0.0f;
    if (qrow < NQ) {
      const size_t rw = size_t(bh) * NQ + qrow;
      nrm = p.norms[rw];
      ta = p.taus[rw];
      if constexpr (REF) {
        c = p.delta[rows + rw];
        sh = p.delta[rw];
      } else {
        c = static_cast<float>(pow(static_cast<double>(nrm + kEps), static_cast<double>(alpha) - 2.0));
      }
    }
    s_cfac[w][lane] = c;
    s_shift[w][lane] = sh;
    s_norm[w][lane] = nrm;
    s_tau[w][lane] = ta;
  }

  // One row's state: its q and dO chunks, clipping, and the fp32 sums
  // A = sum w dp k_j, B = sum w k_j, sum w, sum w dp.
  int rr = 0;  // row within the wave
  bool ok = false;
  size_t row = 0;
  uint4 qv{0u, 0u, 0u, 0u}, dO{0u, 0u, 0u, 0u};
  uint4 nqv{0u, 0u, 0u, 0u}, ndO{0u, 0u, 0u, 0u};  // the next row's, loaded ahead
  ClippedU clip(am1, scale, 0.0f, false);
  float a1[E], a2[E];
  float sw = 0.0f, swdp = 0.0f;
  // q and dO chunks of row r of the wave, for a later start_row(r)
  auto prefetch = [&](int r) {
    const int qrow = qb * kBlock + 16 * w + r;
    nqv = uint4{0u, 0u, 0u, 0u};
    ndO = uint4{0u, 0u, 0u, 0u};
    if (qrow < NQ && colok) {
      nqv = C::raw(Qh + size_t(qrow) * (FULL ? D : p.lq.sn) + sub * E);
      ndO = C::raw(dOh + size_t(qrow) * (FULL ? D : p.ldo.sn) + sub * E);
    }
  };
  auto start_row = [&](int r) {  // after prefetch(r)
    rr = r;
    const int qrow = qb * kBlock + 16 * w + rr;
    ok = qrow < NQ;
    row = size_t(bh) * NQ + (ok ? qrow : 0);
    qv = nqv;
    dO = ndO;
    clip = ClippedU(am1, scale, s_tau[w][rr], ok);
    for (int x = 0; x < E; ++x) a1[x] = a2[x] = 0.0f;
    sw = swdp = 0.0f;
  };
  // entries q .. q + kBatchQ - 1 (those below n) of a key list, in lock step
  // with the other lane groups: gathers first, then the sums
  auto step = [&](const int* lst, int q, int n) {
    int key[kBatchQ];
    bool val[kBatchQ];
    uint4 kraw[kBatchQ], vraw[kBatchQ];
    for (int u = 0; u < kBatchQ; ++u) {
      val[u] = q + u < n;
      key[u] = val[u] ? lst[q + u] : 0;
    }
    for (int u = 0; u < kBatchQ; ++u) {
      kraw[u] = raw_at(Kb, uint32_t(key[u]) * ksb + lcol);
      vraw[u] = raw_at(Vb, uint32_t(key[u]) * vsb + lcol);
    }
    for (int u = 0; u < kBatchQ; ++u) {
      float ps = C::dot(qv, kraw[u]), pd = C::dot(dO, vraw[u]);
      if constexpr (!FULL) {
        ps = colok ? ps : 0.0f;
        pd = colok ? pd : 0.0f;
      }
      float s = group_lanes_sum<LPR>(ps);
      float dp = group_lanes_sum<LPR>(pd);
      // complete here: sunk into the branch below, the last step's DPP
      // move no longer fused into its add
      asm volatile("" : "+v"(s), "+v"(dp));
      if (val[u]) {
        float kr[E];
        C::unpack(kraw[u], kr);
        const float wv = weight(clip(s));
        sw += wv;
        const float wdp = wv * dp;
        swdp += wdp;
        for (int x = 0; x < E; ++x) {
          a1[x] = fmaf(wdp, kr[x], a1[x]);
          a2[x] = fmaf(wv, kr[x], a2[x]);
        }
      }
    }
  };
  // dQ and the row's record for the dK/dV pass
  auto finish_row = [&]() {
    if (!ok) return;
    const float norm = s_norm[w][rr];
    float cfac, shift;
    if constexpr (REF) {
      cfac = s_cfac[w][rr];
      shift = s_shift[w][rr];
    } else {
      cfac = s_cfac[w][rr];
      shift = sw > 0.0f ? swdp / sw : 0.0f;
      if (!finite(shift)) shift = 0.0f;
    }
    // dQ_i = scale c (A - shift B) = scale sum_j c w_j (dp_j - shift) k_j
    const float cs = scale * cfac;
    float o[E];
    for (int x = 0; x < E; ++x) {
      const float v = cs * fmaf(-shift, a2[x], a1[x]);
      o[x] = finite(v) ? v : 0.0f;
    }
    if (colok)
      C::store(static_cast<T*>(p.dq) + head_at(p.ldq, bh, p.d.H) +
                   size_t(qb * kBlock + 16 * w + rr) * (FULL ? D : p.ldq.sn) + sub * E,
               o);
    if (sub == 0)
      p.rowrec[row] = RowRec{clip.nt, 1.0f / (norm + kEps), cfac, -cfac * shift};
  };

  // ---- count the keys each row of the wave lists.  A row's four masks of
  // a tile are one 8-byte word (bit 16 g + 4 f + r <-> key 16 f + 4 g + r);
  // lane (row c16, slot g4) reads the words of tiles e0 + 4 u + g4, eight
  // loads (32 tiles) in flight together.  The first 32 tiles' words stay in
  // registers for the listing below.
  const int c16 = lane & 15, g4 = lane >> 4;
  const uint64_t* lw = reinterpret_cast<const uint64_t*>(wmask + 4 * c16);  // tile e at + e * 64
  constexpr int kWords = 8;  // words per lane per batch of 4 * kWords tiles
  auto load_words = [&](int e8, uint64_t (&wd)[kWords], int (&kbs)[kWords]) {
    for (int u = 0; u < kWords; ++u) {
      const int e = e8 + 4 * u + g4;
      wd[u] = e < e1 ? lw[size_t(e) * 64] : 0ull;
      kbs[u] = e < e1 ? ql[e] * kBlock : 0;
    }
  };
  uint64_t wd0[kWords];
  int kb0[kWords];
  load_words(e0, wd0, kb0);
  int nl = 0;
  for (int u = 0; u < kWords; ++u) nl += __builtin_popcountll(wd0[u]);
  for (int e8 = e0 + 4 * kWords; e8 < e1; e8 += 4 * kWords) {
    uint64_t wd[kWords];
    int kbs[kWords];
    load_words(e8, wd, kbs);
    for (int u = 0; u < kWords; ++u) nl += __builtin_popcountll(wd[u]);
  }
  const int rn = int(group_reduce_bits(uint32_t(nl), [](uint32_t x, uint32_t y) { return x + y; }));
  if (lane < 16) s_rn[w][lane] = rn;
  int cnt16[16];
  for (int i = 0; i < 16; ++i) cnt16[i] = s_rn[w][i];
  int total = 0, off = 0, rank = 0;
  for (int i = 0; i < 16; ++i) {
    total += cnt16[i];
    off += i < c16 ? cnt16[i] : 0;
    rank += (cnt16[i] > rn || (cnt16[i] == rn && i < c16)) ? 1 : 0;
  }

  if (lane < 16) s_rank[w][rank] = lane;  // rows by descending count
  if (total <= kFlat) {  // wave-uniform
    // ---- balanced path.  Every row's whole list in s_flat (tile order,
    // then bit 16 g + 4 f + r: the chunked path's order); the lane groups
    // take the rows in a snake over the descending counts, so each group's
    // total is close to the mean and the lock-step loop runs near its
    // length.
    if (lane < 16) s_off[w][lane] = off;
    // the first row's q and dO load while the lists are built
    prefetch(s_rank[w][grp]);
    int base = off;
    auto list_words = [&](int e8, const uint64_t (&wd)[kWords], const int (&kbs)[kWords]) {
      for (int u = 0; u < kWords && e8 + 4 * u < e1; ++u) {
        uint64_t m = wd[u];
        const uint32_t n = uint32_t(__builtin_popcountll(m));
        // prefix of the counts over the row's four tiles g4 = 0..3 (lanes c16 + 16 g4)
        const auto pa = __builtin_amdgcn_permlane16_swap(n, n, false, false);
        const uint32_t pair = pa[0] + pa[1];
        const auto pb = __builtin_amdgcn_permlane32_swap(pair, pair, false, false);
        const uint32_t tot = pb[0] + pb[1];
        int pos = base + int(((g4 & 1) ? pair - n : 0u) + ((g4 & 2) ? tot - pair : 0u));
        const int kb = kbs[u];
        while (m) {
          const int b = __builtin_ctzll(m);
          m &= m - 1;
          // bit 16 g + 4 f + r -> key 16 f + 4 g + r
          s_flat[w][pos++] = kb + 16 * ((b >> 2) & 3) + 4 * (b >> 4) + (b & 3);
        }
        base += int(tot);
      }
    };
    list_words(e0, wd0, kb0);
    for (int e8 = e0 + 4 * kWords; e8 < e1; e8 += 4 * kWords) {
      uint64_t wd[kWords];
      int kbs[kWords];
      load_words(e8, wd, kbs);
      list_words(e8, wd, kbs);
    }
    auto rank_row = [&](int j) { return s_rank[w][j * RPR + ((j & 1) ? RPR - 1 - grp : grp)]; };
    int j = 0;
    start_row(rank_row(0));  // prefetched before the listing
    if (NR > 1) prefetch(rank_row(1));
    int pos = s_off[w][rr], end = pos + s_rn[w][rr];
    for (;;) {
      while (j < NR && pos >= end) {  // group-uniform
        finish_row();
        if (++j < NR) {
          start_row(rank_row(j));
          if (j + 1 < NR) prefetch(rank_row(j + 1));
          pos = s_off[w][rr];
          end = pos + s_rn[w][rr];
        }
      }
      if (!__any(j < NR)) break;
      if (j < NR) {
        step(s_flat[w], pos, end);
        pos += kBatchQ;
      }
    }
    return;
  }

  // ---- chunked path (a wave with more than kFlat listed keys): rows in
  // rounds of RPR, each row's keys listed kRowList at a time per chunk of
  // tiles and drained in lock step.  A round takes RPR rows of consecutive
  // count ranks (the lock step lasts as long as its longest list).
  int* list = s_list[w][grp];
  for (int r0 = 0; r0 < 16; r0 += RPR) {
    prefetch(s_rank[w][r0 + grp]);
    start_row(s_rank[w][r0 + grp]);
    auto drain = [&](int cnt) {
      const int nmax = groups_max<LPR>(cnt);
      for (int q = 0; q < nmax; q += kBatchQ) step(list, q, cnt);
    };
    for (int c0 = e0; c0 < e1; c0 += kChunk) {
      const int nt = min(kChunk, e1 - c0);
      // the chunk's mask words: 4 tiles (16 rows each) per wave load
      for (int s4 = 0; s4 < kChunk; s4 += 4) {
        const int tt = s4 + (lane >> 4);
        if (tt < nt)
          s_mw[w][tt][lane & 15] =
              *reinterpret_cast<const uint64_t*>(wmask + size_t(c0 + tt) * 256 + 4 * (lane & 15));
      }
      if (lane < nt) s_kb[w][lane] = ql[c0 + lane] * kBlock;
      // phase A over the chunk: list up to kRowList keys per row (tile
      // order, then g, f, r), drain, continue where the list filled up
      int tt = 0, kbase = 0;
      uint64_t bits = 0;
      bool more = ok;
      while (__any(more)) {
        int cnt = 0;
        while (more && cnt < kRowList) {
          if (bits == 0) {
            if (tt >= nt) {
              more = false;
              break;
            }
            bits = s_mw[w][tt][rr];
            kbase = s_kb[w][tt];
            ++tt;
            continue;
          }
          const int b = __builtin_ctzll(bits);
          bits &= bits - 1;
          // bit 16 g + 4 f + r -> key 16 f + 4 g + r
          if (sub == 0) list[cnt] = kbase + 16 * ((b >> 2) & 3) + 4 * (b >> 4) + (b & 3);
          ++cnt;
        }
        drain(cnt);
      }
    }
    finish_row();
  }
}

// ---------------------------------------------------------------------------
// dK, dV
// ---------------------------------------------------------------------------
// Each lane holds kKeyChunks 16-byte chunks of a key's rows.  Two chunks
// (fewer lanes per key, 16 keys per wave at d = 64) spread a pair's fixed
// work over more of the head dimension but lock-step more keys of unequal
// list lengths and hold fewer gathers in flight: at the headline shape the
// dK/dV pass took 330-400 us with two chunks against 271 us with one.
constexpr int kKeyChunks = 1;
template <typename T, int D> constexpr int key_lanes() { return D / (kKeyChunks * Chunk<T>::E); }
template <typename T, int D> constexpr int keys_per_block() { return 4 * (kWave / key_lanes<T, D>()); }

template <typename T, int D, int AC, bool REF, bool FULL>
__global__ __launch_bounds__(kThreads, 4) void dkdv_sparse_kernel(BackwardParams p) {
  constexpr int kBatch = batch_kv<AC>();
  using C = Chunk<T>;
  constexpr int E = C::E;
  constexpr int NC = kKeyChunks;      // 16-byte chunks per lane
  constexpr int EL = NC * E;          // elements per lane
  constexpr int LPR = key_lanes<T, D>();  // lanes per key
  constexpr int KPW = kWave / LPR;    // keys per wave
  constexpr int KPB = 4 * KPW;        // keys per block
  constexpr int SLICES = kBlock / KPB;
  constexpr int PP = AlphaPow<AC>::P, PW = AlphaPow<AC>::W;
  constexpr int kKeyList = key_list<KPW>();
  // phase A: tiles whose mask words are loaded together, and the events
  // held per wave (one group's worth beyond a partly listed chunk)
  constexpr int kTileGroup = KPW > 8 ? 4 : 8;
  constexpr int kEvents = kWave + kTileGroup * kWave;
  // the waves' key lists, [wave][key][kKeyList], then one dump slot per
  // lane for the phase A stores of lanes with nothing to list
  __shared__ int s_lists[4 * KPW * kKeyList + 4 * kWave];
  __shared__ int s_cnt[4][KPW];
  __shared__ int s_rank[4][KPW];  // phase B: the wave's keys by list length
  // phase B: the own sums of the shorter lists' groups while they sum
  // their partners' tails, [wave][pair][lane of the group][dK, dV]
  __shared__ float4 s_save[4][KPW / 2][LPR][2 * EL / 4];
  using Bits = std::conditional_t<(KPW > 8), uint16_t, uint8_t>;
  __shared__ int s_evr[4][kEvents];   // events: a row listing some of the wave's keys
  __shared__ Bits s_evm[4][kEvents];  //   and its key bits (bit k <-> key jb + k)
  const int NQ = p.d.NQ, NK = p.d.NK, nQB = p.d.nQB, nKB = p.d.nKB;
  const int t = threadIdx.x, lane = t & 63;
  const int w = __builtin_amdgcn_readfirstlane(t >> 6);  // wave-uniform: w, jb and b0 in scalar registers
  // Block order: the XCD's heads (contiguous, as xcd_task deals them) go
  // in pairs, and within a pair key block by key block, so the heavy first
  // key blocks of both heads start first (under the causal mask key block
  // kb is listed by the rows of every query block >= kb: the first blocks
  // carry several times the mean work) while two heads' rows share the L2.
  int slice, kb, bh;
  {
    const int BH = p.d.BH;
    if (BH % kXcds == 0) {
      const int x = blockIdx.x % kXcds, jj = blockIdx.x / kXcds, hpx = BH / kXcds;
      const int hg = hpx % 2 == 0 ? 2 : 1;  // heads per group
      const int per = hg * nKB * SLICES;    // blocks per group
      const int r = jj % per, rr = r % (hg * SLICES);
      kb = r / (hg * SLICES);
      bh = x * hpx + (jj / per) * hg + rr / SLICES;
      slice = rr % SLICES;
    } else {
      const int task = xcd_task(blockIdx.x, nKB * SLICES * BH);
      slice = task % SLICES;
      kb = (task / SLICES) % nKB;
      bh = task / (SLICES * nKB);
    }
  }
  const int sub = lane % LPR, grp = lane / LPR;
  const int jb = slice * KPB + w * KPW;  // first key (within the block) of this wave
  const int j = kb * kBlock + jb + grp;  // this group's key
  const bool jok = j < NK;

  const float alpha = p.d.alpha, am1 = alpha - 1.0f;
  const float a = 1.0f / am1, ew = (2.0f - alpha) / am1;
  const float cu = am1 * p.d.scale;  // ClippedU's c
  // the score clamp [-10, 10] on the raw dot product (scale > 0); NaN dots
  // give smin, as the clamp gives NaN -> -10
  const float smax = 10.0f / p.d.scale, smin = -smax;
  const size_t rbase = size_t(bh) * NQ;
  const int H = p.d.H;
  const T* Qb = static_cast<const T*>(p.q) + head_at(p.lq, bh, H);
  const T* dOb = static_cast<const T*>(p.dout) + head_at(p.ldo, bh, H);
  // Chunk c of the lane's rows: inside the head dimension (colok[c]), or
  // past hd, where the lane gathers the row's first chunk instead (an
  // address inside the row) and drops that chunk's partial dot products;
  // its sums there are never stored.  FULL: hd = D, rows of D elements.
  bool colok[NC];
  uint32_t lcol[NC];  // bytes
  for (int c = 0; c < NC; ++c) {
    colok[c] = FULL || sub * EL + c * E < p.d.hd;
    lcol[c] = uint32_t(colok[c] ? sub * EL + c * E : 0) * uint32_t(sizeof(T));
  }
  const uint32_t qsb = uint32_t(FULL ? D : p.lq.sn) * uint32_t(sizeof(T));  // row strides, bytes
  const uint32_t gsb = uint32_t(FULL ? D : p.ldo.sn) * uint32_t(sizeof(T));
  const size_t ksn = FULL ? size_t(D) : size_t(p.lk.sn), vsn = FULL ? size_t(D) : size_t(p.lv.sn);
  const RowRec* rec = p.rowrec + rbase;
  const int32_t* kp = p.k_ptr + size_t(bh) * (nKB + 1);
  const int32_t* kl = p.k_list + size_t(bh) * nKB * nQB;
  const uint16_t* hmask = p.sup.mask + size_t(bh) * nQB * nKB * 256;

  uint4 kv[NC], vv[NC];  // raw 16-byte chunks of the key's rows
  const T* const Kh = static_cast<const T*>(p.k) + head_at(p.lk, bh, H);
  const T* const Vh = static_cast<const T*>(p.v) + head_at(p.lv, bh, H);
  for (int c = 0; c < NC; ++c) {
    kv[c] = uint4{0u, 0u, 0u, 0u};
    vv[c] = uint4{0u, 0u, 0u, 0u};
    if (jok && colok[c]) {
      kv[c] = C::raw(Kh + size_t(j) * ksn + sub * EL + c * E);
      vv[c] = C::raw(Vh + size_t(j) * vsn + sub * EL + c * E);
    }
  }
  float dk[EL], dv[EL];
  for (int x = 0; x < EL; ++x) dk[x] = dv[x] = 0.0f;

  const int* mylist = s_lists + (w * KPW + grp) * kKeyList;
  // chunk c of row `key` (jb + key of the block) of K or V (rows sn
  // elements apart), zero past NK and past hd (returned by value: arrays
  // passed by reference here kept the accumulators out of registers)
  auto key_chunk = [&](const T* base, size_t sn, int key, int c) -> uint4 {
    const int jj = kb * kBlock + jb + key;
    if (jj >= NK || !colok[c]) return uint4{0u, 0u, 0u, 0u};
    return C::raw(base + size_t(jj) * sn + sub * EL + c * E);
  };
  // phase B: the wave's KPW key lists, kBatch entries at a time in every
  // lane group.  The keys pair up by list length (longest with shortest,
  // second with second-shortest, ...): the shorter list's group, after its
  // own rows, takes the tail of its partner's list, so that both end near
  // the pair's mean.  Its sums for the tail reach the partner through LDS
  // after the loop and are added to the head's (a fixed order).  The lists
  // are heavy-tailed (a key with a large norm scores high for many rows),
  // and with one group per list the loop ran as long as the longest.
  auto drain = [&]() __attribute__((always_inline)) {
    const int cnt = s_cnt[w][grp];
    int rank = 0;  // by list length, descending; ties by key
    for (int k = 0; k < KPW; ++k) {
      const int ck = s_cnt[w][k];
      rank += (ck > cnt || (ck == cnt && k < grp)) ? 1 : 0;
    }
    if (sub == 0) s_rank[w][rank] = grp;
    const bool big = rank < KPW / 2;
    const int partner = s_rank[w][KPW - 1 - rank];
    const int pcnt = s_cnt[w][partner];
    const int cb = big ? cnt : pcnt, cs = big ? pcnt : cnt;
    const int pcs = (cs + kBatch - 1) / kBatch * kBatch;  // the shorter list in whole batches
    // the longer list's head: whole batches, about half of the pair's work
    const int ob = min(cb, ((cb + pcs + kBatch) / (2 * kBatch)) * kBatch);
    const int hb = cb - ob;                                // its tail, summed by the shorter's group
    const int tail_at = big || hb == 0 ? INT_MAX : pcs;   // step where this group turns to the tail
    const int nmax = groups_max<LPR>(big ? ob : pcs + hb);
    const int* lst = mylist;
    int lim = big ? ob : cs;  // entries below this step position are valid
    int off = 0;              // list index = step position - off
    for (int q = 0; q < nmax; q += kBatch) {
      if (q == tail_at) {  // lane-group uniform
        float4* sv4 = s_save[w][KPW - 1 - rank][sub];
        for (int x = 0; x < EL; x += 4) {
          sv4[x / 4] = float4{dk[x], dk[x + 1], dk[x + 2], dk[x + 3]};
          sv4[EL / 4 + x / 4] = float4{dv[x], dv[x + 1], dv[x + 2], dv[x + 3]};
        }
        for (int x = 0; x < EL; ++x) dk[x] = dv[x] = 0.0f;
        for (int c = 0; c < NC; ++c) {
          kv[c] = key_chunk(Kh, ksn, partner, c);
          vv[c] = key_chunk(Vh, vsn, partner, c);
        }
        lst = s_lists + (w * KPW + partner) * kKeyList;
        off = pcs - ob;
        lim = pcs + hb;
      }
      int r[kBatch];
      bool val[kBatch];
      uint4 qraw[kBatch][NC], graw[kBatch][NC];
      float rw[kBatch];  // word sub % 4 of the row's record (a 4-byte load: a
                         // 16-byte one per lane costs the address unit 4x)
      for (int u = 0; u < kBatch; ++u) {
        val[u] = q + u < lim;
        r[u] = val[u] ? lst[q + u - off] : 0;
      }
      for (int u = 0; u < kBatch; ++u) {
        for (int c = 0; c < NC; ++c) {
          qraw[u][c] = raw_at(Qb, uint32_t(r[u]) * qsb + lcol[c]);
          graw[u][c] = raw_at(dOb, uint32_t(r[u]) * gsb + lcol[c]);
        }
        rw[u] = *reinterpret_cast<const float*>(reinterpret_cast<const unsigned char*>(rec) +
                                                (uint32_t(r[u]) * uint32_t(sizeof(RowRec)) + 4u * (sub & 3)));
      }
      for (int u = 0; u < kBatch; ++u) {
        float s = 0.0f, dp = 0.0f;
        for (int c = 0; c < NC; ++c) {
          if (FULL || colok[c]) {
            s = C::dot(qraw[u][c], kv[c], s);
            dp = C::dot(graw[u][c], vv[c], dp);
          }
        }
        s = group_lanes_sum<LPR>(s);
        dp = group_lanes_sum<LPR>(dp);
        // complete here: sunk into the branch below, the last step's DPP
        // move no longer fused into its add
        asm volatile("" : "+v"(s), "+v"(dp));
        // the record's words to every lane of each quad (DPP broadcasts)
        const RowRec rc{quad_bcast<0>(rw[u]), quad_bcast<1>(rw[u]), quad_bcast<2>(rw[u]),
                        quad_bcast<3>(rw[u])};
        if (val[u]) {
          float qr[EL], gr[EL];
          for (int c = 0; c < NC; ++c) {
            float x8[E];
            C::unpack(qraw[u][c], x8);
            for (int x = 0; x < E; ++x) qr[c * E + x] = x8[x];
            C::unpack(graw[u][c], x8);
            for (int x = 0; x < E; ++x) gr[c * E + x] = x8[x];
          }
          // max(u, 0) of a valid row (the lists hold valid rows only) with
          // the score clamp on s itself: three instructions instead of
          // ClippedU's bounds per pair (u differs from ClippedU's only for
          // clamped scores, by the rounding of 10 / scale)
          const float v = fmaxf(fmaf(cu, __builtin_amdgcn_fmed3f(s, smin, smax), rc.nt), 0.0f);
          const float pn = pow_clipped<PP>(v, a) * rc.invn;
          float wv = pow_clipped<PW>(v, ew);
          if constexpr (REF) wv = v > kEps ? wv : 0.0f;  // the reference's u > EPS
          float ds = wv * fmaf(rc.c, dp, rc.cs);
          ds = finite(ds) ? ds : 0.0f;
          for (int x = 0; x < EL; ++x) {
            dk[x] = fmaf(ds, qr[x], dk[x]);
            dv[x] = fmaf(pn, gr[x], dv[x]);
          }
        }
      }
    }
    // The tails' sums, through the wave's (now read) list region: slot
    // rank of the longer list, LPR lanes x 2 EL floats (at most 8 d bytes
    // per pair; the region holds KPW * kKeyList ints >= (KPW / 2) * 2 d).
    float4* slots = reinterpret_cast<float4*>(s_lists + w * KPW * kKeyList);
    constexpr int F4 = 2 * EL / 4;  // float4s per lane
    static_assert(KPW * kKeyList >= (KPW / 2) * LPR * 2 * EL, "tail slots must fit the list region");
    if (tail_at != INT_MAX) {  // the shorter list's group: hand over, take its own sums back
      float4* sl = slots + ((KPW - 1 - rank) * LPR + sub) * F4;
      for (int x = 0; x < EL; x += 4) {
        sl[x / 4] = float4{dk[x], dk[x + 1], dk[x + 2], dk[x + 3]};
        sl[EL / 4 + x / 4] = float4{dv[x], dv[x + 1], dv[x + 2], dv[x + 3]};
      }
      const float4* sv4 = s_save[w][KPW - 1 - rank][sub];
      for (int x = 0; x < EL; x += 4) {
        const float4 a4 = sv4[x / 4], b4 = sv4[EL / 4 + x / 4];
        dk[x] = a4.x; dk[x + 1] = a4.y; dk[x + 2] = a4.z; dk[x + 3] = a4.w;
        dv[x] = b4.x; dv[x + 1] = b4.y; dv[x + 2] = b4.z; dv[x + 3] = b4.w;
      }
      for (int c = 0; c < NC; ++c) {
        kv[c] = key_chunk(Kh, ksn, grp, c);
        vv[c] = key_chunk(Vh, vsn, grp, c);
      }
    }
    if (big && hb > 0) {  // the longer list's group: add its tail's sums
      const float4* sl = slots + (rank * LPR + sub) * F4;
      for (int x = 0; x < EL; x += 4) {
        const float4 a4 = sl[x / 4], b4 = sl[EL / 4 + x / 4];
        dk[x] += a4.x; dk[x + 1] += a4.y; dk[x + 2] += a4.z; dk[x + 3] += a4.w;
        dv[x] += b4.x; dv[x + 1] += b4.y; dv[x + 2] += b4.z; dv[x + 3] += b4.w;
      }
    }
  };

  // phase A over the key block's query tiles (ascending query blocks).
  // Lane L <-> row L of a tile.  The tiles' query blocks and q_list
  // positions are fetched for up to 64 tiles at once (one lane each); the
  // mask words then come kTileGroup tiles at a time, the next group's
  // loads in flight while the current group is listed.  A tile's rows that
  // list any of the wave's keys (a few of its 64) become events in LDS: the
  // row and its KPW key bits.  Once a group leaves fewer than a group's
  // worth of free event slots, one lane per event appends the rows to the
  // keys' lists (one ballot per key and 64 events), so the per-key ballots
  // run per 64 events instead of per tile, and a drain can start only
  // between groups.  Events and lists keep ascending row order.  The list
  // lengths are wave-uniform (scalar registers); drain() reads them from
  // s_cnt.
  int cnt[KPW];
  for (int k = 0; k < KPW; ++k) cnt[k] = 0;
  auto drain_lists = [&]() __attribute__((always_inline)) {
    for (int k = 0; k < KPW; ++k)
      if (lane == k) s_cnt[w][k] = cnt[k];
    drain();
    for (int k = 0; k < KPW; ++k) cnt[k] = 0;
  };
  const int dump = 4 * KPW * kKeyList + w * kWave + lane;
  int nev = 0;  // events held (wave-uniform), at most kEvents
  auto list_events = [&]() __attribute__((always_inline)) {
    for (int c0 = 0; c0 < nev; c0 += kWave) {
      const bool live = c0 + lane < nev;
      const int row = live ? s_evr[w][c0 + lane] : 0;
      const uint32_t bits = live ? uint32_t(s_evm[w][c0 + lane]) : 0u;
      uint64_t col[KPW];
      bool room = true;  // for these events in every list of the wave, else drain first
      for (int k = 0; k < KPW; ++k) {
        col[k] = __ballot(((bits >> k) & 1u) != 0);
        room = room && cnt[k] + __builtin_popcountll(col[k]) <= kKeyList;
      }
      if (!room) drain_lists();
      // Every lane stores: a lane whose event does not list the key writes
      // its dump slot instead of branching around the store.
      for (int k = 0; k < KPW; ++k) {
        const bool on = ((bits >> k) & 1u) != 0;
        const int at = (w * KPW + k) * kKeyList + cnt[k] + lane_rank(col[k]);
        s_lists[on ? at : dump] = row;
        cnt[k] += __builtin_popcountll(col[k]);
      }
    }
    nev = 0;
  };
  const int32_t* pm = p.posmap + size_t(bh) * nQB * nKB + kb;  // tile (qb, kb) at + qb * nKB
  const int x0 = kp[kb], x1 = kp[kb + 1];
  static_assert(KPW == 2 || KPW == 4 || KPW == 8 || KPW == 16, "a wave's keys: 2, 4, 8 or 16");
  // The wave's keys jb .. jb + KPW - 1 in row L's masks (bit 16 g + 4 f + r
  // of its 64-bit word <-> key 16 f + 4 g + r).  Up to eight keys lie in
  // masks g and g + 1 (g = gb, even): a 32-bit load at mask gb, where two
  // or four keys are consecutive bits from b0 and eight (jb a multiple of
  // 8) the nibbles at b0 and b0 + 16.  Sixteen keys (jb = 16 f) are the nibbles at 4 f, 16 +
  // 4 f, 32 + 4 f and 48 + 4 f of the whole word.
  using Word = std::conditional_t<(KPW > 8), uint64_t, uint32_t>;
  const int gb = KPW > 8 ? 0 : ((jb >> 2) & 3) & ~1;
  const int b0 = 16 * (((jb >> 2) & 3) - gb) + 4 * (jb >> 4) + (jb & 3);
  auto key_bits = [&](Word word) -> uint32_t {
    if constexpr (KPW == 16) {
      const uint32_t lo = uint32_t(word), hi = uint32_t(word >> 32);
      return ((lo >> b0) & 0xFu) | (((lo >> (b0 + 16)) & 0xFu) << 4) | (((hi >> b0) & 0xFu) << 8) |
             (((hi >> (b0 + 16)) & 0xFu) << 12);
    } else if constexpr (KPW == 8) {
      return ((word >> b0) & 0xFu) | (((word >> (b0 + 16)) & 0xFu) << 4);
    } else {
      return (word >> b0) & ((1u << KPW) - 1u);
    }
  };
  for (int m0 = x0; m0 < x1; m0 += kWave) {
    const int nm = min(kWave, x1 - m0);
    const int my_qb = lane < nm ? kl[m0 + lane] : 0;
    const int my_e = lane < nm ? pm[size_t(my_qb) * nKB] : 0;
    const uint16_t* rowm = hmask + (lane >> 4) * 64 + 4 * (lane & 15) + gb;
    // (slots past the last tile re-read the last tile and are not used)
    auto fetch = [&](int g0, Word (&wd)[kTileGroup]) {
      for (int u = 0; u < kTileGroup; ++u) {
        const int e = __builtin_amdgcn_readlane(my_e, min(g0 + u, nm - 1));
        wd[u] = *reinterpret_cast<const Word*>(rowm + size_t(e) * 256);
      }
    };
    // A group's words give way to its key bits before the next group's
    // loads are issued; the listing (and any drain it starts) runs after
    // the group, with only those loads in flight live.
    Word word[kTileGroup];
    fetch(0, word);
    for (int g0 = 0; g0 < nm; g0 += kTileGroup) {
      uint32_t kbits[kTileGroup];
      for (int u = 0; u < kTileGroup; ++u) kbits[u] = key_bits(word[u]);
      fetch(g0 + kTileGroup, word);  // unconditional: the waits stay exact
#pragma unroll
      for (int u = 0; u < kTileGroup; ++u) {
        if (g0 + u >= nm) break;
        const uint32_t bits = kbits[u];
        const uint64_t any = __ballot(bits != 0u);
        if (any != 0ull) {  // wave-uniform
          // the tile's first row, read in wave-uniform flow: a lane read
          // inside the divergent branch below could meet a value that the
          // compiler reloaded there for the active lanes only
          const int row0 = __builtin_amdgcn_readlane(my_qb, g0 + u) * kBlock;
          if (bits != 0u) {
            const int at = nev + lane_rank(any);
            s_evr[w][at] = row0 + lane;
            s_evm[w][at] = Bits(bits);
          }
          nev += __builtin_popcountll(any);
        }
      }
      if (nev > kEvents - kTileGroup * kWave) list_events();  // room for the next group's events
    }
  }
  list_events();
  drain_lists();

  if (jok) {
    for (int x = 0; x < EL; ++x) {
      // NaN -> 0; a sum that overflowed stays +-inf, as the reference's
      // atomic sums do (its host fix-up clamps them, cu:684-697)
      const float vk = p.d.scale * dk[x];
      dk[x] = __builtin_isnan(vk) ? 0.0f : vk;
      dv[x] = __builtin_isnan(dv[x]) ? 0.0f : dv[x];
    }
    for (int c = 0; c < NC; ++c) {
      float k8[E], v8[E];
      for (int x = 0; x < E; ++x) {
        k8[x] = dk[c * E + x];
        v8[x] = dv[c * E + x];
      }
      if (colok[c]) {
        C::store(static_cast<T*>(p.dk) + head_at(p.ldk, bh, H) + size_t(j) * (FULL ? D : p.ldk.sn) +
                     sub * EL + c * E,
                 k8);
        C::store(static_cast<T*>(p.dv) + head_at(p.ldv, bh, H) + size_t(j) * (FULL ? D : p.ldv.sn) +
                     sub * EL + c * E,
                 v8);
      }
    }
  }
}

// Rows of exactly D elements in every operand (hd = D): the kernels'
// compile-time-stride variant.
inline bool rows_dense(const BackwardParams& p) {
  const int64_t D = p.d.D;
  return p.d.hd == D && p.lq.sn == D && p.lk.sn == D && p.lv.sn == D && p.ldo.sn == D &&
         p.ldq.sn == D && p.ldk.sn == D && p.ldv.sn == D;
}

template <typename T, int D, bool REF, bool DKDV>
hipError_t launch_sparse_m(const BackwardParams& p, hipStream_t s) {
  const dim3 grid(DKDV ? p.d.nKB * (kBlock / keys_per_block<T, D>()) * p.d.BH : p.d.nQB * p.d.BH);
  const bool full = rows_dense(p);
  auto go = [&](auto ac) {
    constexpr int AC = decltype(ac)::value;
    if constexpr (DKDV) {
      if (full) hipLaunchKernelGGL((dkdv_sparse_kernel<T, D, AC, REF, true>), grid, dim3(kThreads), 0, s, p);
      else hipLaunchKernelGGL((dkdv_sparse_kernel<T, D, AC, REF, false>), grid, dim3(kThreads), 0, s, p);
    } else {
      if (full) hipLaunchKernelGGL((dq_sparse_kernel<T, D, AC, REF, true>), grid, dim3(kThreads), 0, s, p);
      else hipLaunchKernelGGL((dq_sparse_kernel<T, D, AC, REF, false>), grid, dim3(kThreads), 0, s, p);
    }
  };
  switch (alpha_class_of(p.d.alpha)) {
    case kA15: go(std::integral_constant<int, kA15>{}); break;
    case kA20: go(std::integral_constant<int, kA20>{}); break;
    case kA125: go(std::integral_constant<int, kA125>{}); break;
    default: go(std::integral_constant<int, kAGen>{}); break;
  }
  return hipGetLastError();
}
template <bool DKDV>
hipError_t launch_sparse(const BackwardParams& p, int dtype, hipStream_t s) {
  const bool ref = p.mode == 1;
  if (dtype == kElemBF16) {
    if (p.d.D == 64)
      return ref ? launch_sparse_m<u16, 64, true, DKDV>(p, s) : launch_sparse_m<u16, 64, false, DKDV>(p, s);
    if (p.d.D == 128)
      return ref ? launch_sparse_m<u16, 128, true, DKDV>(p, s) : launch_sparse_m<u16, 128, false, DKDV>(p, s);
  } else if (dtype == kElemF16) {
    if (p.d.D == 64)
      return ref ? launch_sparse_m<h16, 64, true, DKDV>(p, s) : launch_sparse_m<h16, 64, false, DKDV>(p, s);
    if (p.d.D == 128)
      return ref ? launch_sparse_m<h16, 128, true, DKDV>(p, s) : launch_sparse_m<h16, 128, false, DKDV>(p, s);
  } else {
    if (p.d.D == 64)
      return ref ? launch_sparse_m<float, 64, true, DKDV>(p, s) : launch_sparse_m<float, 64, false, DKDV>(p, s);
    if (p.d.D == 128)
      return ref ? launch_sparse_m<float, 128, true, DKDV>(p, s) : launch_sparse_m<float, 128, false, DKDV>(p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_bwd_dq_sparse(const BackwardParams& p, int dtype, hipStream_t s) {
  return launch_sparse<false>(p, dtype, s);
}
hipError_t launch_bwd_dkdv_sparse(const BackwardParams& p, int dtype, hipStream_t s) {
  return launch_sparse<true>(p, dtype, s);  // after the dQ pass, which writes the position map
}

}  // namespace asa
