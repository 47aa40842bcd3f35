// Score pass: scores, per-row top-k, tau and block mask.
//
// Reference: build_mask_kernel + insert_topk + entmax_threshold
// (adasplashattention.cu:35-217).  One 64-lane wave owns one 64-row query
// block of one (batch, head):
//   1. For every key block that holds a key visible to some row of the
//      block, S^T = K Q^T is formed on MFMA (K fragments straight from
//      global memory, Q^T fragments kept in registers), scaled, clamped to
//      [-10, 10], masked by K_idx <= Q_idx, and written to a 64x64 fp32 tile
//      in LDS.  (The scores path instead copies caller-given scores.)
//   2. Lane L takes row L of the tile.  Its kept top-k lives in LDS as a
//      min-heap of 64-bit keys (score order, then lower key index wins), so
//      a new score costs one compare against the heap root, and an accepted
//      one a log2(k) sift.
//   3. After the last block the heap is sorted in place (best first), the
//      tau recurrence runs on the sorted values, and the row's top-k key
//      blocks are OR-ed into the block's mask bitmap.
#include <climits>

#include "asa_device.hpp"
#include "asa_launch.hpp"

namespace asa {
namespace {

constexpr int kRowStride = 68;  // floats per tile row: 16-byte aligned, spreads LDS banks
constexpr size_t kTileBytes = size_t(kBlock) * kRowStride * sizeof(float);
constexpr size_t kKidBytes = size_t(kBlock) * sizeof(int);

__device__ __forceinline__ int wave_min(int v) {
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, kWave));
  return v;
}
__device__ __forceinline__ int wave_max(int v) {
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, kWave));
  return v;
}

// Lane L's heap occupies h[j * 64 + L], j < n; h[L] is the worst kept key.
// Replaces the root by `key` (known to beat it) and restores heap order.
__device__ __forceinline__ void heap_sift(uint64_t* h, int L, int n, uint64_t key) {
  int pos = 0;
  for (;;) {
    int c = 2 * pos + 1;
    if (c >= n) break;
    uint64_t cv = h[c * kWave + L];
    if (c + 1 < n) {
      const uint64_t c2 = h[(c + 1) * kWave + L];
      if (c2 < cv) {
        cv = c2;
        ++c;
      }
    }
    if (key <= cv) break;
    h[pos * kWave + L] = cv;
    pos = c;
  }
  h[pos * kWave + L] = key;
}

// tau from the sorted top-k of lane L (best first), following the
// reference recurrence step by step (adasplashattention.cu:51-125):
// bracket from the extreme kept values, midpoint start, up to five rounds of
// {f, f', f'' over the leading positive terms; exit when |f| < 1e-4; Halley
// step with the reference's f'' coefficient a(a + 1 - alpha); bracket
// midpoint when the step leaves the bracket; bracket update from f at the
// new point; clamp}.  No contraction, powers via pow_exact, so the result
// is bit-identical to the CPU oracle on identical inputs.
__device__ float entmax_tau(const uint64_t* h, int L, int k, float alpha_in) {
#pragma clang fp contract(off)
  const float alpha = fmaxf(1.05f, fminf(alpha_in, 3.0f));
  const float am1 = alpha - 1.0f;
  const float a = 1.0f / am1;
  const float e1 = (2.0f - alpha) * a;
  const float e2 = (3.0f - 2.0f * alpha) * a;
  const float c2 = a * ((a + 1.0f) - alpha);
  const float top = key_score(h[L]);
  const float bottom = key_score(h[(k - 1) * kWave + L]);
  float lo = am1 * bottom - 2.0f;
  float hi = am1 * top + 2.0f;
  float tau = 0.5f * (lo + hi);
  for (int it = 0; it < 5; ++it) {
    float f = -1.0f, df = 0.0f, d2f = 0.0f;
    for (int j = 0; j < k; ++j) {
      const float u = am1 * key_score(h[j * kWave + L]) - tau;
      if (u <= 0.0f) break;
      const float ue = fmaxf(u, kEps);
      float t = pow_exact(ue, a);
      if (!finite(t)) t = 0.0f;
      f = f + t;
      const float t1 = -a * pow_exact(ue, e1);
      if (finite(t1)) df = df + t1;
      const float t2 = c2 * pow_exact(ue, e2);
      if (finite(t2)) d2f = d2f + t2;
    }
    if (fabsf(f) < 1e-4f) break;
    float next = tau;
    if (fabsf(df) > kEps) {
      const float den = 2.0f * df * df - f * d2f;
      if (fabsf(den) > kEps) next = tau - 2.0f * f * df / den;
    }
    if (!(next >= lo && next <= hi)) next = 0.5f * (lo + hi);
    float gsum = -1.0f;
    for (int j = 0; j < k; ++j) {
      const float u = am1 * key_score(h[j * kWave + L]) - next;
      if (u <= 0.0f) break;
      const float t = pow_exact(fmaxf(u, kEps), a);
      if (finite(t)) gsum = gsum + t;
    }
    if (gsum > 0.0f) lo = next;
    else hi = next;
    tau = next;
    tau = fmaxf(tau, bottom * am1 - 10.0f);
    tau = fminf(tau, top * am1 + 10.0f);
  }
  return tau;
}

// Q^T operand fragments of the 64 query rows: 4 column groups (16 rows
// each) x the head dimension in MFMA k-chunks.
template <typename T, int D> struct QFrags;
template <int D> struct QFrags<u16, D> {
  bf16x8 v[4][D / 32];
  __device__ void load(const u16* Q, int row0, int NQ, int lane) {
    const int g = lane >> 4, c = lane & 15;
    for (int m = 0; m < 4; ++m) {
      const int row = row0 + 16 * m + c;
      for (int s = 0; s < D / 32; ++s) {
        if (row < NQ) v[m][s] = *reinterpret_cast<const bf16x8*>(Q + size_t(row) * D + 32 * s + 8 * g);
        else v[m][s] = bf16x8{};
      }
    }
  }
};
template <int D> struct QFrags<float, D> {
  f32x4 v[4][D / 16];
  __device__ void load(const float* Q, int row0, int NQ, int lane) {
    const int g = lane >> 4, c = lane & 15;
    for (int m = 0; m < 4; ++m) {
      const int row = row0 + 16 * m + c;
      for (int j = 0; j < D / 16; ++j) {
        if (row < NQ) v[m][j] = *reinterpret_cast<const f32x4*>(Q + size_t(row) * D + 16 * j + 4 * g);
        else v[m][j] = f32x4{};
      }
    }
  }
};

// acc[f][m] += K[key block rows 16f..16f+15] . Q[rows 16m..16m+15]^T
template <int D>
__device__ __forceinline__ void score_tile(f32x4 (&acc)[4][4], const QFrags<u16, D>& qf,
                                           const u16* K, int kbase, int NK, int lane) {
  const int g = lane >> 4, c = lane & 15;
  for (int s = 0; s < D / 32; ++s) {
    bf16x8 kf[4];
    for (int f = 0; f < 4; ++f) {
      const int row = min(kbase + 16 * f + c, NK - 1);
      kf[f] = *reinterpret_cast<const bf16x8*>(K + size_t(row) * D + 32 * s + 8 * g);
    }
    for (int f = 0; f < 4; ++f)
      for (int m = 0; m < 4; ++m) acc[f][m] = mfma(kf[f], qf.v[m][s], acc[f][m]);
  }
}
template <int D>
__device__ __forceinline__ void score_tile(f32x4 (&acc)[4][4], const QFrags<float, D>& qf,
                                           const float* K, int kbase, int NK, int lane) {
  const int g = lane >> 4, c = lane & 15;
  for (int j = 0; j < D / 16; ++j) {
    f32x4 kf[4];
    for (int f = 0; f < 4; ++f) {
      const int row = min(kbase + 16 * f + c, NK - 1);
      kf[f] = *reinterpret_cast<const f32x4*>(K + size_t(row) * D + 16 * j + 4 * g);
    }
    for (int r = 0; r < 4; ++r)
      for (int f = 0; f < 4; ++f)
        for (int m = 0; m < 4; ++m) acc[f][m] = mfma(kf[f][r], qf.v[m][j][r], acc[f][m]);
  }
}

template <typename T, int D, bool kFromScores>
__global__ __launch_bounds__(64) void select_kernel(SelectParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int k = p.d.k, NQ = p.d.NQ, NK = p.d.NK, nKB = p.d.nKB, nQB = p.d.nQB;
  float* stile = reinterpret_cast<float*>(smem);
  int* ktile = reinterpret_cast<int*>(smem + kTileBytes);
  uint64_t* heap = reinterpret_cast<uint64_t*>(smem + kTileBytes + kKidBytes);
  uint32_t* bits = reinterpret_cast<uint32_t*>(heap + size_t(k) * kWave);
  const int nbw = (nKB + 31) >> 5;

  const int L = threadIdx.x;
  const int g = L >> 4, c16 = L & 15;
  const int qb = blockIdx.x, bh = blockIdx.y;
  const int q0 = qb * kBlock;

  // Row owned by this lane in the selection phase.
  const int myq = q0 + L;
  const bool qvalid = myq < NQ;
  const int myqidx = qvalid ? p.q_idx[size_t(bh) * NQ + myq] : 0;
  const int qmax = wave_max(qvalid ? myqidx : INT_MIN);

  const uint64_t sentinel = make_key(kSentinel, -1);
  for (int j = 0; j < k; ++j) heap[j * kWave + L] = sentinel;
  for (int w = L; w < nbw; w += kWave) bits[w] = 0u;

  // Rows of this lane in the MFMA accumulator layout (columns 16m + c16).
  int qid_m[4];
  bool qok_m[4];
  for (int m = 0; m < 4; ++m) {
    const int qq = q0 + 16 * m + c16;
    qok_m[m] = qq < NQ;
    qid_m[m] = qok_m[m] ? p.q_idx[size_t(bh) * NQ + qq] : 0;
  }

  QFrags<T, D> qf;
  const T* Kb = nullptr;
  if constexpr (!kFromScores) {
    qf.load(static_cast<const T*>(p.q) + size_t(bh) * NQ * D, q0, NQ, L);
    Kb = static_cast<const T*>(p.k) + size_t(bh) * NK * D;
  }

  for (int kt = 0; kt < nKB; ++kt) {
    const int kbase = kt * kBlock;
    const int kj = kbase + L;
    const int kid = kj < NK ? p.k_idx[size_t(bh) * NK + kj] : INT_MAX;
    if (wave_min(kid) > qmax) continue;  // nothing in this key block is visible
    ktile[L] = kid;
    __syncthreads();

    if constexpr (kFromScores) {
      const float* srow = p.scores + (size_t(bh) * NQ + (qvalid ? myq : 0)) * NK;
      for (int c = 0; c < kBlock; c += 4) {
        f32x4 v;
        for (int r = 0; r < 4; ++r) {
          const int key = kbase + c + r;
          const bool ok = qvalid && key < NK && ktile[c + r] <= myqidx;
          v[r] = ok ? clamp_score(srow[key]) : -__builtin_inff();
        }
        *reinterpret_cast<f32x4*>(stile + L * kRowStride + c) = v;
      }
    } else {
      f32x4 acc[4][4];
      for (int f = 0; f < 4; ++f)
        for (int m = 0; m < 4; ++m) acc[f][m] = f32x4{0.f, 0.f, 0.f, 0.f};
      score_tile<D>(acc, qf, Kb, kbase, NK, L);
      const float scale = p.d.scale;
      for (int f = 0; f < 4; ++f) {
        const int kb4 = 16 * f + 4 * g;
        int kid4[4];
        for (int r = 0; r < 4; ++r) kid4[r] = ktile[kb4 + r];
        for (int m = 0; m < 4; ++m) {
          f32x4 v;
          for (int r = 0; r < 4; ++r) {
            const bool ok = qok_m[m] && (kbase + kb4 + r) < NK && kid4[r] <= qid_m[m];
            v[r] = ok ? clamp_score(acc[f][m][r] * scale) : -__builtin_inff();
          }
          *reinterpret_cast<f32x4*>(stile + (16 * m + c16) * kRowStride + kb4) = v;
        }
      }
    }
    __syncthreads();

    // Selection: lane L scans row L of the tile.
    uint64_t root = heap[L];
    const float thr = key_score(root);
    const float* row = stile + L * kRowStride;
    uint32_t mlo = 0u, mhi = 0u;
    for (int c = 0; c < 32; c += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(row + c);
      for (int r = 0; r < 4; ++r) mlo |= (v[r] >= thr ? 1u : 0u) << (c + r);
    }
    for (int c = 0; c < 32; c += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(row + 32 + c);
      for (int r = 0; r < 4; ++r) mhi |= (v[r] >= thr ? 1u : 0u) << (c + r);
    }
    uint64_t cand = (uint64_t(mhi) << 32) | mlo;
    while (cand) {
      const int c = __builtin_ctzll(cand);
      cand &= cand - 1;
      const uint64_t key = make_key(row[c], kbase + c);
      if (key > root) {
        heap_sift(heap, L, k, key);
        root = heap[L];
      }
    }
    __syncthreads();
  }

  // Sort the heap in place, best first: repeatedly move the worst kept key
  // to the end of the shrinking heap.
  for (int end = k - 1; end > 0; --end) {
    const uint64_t worst = heap[L];
    const uint64_t last = heap[end * kWave + L];
    heap[end * kWave + L] = worst;
    heap_sift(heap, L, end, last);
  }

  if (qvalid) {
    const float tau = entmax_tau(heap, L, k, p.d.alpha);
    const size_t r = size_t(bh) * NQ + myq;
    p.taus[r] = tau;
    for (int j = 0; j < k; ++j) {
      const uint64_t key = heap[j * kWave + L];
      const int idx = key_index(key);
      if (p.topk_idx) p.topk_idx[r * k + j] = idx;
      if (p.topk_val) p.topk_val[r * k + j] = key_score(key);
      if (idx >= 0) {
        const int kb = idx / kBlock;
        atomicOr(&bits[kb >> 5], 1u << (kb & 31));
      }
    }
  }
  __syncthreads();
  uint8_t* mrow = p.mask + (size_t(bh) * nQB + qb) * nKB;
  for (int kb = L; kb < nKB; kb += kWave) mrow[kb] = uint8_t((bits[kb >> 5] >> (kb & 31)) & 1u);
}

template <typename T, int D, bool kFromScores>
hipError_t launch_one(const SelectParams& p, hipStream_t s) {
  const size_t lds = select_lds_bytes(p.d);
  auto kern = select_kernel<T, D, kFromScores>;
  if (lds > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) return e;
  }
  dim3 grid(p.d.nQB, p.d.BH);
  hipLaunchKernelGGL(kern, grid, dim3(kWave), lds, s, p);
  return hipGetLastError();
}

}  // namespace

size_t select_lds_bytes(const Dims& d) {
  const size_t nbw = size_t(d.nKB + 31) / 32;
  size_t b = kTileBytes + kKidBytes + size_t(d.k) * kWave * sizeof(uint64_t) + nbw * 4;
  return (b + 15) & ~size_t(15);
}

hipError_t launch_select(const SelectParams& p, bool bf16, bool from_scores, hipStream_t s) {
  if (from_scores) return launch_one<float, 64, true>(p, s);
  if (bf16) {
    if (p.d.D == 64) return launch_one<u16, 64, false>(p, s);
    if (p.d.D == 128) return launch_one<u16, 128, false>(p, s);
  } else {
    if (p.d.D == 64) return launch_one<float, 64, false>(p, s);
    if (p.d.D == 128) return launch_one<float, 128, false>(p, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace asa
