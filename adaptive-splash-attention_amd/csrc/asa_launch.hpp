// Host-side launch interface between the C ABI (capi.cpp) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace asa {

// Storage type of Q, K, V, Out, dOut and the gradients (values as asa_dtype).
enum ElemType : int { kElemF32 = 0, kElemBF16 = 1, kElemF16 = 2 };
inline int elem_bytes(int dtype) { return dtype == kElemF32 ? 4 : 2; }

// Problem constants shared by every kernel.  D is the head dimension the
// kernels compute at (64 or 128, compile-time in each kernel); hd <= D is
// the tensors' own head dimension (a multiple of one 16-byte chunk: 8
// elements for 16-bit types, 4 for fp32).  Columns hd .. D - 1 are never
// read or written: loads of them give zeros, so every dot product is the
// hd-dimensional one, and stores skip them.
struct Dims {
  int BH, H, NQ, NK, D, hd, k, nQB, nKB;
  float alpha;  // already clamped to [1.05, 3]
  float scale;
};

// Where the rows of a [B, H, N, hd] operand are: element strides of batch,
// head and row (the head dimension is contiguous).  Every stride is a
// multiple of a 16-byte chunk's elements, so that every chunk the kernels
// load is 16-byte aligned, and the offsets of a head's rows from its first
// fit 32 bits (checked by the C ABI).
struct Lay {
  int64_t sb, sh, sn;
};
// Offset (elements) of head bh = b * H + h's first row.
__host__ __device__ inline size_t head_at(const Lay& l, int bh, int H) {
  return size_t(bh / H) * size_t(l.sb) + size_t(bh % H) * size_t(l.sh);
}
// The contiguous layout of a [B, H, N, hd] tensor.
__host__ __device__ inline Lay contiguous_lay(int H, int N, int hd) {
  return Lay{int64_t(H) * N * hd, int64_t(N) * hd, hd};
}
// Whether an operand is a contiguous [B, H, N, D] tensor (then its row n
// of head bh is at (bh N + n) D: the kernels' compile-time-stride case).
__host__ __device__ inline bool lay_dense(const Lay& l, int H, int N, int D) {
  const Lay c = contiguous_lay(H, N, D);
  return l.sb == c.sb && l.sh == c.sh && l.sn == c.sn;
}
// Row n of head bh of an operand: at (bh N + n) D when DENSE (a contiguous
// [B, H, N, D] tensor), else from its strides.
template <bool DENSE, int D, typename T>
__host__ __device__ inline T* row_at(T* base, const Lay& l, int bh, int H, int N, int n) {
  if constexpr (DENSE) return base + (size_t(bh) * N + n) * D;
  else return base + head_at(l, bh, H) + size_t(n) * size_t(l.sn);
}

// Support masks written by the forward and read by the backward: for the
// tile at the head's q_list position e (query block qb, key block kb), bit
// 4 f + r of
//   mask[((bh * nQB * nKB + e) * 4 + w) * 64 + 4 c + g]
// is set iff u > 0 for row qb * 64 + 16 w + c and key kb * 64 + 16 f + 4 g + r
// (w, c < 16, g, f, r < 4): a row's four masks of a tile form one 8-byte
// word, a tile's masks 512 bytes.
struct SupportMasks {
  uint16_t* mask;  // nullptr: no masks (the backward runs the dense passes)
};

// 32-row mask blocks (the reference's BLOCK_M = 32): the kernels still work
// on 64-row query blocks, over the union of the two 32-row halves' key
// blocks, and a half whose own mask row lacks a key block contributes
// nothing to that tile.  half[(bh * nQH + h) * nKB + kb], nQH = ceil(NQ / 32),
// is that mask; nullptr for 64-row blocks.
__host__ __device__ inline int half_blocks(int NQ) { return (NQ + 31) / 32; }

struct SelectParams {
  Dims d;
  const void* q;          // MFMA path
  const void* k;
  Lay lq, lk;
  const float* scores;    // scores path: [BH, NQ, NK]
  const int32_t* q_idx;
  const int32_t* k_idx;
  float* taus;
  uint8_t* mask;          // [BH, nQB, nKB], 64-row blocks
  uint8_t* half;          // 32-row blocks: also [BH, nQH, nKB] (else nullptr)
  int32_t* topk_idx;      // optional
  float* topk_val;        // optional
  float* tkv;             // workspace: sorted top-k values, [k][BH * NQ]
  int2* kbounds;          // workspace: (min, max) position per key block, [BH * nKB]
  int cap;                // candidate keys per row in LDS (select_capacity)
  int lcap;               // refine pass: listed keys per row in LDS (refine_list_capacity)
  uint32_t* status;       // optional per-call status word (kStatus* bits), zeroed by bounds_kernel
};

// Bits of the per-call status word.  Bits 8-15 hold the largest number of
// overflow rounds a select block ran (saturating at 255): information only.
// Values as ASA_STATUS_* in adasplash.h.
constexpr uint32_t kStatusSelectRounds = 1u;  // select stopped at its proven round bound
constexpr uint32_t kStatusRefineSweeps = 2u;  // exact-mode refine stopped at its sweep cap

struct CompactParams {
  int BH, nQB, nKB;
  const uint8_t* mask;
  int32_t* q_ptr;
  int32_t* q_list;
  int32_t* k_ptr;
  int32_t* k_list;
};

struct ForwardParams {
  Dims d;
  const void* q;
  const void* k;
  const void* v;
  Lay lq, lk, lv, lo;  // lo: out
  const int32_t* q_idx;
  const int32_t* k_idx;
  const float* taus;
  const int32_t* q_ptr;
  const int32_t* q_list;
  void* out;
  float* norms;
  const int2* kbounds;  // (min, max) position per key block [BH * nKB], from the score pass
  const uint8_t* half;  // 32-row mask (32-row blocks only, else nullptr)
  const float* top1;    // each row's best score (the score pass's first sorted value)
  // Support masks (optional: sup.mask == nullptr writes none).
  SupportMasks sup;
  // Two query blocks per workgroup (16-bit inputs): 0 when the pairs fill
  // at least one wave of resident workgroups on `cus` compute units, 1
  // wherever the paired kernel applies, 2 never (asa_set_pairing).
  int pairing;
  int cus;
};

// Per-row constants of the support-mask backward, written by its dQ pass
// for its dK/dV pass: ClippedU's nt (its lo and hi follow from nt and
// alpha), 1/(sum p + EPS), the gradient factor c and cs = -c shift
// (ds = w (c dp + cs)).  16 bytes: one load per listed row.
struct alignas(16) RowRec {
  float nt, invn, c, cs;
};

struct BackwardParams {
  Dims d;
  int mode;  // 0 entmax Jacobian, 1 reference kernel's gradient
  const void* q;
  const void* k;
  const void* v;
  const void* out;
  const void* dout;
  const int32_t* q_idx;
  const int32_t* k_idx;
  const float* taus;
  const float* norms;
  const uint8_t* mask;
  const uint8_t* half;  // 32-row mask (32-row blocks only, else nullptr)
  const int32_t* q_ptr;
  const int32_t* q_list;
  const int32_t* k_ptr;
  const int32_t* k_list;
  float* delta;  // workspace [BH, NQ]
  void* dq;
  void* dk;
  void* dv;
  Lay lq, lk, lv, lo, ldo, ldq, ldk, ldv;  // lo: out, ldo: dout
  SupportMasks sup;  // mask == nullptr: dense passes
  RowRec* rowrec;    // workspace [BH * NQ] (support-mask passes)
  int32_t* posmap;   // workspace [BH, nQB * nKB] (support-mask dK/dV pass)
};

// Each launcher returns the launch status; `name` receives the kernel's
// name for the profiler.
hipError_t launch_select(const SelectParams& p, int dtype, bool from_scores, hipStream_t s);
// LDS bytes of one select block holding `cap` candidate keys per row.
size_t select_lds_bytes(const Dims& d, int dtype, bool from_scores, int cap);
// Candidate keys per row that fit `max_lds` bytes (k + 32 at most; -1 if
// not even k + 8 fit).
int select_capacity(const Dims& d, int dtype, bool from_scores, size_t max_lds);
hipError_t launch_bounds(const SelectParams& p, hipStream_t s);
hipError_t launch_tau(const SelectParams& p, hipStream_t s);
// Exact-threshold pass (tau mode "exact"): after launch_tau, before
// compaction; reads tkv and kbounds, rewrites taus and ORs blocks into mask.
hipError_t launch_refine(const SelectParams& p, int dtype, hipStream_t s);
// LDS bytes of one refine block holding `lcap` listed keys per row.
size_t refine_lds_bytes(const Dims& d, int dtype, int lcap);
// Listed keys per row that fit `max_lds` bytes (max(64, k + 32) at most;
// 0: none fit, every row sweeps; -1: not even the sweep stage fits).
int refine_list_capacity(const Dims& d, int dtype, size_t max_lds);
hipError_t launch_compact(const CompactParams& p, hipStream_t s);
// launch_tau and launch_compact(cp) as one launch (the tau rows' blocks
// first); for a mask that no pass changes between the two.
hipError_t launch_tau_compact(const SelectParams& p, const CompactParams& cp, hipStream_t s);
// 64-row mask from a 32-row one: mask[bh, qb, kb] = half[bh, 2 qb, kb] |
// half[bh, 2 qb + 1, kb] (the second row when it exists).
hipError_t launch_fold_halves(const uint8_t* half, uint8_t* mask, int BH, int NQ, int nQB,
                              int nKB, hipStream_t s);
hipError_t launch_forward(const ForwardParams& p, int dtype, hipStream_t s);
hipError_t launch_bwd_delta(const BackwardParams& p, int dtype, hipStream_t s);
hipError_t launch_bwd_dq(const BackwardParams& p, int dtype, hipStream_t s);
hipError_t launch_bwd_dkdv(const BackwardParams& p, int dtype, hipStream_t s);
// The support-pair passes: dQ writes the row records and the position map
// that dK/dV reads, so dK/dV must follow it on the stream.
hipError_t launch_bwd_dq_sparse(const BackwardParams& p, int dtype, hipStream_t s);
hipError_t launch_bwd_dkdv_sparse(const BackwardParams& p, int dtype, hipStream_t s);

// Kernel-timing hooks implemented in capi.cpp (no-ops unless profiling).
void profile_begin(const char* name, hipStream_t s);
void profile_end(hipStream_t s);

}  // namespace asa
