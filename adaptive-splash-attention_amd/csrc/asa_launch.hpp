// Host-side launch interface between the C ABI (capi.cpp) and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace asa {

// Problem constants shared by every kernel.
struct Dims {
  int BH, NQ, NK, D, k, nQB, nKB;
  float alpha;  // already clamped to [1.05, 3]
  float scale;
};

// Support-list buffers shared by the forward (writer) and the backward.
struct SupportLists {
  uint32_t* key;
  float* val;
  float* ds;       // backward: ds of every entry (written by the dQ pass)
  int32_t* off;
  int32_t* cnt;
  int cap;         // entries per wave region
};

struct SelectParams {
  Dims d;
  const void* q;          // MFMA path
  const void* k;
  const float* scores;    // scores path: [BH, NQ, NK]
  const int32_t* q_idx;
  const int32_t* k_idx;
  float* taus;
  uint8_t* mask;
  int32_t* topk_idx;      // optional
  float* topk_val;        // optional
  float* tkv;             // workspace: sorted top-k values, [k][BH * NQ]
  int2* kbounds;          // workspace: (min, max) position per key block, [BH * nKB]
  int cap;                // candidate keys per row in LDS (select_capacity)
};

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
  const int32_t* q_idx;
  const int32_t* k_idx;
  const float* taus;
  const int32_t* q_ptr;
  const int32_t* q_list;
  void* out;
  float* norms;
  // Support lists (optional: sup_key == nullptr emits nothing).  Every wave
  // of a query block (16 rows) owns a region of sup_cap entries at
  // ((bh * nQB + qb) * 4 + w) * sup_cap; entry = key index | row-in-wave << 28
  // in sup_key and v = max(u, 0) in sup_val, for every score of the forward
  // with u > 0, in (tile, score slot, lane) order.  sup_off[(bh * nQB * nKB
  // + e) * 4 + w] = the wave's entry count before tile e (the head's
  // q_list position e); sup_cnt[(bh * nQB + qb) * 4 + w] = its total, which
  // may exceed sup_cap (then only the first sup_cap entries were written).
  SupportLists sup;
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
  const int32_t* q_ptr;
  const int32_t* q_list;
  const int32_t* k_ptr;
  const int32_t* k_list;
  float* delta;  // workspace [BH, NQ]
  void* dq;
  void* dk;
  void* dv;
};

// Each launcher returns the launch status; `name` receives the kernel's
// name for the profiler.
hipError_t launch_select(const SelectParams& p, bool bf16, bool from_scores, hipStream_t s);
// LDS bytes of one select block holding `cap` candidate keys per row.
size_t select_lds_bytes(const Dims& d, bool bf16, bool from_scores, int cap);
// Candidate keys per row that fit `max_lds` bytes (k + 32 at most; -1 if
// not even k + 8 fit).
int select_capacity(const Dims& d, bool bf16, bool from_scores, size_t max_lds);
hipError_t launch_bounds(const SelectParams& p, hipStream_t s);
hipError_t launch_tau(const SelectParams& p, hipStream_t s);
hipError_t launch_compact(const CompactParams& p, hipStream_t s);
hipError_t launch_forward(const ForwardParams& p, bool bf16, hipStream_t s);
hipError_t launch_bwd_delta(const BackwardParams& p, bool bf16, hipStream_t s);
hipError_t launch_bwd_dq(const BackwardParams& p, bool bf16, hipStream_t s);
hipError_t launch_bwd_dkdv(const BackwardParams& p, bool bf16, hipStream_t s);

// Kernel-timing hooks implemented in capi.cpp (no-ops unless profiling).
void profile_begin(const char* name, hipStream_t s);
void profile_end(hipStream_t s);

}  // namespace asa
