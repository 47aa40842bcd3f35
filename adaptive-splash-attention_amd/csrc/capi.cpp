// C ABI of libadasplash (declared in include/adasplash.h).
//
// Host side of the reference's forward_splash / backward_splash
// (adasplashattention.cu:537-700): argument validation, the kernel sequence
// on the caller's stream, and error reporting.  Unlike the reference it
// allocates nothing, never synchronises, and reports errors through status
// codes plus a thread-local message instead of exceptions.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/adasplash.h"
#include "asa_launch.hpp"

static_assert(int(ASA_DTYPE_F32) == asa::kElemF32 && int(ASA_DTYPE_BF16) == asa::kElemBF16 &&
                  int(ASA_DTYPE_F16) == asa::kElemF16,
              "asa_dtype and asa::ElemType must agree");

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int ok() {
  g_error.clear();
  return ASA_OK;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return ASA_OK;
  return fail(ASA_ERR_DEVICE, "%s failed: %s", what, hipGetErrorString(e));
}

struct Shape {
  int BH, H, NQ, NK, D, k;
  int hd;   // the tensors' head dimension (D: the kernels' compute width)
  asa::Lay lq, lk, lv, ldo;  // input strides (validated)
  int nQB;  // 64-row query blocks (the kernels' tiles)
  int nKB;
  int bm;   // block_m: 64, or 32 (the reference's BLOCK_M)
  int nQBm; // block_m-row query blocks: rows of the state's mask and CSR
  int dtype;  // asa_dtype (= asa::ElemType)
  bool exact;  // ASA_TAU_EXACT
  float alpha, scale;
};

// Strides of a contiguous [batch, heads, n, hd] tensor.
asa::Lay contiguous(int heads, int n, int hd) { return asa::contiguous_lay(heads, n, hd); }

// 16-byte alignment of every tensor pointer (the kernels' 16-byte loads
// and stores).
int check_aligned(std::initializer_list<const void*> ptrs) {
  for (const void* q : ptrs)
    if (reinterpret_cast<uintptr_t>(q) % 16)
      return fail(ASA_ERR_INVALID_ARGUMENT, "tensor pointer %p is not 16-byte aligned", q);
  return ASA_OK;
}

int validate(const asa_problem* p, Shape* sh) {
  if (!p) return fail(ASA_ERR_INVALID_ARGUMENT, "problem descriptor is NULL");
  if (p->batch < 1 || p->heads < 1)
    return fail(ASA_ERR_INVALID_ARGUMENT, "batch (%d) and heads (%d) must be >= 1", p->batch,
                p->heads);
  if (p->nq < 1 || p->nk < 1)
    return fail(ASA_ERR_INVALID_ARGUMENT, "nq (%d) and nk (%d) must be >= 1", p->nq, p->nk);
  if (p->nk >= (1 << 28))
    return fail(ASA_ERR_INVALID_ARGUMENT, "nk (%d) must be below 2^28", p->nk);
  if (p->head_dim > 128)
    return fail(ASA_ERR_INVALID_ARGUMENT, "Head dimension too large (%d > 128)", p->head_dim);
  if (p->head_dim < 1)
    return fail(ASA_ERR_INVALID_ARGUMENT, "head_dim %d must be >= 1", p->head_dim);
  if (p->k_keep < 1 || p->k_keep > 128)
    return fail(ASA_ERR_INVALID_ARGUMENT, "k_keep %d out of range [1, 128]", p->k_keep);
  if ((p->block_m != 64 && p->block_m != 32) || p->block_n != 64)
    return fail(ASA_ERR_UNSUPPORTED,
                "block_m x block_n = %d x %d not supported (64 x 64 or 32 x 64)", p->block_m,
                p->block_n);
  if (p->block_m == 32 && p->tau_mode == ASA_TAU_EXACT)
    return fail(ASA_ERR_UNSUPPORTED, "exact tau mode needs block_m = 64");
  if (p->dtype != ASA_DTYPE_F32 && p->dtype != ASA_DTYPE_BF16 && p->dtype != ASA_DTYPE_F16)
    return fail(ASA_ERR_INVALID_ARGUMENT, "unknown dtype %d", p->dtype);
  if (p->tau_mode != ASA_TAU_REFERENCE && p->tau_mode != ASA_TAU_EXACT)
    return fail(ASA_ERR_INVALID_ARGUMENT, "unknown tau_mode %d", p->tau_mode);
  // 16-byte chunks: the kernels' unit of every load and store
  const int epc = p->dtype == ASA_DTYPE_F32 ? 4 : 8;
  if (p->head_dim % epc)
    return fail(ASA_ERR_UNSUPPORTED, "head_dim %d must be a multiple of %d for this dtype",
                p->head_dim, epc);
  if (!std::isfinite(p->alpha)) return fail(ASA_ERR_INVALID_ARGUMENT, "alpha is not finite");
  if (!std::isfinite(p->sm_scale)) return fail(ASA_ERR_INVALID_ARGUMENT, "sm_scale is not finite");
  const long long bh = (long long)p->batch * p->heads;
  const long long nqb = (p->nq + 63) / 64, nkb = (p->nk + 63) / 64;
  const long long nqbm = (p->nq + p->block_m - 1) / p->block_m;
  if (bh > (1LL << 31) - 1 || nqbm * nkb > (1LL << 31) - 1 ||
      bh * (long long)p->nq > (1LL << 40) || bh * (long long)p->nk > (1LL << 40))
    return fail(ASA_ERR_INVALID_ARGUMENT, "problem too large");
  sh->BH = int(bh);
  sh->H = p->heads;
  sh->NQ = p->nq;
  sh->NK = p->nk;
  sh->hd = p->head_dim;
  sh->D = p->head_dim <= 64 ? 64 : 128;
  const int64_t ebytes = p->dtype == ASA_DTYPE_F32 ? 4 : 2;
  struct {
    const int64_t* st;
    int n;
    asa::Lay* lay;
    const char* name;
  } ops[] = {{p->q_strides, p->nq, &sh->lq, "q"},
             {p->k_strides, p->nk, &sh->lk, "k"},
             {p->v_strides, p->nk, &sh->lv, "v"},
             {p->dout_strides, p->nq, &sh->ldo, "dout"}};
  for (auto& o : ops) {
    if (o.st[0] == 0 && o.st[1] == 0 && o.st[2] == 0) {
      *o.lay = contiguous(p->heads, o.n, p->head_dim);
      continue;
    }
    for (int i = 0; i < 3; ++i)
      if (o.st[i] < 0 || o.st[i] % epc)
        return fail(ASA_ERR_INVALID_ARGUMENT,
                    "%s_strides[%d] = %lld must be >= 0 and a multiple of %d elements", o.name, i,
                    (long long)o.st[i], epc);
    // a head's rows within 2^31 bytes of its first (32-bit row offsets)
    if (((int64_t(o.n) - 1) * o.st[2] + p->head_dim) * ebytes >= (int64_t(1) << 31))
      return fail(ASA_ERR_UNSUPPORTED, "%s row stride %lld spans 2^31 bytes or more per head",
                  o.name, (long long)o.st[2]);
    // a dimension of size 1 takes its contiguous stride (its stride is
    // never used), so that a contiguous tensor compares equal to one
    const asa::Lay c = contiguous(p->heads, o.n, p->head_dim);
    *o.lay = asa::Lay{p->batch == 1 ? c.sb : o.st[0], p->heads == 1 ? c.sh : o.st[1],
                      o.n == 1 ? c.sn : o.st[2]};
  }
  sh->k = p->k_keep;
  sh->nQB = int(nqb);
  sh->nKB = int(nkb);
  sh->bm = p->block_m;
  sh->nQBm = int(nqbm);
  sh->dtype = p->dtype;
  sh->exact = p->tau_mode == ASA_TAU_EXACT;
  // alpha is clamped to [1.05, 3] as the reference does (adasplashattention.cu:547).
  sh->alpha = std::fmax(1.05f, std::fmin(p->alpha, 3.0f));
  sh->scale = p->sm_scale;
  return ASA_OK;
}

asa::Dims dims_of(const Shape& s) {
  return asa::Dims{s.BH, s.H, s.NQ, s.NK, s.D, s.hd, s.k, s.nQB, s.nKB, s.alpha, s.scale};
}

// Bytes of the sorted top-k values at the start of the forward workspace,
// rounded up so that the key-block bounds after them are 16-byte aligned.
size_t tkv_bytes(const Shape& s) {
  const size_t b = size_t(s.BH) * s.NQ * s.k * sizeof(float);
  return (b + 15) & ~size_t(15);
}

// Byte offset of the per-row records of the support-mask backward in its
// workspace (after the two floats per row), 16-byte aligned.
size_t bwd_rec_offset(const Shape& s) {
  return (2 * size_t(s.BH) * s.NQ * sizeof(float) + 15) & ~size_t(15);
}

// Then the tile position map of the support-mask dK/dV pass.
size_t bwd_map_offset(const Shape& s) {
  return bwd_rec_offset(s) + size_t(s.BH) * s.NQ * sizeof(asa::RowRec);
}

size_t align16(size_t b) { return (b + 15) & ~size_t(15); }

// With 32-row mask blocks the kernels run over the 64-row union of each
// pair of 32-row mask rows: that mask and its CSR lists live in the
// workspace (the state holds the block_m-row ones).
struct Csr64 {
  uint8_t* mask;
  int32_t *q_ptr, *q_list, *k_ptr, *k_list;
};

size_t csr64_bytes(const Shape& s) {
  const size_t blocks = size_t(s.BH) * s.nQB * s.nKB;
  return align16(blocks) + align16(size_t(s.BH) * (s.nQB + 1) * 4) + align16(blocks * 4) +
         align16(size_t(s.BH) * (s.nKB + 1) * 4) + align16(blocks * 4);
}

Csr64 csr64_at(const Shape& s, char* base) {
  const size_t blocks = size_t(s.BH) * s.nQB * s.nKB;
  Csr64 c;
  c.mask = reinterpret_cast<uint8_t*>(base);
  base += align16(blocks);
  c.q_ptr = reinterpret_cast<int32_t*>(base);
  base += align16(size_t(s.BH) * (s.nQB + 1) * 4);
  c.q_list = reinterpret_cast<int32_t*>(base);
  base += align16(blocks * 4);
  c.k_ptr = reinterpret_cast<int32_t*>(base);
  base += align16(size_t(s.BH) * (s.nKB + 1) * 4);
  c.k_list = reinterpret_cast<int32_t*>(base);
  return c;
}

// Workspace offsets of that 64-row structure in the forward and backward.
size_t fwd_csr_offset(const Shape& s) {
  return tkv_bytes(s) + align16(size_t(s.BH) * s.nKB * 2 * sizeof(int32_t));
}
size_t bwd_csr_offset(const Shape& s) {
  return align16(bwd_map_offset(s) + size_t(s.BH) * s.nQB * s.nKB * sizeof(int32_t));
}

// The 64-row mask and lists the kernels use: the state's own (64-row
// blocks) or the workspace's (32-row blocks).
Csr64 kernel_csr(const Shape& s, const asa_state* st, void* workspace, size_t offset) {
  if (s.bm == 64) return Csr64{st->mask, st->q_ptr, st->q_list, st->k_ptr, st->k_list};
  return csr64_at(s, static_cast<char*>(workspace) + offset);
}

void sizes_of(const Shape& s, asa_sizes* z) {
  const size_t rows = size_t(s.BH) * s.NQ;
  const size_t blocks = size_t(s.BH) * s.nQB * s.nKB;    // 64-row tiles
  const size_t mblocks = size_t(s.BH) * s.nQBm * s.nKB;  // block_m-row mask entries
  z->taus = rows * sizeof(float);
  z->norms = rows * sizeof(float);
  z->mask = mblocks;
  z->q_ptr = size_t(s.BH) * (s.nQBm + 1) * sizeof(int32_t);
  z->q_list = mblocks * sizeof(int32_t);
  z->k_ptr = size_t(s.BH) * (s.nKB + 1) * sizeof(int32_t);
  z->k_list = mblocks * sizeof(int32_t);
  z->topk_idx = rows * s.k * sizeof(int32_t);
  z->topk_val = rows * s.k * sizeof(float);
  z->sup_mask = blocks * 256 * sizeof(uint16_t);
  // forward: the rows' sorted top-k values and the key blocks' position
  // bounds; backward: two floats per row, a 16-byte record per row and an
  // int per tile; both, with 32-row blocks, the 64-row mask and lists
  const size_t extra = s.bm == 32 ? csr64_bytes(s) : 0;
  const size_t fwd_ws = s.bm == 32 ? fwd_csr_offset(s) + extra
                                   : tkv_bytes(s) + size_t(s.BH) * s.nKB * 2 * sizeof(int32_t);
  const size_t bwd_ws = s.bm == 32 ? bwd_csr_offset(s) + extra
                                   : bwd_map_offset(s) + blocks * sizeof(int32_t);
  z->workspace = fwd_ws > bwd_ws ? fwd_ws : bwd_ws;
}

int check_state(const asa_state* st, bool need_norms) {
  if (!st) return fail(ASA_ERR_INVALID_ARGUMENT, "state is NULL");
  if (!st->taus || !st->mask || !st->q_ptr || !st->q_list || !st->k_ptr || !st->k_list ||
      (need_norms && !st->norms))
    return fail(ASA_ERR_INVALID_ARGUMENT, "a required state buffer is NULL");
  if ((st->topk_idx == nullptr) != (st->topk_val == nullptr))
    return fail(ASA_ERR_INVALID_ARGUMENT, "topk_idx and topk_val must be both set or both NULL");
  return ASA_OK;
}

// asa_set_pairing's mode (process-wide).
std::atomic<int> g_pairing{ASA_PAIRING_AUTO};

// Compute units of the current device, cached per device ordinal.
int device_cus(int* cus) {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev >= 0 && dev < 64 && cached[dev].load() > 0) {
    *cus = cached[dev].load();
    return ASA_OK;
  }
  int n = 0;
  if (int rc = check_hip(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev),
                         "hipDeviceGetAttribute"))
    return rc;
  if (dev >= 0 && dev < 64) cached[dev].store(n);
  *cus = n;
  return ASA_OK;
}

// Candidate capacity per row of the select kernel on the current device
// (*cap), or an error when even the smallest capacity does not fit its LDS.
int select_cap(const Shape& s, bool from_scores, int* cap) {
  int dev = 0, max_lds = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (int rc = check_hip(hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock,
                                               dev),
                         "hipDeviceGetAttribute"))
    return rc;
  const asa::Dims d = dims_of(s);
  *cap = asa::select_capacity(d, s.dtype, from_scores, size_t(max_lds));
  if (*cap < 0)
    return fail(ASA_ERR_UNSUPPORTED, "k_keep %d needs %zu bytes of LDS per block, device has %d",
                s.k, asa::select_lds_bytes(d, s.dtype, from_scores, s.k + 8), max_lds);
  return ASA_OK;
}

// ---------------------------------------------------------------------------
// Kernel timing (asa_profile_*).  Process-wide: a backward pass may run on
// another thread than the one that enabled profiling (e.g. an autograd
// worker).
// ---------------------------------------------------------------------------
struct Rec {
  const char* name;
  hipEvent_t start, stop;
  hipStream_t stream;
};
std::atomic<bool> g_prof{false};
std::mutex g_prof_mu;
std::vector<Rec> g_recs;
thread_local int g_open = -1;  // index of this thread's launch being timed

// Score pass and compaction: the kernels' 64-row mask and lists into c64,
// and with 32-row blocks the state's 32-row mask and lists as well.
int run_select(const Shape& sh, const void* q, const void* k, const float* scores,
               const int32_t* q_idx, const int32_t* k_idx, const asa_state* st, const Csr64& c64,
               void* workspace, hipStream_t s) {
  asa::SelectParams sp{};
  sp.tkv = static_cast<float*>(workspace);
  sp.kbounds = reinterpret_cast<int2*>(static_cast<char*>(workspace) + tkv_bytes(sh));
  if (int rc = select_cap(sh, scores != nullptr, &sp.cap)) return rc;
  sp.d = dims_of(sh);
  if (sh.exact) {
    // the refine pass's key lists: checked before anything is launched
    int dev = 0, max_lds = 0;
    if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
    if (int rc = check_hip(hipDeviceGetAttribute(&max_lds,
                                                 hipDeviceAttributeMaxSharedMemoryPerBlock, dev),
                           "hipDeviceGetAttribute"))
      return rc;
    sp.lcap = asa::refine_list_capacity(sp.d, sh.dtype, size_t(max_lds));
    if (sp.lcap < 0)
      return fail(ASA_ERR_UNSUPPORTED,
                  "exact tau mode needs %zu bytes of LDS per block, device has %d",
                  asa::refine_lds_bytes(sp.d, sh.dtype, 0), max_lds);
  }
  sp.q = q;
  sp.k = k;
  sp.lq = sh.lq;
  sp.lk = sh.lk;
  sp.scores = scores;
  sp.q_idx = q_idx;
  sp.k_idx = k_idx;
  sp.taus = st->taus;
  sp.mask = c64.mask;
  sp.half = sh.bm == 32 ? st->mask : nullptr;
  sp.topk_idx = st->topk_idx;
  sp.topk_val = st->topk_val;
  sp.status = st->status;
  asa::profile_begin("bounds", s);
  hipError_t eb = asa::launch_bounds(sp, s);
  asa::profile_end(s);
  if (int rc = check_hip(eb, "bounds kernel launch")) return rc;
  asa::profile_begin(scores ? "select_scores" : "select", s);
  hipError_t e = asa::launch_select(sp, sh.dtype, scores != nullptr, s);
  asa::profile_end(s);
  if (int rc = check_hip(e, "select kernel launch")) return rc;
  asa::CompactParams cp{sh.BH, sh.nQB, sh.nKB, c64.mask, c64.q_ptr, c64.q_list, c64.k_ptr,
                        c64.k_list};
  if (sh.exact) {
    asa::profile_begin("tau", s);
    e = asa::launch_tau(sp, s);
    asa::profile_end(s);
    if (int rc = check_hip(e, "tau kernel launch")) return rc;
    // exact threshold over the whole row; adds the support's key blocks
    asa::profile_begin("refine", s);
    e = asa::launch_refine(sp, sh.dtype, s);
    asa::profile_end(s);
    if (int rc = check_hip(e, "refine kernel launch")) return rc;
    asa::profile_begin("compact", s);
    e = asa::launch_compact(cp, s);
    asa::profile_end(s);
    if (int rc = check_hip(e, "compact kernel launch")) return rc;
  } else {
    // the mask is final after the score pass: tau and the lists in one launch
    asa::profile_begin("tau_compact", s);
    e = asa::launch_tau_compact(sp, cp, s);
    asa::profile_end(s);
    if (int rc = check_hip(e, "tau/compact kernel launch")) return rc;
  }
  if (sh.bm == 32) {
    asa::CompactParams cm{sh.BH, sh.nQBm, sh.nKB, st->mask, st->q_ptr, st->q_list, st->k_ptr,
                          st->k_list};
    asa::profile_begin("compact_m", s);
    e = asa::launch_compact(cm, s);
    asa::profile_end(s);
    if (int rc = check_hip(e, "compact kernel launch")) return rc;
  }
  return ASA_OK;
}

}  // namespace

namespace asa {

void profile_begin(const char* name, hipStream_t s) {
  g_open = -1;
  if (!g_prof.load(std::memory_order_relaxed)) return;
  Rec r{name, nullptr, nullptr, s};
  if (hipEventCreate(&r.start) != hipSuccess) return;
  if (hipEventCreate(&r.stop) != hipSuccess) {
    hipEventDestroy(r.start);
    return;
  }
  hipEventRecord(r.start, s);
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_open = int(g_recs.size());
  g_recs.push_back(r);
}

void profile_end(hipStream_t s) {
  if (g_open < 0) return;
  hipEvent_t stop;
  {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    if (g_open >= int(g_recs.size())) {
      g_open = -1;
      return;
    }
    stop = g_recs[g_open].stop;
  }
  hipEventRecord(stop, s);
  g_open = -1;
}

}  // namespace asa

extern "C" {

int asa_abi_version(void) { return ASA_ABI_VERSION; }

const char* asa_last_error(void) { return g_error.c_str(); }

int asa_query_sizes(const asa_problem* p, asa_sizes* out) {
  Shape sh;
  if (int rc = validate(p, &sh)) return rc;
  if (!out) return fail(ASA_ERR_INVALID_ARGUMENT, "output pointer is NULL");
  sizes_of(sh, out);
  return ok();
}

}  // extern "C"

namespace {

// The forward's kernel sequence on `workspace` (asa_sizes.workspace bytes);
// the problem is already validated.
int forward_impl(const Shape& sh, const void* q, const void* k, const void* v,
                 const int32_t* q_idx, const int32_t* k_idx, void* out, const asa_state* st,
                 void* workspace, void* stream) {
  hipStream_t s = static_cast<hipStream_t>(stream);

  const Csr64 c64 = kernel_csr(sh, st, workspace, fwd_csr_offset(sh));
  if (int rc = run_select(sh, q, k, nullptr, q_idx, k_idx, st, c64, workspace, s)) return rc;

  asa::ForwardParams fp{};
  fp.d = dims_of(sh);
  fp.q = q;
  fp.k = k;
  fp.v = v;
  fp.lq = sh.lq;
  fp.lk = sh.lk;
  fp.lv = sh.lv;
  fp.lo = contiguous(sh.H, sh.NQ, sh.hd);
  fp.q_idx = q_idx;
  fp.k_idx = k_idx;
  fp.taus = st->taus;
  fp.q_ptr = c64.q_ptr;
  fp.q_list = c64.q_list;
  fp.half = sh.bm == 32 ? st->mask : nullptr;
  fp.top1 = static_cast<const float*>(workspace);  // slot 0 of the sorted top-k values
  fp.out = out;
  fp.norms = st->norms;
  fp.kbounds = reinterpret_cast<const int2*>(static_cast<const char*>(workspace) + tkv_bytes(sh));
  fp.sup.mask = st->sup_mask;
  fp.pairing = g_pairing.load();
  if (int rc = device_cus(&fp.cus)) return rc;
  asa::profile_begin("forward", s);
  hipError_t e = asa::launch_forward(fp, sh.dtype, s);
  asa::profile_end(s);
  if (int rc = check_hip(e, "forward kernel launch")) return rc;
  return ok();
}

// Workspace of asa_forward_noalloc: a file-scope device array (each GPU the
// library runs on holds its own copy until the process ends).  In host code
// `scratch` only names the symbol; its device address comes from
// hipGetSymbolAddress, once per device, and only that address is passed on.
constexpr size_t kScratchBytes = size_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's `scratch`.
int scratch_address(void** ptr) {
  int dev = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev < 0 || dev >= kMaxDevices)
    return fail(ASA_ERR_UNSUPPORTED, "device ordinal %d above %d", dev, kMaxDevices - 1);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* a = nullptr;
    if (int rc = check_hip(hipGetSymbolAddress(&a, HIP_SYMBOL(scratch)), "hipGetSymbolAddress"))
      return rc;
    g_scratch_ptr[dev] = a;
  }
  *ptr = g_scratch_ptr[dev];
  return ASA_OK;
}

}  // namespace

extern "C" {

int asa_forward(const asa_problem* p, const void* q, const void* k, const void* v,
                const int32_t* q_idx, const int32_t* k_idx, void* out, const asa_state* st,
                void* workspace, void* stream) {
  Shape sh;
  if (int rc = validate(p, &sh)) return rc;
  if (!q || !k || !v || !q_idx || !k_idx || !out)
    return fail(ASA_ERR_INVALID_ARGUMENT, "a tensor argument is NULL");
  if (int rc = check_aligned({q, k, v, out})) return rc;
  if (int rc = check_state(st, true)) return rc;
  if (!workspace) return fail(ASA_ERR_INVALID_ARGUMENT, "workspace is NULL");
  return forward_impl(sh, q, k, v, q_idx, k_idx, out, st, workspace, stream);
}

int asa_forward_noalloc(const asa_problem* p, const void* q, const void* k, const void* v,
                        const int32_t* q_idx, const int32_t* k_idx, void* out,
                        const asa_state* st, void* stream) {
  Shape sh;
  if (int rc = validate(p, &sh)) return rc;
  asa_sizes z;
  sizes_of(sh, &z);
  if (z.workspace > kScratchBytes)
    return fail(ASA_ERR_UNSUPPORTED,
                "problem needs %zu bytes of workspace; asa_forward_noalloc holds %zu "
                "(use asa_forward with a caller-owned workspace)",
                z.workspace, kScratchBytes);
  if (!q || !k || !v || !q_idx || !k_idx || !out)
    return fail(ASA_ERR_INVALID_ARGUMENT, "a tensor argument is NULL");
  if (int rc = check_aligned({q, k, v, out})) return rc;
  if (int rc = check_state(st, true)) return rc;
  void* ws = nullptr;
  if (int rc = scratch_address(&ws)) return rc;
  return forward_impl(sh, q, k, v, q_idx, k_idx, out, st, ws, stream);
}

int asa_backward(const asa_problem* p, int32_t grad_mode, const void* q, const void* k,
                 const void* v, const int32_t* q_idx, const int32_t* k_idx, const void* out,
                 const void* dout, const asa_state* st, void* dq, void* dk, void* dv,
                 void* workspace, void* stream) {
  Shape sh;
  if (int rc = validate(p, &sh)) return rc;
  if (grad_mode != ASA_GRAD_ENTMAX && grad_mode != ASA_GRAD_REFERENCE)
    return fail(ASA_ERR_INVALID_ARGUMENT, "unknown grad_mode %d", grad_mode);
  if (!q || !k || !v || !q_idx || !k_idx || !dout || !dq || !dk || !dv)
    return fail(ASA_ERR_INVALID_ARGUMENT, "a tensor argument is NULL");
  if (grad_mode == ASA_GRAD_REFERENCE && !out)
    return fail(ASA_ERR_INVALID_ARGUMENT, "reference-gradient mode needs the forward output");
  if (int rc = check_aligned({q, k, v, out, dout, dq, dk, dv})) return rc;
  if (!workspace) return fail(ASA_ERR_INVALID_ARGUMENT, "workspace is NULL");
  if (int rc = check_state(st, true)) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);

  asa::BackwardParams bp{};
  bp.d = dims_of(sh);
  bp.mode = grad_mode;
  bp.q = q;
  bp.k = k;
  bp.v = v;
  bp.out = out;
  bp.dout = dout;
  bp.lq = sh.lq;
  bp.lk = sh.lk;
  bp.lv = sh.lv;
  bp.ldo = sh.ldo;
  bp.lo = contiguous(sh.H, sh.NQ, sh.hd);
  bp.ldq = contiguous(sh.H, sh.NQ, sh.hd);
  bp.ldk = contiguous(sh.H, sh.NK, sh.hd);
  bp.ldv = contiguous(sh.H, sh.NK, sh.hd);
  bp.q_idx = q_idx;
  bp.k_idx = k_idx;
  bp.taus = st->taus;
  bp.norms = st->norms;
  // with 32-row blocks, the 64-row union and its lists first (the same
  // kernels as the forward's, so the tiles' list positions, which index the
  // support masks, are the forward's)
  const Csr64 c64 = kernel_csr(sh, st, workspace, bwd_csr_offset(sh));
  if (sh.bm == 32) {
    asa::profile_begin("fold_halves", s);
    hipError_t ef = asa::launch_fold_halves(st->mask, c64.mask, sh.BH, sh.NQ, sh.nQB, sh.nKB, s);
    asa::profile_end(s);
    if (int rc = check_hip(ef, "fold kernel launch")) return rc;
    asa::CompactParams cp{sh.BH, sh.nQB, sh.nKB, c64.mask, c64.q_ptr, c64.q_list, c64.k_ptr,
                          c64.k_list};
    asa::profile_begin("compact", s);
    ef = asa::launch_compact(cp, s);
    asa::profile_end(s);
    if (int rc = check_hip(ef, "compact kernel launch")) return rc;
  }
  bp.mask = c64.mask;
  bp.half = sh.bm == 32 ? st->mask : nullptr;
  bp.q_ptr = c64.q_ptr;
  bp.q_list = c64.q_list;
  bp.k_ptr = c64.k_ptr;
  bp.k_list = c64.k_list;
  bp.delta = static_cast<float*>(workspace);
  bp.dq = dq;
  bp.dk = dk;
  bp.dv = dv;
  bp.sup.mask = st->sup_mask;
  bp.rowrec = reinterpret_cast<asa::RowRec*>(static_cast<char*>(workspace) + bwd_rec_offset(sh));
  bp.posmap = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) + bwd_map_offset(sh));

  hipError_t e;
  if (grad_mode == ASA_GRAD_REFERENCE) {
    asa::profile_begin("bwd_delta", s);
    e = asa::launch_bwd_delta(bp, sh.dtype, s);
    asa::profile_end(s);
    if (int rc = check_hip(e, "backward delta kernel launch")) return rc;
  }
  if (bp.sup.mask) {
    // support masks: only the listed (row, key) pairs
    asa::profile_begin("bwd_dq_sparse", s);
    e = asa::launch_bwd_dq_sparse(bp, sh.dtype, s);
    asa::profile_end(s);
    if (int rc = check_hip(e, "backward sparse dQ kernel launch")) return rc;
    asa::profile_begin("bwd_dkdv_sparse", s);
    e = asa::launch_bwd_dkdv_sparse(bp, sh.dtype, s);
    asa::profile_end(s);
    if (int rc = check_hip(e, "backward sparse dK/dV kernel launch")) return rc;
    return ok();
  }
  asa::profile_begin("bwd_dq", s);
  e = asa::launch_bwd_dq(bp, sh.dtype, s);
  asa::profile_end(s);
  if (int rc = check_hip(e, "backward dQ kernel launch")) return rc;
  asa::profile_begin("bwd_dkdv", s);
  e = asa::launch_bwd_dkdv(bp, sh.dtype, s);
  asa::profile_end(s);
  if (int rc = check_hip(e, "backward dK/dV kernel launch")) return rc;
  return ok();
}

int asa_select_from_scores(const asa_problem* p, const float* scores, const int32_t* q_idx,
                           const int32_t* k_idx, const asa_state* st, void* workspace,
                           void* stream) {
  Shape sh;
  if (int rc = validate(p, &sh)) return rc;
  if (sh.exact)
    return fail(ASA_ERR_UNSUPPORTED, "exact tau mode needs Q and K (asa_forward)");
  if (!scores || !q_idx || !k_idx)
    return fail(ASA_ERR_INVALID_ARGUMENT, "a tensor argument is NULL");
  if (int rc = check_state(st, false)) return rc;
  if (!workspace) return fail(ASA_ERR_INVALID_ARGUMENT, "workspace is NULL");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const Csr64 c64 = kernel_csr(sh, st, workspace, fwd_csr_offset(sh));
  if (int rc = run_select(sh, nullptr, nullptr, scores, q_idx, k_idx, st, c64, workspace, s))
    return rc;
  return ok();
}

int asa_set_pairing(int mode) {
  if (mode != ASA_PAIRING_AUTO && mode != ASA_PAIRING_ALWAYS && mode != ASA_PAIRING_NEVER)
    return fail(ASA_ERR_INVALID_ARGUMENT, "unknown pairing mode %d", mode);
  g_pairing.store(mode);
  return ok();
}

int asa_profile_enable(int on) {
  g_prof = on != 0;
  return ok();
}

int asa_profile_read(int max, char (*names)[64], int* counts, double* total_ms) {
  struct Acc {
    const char* name;
    int n;
    double ms;
  };
  std::vector<Acc> acc;
  std::vector<Rec> recs;
  {
    std::lock_guard<std::mutex> lk(g_prof_mu);
    recs.swap(g_recs);
  }
  for (const Rec& r : recs) {
    float ms = 0.0f;
    if (hipEventSynchronize(r.stop) == hipSuccess) hipEventElapsedTime(&ms, r.start, r.stop);
    hipEventDestroy(r.start);
    hipEventDestroy(r.stop);
    bool found = false;
    for (Acc& a : acc)
      if (std::strcmp(a.name, r.name) == 0) {
        a.n += 1;
        a.ms += ms;
        found = true;
        break;
      }
    if (!found) acc.push_back(Acc{r.name, 1, double(ms)});
  }
  int n = 0;
  for (const Acc& a : acc) {
    if (n >= max) break;
    if (names) {
      std::strncpy(names[n], a.name, 63);
      names[n][63] = '\0';
    }
    if (counts) counts[n] = a.n;
    if (total_ms) total_ms[n] = a.ms;
    ++n;
  }
  ok();
  return n;
}

}  // extern "C"
