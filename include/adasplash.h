/*
 * adasplash.h -- C ABI of libadasplash, block-sparse alpha-entmax ("splash")
 * attention for AMD Instinct MI355X (gfx950).
 *
 * This is the drop-in boundary for the reference extension's native entry
 * points (mvideet/Adaptive-Splash-Attention, source/adasplashattention.cu):
 *
 *   asa_forward   replaces  forward_splash  (adasplashattention.cu:537-609,
 *                           bound as "forward" at :703)
 *   asa_backward  replaces  backward_splash (adasplashattention.cu:611-700,
 *                           bound as "backward" at :704)
 *
 * Differences from the reference boundary, all deliberate:
 *   - Plain pointers, sizes and a POD problem descriptor instead of torch
 *     tensors; the caller owns every buffer (outputs, per-call state and
 *     workspace) and the library never allocates device memory.
 *   - Work is launched on the caller's stream; nothing synchronises the
 *     device (the reference calls cudaDeviceSynchronize, :597 / :682).
 *   - The forward returns its selection state (tau, row sums, block mask,
 *     CSR lists) so that the backward does not rebuild it (the reference
 *     recomputes the mask in backward, :669-676).
 *   - k_keep is a run-time argument (the reference fixes K_KEEP=8 at
 *     compile time, :17-19).
 *   - bf16 and fp16 are accepted besides fp32 (reference: fp32 only,
 *     :575-578); 16-bit inputs compute in fp32 with 16-bit MFMA operands.
 *
 * Semantics kept from the reference: visibility K_idx[j] <= Q_idx[i]
 * (:181); scores clamped to [-10, 10] (:195-197); alpha clamped to
 * [1.05, 3] (:547); top-k ties to the lower key index (:35-49); the
 * 5-step tau recurrence (:51-125); block mask = union over a query block
 * of its rows' top-k key blocks (:210-216); CSR in ascending key-block
 * order (:219-242); forward weights over active blocks (:244-341);
 * non-finite intermediate values replaced by zero (:75-77, :314-316,
 * :335-337, :505-507, :529-531).
 *
 * All functions return ASA_OK (0) or an asa_status error code; the message
 * of the last error on the calling thread is available from
 * asa_last_error().
 */
#ifndef ADASPLASH_H
#define ADASPLASH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ASA_ABI_VERSION 8

typedef enum asa_status {
  ASA_OK = 0,
  ASA_ERR_INVALID_ARGUMENT = 1, /* shape, pointer or parameter out of range   */
  ASA_ERR_UNSUPPORTED = 2,      /* valid but not implemented (e.g. head_dim)  */
  ASA_ERR_DEVICE = 3            /* a HIP runtime call failed                  */
} asa_status;

typedef enum asa_dtype { ASA_DTYPE_F32 = 0, ASA_DTYPE_BF16 = 1, ASA_DTYPE_F16 = 2 } asa_dtype;

typedef enum asa_tau_mode {
  /* The reference's threshold: its 5-step recurrence on the row's top-k
   * scores (adasplashattention.cu:51-125); block mask = union of the rows'
   * top-k key blocks (:210-216).                                          */
  ASA_TAU_REFERENCE = 0,
  /* The alpha-entmax threshold over every visible key of the row (dense
   * alpha-entmax), found by safeguarded Newton steps started from the
   * top-k root; key blocks holding a key with u > 0 at that threshold are
   * added to the mask, so the forward weights the exact alpha-entmax
   * support.  No reference counterpart (the reference has only the top-k
   * threshold); asa_forward only.                                         */
  ASA_TAU_EXACT = 1
} asa_tau_mode;

typedef enum asa_grad_mode {
  /* ds = g (dp - sum(g dp)/sum(g)), g = P^(2-alpha): the alpha-entmax
   * Jacobian applied to the forward's normalised weights.               */
  ASA_GRAD_ENTMAX = 0,
  /* The gradient the reference kernel computes (adasplashattention.cu:343-535):
   * tau held fixed, ds = p^(2-alpha) (dp - out.dO) / (sum p + EPS).      */
  ASA_GRAD_REFERENCE = 1
} asa_grad_mode;

/* Problem descriptor.  Q, Out, dOut, dQ: [batch, heads, nq, head_dim];
 * K, V, dK, dV: [batch, heads, nk, head_dim], row-major with the head
 * dimension contiguous.  Out, dQ, dK and dV are contiguous; Q, K, V and
 * dOut may have any batch, head and row strides (q_strides ... below).
 * Every tensor pointer is 16-byte aligned.
 * Q_idx: [batch*heads, nq], K_idx: [batch*heads, nk], int32 positions.
 * Reference argument list: forward_splash(Q, K, V, Q_idx, K_idx, sm_scale,
 * alpha) (adasplashattention.cu:537-541).                                 */
typedef struct asa_problem {
  int32_t batch;
  int32_t heads;
  int32_t nq;
  int32_t nk;
  int32_t head_dim; /* <= 128 (reference limit, :542), a multiple of 8
                     * for bf16 / fp16 and of 4 for fp32 (one 16-byte
                     * chunk); the kernels compute at 64 (head_dim <= 64)
                     * or 128 and never touch the columns past head_dim */
  int32_t k_keep;   /* 1..128 (reference: compile-time 8, :17-19)        */
  int32_t block_m;  /* query rows per mask block: 64, or 32 (the
                     * reference's BLOCK_M, :8-9; reference tau mode
                     * only): the mask and CSR lists of the state are
                     * then per 32 rows, as the reference's            */
  int32_t block_n;  /* keys per mask block: 64                            */
  float alpha;      /* clamped to [1.05, 3]                               */
  float sm_scale;
  int32_t dtype;    /* asa_dtype of Q, K, V, Out, dOut, dQ, dK, dV        */
  int32_t tau_mode; /* asa_tau_mode (asa_forward; ignored by asa_backward) */
  /* Element strides {batch, head, row} of Q, K, V and dOut (dout_strides:
   * asa_backward only).  {0, 0, 0}: contiguous, {heads*n*head_dim,
   * n*head_dim, head_dim}.  Otherwise each stride is >= 0 and a multiple of
   * 8 elements for bf16 / fp16, 4 for fp32, and a head's rows lie within
   * 2^31 bytes of its first ((n - 1) * row stride + head_dim elements), so
   * that views such as a [batch, n, heads, head_dim] tensor transposed to
   * [batch, heads, n, head_dim], or K and V shared across heads (head
   * stride 0), are read in place.  The stride of a dimension of size 1 is
   * not used.  {0, 0, 0} always means contiguous, so an operand broadcast
   * along all three (every stride 0) is passed materialised.  No
   * reference counterpart (the reference
   * reads contiguous tensors through data_ptr, adasplashattention.cu:
   * 568-571).                                                            */
  int64_t q_strides[3];
  int64_t k_strides[3];
  int64_t v_strides[3];
  int64_t dout_strides[3];
} asa_problem;

/* Per-call selection state written by asa_forward (and by
 * asa_select_from_scores) and read by asa_backward.  Sizes in elements,
 * nQB = ceil(nq / block_m), nKB = ceil(nk / block_n), BH = batch*heads:
 *   taus     float   [BH, nq]       tau of every query row
 *   norms    float   [BH, nq]       sum of weights p of every row
 *   mask     uint8   [BH, nQB, nKB] 1 where a key block is active
 *   q_ptr    int32   [BH, nQB + 1]  query-major CSR offsets (reference Qi_ptr)
 *   q_list   int32   [BH, nQB*nKB]  ascending active key blocks (reference Qi_idx;
 *                                   unused tail zero)
 *   k_ptr    int32   [BH, nKB + 1]  key-major CSR offsets
 *   k_list   int32   [BH, nKB*nQB]  ascending query blocks per key block
 *   topk_idx int32   [BH, nq, k_keep] optional (NULL): row top-k key indices,
 *                                   best first, -1 in empty slots
 *   topk_val float   [BH, nq, k_keep] optional (NULL): matching scores,
 *                                   -1e6 in empty slots
 * Support masks, optional (NULL: not written, and the backward computes
 * every active block densely):
 *   sup_mask uint16  [BH, nQ64*nKB, 4, 64], nQ64 = ceil(nq / 64): for the
 *                                   tile at the head's position e of the
 *                                   64-row list (q_list itself when
 *                                   block_m = 64; with block_m = 32 the
 *                                   list of the union of mask rows 2i and
 *                                   2i + 1, which the library derives in
 *                                   its workspace) (64-row query block
 *                                   qb, key block
 *                                   kb), bit 4f + r of element [e][w][4c + g]
 *                                   is set iff the forward weighted row
 *                                   qb*64 + 16w + c, key kb*64 + 16f + 4g + r
 *                                   with u = (alpha-1) s - tau > 0
 *                                   (w, c < 16; g, f, r < 4).  These are
 *                                   the rows' exact supports, on which
 *                                   every backward term lives: with them
 *                                   the backward visits only those pairs.
 * Status word, optional (NULL: not written):
 *   status   uint32  [1]            written by asa_forward and
 *                                   asa_select_from_scores on the stream
 *                                   (cleared by their first kernel): the
 *                                   ASA_STATUS_* bits below, and in bits
 *                                   8-15 the largest number of candidate
 *                                   overflow rounds a query block of the
 *                                   score pass ran (saturating at 255).  Read
 *                                   it after the call has completed (e.g.
 *                                   in a debug check); the call itself never
 *                                   synchronises.
 */
/* Score pass: a query block's candidate rounds reached their proven bound
 * (2 + (nk - cap) / (cap - k) rounds always suffice; set only if that proof
 * were wrong, never observed).  Top-k of that block may be incomplete.     */
#define ASA_STATUS_SELECT_ROUNDS 0x1u
/* tau_mode = ASA_TAU_EXACT: a row's Newton iteration reached the refine
 * pass's sweep cap before |f| <= 1e-6; its tau is the last iterate.        */
#define ASA_STATUS_REFINE_SWEEPS 0x2u
typedef struct asa_state {
  float *taus;
  float *norms;
  uint8_t *mask;
  int32_t *q_ptr;
  int32_t *q_list;
  int32_t *k_ptr;
  int32_t *k_list;
  int32_t *topk_idx;
  float *topk_val;
  uint16_t *sup_mask;
  uint32_t *status;
} asa_state;

/* Byte sizes of every state buffer and of the workspace the entry points
 * need for this problem.                                                   */
typedef struct asa_sizes {
  size_t taus, norms, mask, q_ptr, q_list, k_ptr, k_list, topk_idx, topk_val;
  size_t sup_mask;
  size_t workspace;
} asa_sizes;

/* ABI version of the loaded library (ASA_ABI_VERSION when it matches).     */
int asa_abi_version(void);

/* Message of the last failed call on this thread ("" if none).            */
const char *asa_last_error(void);

/* Validates *p and fills *out.  Host-only; no device call.                 */
int asa_query_sizes(const asa_problem *p, asa_sizes *out);

/* Forward pass (reference: forward_splash, adasplashattention.cu:537-609):
 * score pass (QK^T on MFMA, top-k, tau, block mask), with p->tau_mode ==
 * ASA_TAU_EXACT the exact-threshold pass (tau over the whole row, support
 * blocks added to the mask), CSR compaction and the block-sparse weighted
 * sum.  Writes `out` and every non-NULL field of *st.
 * `workspace` must hold asa_sizes.workspace bytes.  `stream` is a
 * hipStream_t (NULL: the null stream).                                     */
int asa_forward(const asa_problem *p, const void *q, const void *k, const void *v,
                const int32_t *q_idx, const int32_t *k_idx, void *out, const asa_state *st,
                void *workspace, void *stream);

/* asa_forward without a workspace argument.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Its workspace is a file-scope device array of the library
 * of ASA_NOALLOC_WORKSPACE_BYTES, one per GPU, held until the process ends;
 * the call allocates nothing.  Problems whose asa_sizes.workspace exceeds it
 * (batch*heads*nq*k_keep*4 + batch*heads*ceil(nk/64)*8 bytes, rounded; the
 * B4 H16 N4096 k32 shape needs 33.6 MB) fail with ASA_ERR_UNSUPPORTED.
 * Every call on one GPU shares that GPU's array: calls that overlap on one
 * GPU (other streams or threads) race.  Same outputs as asa_forward.       */
#define ASA_NOALLOC_WORKSPACE_BYTES (64u << 20)
int asa_forward_noalloc(const asa_problem *p, const void *q, const void *k, const void *v,
                        const int32_t *q_idx, const int32_t *k_idx, void *out,
                        const asa_state *st, void *stream);

/* Backward pass (reference: backward_splash, adasplashattention.cu:611-700)
 * from the state a matching asa_forward wrote.  `out` is that forward's
 * output (read in ASA_GRAD_REFERENCE mode only; may be NULL otherwise).
 * Writes dq, dk, dv (overwritten, not accumulated).  Deterministic: no
 * atomics, fixed reduction order.                                          */
int asa_backward(const asa_problem *p, int32_t grad_mode, const void *q, const void *k,
                 const void *v, const int32_t *q_idx, const int32_t *k_idx, const void *out,
                 const void *dout, const asa_state *st, void *dq, void *dk, void *dv,
                 void *workspace, void *stream);

/* Selection from given scores (no reference counterpart; it exposes the
 * reference's selection stage, adasplashattention.cu:199-216, for checking
 * on identical inputs).  scores: float [BH, nq, nk], clamped to [-10, 10]
 * by the kernel; visibility from q_idx / k_idx as in asa_forward.  Writes
 * taus, mask, q_ptr, q_list, k_ptr, k_list and the optional top-k arrays;
 * norms is not touched.                                                    */
int asa_select_from_scores(const asa_problem *p, const float *scores, const int32_t *q_idx,
                           const int32_t *k_idx, const asa_state *st, void *workspace,
                           void *stream);

/* Kernel timing for benchmarks (no reference counterpart).  While enabled
 * (process-wide), every kernel launch of the library is bracketed by HIP
 * events recorded on its launch stream; asa_profile_read() synchronises on
 * them and reports, per kernel name, the number of launches and the summed
 * duration in milliseconds, then clears the record.  Call it when no other
 * thread is launching.  Returns the number of distinct kernels (<= max).  */
/* Which forward kernel runs for 16-bit inputs (no reference counterpart;
 * for tuning and tests): ASA_PAIRING_AUTO (default) runs two query blocks
 * per workgroup when those workgroups fill at least one wave of the GPU
 * (three per compute unit at head_dim <= 64, two above) and one block per
 * workgroup otherwise; ASA_PAIRING_ALWAYS pairs wherever the paired
 * kernel applies; ASA_PAIRING_NEVER never pairs.  The two kernels give
 * the same results to the last ulps.  Process-wide; read by each
 * asa_forward / asa_forward_noalloc call. */
typedef enum asa_pairing {
  ASA_PAIRING_AUTO = 0,
  ASA_PAIRING_ALWAYS = 1,
  ASA_PAIRING_NEVER = 2
} asa_pairing;
int asa_set_pairing(int mode);

int asa_profile_enable(int on);
int asa_profile_read(int max, char (*names)[64], int *counts, double *total_ms);

#ifdef __cplusplus
}
#endif

#endif /* ADASPLASH_H */
