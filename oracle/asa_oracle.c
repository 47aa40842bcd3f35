/*
 * asa_oracle.c -- CPU oracle for block-sparse alpha-entmax ("splash") attention.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates, in plain C, the algorithm of
 * the reference extension (source/adasplashattention.cu of
 * mvideet/Adaptive-Splash-Attention) so that tests/, __graft_entry__.smoke()
 * and the cpu_baseline leg of bench.py can check the HIP product against it.
 * The product library (libadasplash.so) never links, loads or calls this code.
 *
 * It is compiled twice (oracle/Makefile):
 *   liboracle_f32.so : `real` = float.  The selection recurrence (top-k order,
 *                      tau iteration, u and p) follows the reference's fp32
 *                      arithmetic step by step; reductions over keys are
 *                      accumulated in double so that the oracle is at least
 *                      as accurate as any summation order the GPU may pick.
 *   liboracle_f64.so : `real` = double.  Same recurrences in fp64; used for
 *                      finite-difference checks of the two gradients.
 *
 * Conventions shared with the HIP kernels (so that the two agree bit-for-bit
 * on the tau recurrence when they see the same top-k values):
 *   - no floating-point contraction: every a*b+c below is two roundings
 *     (the Makefile passes -ffp-contract=off);
 *   - x^e for x > 0 is evaluated by pow_pos(): exact small-integer exponents
 *     use a double-precision product chain rounded once to `real`, other
 *     exponents use double pow() rounded once.  The reference calls powf();
 *     this is the same function up to the last-ulp rounding of the libm in
 *     use, which is not reproducible across toolchains anyway.
 *
 * Semantics (reference file:line citations are to source/adasplashattention.cu):
 *   visibility  key j visible to query i iff K_idx[j] <= Q_idx[i]     (:181, :189)
 *   score       s = clamp(sm_scale * (q . k), -10, 10)                 (:190-197)
 *   top-k       first k of the keys ordered by (score desc, index asc);
 *               empty slots hold score -1e6 and index -1              (:35-49, :166-172)
 *   tau         5-step Halley/bisection recurrence on the top-k values (:51-125)
 *   mask        M[qb][j/block_n] = 1 for every top-k index of every row
 *               of query block qb                                      (:210-216)
 *   CSR         q_ptr = prefix of row popcounts, q_list = ascending
 *               active key blocks per query block                      (:219-242)
 *   forward     p = (u > 0) ? max(u,EPS)^(1/(a-1)) : 0 with
 *               u = (a-1)s - tau over visible keys of active blocks;
 *               out = sum p v / (sum p + EPS)                          (:244-341)
 *   backward    mode 1 ("reference"): the gradient the reference kernel
 *               computes (tau held fixed, renormalised p)              (:343-535)
 *               mode 0 ("entmax"): ds = g (dp - sum g dp / sum g) with
 *               g = P^(2-a), P = p / (sum p + EPS), dp = dO . v.
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef ASAO_DOUBLE
typedef double real;
#define ASAO_REAL_BYTES 8
#else
typedef float real;
#define ASAO_REAL_BYTES 4
#endif

#define ASAO_ABI 4
#define ASAO_EPS ((real)1e-8f)
#define ASAO_TAU_ITERS 5
#define ASAO_SENTINEL_S ((real)-1e6f)

int asao_abi_version(void) { return ASAO_ABI; }
/* Thread count of the OpenMP regions that follow (the CPU baseline times one
 * thread and the host's share). */
void asao_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int asao_max_threads(void) { return omp_get_max_threads(); }
int asao_real_bytes(void) { return ASAO_REAL_BYTES; }

static real rmax(real a, real b) { return a > b ? a : (b != b ? a : b); }
static real rmin(real a, real b) { return a < b ? a : (b != b ? a : b); }
static int rfinite(real x) { return isfinite(x); }

/* x^e for x > 0, rounded once to `real` (see header). */
static real pow_pos(real x, real e)
{
    double xd = (double)x;
    if (e == (real)2) return (real)(xd * xd);
    if (e == (real)1) return x;
    if (e == (real)0) return (real)1;
    if (e == (real)3) return (real)(xd * xd * xd);
    if (e == (real)4) { double x2 = xd * xd; return (real)(x2 * x2); }
    if (e == (real)-1) return (real)(1.0 / xd);
    return (real)pow(xd, (double)e);
}

/* alpha as the reference sees it: clamped to [1.05, 3] (:52, :547). */
static real clamp_alpha(real a)
{
    return rmax((real)1.05f, rmin(a, (real)3.0f));
}

/*
 * tau for one row from its top-k values s[0..k-1] (descending, sentinel
 * -1e6 in unused slots).  Follows the reference recurrence (:51-125):
 * bracket from the smallest and largest kept value, midpoint start, at most
 * five rounds of {evaluate f, f', f''; stop if |f| < 1e-4; Halley step;
 * fall back to the bracket midpoint when the step leaves the bracket;
 * re-evaluate f at the new point and shrink the bracket; clamp tau}.
 * Two details are kept as the reference has them: f'' uses the coefficient
 * a(a + 1 - alpha) with a = 1/(alpha-1), and every term loop stops at the
 * first non-positive u.
 */
real asao_entmax_threshold(const real *s, int k, real alpha_in)
{
    const real alpha = clamp_alpha(alpha_in);
    const real am1 = alpha - (real)1;
    const real a = (real)1 / am1;
    const real e1 = ((real)2 - alpha) * a;          /* exponent of f' terms  */
    const real e2 = ((real)3 - (real)2 * alpha) * a; /* exponent of f'' terms */
    const real c2 = a * ((a + (real)1) - alpha);     /* f'' coefficient       */
    const real top = s[0];
    const real bottom = s[k - 1];
    real lo = am1 * bottom - (real)2;
    real hi = am1 * top + (real)2;
    real tau = (real)0.5f * (lo + hi);

    for (int it = 0; it < ASAO_TAU_ITERS; ++it) {
        real f = (real)-1, df = (real)0, d2f = (real)0;
        for (int j = 0; j < k; ++j) {
            const real u = am1 * s[j] - tau;
            if (u <= (real)0) break;
            const real ue = rmax(u, ASAO_EPS);
            real t = pow_pos(ue, a);
            if (!rfinite(t)) t = (real)0;
            f = f + t;
            const real t1 = -a * pow_pos(ue, e1);
            if (rfinite(t1)) df = df + t1;
            const real t2 = c2 * pow_pos(ue, e2);
            if (rfinite(t2)) d2f = d2f + t2;
        }
        if (fabs(f) < (real)1e-4f) break;

        real next = tau;
        if (fabs(df) > ASAO_EPS) {
            const real den = (real)2 * df * df - f * d2f;
            if (fabs(den) > ASAO_EPS)
                next = tau - (real)2 * f * df / den;
        }
        if (!(next >= lo && next <= hi)) next = (real)0.5f * (lo + hi);

        real g = (real)-1;
        for (int j = 0; j < k; ++j) {
            const real u = am1 * s[j] - next;
            if (u <= (real)0) break;
            const real t = pow_pos(rmax(u, ASAO_EPS), a);
            if (rfinite(t)) g = g + t;
        }
        if (g > (real)0) lo = next; else hi = next;

        tau = next;
        tau = rmax(tau, bottom * am1 - (real)10);
        tau = rmin(tau, top * am1 + (real)10);
    }
    return tau;
}

/* score of one (query, key) pair: dot in double, rounded, scaled, clamped. */
static real score_of(const real *q, const real *kr, int d, real scale)
{
    double acc = 0.0;
    for (int t = 0; t < d; ++t) acc += (double)q[t] * (double)kr[t];
    real s = (real)acc * scale;
    s = rmax(s, (real)-10);
    s = rmin(s, (real)10);
    return s;
}

/*
 * Full score matrix S[bh][i][j] and visibility vis[bh][i][j].
 * Invisible entries get S = 0 and vis = 0.
 */
void asao_scores(const real *Q, const real *K, const int32_t *qidx, const int32_t *kidx,
                 int BH, int NQ, int NK, int d, real scale, real *S, uint8_t *vis)
{
    #pragma omp parallel for schedule(static)
    for (long r = 0; r < (long)BH * NQ; ++r) {
        const long bh = r / NQ;
        const real *q = Q + r * d;
        const int32_t qpos = qidx[r];
        for (int j = 0; j < NK; ++j) {
            const long kj = bh * NK + j;
            const int ok = kidx[kj] <= qpos;
            vis[r * NK + j] = (uint8_t)ok;
            S[r * NK + j] = ok ? score_of(q, K + kj * d, d, scale) : (real)0;
        }
    }
}

/*
 * Running top-k of one row: the kept list is sorted by score descending;
 * a new (s, j) enters only if it is strictly greater than some kept score,
 * and lands after every kept entry with score >= s.  Scanning keys in
 * ascending index order therefore yields the first k keys under the order
 * (score desc, index asc), which is what the reference's insertion produces.
 */
static void topk_push(real s, int j, real *vals, int32_t *inds, int k)
{
    if (!(s > vals[k - 1])) return;
    int pos = k - 1;
    while (pos > 0 && s > vals[pos - 1]) {
        vals[pos] = vals[pos - 1];
        inds[pos] = inds[pos - 1];
        --pos;
    }
    vals[pos] = s;
    inds[pos] = j;
}

static void select_row(const real *srow, const uint8_t *vrow, int NK, int k, real alpha,
                       real *tau_out, int32_t *inds, real *vals)
{
    for (int i = 0; i < k; ++i) { vals[i] = ASAO_SENTINEL_S; inds[i] = -1; }
    for (int j = 0; j < NK; ++j)
        if (vrow[j]) topk_push(srow[j], j, vals, inds, k);
    *tau_out = asao_entmax_threshold(vals, k, alpha);
}

/*
 * Selection from given scores: per-row top-k (indices and values), tau,
 * and the block mask M[bh][qb][kb] (union over the rows of a query block
 * of the key blocks holding a top-k index).  `mask` must be zeroed by the
 * caller.  topk_idx / topk_val may be NULL.
 */
void asao_select(const real *S, const uint8_t *vis, int BH, int NQ, int NK, int k,
                 real alpha, int block_m, int block_n, real *taus, int32_t *topk_idx,
                 real *topk_val, uint8_t *mask)
{
    const int nQB = (NQ + block_m - 1) / block_m;
    const int nKB = (NK + block_n - 1) / block_n;
    #pragma omp parallel
    {
        int32_t *inds = (int32_t *)malloc(sizeof(int32_t) * (size_t)k);
        real *vals = (real *)malloc(sizeof(real) * (size_t)k);
        #pragma omp for schedule(static)
        for (long r = 0; r < (long)BH * NQ; ++r) {
            real tau;
            select_row(S + r * NK, vis + r * NK, NK, k, alpha, &tau, inds, vals);
            taus[r] = tau;
            if (topk_idx) memcpy(topk_idx + r * k, inds, sizeof(int32_t) * (size_t)k);
            if (topk_val) memcpy(topk_val + r * k, vals, sizeof(real) * (size_t)k);
            const long bh = r / NQ;
            const int qb = (int)(r % NQ) / block_m;
            uint8_t *mrow = mask + ((size_t)bh * nQB + qb) * nKB;
            for (int i = 0; i < k; ++i)
                if (inds[i] >= 0) mrow[inds[i] / block_n] = 1; /* benign race: all write 1 */
        }
        free(inds);
        free(vals);
    }
}

/*
 * Block mask -> query-major CSR (q_ptr[bh][nQB+1], q_list[bh][nQB*nKB],
 * ascending key blocks, unused tail zero) and key-major CSR
 * (k_ptr[bh][nKB+1], k_list[bh][nKB*nQB], ascending query blocks).
 */
void asao_csr(const uint8_t *mask, int BH, int nQB, int nKB, int32_t *q_ptr,
              int32_t *q_list, int32_t *k_ptr, int32_t *k_list)
{
    for (int bh = 0; bh < BH; ++bh) {
        const uint8_t *m = mask + (size_t)bh * nQB * nKB;
        int32_t *qp = q_ptr + (size_t)bh * (nQB + 1);
        int32_t *ql = q_list + (size_t)bh * nQB * nKB;
        int32_t *kp = k_ptr + (size_t)bh * (nKB + 1);
        int32_t *kl = k_list + (size_t)bh * nKB * nQB;
        memset(ql, 0, sizeof(int32_t) * (size_t)nQB * nKB);
        memset(kl, 0, sizeof(int32_t) * (size_t)nQB * nKB);
        int w = 0;
        qp[0] = 0;
        for (int i = 0; i < nQB; ++i) {
            for (int j = 0; j < nKB; ++j)
                if (m[(size_t)i * nKB + j]) ql[w++] = j;
            qp[i + 1] = w;
        }
        w = 0;
        kp[0] = 0;
        for (int j = 0; j < nKB; ++j) {
            for (int i = 0; i < nQB; ++i)
                if (m[(size_t)i * nKB + j]) kl[w++] = i;
            kp[j + 1] = w;
        }
    }
}

/* p for one score against tau, as the forward pass defines it (:311-316). */
static real weight_of(real s, real tau, real am1, real a)
{
    const real u = am1 * s - tau;
    if (!(u > (real)0)) return (real)0;
    real p = pow_pos(rmax(u, ASAO_EPS), a);
    if (!rfinite(p)) p = (real)0;
    return p;
}

/*
 * Forward output for given taus and query-major CSR.
 * norms[bh][i] = sum of p over the row (the denominator before +EPS).
 */
static void sparse_forward(const real *Q, const real *K, const real *V, const int32_t *qidx,
                           const int32_t *kidx, int BH, int NQ, int NK, int d, real alpha,
                           real scale, int block_m, int block_n, const real *taus,
                           const int32_t *q_ptr, const int32_t *q_list, real *norms, real *out)
{
    const int nQB = (NQ + block_m - 1) / block_m;
    const int nKB = (NK + block_n - 1) / block_n;
    const real am1 = clamp_alpha(alpha) - (real)1;
    const real a = (real)1 / am1;
    #pragma omp parallel
    {
        double *acc = (double *)malloc(sizeof(double) * (size_t)d);
        #pragma omp for schedule(static)
        for (long r = 0; r < (long)BH * NQ; ++r) {
            const long bh = r / NQ;
            const int i = (int)(r % NQ);
            const int qb = i / block_m;
            const int32_t *qp = q_ptr + bh * (nQB + 1);
            const int32_t *ql = q_list + bh * (long)nQB * nKB;
            const real *q = Q + r * d;
            const real tau = taus[r];
            double nsum = 0.0;
            for (int t = 0; t < d; ++t) acc[t] = 0.0;
            for (int e = qp[qb]; e < qp[qb + 1]; ++e) {
                const int kb = ql[e];
                for (int j = kb * block_n; j < (kb + 1) * block_n && j < NK; ++j) {
                    const long kj = bh * NK + j;
                    if (kidx[kj] > qidx[r]) continue;
                    const real p = weight_of(score_of(q, K + kj * d, d, scale), tau, am1, a);
                    if (p == (real)0) continue;
                    nsum += (double)p;
                    const real *v = V + kj * d;
                    for (int t = 0; t < d; ++t) acc[t] += (double)p * (double)v[t];
                }
            }
            norms[r] = (real)nsum;
            const double inv = 1.0 / (nsum + (double)ASAO_EPS);
            for (int t = 0; t < d; ++t) {
                real o = (real)(acc[t] * inv);
                if (!rfinite(o)) o = (real)0;
                out[r * d + t] = o;
            }
        }
        free(acc);
    }
}

/*
 * Whole forward pass: scores -> top-k / tau / mask -> CSR -> output.
 * If taus_in is non-NULL those taus are used for the output instead of the
 * recurrence (the mask still comes from the top-k indices); `taus` then
 * receives a copy.  topk_idx, topk_val may be NULL.  mask, q_ptr, q_list,
 * k_ptr, k_list are outputs sized as in asao_csr().
 */
void asao_forward(const real *Q, const real *K, const real *V, const int32_t *qidx,
                  const int32_t *kidx, int BH, int NQ, int NK, int d, real alpha, real scale,
                  int k, int block_m, int block_n, const real *taus_in, real *taus,
                  real *norms, int32_t *topk_idx, real *topk_val, uint8_t *mask,
                  int32_t *q_ptr, int32_t *q_list, int32_t *k_ptr, int32_t *k_list, real *out)
{
    const int nQB = (NQ + block_m - 1) / block_m;
    const int nKB = (NK + block_n - 1) / block_n;
    memset(mask, 0, (size_t)BH * nQB * nKB);
    #pragma omp parallel
    {
        int32_t *inds = (int32_t *)malloc(sizeof(int32_t) * (size_t)k);
        real *vals = (real *)malloc(sizeof(real) * (size_t)k);
        #pragma omp for schedule(static)
        for (long r = 0; r < (long)BH * NQ; ++r) {
            const long bh = r / NQ;
            const real *q = Q + r * d;
            for (int i = 0; i < k; ++i) { vals[i] = ASAO_SENTINEL_S; inds[i] = -1; }
            for (int j = 0; j < NK; ++j) {
                const long kj = bh * NK + j;
                if (kidx[kj] > qidx[r]) continue;
                topk_push(score_of(q, K + kj * d, d, scale), j, vals, inds, k);
            }
            taus[r] = taus_in ? taus_in[r] : asao_entmax_threshold(vals, k, alpha);
            if (topk_idx) memcpy(topk_idx + r * k, inds, sizeof(int32_t) * (size_t)k);
            if (topk_val) memcpy(topk_val + r * k, vals, sizeof(real) * (size_t)k);
            const int qb = (int)(r % NQ) / block_m;
            uint8_t *mrow = mask + ((size_t)bh * nQB + qb) * nKB;
            for (int i = 0; i < k; ++i)
                if (inds[i] >= 0) mrow[inds[i] / block_n] = 1;
        }
        free(inds);
        free(vals);
    }
    asao_csr(mask, BH, nQB, nKB, q_ptr, q_list, k_ptr, k_list);
    sparse_forward(Q, K, V, qidx, kidx, BH, NQ, NK, d, alpha, scale, block_m, block_n, taus,
                   q_ptr, q_list, norms, out);
}

/*
 * Backward for given taus and query-major CSR.  dQ, dK, dV are written
 * (zeroed first).  mode 0: entmax-Jacobian gradient; mode 1: the
 * gradient of the reference kernel (:343-535).  Non-finite contributions
 * are dropped and non-finite dQ set to zero, as the reference does; dK and
 * dV keep an overflowed (+-inf) sum and zero NaN.
 */
void asao_backward(const real *Q, const real *K, const real *V, const int32_t *qidx,
                   const int32_t *kidx, const real *dO, int BH, int NQ, int NK, int d,
                   real alpha, real scale, int block_m, int block_n, const real *taus,
                   const int32_t *q_ptr, const int32_t *q_list, int mode, real *dQ, real *dK,
                   real *dV)
{
    const int nQB = (NQ + block_m - 1) / block_m;
    const int nKB = (NK + block_n - 1) / block_n;
    const real alpha_c = clamp_alpha(alpha);
    const real am1 = alpha_c - (real)1;
    const real a = (real)1 / am1;
    const real ew = ((real)2 - alpha_c) / am1; /* exponent of u in p^(2-alpha) */

    #pragma omp parallel
    {
        double *acc = (double *)malloc(sizeof(double) * (size_t)d);
        double *dq = (double *)malloc(sizeof(double) * (size_t)d);
        double *gk = (double *)malloc(sizeof(double) * (size_t)NK * 2 * d);
        #pragma omp for schedule(dynamic, 1)
        for (int bh = 0; bh < BH; ++bh) {
            double *dk_acc = gk;
            double *dv_acc = gk + (size_t)NK * d;
            memset(gk, 0, sizeof(double) * (size_t)NK * 2 * d);
            const int32_t *qp = q_ptr + (long)bh * (nQB + 1);
            const int32_t *ql = q_list + (long)bh * nQB * nKB;
            for (int i = 0; i < NQ; ++i) {
                const long r = (long)bh * NQ + i;
                const int qb = i / block_m;
                const real *q = Q + r * d;
                const real *go = dO + r * d;
                const real tau = taus[r];
                /* pass 1: norm and unnormalised accumulator, as the forward */
                double nsum = 0.0;
                for (int t = 0; t < d; ++t) { acc[t] = 0.0; dq[t] = 0.0; }
                for (int e = qp[qb]; e < qp[qb + 1]; ++e) {
                    const int kb = ql[e];
                    for (int j = kb * block_n; j < (kb + 1) * block_n && j < NK; ++j) {
                        const long kj = (long)bh * NK + j;
                        if (kidx[kj] > qidx[r]) continue;
                        const real p = weight_of(score_of(q, K + kj * d, d, scale), tau, am1, a);
                        nsum += (double)p;
                        for (int t = 0; t < d; ++t) acc[t] += (double)p * (double)V[kj * d + t];
                    }
                }
                const double invn = 1.0 / (nsum + (double)ASAO_EPS);
                /* row constants */
                double shift = 0.0, cg = 0.0;
                if (mode == 1) {
                    double od = 0.0; /* (sum p v) . dO / N, i.e. out . dO */
                    for (int t = 0; t < d; ++t) od += acc[t] * (double)go[t];
                    shift = od * invn;
                    cg = invn;
                } else {
                    double sw = 0.0, swdp = 0.0;
                    for (int e = qp[qb]; e < qp[qb + 1]; ++e) {
                        const int kb = ql[e];
                        for (int j = kb * block_n; j < (kb + 1) * block_n && j < NK; ++j) {
                            const long kj = (long)bh * NK + j;
                            if (kidx[kj] > qidx[r]) continue;
                            const real u = am1 * score_of(q, K + kj * d, d, scale) - tau;
                            if (!(u > (real)0)) continue;
                            const double w = (double)pow_pos(rmax(u, ASAO_EPS), ew);
                            double dp = 0.0;
                            for (int t = 0; t < d; ++t) dp += (double)V[kj * d + t] * (double)go[t];
                            sw += w;
                            swdp += w * dp;
                        }
                    }
                    shift = sw > 0.0 ? swdp / sw : 0.0;
                    cg = pow(nsum + (double)ASAO_EPS, (double)alpha_c - 2.0);
                }
                /* pass 2: per-key gradient terms */
                for (int e = qp[qb]; e < qp[qb + 1]; ++e) {
                    const int kb = ql[e];
                    for (int j = kb * block_n; j < (kb + 1) * block_n && j < NK; ++j) {
                        const long kj = (long)bh * NK + j;
                        if (kidx[kj] > qidx[r]) continue;
                        const real *kr = K + kj * d;
                        const real *v = V + kj * d;
                        const real u = am1 * score_of(q, kr, d, scale) - tau;
                        const real p = weight_of(score_of(q, kr, d, scale), tau, am1, a);
                        const double pn = (double)p * invn;
                        for (int t = 0; t < d; ++t) dv_acc[(size_t)j * d + t] += pn * (double)go[t];
                        double w = 0.0;
                        if (mode == 1 ? (u > ASAO_EPS) : (u > (real)0)) {
                            const real wr = pow_pos(rmax(u, ASAO_EPS), ew);
                            w = rfinite(wr) ? (double)wr : 0.0;
                        }
                        if (w == 0.0) continue;
                        double dp = 0.0;
                        for (int t = 0; t < d; ++t) dp += (double)v[t] * (double)go[t];
                        double ds = cg * w * (dp - shift);
                        if (!isfinite(ds)) ds = 0.0;
                        for (int t = 0; t < d; ++t) {
                            dq[t] += ds * (double)kr[t] * (double)scale;
                            dk_acc[(size_t)j * d + t] += ds * (double)q[t] * (double)scale;
                        }
                    }
                }
                for (int t = 0; t < d; ++t) {
                    real g = (real)dq[t];
                    dQ[r * d + t] = rfinite(g) ? g : (real)0;
                }
            }
            for (int j = 0; j < NK; ++j) {
                const long kj = (long)bh * NK + j;
                for (int t = 0; t < d; ++t) {
                    /* a sum beyond the float range is +-inf, as the
                     * reference's fp32 atomic sums give (:477, :518); its
                     * host fix-up (:684-697) then clamps it */
                    real gkv = (real)dk_acc[(size_t)j * d + t];
                    real gvv = (real)dv_acc[(size_t)j * d + t];
                    dK[kj * d + t] = isnan(gkv) ? (real)0 : gkv;
                    dV[kj * d + t] = isnan(gvv) ? (real)0 : gvv;
                }
            }
        }
        free(acc);
        free(dq);
        free(gk);
    }
}
