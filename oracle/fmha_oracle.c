/*
 * fmha_oracle.c — CPU oracle for the D64 BF16 FMHA forward path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the
 * bench CLI, bench.py's timed leg) may link, load or call this file.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and
 * only as the checker / the timed CPU baseline.
 *
 * It restates the reference's CPU reference, src/runner/cpu_ref.cpp:73-153,
 * per query row and in the same arithmetic order:
 *   1. s_j = (sum_d q_d*k_{j,d}) * (1/sqrt(D)), d accumulated in order, fp32
 *      (cpu_ref.cpp:107-114)
 *   2. causal: s_j = -inf when j > i + (Sk_b - Sq_b)         (cpu_ref.cpp:115-120)
 *   3. m = max_j s_j; if m == -inf every P_j = 0              (cpu_ref.cpp:124-129)
 *   4. P_j = expf(s_j - m) (0 for -inf), sum in j order       (cpu_ref.cpp:130-136)
 *   5. P_j = bf16_trunc(P_j * (1/sum))                        (cpu_ref.cpp:137-144)
 *   6. O_d = sum_j P_j * v_{j,d}, j in order                  (cpu_ref.cpp:148-153)
 * plus the LSE the reference computes only in its GPU oracle,
 * src/runner/gpu_ref.cpp:116-117: lse = logf(sum) + m, -inf when sum == 0.
 * bf16 <-> fp32 is by truncation / zero-extension (src/runner/bf16_utils.hpp:18-30).
 *
 * Entry points (the first two compute the same numbers):
 *  - oracle_fmha_fwd_faithful(): the reference's loop nest (rows, then d-outer
 *    / j-inner for P.V) with its OpenMP collapse(2) over (batch, head)
 *    (cpu_ref.cpp:73-87).  Timed as the CPU baseline.
 *  - oracle_fmha_fwd(): the same per-element operation order, restructured so
 *    the compiler can vectorise across keys (scores) and head dims (P.V), with
 *    masked keys skipped (they contribute exact zeros) and rows parallelised.
 *    Bit-identical to the faithful form; tests check that.
 *  - oracle_fmha_fwd_ex(..., ORACLE_NO_P_TRUNC): the same computation without
 *    step 5's bf16 truncation of P (the one quantisation the reference adds to
 *    imitate its kernel).  Its difference to the faithful result is the
 *    oracle's own truncation error, used as an explicit allowance in tests.
 *  - oracle_fmha_fwd_ex(..., ORACLE_P_RNE_UNNORM): not the reference's
 *    arithmetic but a model of this build's kernel (P = exp(s - m) rounded to
 *    nearest-even bf16 before P.V, the row sum and the division by it in
 *    fp32 on the unrounded P, O = (sum_j bf16(P_j) v_j) / sum_j P_j).  Tests
 *    use it, on the CPU, to show that the parity bounds recorded for the
 *    benchmark configurations fail when a mistake is planted in that model.
 *  - oracle_merge_d64(): the merge of partial results over disjoint key sets
 *    (no reference counterpart; it checks this build's fmha_merge_d64_bf16):
 *    LSE = log sum_i exp(LSE_i), O = sum_i exp(LSE_i - LSE) O_i in float64,
 *    O rounded to nearest even bf16; O = 0, LSE = -inf when every part is -inf.
 *    Pinned in tests/test_oracle.py by closed forms (one part is the identity,
 *    equal LSEs average, -inf parts drop out) and by the identity that merging
 *    the float64 attention of key chunks gives the attention of all keys.
 * Build with -ffp-contract=off so no multiply-add is fused (the reference's
 * host build has no FMA contraction either).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "fmha_oracle.h"

static inline float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline uint16_t f32_to_bf16_trunc(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)(u >> 16);
}

static inline uint16_t f32_to_bf16_rne(float f);

static int seq_lengths(const oracle_params* p, int b, int* sq, int* sk, int64_t* off_q, int64_t* off_k) {
    if (p->seqstart_q) {
        *off_q = p->seqstart_q[b];
        *off_k = p->seqstart_k[b];
        *sq = p->seqstart_q[b + 1] - p->seqstart_q[b];
        *sk = p->seqstart_k[b + 1] - p->seqstart_k[b];
    } else {
        *off_q = 0;
        *off_k = 0;
        *sq = p->seqlen_q;
        *sk = p->seqlen_k;
    }
    return 0;
}

/* Base element offsets of (b, hq) for q/o and of (b, hkv) for k/v. */
static void head_bases(const oracle_params* p, int b, int hq, int64_t off_q, int64_t off_k,
                       int64_t* qb, int64_t* kb, int64_t* vb, int64_t* ob) {
    const int hkv = hq / (p->nhead_q / p->nhead_k);
    if (p->seqstart_q) {
        *qb = (int64_t)hq * p->nhead_stride_q + off_q * p->stride_q;
        *kb = (int64_t)hkv * p->nhead_stride_k + off_k * p->stride_k;
        *vb = (int64_t)hkv * p->nhead_stride_v + off_k * p->stride_v;
        *ob = (int64_t)hq * p->nhead_stride_o + off_q * p->stride_o;
    } else {
        *qb = (int64_t)b * p->batch_stride_q + (int64_t)hq * p->nhead_stride_q;
        *kb = (int64_t)b * p->batch_stride_k + (int64_t)hkv * p->nhead_stride_k;
        *vb = (int64_t)b * p->batch_stride_v + (int64_t)hkv * p->nhead_stride_v;
        *ob = (int64_t)b * p->batch_stride_o + (int64_t)hq * p->nhead_stride_o;
    }
}

/* LSE element index, the kernel's convention (src/fused/pipeline.hpp:408-418). */
static int64_t lse_index(const oracle_params* p, int b, int hq, int64_t off_q, int i) {
    if (p->seqstart_q)
        return (int64_t)hq * (p->nhead_stride_q / p->stride_q) + off_q + i;
    return (int64_t)b * p->nhead_q * p->seqlen_q + (int64_t)hq * p->seqlen_q + i;
}

static int check_params(const oracle_params* p, int batch) {
    if (!p || !p->q || !p->k || !p->v || !p->o) return -1;
    if (batch < 0 || p->nhead_q <= 0 || p->nhead_k <= 0 || p->nhead_q % p->nhead_k) return -1;
    if (p->head_dim <= 0 || p->head_dim > ORACLE_MAX_HEAD_DIM) return -1;
    if ((p->seqstart_q == NULL) != (p->seqstart_k == NULL)) return -1;
    return 0;
}

/* One query row, reference loop order (cpu_ref.cpp:86-153). S and P are
 * caller scratch of length >= sk. */
static void row_faithful(const oracle_params* p, int causal, int i, int sq, int sk,
                         const uint16_t* qrow, const uint16_t* kbase, const uint16_t* vbase,
                         float* orow, float* lse_out, float* S, float* P) {
    const int D = p->head_dim;
    for (int j = 0; j < sk; j++) {
        float s = 0;
        for (int d = 0; d < D; d++) {
            float q = bf16_to_f32(qrow[d]);
            float k = bf16_to_f32(kbase[(int64_t)j * p->stride_k + d]);
            s += q * k;
        }
        S[j] = s * p->softmax_scale;
        if (causal && j > i + (sk - sq)) S[j] = -INFINITY;
    }
    float m = sk > 0 ? S[0] : -INFINITY;
    for (int j = 1; j < sk; j++)
        if (S[j] > m) m = S[j];
    float sum = 0;
    if (m == -INFINITY) {
        for (int j = 0; j < sk; j++) P[j] = 0.0f;
    } else {
        for (int j = 0; j < sk; j++) {
            P[j] = (isinf(S[j]) && S[j] < 0) ? 0.0f : expf(S[j] - m);
            sum += P[j];
        }
        float inv_sum = 1.0f / sum;
        for (int j = 0; j < sk; j++) {
            P[j] *= inv_sum;
            P[j] = bf16_to_f32(f32_to_bf16_trunc(P[j]));
        }
    }
    for (int d = 0; d < D; d++) {
        float o_ref = 0;
        for (int j = 0; j < sk; j++) {
            float v = bf16_to_f32(vbase[(int64_t)j * p->stride_v + d]);
            o_ref += P[j] * v;
        }
        orow[d] = o_ref;
    }
    if (lse_out) *lse_out = (sum > 0) ? logf(sum) + m : -INFINITY;
}

int oracle_fmha_fwd_faithful(const oracle_params* p, int batch, int causal, int nthreads,
                             int row_begin, int row_end) {
    if (check_params(p, batch)) return -1;
    const int Hq = p->nhead_q;
    const int max_sk = p->seqstart_k ? 0 : p->seqlen_k;
    int alloc_sk = max_sk;
    if (p->seqstart_k)
        for (int b = 0; b < batch; b++) {
            int l = p->seqstart_k[b + 1] - p->seqstart_k[b];
            if (l > alloc_sk) alloc_sk = l;
        }
    int err = 0;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
#pragma omp parallel
    {
        float* S = (float*)malloc(sizeof(float) * (alloc_sk + 1));
        float* P = (float*)malloc(sizeof(float) * (alloc_sk + 1));
        if (!S || !P) {
#pragma omp atomic write
            err = -2;
        }
#pragma omp for collapse(2) schedule(dynamic, 16)
        for (int b = 0; b < batch; b++)
            for (int hq = 0; hq < Hq; hq++) {
                if (!S || !P) continue;
                int sq, sk;
                int64_t off_q, off_k, qb, kb, vb, ob;
                seq_lengths(p, b, &sq, &sk, &off_q, &off_k);
                head_bases(p, b, hq, off_q, off_k, &qb, &kb, &vb, &ob);
                int lo = row_begin < 0 ? 0 : row_begin;
                int hi = (row_end < 0 || row_end > sq) ? sq : row_end;
                for (int i = lo; i < hi; i++) {
                    float lse_v;
                    row_faithful(p, causal, i, sq, sk, p->q + qb + (int64_t)i * p->stride_q, p->k + kb, p->v + vb,
                                 p->o + ob + (int64_t)i * p->stride_o, p->lse ? &lse_v : NULL, S, P);
                    if (p->lse) p->lse[lse_index(p, b, hq, off_q, i)] = lse_v;
                }
            }
        free(S);
        free(P);
    }
    return err;
}

/* Same numbers as row_faithful, vectorisable loop order.  KT is the key block
 * transposed to [d][j] (fp32), VF the value rows widened to fp32 [j][d]. */
static void row_fast(const oracle_params* p, int causal, int i, int sq, int sk, const float* qf,
                     const float* KT, const float* VF, float* orow, float* lse_out, float* S, float* P,
                     int flags) {
    const int D = p->head_dim;
    /* keys past the causal limit are -inf in the reference and contribute
     * exact zeros to max/sum/P.V; skipping them leaves every result bit-equal */
    int n = sk;
    if (causal) {
        long lim = (long)i + (sk - sq) + 1;
        n = lim < 0 ? 0 : (lim < sk ? (int)lim : sk);
    }
    for (int j = 0; j < n; j++) S[j] = 0.0f;
    for (int d = 0; d < D; d++) {
        const float qd = qf[d];
        const float* kt = KT + (int64_t)d * sk;
        for (int j = 0; j < n; j++) S[j] += qd * kt[j];
    }
    for (int j = 0; j < n; j++) S[j] = S[j] * p->softmax_scale;
    float m = -INFINITY;
    if (n > 0) {
        m = S[0];
        for (int j = 1; j < n; j++)
            if (S[j] > m) m = S[j];
    }
    for (int d = 0; d < D; d++) orow[d] = 0.0f;
    float sum = 0;
    if (n > 0 && m != -INFINITY) {
        for (int j = 0; j < n; j++) {
            P[j] = expf(S[j] - m);
            sum += P[j];
        }
        float inv_sum = 1.0f / sum;
        if (flags & ORACLE_P_TRUNC_UNNORM)
            for (int j = 0; j < n; j++) P[j] = bf16_to_f32(f32_to_bf16_trunc(P[j]));
        else if (flags & ORACLE_P_RNE_UNNORM)
            for (int j = 0; j < n; j++) P[j] = bf16_to_f32(f32_to_bf16_rne(P[j]));
        else if (flags & ORACLE_NO_P_TRUNC)
            for (int j = 0; j < n; j++) P[j] = P[j] * inv_sum;
        else
            for (int j = 0; j < n; j++) P[j] = bf16_to_f32(f32_to_bf16_trunc(P[j] * inv_sum));
        float acc[ORACLE_MAX_HEAD_DIM];
        for (int d = 0; d < D; d++) acc[d] = 0.0f;
        for (int j = 0; j < n; j++) {
            const float pj = P[j];
            const float* vr = VF + (int64_t)j * D;
            for (int d = 0; d < D; d++) acc[d] += pj * vr[d];
        }
        if (flags & (ORACLE_P_RNE_UNNORM | ORACLE_P_TRUNC_UNNORM))
            for (int d = 0; d < D; d++) orow[d] = acc[d] * inv_sum;
        else
            for (int d = 0; d < D; d++) orow[d] = acc[d];
    }
    if (lse_out) *lse_out = (sum > 0) ? logf(sum) + m : -INFINITY;
}

int oracle_fmha_fwd(const oracle_params* p, int batch, int causal, int nthreads) {
    return oracle_fmha_fwd_ex(p, batch, causal, nthreads, 0);
}

int oracle_fmha_fwd_ex(const oracle_params* p, int batch, int causal, int nthreads, int flags) {
    if (check_params(p, batch)) return -1;
    const int Hq = p->nhead_q, Hk = p->nhead_k, D = p->head_dim;
    const int gqa = Hq / Hk;
    int err = 0;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
    for (int b = 0; b < batch; b++) {
        int sq, sk;
        int64_t off_q, off_k;
        seq_lengths(p, b, &sq, &sk, &off_q, &off_k);
        if (sq <= 0) continue;
        float* KT = (float*)malloc(sizeof(float) * ((size_t)D * sk + 1));
        float* VF = (float*)malloc(sizeof(float) * ((size_t)D * sk + 1));
        if (!KT || !VF) {
            free(KT);
            free(VF);
            return -2;
        }
        for (int hkv = 0; hkv < Hk; hkv++) {
            int64_t qb, kb, vb, ob;
            head_bases(p, b, hkv * gqa, off_q, off_k, &qb, &kb, &vb, &ob);
#pragma omp parallel for schedule(static)
            for (int j = 0; j < sk; j++)
                for (int d = 0; d < D; d++) {
                    KT[(int64_t)d * sk + j] = bf16_to_f32(p->k[kb + (int64_t)j * p->stride_k + d]);
                    VF[(int64_t)j * D + d] = bf16_to_f32(p->v[vb + (int64_t)j * p->stride_v + d]);
                }
            for (int g = 0; g < gqa; g++) {
                const int hq = hkv * gqa + g;
                head_bases(p, b, hq, off_q, off_k, &qb, &kb, &vb, &ob);
#pragma omp parallel
                {
                    float* S = (float*)malloc(sizeof(float) * (sk + 1));
                    float* P = (float*)malloc(sizeof(float) * (sk + 1));
                    if (!S || !P) {
#pragma omp atomic write
                        err = -2;
                    }
#pragma omp for schedule(dynamic, 16)
                    for (int i = 0; i < sq; i++) {
                        if (!S || !P) continue;
                        float qf[ORACLE_MAX_HEAD_DIM];
                        const uint16_t* qrow = p->q + qb + (int64_t)i * p->stride_q;
                        for (int d = 0; d < D; d++) qf[d] = bf16_to_f32(qrow[d]);
                        float lse_v;
                        row_fast(p, causal, i, sq, sk, qf, KT, VF, p->o + ob + (int64_t)i * p->stride_o,
                                 p->lse ? &lse_v : NULL, S, P, flags);
                        if (p->lse) p->lse[lse_index(p, b, hq, off_q, i)] = lse_v;
                    }
                    free(S);
                    free(P);
                }
            }
        }
        free(KT);
        free(VF);
    }
    return err;
}

/* Brute-force float64 attention: no bf16 truncation of P, exact softmax.
 * Independent of both forms above (different precision and formula order);
 * used to pin them at small sizes. */
int oracle_fmha_fwd_f64(const oracle_params* p, int batch, int causal, double* o64, double* lse64) {
    if (check_params(p, batch)) return -1;
    const int Hq = p->nhead_q, D = p->head_dim;
    for (int b = 0; b < batch; b++) {
        int sq, sk;
        int64_t off_q, off_k;
        seq_lengths(p, b, &sq, &sk, &off_q, &off_k);
        for (int hq = 0; hq < Hq; hq++) {
            int64_t qb, kb, vb, ob;
            head_bases(p, b, hq, off_q, off_k, &qb, &kb, &vb, &ob);
            double* s = (double*)malloc(sizeof(double) * (sk + 1));
            if (!s) return -2;
            for (int i = 0; i < sq; i++) {
                double m = -INFINITY;
                for (int j = 0; j < sk; j++) {
                    double acc = 0;
                    for (int d = 0; d < D; d++)
                        acc += (double)bf16_to_f32(p->q[qb + (int64_t)i * p->stride_q + d]) *
                               (double)bf16_to_f32(p->k[kb + (int64_t)j * p->stride_k + d]);
                    s[j] = acc * (double)p->softmax_scale;
                    if (causal && j > i + (sk - sq)) s[j] = -INFINITY;
                    if (s[j] > m) m = s[j];
                }
                double sum = 0;
                for (int j = 0; j < sk; j++) sum += (s[j] == -INFINITY) ? 0.0 : exp(s[j] - m);
                double* orow = o64 + ob + (int64_t)i * p->stride_o;
                for (int d = 0; d < D; d++) {
                    double acc = 0;
                    if (sum > 0)
                        for (int j = 0; j < sk; j++)
                            if (s[j] != -INFINITY)
                                acc += exp(s[j] - m) / sum * (double)bf16_to_f32(p->v[vb + (int64_t)j * p->stride_v + d]);
                    orow[d] = acc;
                }
                if (lse64) lse64[lse_index(p, b, hq, off_q, i)] = sum > 0 ? log(sum) + m : -INFINITY;
            }
            free(s);
        }
    }
    return 0;
}

/* The reference's input generator, src/runner/buffers.cpp:99-127: one glibc
 * srand(seed) stream, then Q, K, V filled in that order, each value
 * bf16_trunc(((rand() % 1000) - 500) / 5000.0f).  Also the generator of the
 * two BSHD smoke tests (tests/test_fmha_fwd_d64.cpp:209-212, 362-365). */
void oracle_fill_ref(unsigned seed, uint16_t* q, size_t nq, uint16_t* k, size_t nk, uint16_t* v, size_t nv) {
    srand(seed);
    uint16_t* bufs[3] = {q, k, v};
    size_t ns[3] = {nq, nk, nv};
    for (int t = 0; t < 3; t++)
        for (size_t i = 0; i < ns[t]; i++) {
            float x = ((rand() % 1000) - 500) / 5000.0f;
            bufs[t][i] = f32_to_bf16_trunc(x);
        }
}

static inline uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* NaN stays NaN */
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void oracle_merge_d64(int n_parts, int64_t rows, const uint16_t* o_parts, int64_t o_part_stride,
                      const float* lse_parts, int64_t lse_part_stride, int64_t o_row_stride, uint16_t* o,
                      float* lse) {
    for (int64_t r = 0; r < rows; r++) {
        double m = -INFINITY;
        for (int i = 0; i < n_parts; i++) {
            const double l = lse_parts[i * lse_part_stride + r];
            if (l > m) m = l;
        }
        uint16_t* orow = o + r * o_row_stride;
        if (m == -INFINITY) {
            for (int d = 0; d < 64; d++) orow[d] = 0;
            if (lse) lse[r] = -INFINITY;
            continue;
        }
        double acc[64] = {0};
        double w_sum = 0.0;
        for (int i = 0; i < n_parts; i++) {
            const double w = exp((double)lse_parts[i * lse_part_stride + r] - m);
            const uint16_t* prow = o_parts + i * o_part_stride + r * o_row_stride;
            w_sum += w;
            for (int d = 0; d < 64; d++) acc[d] += w * (double)bf16_to_f32(prow[d]);
        }
        for (int d = 0; d < 64; d++) orow[d] = f32_to_bf16_rne((float)(acc[d] / w_sum));
        if (lse) lse[r] = (float)(m + log(w_sum));
    }
}
