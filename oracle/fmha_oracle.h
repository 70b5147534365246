/*
 * fmha_oracle.h — CPU oracle interface (test infrastructure only; see
 * fmha_oracle.c).  Host pointers everywhere; bf16 tensors are uint16_t bit
 * patterns; O outputs are fp32 (the reference keeps its O_ref in fp32,
 * src/runner/cpu_ref.cpp:148-153) and are written with the o strides.
 */
#ifndef FMHA_ORACLE_H_
#define FMHA_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORACLE_MAX_HEAD_DIM 256

typedef struct oracle_params {
    const uint16_t *q, *k, *v; /* bf16 bit patterns */
    float* o;                  /* fp32 O_ref, element (b,h,s,d) at the o strides */
    float* lse;                /* NULL = skip; same indexing as the kernel's LSE */
    int seqlen_q, seqlen_k;    /* dense lengths (ignored in varlen mode) */
    int nhead_q, nhead_k;
    int head_dim;
    float softmax_scale; /* plain 1/sqrt(head_dim), natural-e softmax */
    int stride_q, nhead_stride_q, batch_stride_q;
    int stride_k, nhead_stride_k, batch_stride_k;
    int stride_v, nhead_stride_v, batch_stride_v;
    int stride_o, nhead_stride_o, batch_stride_o;
    const int32_t* seqstart_q; /* host arrays of batch+1 offsets, or NULL */
    const int32_t* seqstart_k;
} oracle_params;

/* Reference loop nest; rows [row_begin, row_end) of every (b, h) (-1 = all). */
int oracle_fmha_fwd_faithful(const oracle_params* p, int batch, int causal, int nthreads,
                             int row_begin, int row_end);
/* Same results, vectorisable and row-parallel. */
int oracle_fmha_fwd(const oracle_params* p, int batch, int causal, int nthreads);
/* flags: ORACLE_NO_P_TRUNC keeps P in fp32 (no bf16 truncation before P.V). */
#define ORACLE_NO_P_TRUNC 1
/* flags: ORACLE_P_RNE_UNNORM models this build's kernel instead of the
 * reference: P rounded to nearest-even bf16 before normalisation, O divided by
 * the fp32 row sum at the end. */
#define ORACLE_P_RNE_UNNORM 2
/* flags: the same model with P truncated instead of rounded (a mistake planted
 * in the model by tests, to show that their parity bounds catch it). */
#define ORACLE_P_TRUNC_UNNORM 4
int oracle_fmha_fwd_ex(const oracle_params* p, int batch, int causal, int nthreads, int flags);
/* float64 brute force (exact softmax, no P truncation); o64/lse64 use the
 * o / lse indexing of p. */
int oracle_fmha_fwd_f64(const oracle_params* p, int batch, int causal, double* o64, double* lse64);
/* The reference's srand/rand +-0.1 generator for Q, K, V in sequence. */
void oracle_fill_ref(unsigned seed, uint16_t* q, size_t nq, uint16_t* k, size_t nk, uint16_t* v, size_t nv);

/* Merge of partial results over disjoint key sets (the LSE merge; no
 * reference counterpart), in float64, O rounded to nearest even bf16.
 * Layout as the product's fmha_merge_d64_bf16 (strides in elements). */
void oracle_merge_d64(int n_parts, int64_t rows, const uint16_t* o_parts, int64_t o_part_stride,
                      const float* lse_parts, int64_t lse_part_stride, int64_t o_row_stride, uint16_t* o,
                      float* lse);

#ifdef __cplusplus
}
#endif
#endif
