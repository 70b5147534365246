/*
 * fmha_runner.h — host-side input generators of the FMHA forward harness
 * (the counterpart of the reference's src/runner/buffers.hpp fill_random).
 * bf16 values are returned as uint16_t bit patterns, truncated from fp32 as
 * the reference does (src/runner/bf16_utils.hpp:18-22).
 */
#ifndef FMHA_RUNNER_H_
#define FMHA_RUNNER_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The reference generator (src/runner/buffers.cpp:99-127): glibc srand(seed),
 * then Q, K, V in sequence, each value bf16(((rand() % 1000) - 500) / 5000). */
void fmha_runner_fill_ref(unsigned seed, uint16_t* q, size_t nq, uint16_t* k, size_t nk, uint16_t* v, size_t nv);

/* i.i.d. N(0,1) * mult, counter-based (splitmix64 -> Box-Muller), identical on
 * every host and for any thread count.  Streams: Q = seed, K = seed+1, V = seed+2. */
void fmha_runner_fill_normal(uint64_t seed, float mult, uint16_t* out, size_t n);

/* n sequence lengths uniform in [lo, hi], at least half not multiples of 64. */
int fmha_runner_varlen_lengths(uint64_t seed, int n, int lo, int hi, int* out);

#ifdef __cplusplus
}
#endif
#endif
