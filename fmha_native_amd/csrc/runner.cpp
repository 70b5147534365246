// runner.cpp — host-side input generation for the FMHA forward harness.
//
// Mirrors the reference's src/runner/buffers.cpp:99-127 (fill_random) and adds
// the seeded N(0,1) generator the benchmark configurations need.  Host only;
// exported with a C ABI so the C++ bench CLI, Python tests and bench.py all
// draw bit-identical inputs.

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "fmha_runner.h"

namespace {

inline uint16_t f32_to_bf16_trunc(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)(u >> 16);
}

// splitmix64 finaliser (Steele, Lea, Flood 2014), used as a counter-based
// generator: element i of stream `seed` is mix(seed_base + (i+1)*golden).
inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}
constexpr uint64_t kGolden = 0x9e3779b97f4a7c15ULL;

inline double uniform01_open(uint64_t bits) {  // (0, 1)
    return ((double)(bits >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

}  // namespace

extern "C" void fmha_runner_fill_ref(unsigned seed, uint16_t* q, size_t nq, uint16_t* k, size_t nk, uint16_t* v,
                                     size_t nv) {
    srand(seed);
    uint16_t* bufs[3] = {q, k, v};
    const size_t ns[3] = {nq, nk, nv};
    for (int t = 0; t < 3; t++)
        for (size_t i = 0; i < ns[t]; i++) bufs[t][i] = f32_to_bf16_trunc(((rand() % 1000) - 500) / 5000.0f);
}

extern "C" void fmha_runner_fill_normal(uint64_t seed, float mult, uint16_t* out, size_t n) {
    const uint64_t base = mix64(seed ^ 0x6a09e667f3bcc909ULL);
    const int64_t npairs = (int64_t)((n + 1) / 2);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < npairs; i++) {
        const double u1 = uniform01_open(mix64(base + (uint64_t)(2 * i + 1) * kGolden));
        const double u2 = uniform01_open(mix64(base + (uint64_t)(2 * i + 2) * kGolden));
        const double r = sqrt(-2.0 * log(u1));
        const double a = 6.283185307179586476925 * u2;
        out[2 * i] = f32_to_bf16_trunc((float)(r * cos(a)) * mult);
        if ((size_t)(2 * i + 1) < n) out[2 * i + 1] = f32_to_bf16_trunc((float)(r * sin(a)) * mult);
    }
}

extern "C" int fmha_runner_varlen_lengths(uint64_t seed, int n, int lo, int hi, int* out) {
    if (n <= 0 || lo <= 0 || hi < lo || out == nullptr) return -1;
    const uint64_t base = mix64(seed ^ 0xbb67ae8584caa73bULL);
    const uint64_t span = (uint64_t)(hi - lo + 1);
    for (int i = 0; i < n; i++) out[i] = lo + (int)(mix64(base + (uint64_t)(i + 1) * kGolden) % span);
    // at least half of the lengths must not be multiples of 64 (ragged tiles)
    int ragged = 0;
    for (int i = 0; i < n; i++) ragged += (out[i] % 64) != 0;
    for (int i = 0; i < n && 2 * ragged < n; i++)
        if (out[i] % 64 == 0) {
            out[i] = out[i] + 1 <= hi ? out[i] + 1 : out[i] - 1;
            ragged++;
        }
    return 0;
}
