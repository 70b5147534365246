// probe_coissue.hip — gfx950 microbenchmark behind the kernel's performance
// ceiling (a measurement tool; the library does not use it).
//
// One block per compute unit, 4 * W waves per block, so every SIMD runs W
// waves.  Each wave repeats a fixed instruction mix; the SIMD's cycles per
// repetition come from the elapsed time and the shader clock (s_memtime
// against the 100 MHz s_memrealtime).  All measured instructions are inline
// asm, so the mix is exactly the one listed.
//
//  1. issue cost: 64 instances of one VALU instruction per repetition, over
//     8 independent registers, at 2 waves per SIMD -> SIMD cycles per wave64
//     instruction;
//  2. MFMA alone: 16 v_mfma_f32_32x32x16_bf16 per repetition on 4
//     independent accumulators -> SIMD cycles per MFMA (the 32 the busy
//     figure below divides by);
//  3. the softmax work of one 64-key tile as the kernel issues it per wave
//     (32 x {fma with two VGPR operands, exp, add} and 16 cvt_pk, each score's
//     exp two MFMA slots after its fma), alone and beside the tile's 16 MFMAs,
//     at 1-4 waves per SIMD -> MFMA busy = 16 * 32 * W / SIMD cycles per
//     repetition.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

#define CK(x)                                                                              \
    do {                                                                                   \
        hipError_t e_ = (x);                                                               \
        if (e_ != hipSuccess) {                                                            \
            std::fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__); \
            std::exit(1);                                                                  \
        }                                                                                  \
    } while (0)

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

enum Op { kExp, kCvtPk, kFmaV, kFmaS, kAdd, kMov };
constexpr int kCycPerMfma = 32;  // v_mfma_f32_32x32x16_bf16: 8 passes of 4 cycles

struct Timing {
    unsigned long long cycles;  // s_memtime delta of wave 0 of block 0
    unsigned long long ticks;   // s_memrealtime delta (100 MHz)
};

__device__ __forceinline__ void record(Timing* t, unsigned long long c0, unsigned long long r0) {
    const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        t->cycles = c1 - c0;
        t->ticks = r1 - r0;
    }
}

template <int kOp>
__global__ void issue_cost(float* sink, Timing* tm, int reps, float sc) {
    float x[8];
    unsigned y[8];
    for (int i = 0; i < 8; ++i) {
        x[i] = threadIdx.x * 1e-7f + i * 1e-8f;
        y[i] = threadIdx.x + i;
    }
    const float vs = sc + threadIdx.x * 1e-9f;  // a per-lane value: lives in a VGPR
    const unsigned long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int r = 0; r < reps; ++r) {
#pragma unroll
        for (int i = 0; i < 64; ++i) {
            float& a = x[i % 8];
            if constexpr (kOp == kExp) asm volatile("v_exp_f32 %0, %0" : "+v"(a));
            if constexpr (kOp == kCvtPk)
                asm volatile("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(y[i % 8]) : "v"(a), "v"(x[(i + 1) % 8]));
            if constexpr (kOp == kFmaV) asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(a) : "v"(vs), "v"(x[(i + 3) % 8]));
            if constexpr (kOp == kFmaS) asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(a) : "s"(sc), "v"(x[(i + 3) % 8]));
            if constexpr (kOp == kAdd) asm volatile("v_add_f32 %0, %0, %1" : "+v"(a) : "v"(x[(i + 3) % 8]));
            if constexpr (kOp == kMov) asm volatile("v_mov_b32 %0, %1" : "=v"(a) : "v"(x[(i + 3) % 8]));
        }
    }
    record(tm, c0, r0);
    float s = 0.f;
    for (int i = 0; i < 8; ++i) s += x[i] + (float)y[i];
    if (s == 1234.5f) sink[threadIdx.x] = s;  // keeps the work observable; never true in practice
}

// the per-wave work of one 64-key tile, slot m of 16 (two scores per slot)
__device__ __forceinline__ void softmax_slot(float* s, float* t, float& acc, unsigned* y, float vs, float vb, int m) {
    const int i0 = (2 * m) % 16;
    asm volatile("v_fma_f32 %0, %1, %2, %3" : "=v"(t[i0]) : "v"(s[i0]), "v"(vs), "v"(vb));
    asm volatile("v_fma_f32 %0, %1, %2, %3" : "=v"(t[i0 + 1]) : "v"(s[i0 + 1]), "v"(vs), "v"(vb));
    const int j0 = (2 * (m + 14)) % 16;  // the scores of two slots back
    asm volatile("v_exp_f32 %0, %0" : "+v"(t[j0]));
    asm volatile("v_exp_f32 %0, %0" : "+v"(t[j0 + 1]));
    const int k0 = (2 * (m + 12)) % 16;  // and of four slots back
    asm volatile("v_add_f32 %0, %0, %1" : "+v"(acc) : "v"(t[k0]));
    asm volatile("v_add_f32 %0, %0, %1" : "+v"(acc) : "v"(t[k0 + 1]));
    asm volatile("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(y[m % 8]) : "v"(t[k0]), "v"(t[k0 + 1]));
}

template <bool kMfma, bool kSoftmax>
__global__ void tile_mix(float* sink, Timing* tm, int reps, float sc) {
    bf16x8 a, b;
    for (int e = 0; e < 8; ++e) {
        a[e] = (__bf16)(threadIdx.x * 0.001f + e);
        b[e] = (__bf16)(e * 0.5f);
    }
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    float s[16], t[16], acc = 0.f;
    for (int i = 0; i < 16; ++i) {
        s[i] = threadIdx.x * 1e-7f + i * 1e-8f;
        t[i] = 0.f;
    }
    unsigned y[8] = {};
    const float vs = sc * (1.0f + threadIdx.x * 1e-9f), vb = -sc;
    const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int r = 0; r < reps; ++r) {
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            if constexpr (kMfma) {
                if (m % 4 == 0) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c0) : "v"(a), "v"(b));
                if (m % 4 == 1) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c1) : "v"(a), "v"(b));
                if (m % 4 == 2) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c2) : "v"(a), "v"(b));
                if (m % 4 == 3) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c3) : "v"(a), "v"(b));
            }
            if constexpr (kSoftmax) softmax_slot(s, t, acc, y, vs, vb, m);
        }
    }
    record(tm, t0, r0);
    float res = acc;
    for (int i = 0; i < 16; ++i) res += t[i];
    for (int i = 0; i < 8; ++i) res += (float)y[i];
    for (int i = 0; i < 16; ++i) res += c0[i] + c1[i] + c2[i] + c3[i];
    if (res == 1234.5f) sink[threadIdx.x] = res;
}

struct Result {
    double simd_cycles_per_rep;
    double ghz;
};

template <typename K>
Result measure(K kern, int ncu, int waves_per_simd, int reps, float* sink, Timing* tm) {
    const dim3 grid(ncu), block(256 * waves_per_simd);
    hipLaunchKernelGGL(kern, grid, block, 0, 0, sink, tm, 4, 0.5f);  // warm-up
    CK(hipGetLastError());
    CK(hipDeviceSynchronize());
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    CK(hipEventRecord(e0, 0));
    hipLaunchKernelGGL(kern, grid, block, 0, 0, sink, tm, reps, 0.5f);
    CK(hipGetLastError());
    CK(hipEventRecord(e1, 0));
    CK(hipEventSynchronize(e1));
    float ms = 0.f;
    CK(hipEventElapsedTime(&ms, e0, e1));
    CK(hipEventDestroy(e0));
    CK(hipEventDestroy(e1));
    Timing h{};
    CK(hipMemcpy(&h, tm, sizeof(h), hipMemcpyDeviceToHost));
    const double ghz = (double)h.cycles / ((double)h.ticks * 10.0);  // cycles per ns
    return {ms * 1e6 * ghz / reps, ghz};
}

}  // namespace

int main() {
    hipDeviceProp_t prop;
    CK(hipGetDeviceProperties(&prop, 0));
    const int ncu = prop.multiProcessorCount;
    float* sink = nullptr;
    Timing* tm = nullptr;
    CK(hipMalloc(&sink, 4096 * sizeof(float)));
    CK(hipMalloc(&tm, sizeof(Timing)));
    std::printf("device %s, %d compute units; one block per CU, W waves per SIMD\n\n", prop.gcnArchName, ncu);

    std::printf("1. issue cost at W = 2 (SIMD cycles per wave64 instruction)\n");
    const int reps1 = 4000;
    struct {
        const char* name;
        Result r;
    } ops[] = {
        {"v_exp_f32", measure(issue_cost<kExp>, ncu, 2, reps1, sink, tm)},
        {"v_cvt_pk_bf16_f32", measure(issue_cost<kCvtPk>, ncu, 2, reps1, sink, tm)},
        {"v_fma_f32 (VGPR operands)", measure(issue_cost<kFmaV>, ncu, 2, reps1, sink, tm)},
        {"v_fma_f32 (one SGPR operand)", measure(issue_cost<kFmaS>, ncu, 2, reps1, sink, tm)},
        {"v_add_f32", measure(issue_cost<kAdd>, ncu, 2, reps1, sink, tm)},
        {"v_mov_b32", measure(issue_cost<kMov>, ncu, 2, reps1, sink, tm)},
    };
    for (const auto& o : ops)
        std::printf("   %-30s %5.2f cycles   (clock %.2f GHz)\n", o.name, o.r.simd_cycles_per_rep / (2 * 64), o.r.ghz);

    std::printf("\n2. MFMA alone (16 v_mfma_f32_32x32x16_bf16 per wave and repetition)\n");
    const int reps = 3000;
    for (int w = 1; w <= 2; ++w) {
        const Result r = measure(tile_mix<true, false>, ncu, w, reps, sink, tm);
        std::printf("   W=%d  SIMD cycles per MFMA %6.2f   (clock %.2f GHz)\n", w, r.simd_cycles_per_rep / (16.0 * w), r.ghz);
    }

    std::printf("\n3. one 64-key tile per wave: 32 x {fma, exp, add} + 16 cvt_pk, alone and beside 16 MFMAs\n");
    for (int w = 1; w <= 4; ++w) {
        const Result alone = measure(tile_mix<false, true>, ncu, w, reps, sink, tm);
        const Result both = measure(tile_mix<true, true>, ncu, w, reps, sink, tm);
        std::printf("   W=%d  softmax alone %7.1f  with MFMAs %7.1f SIMD cycles per tile-step   MFMA busy %5.1f%%   (clock %.2f GHz)\n",
                    w, alone.simd_cycles_per_rep, both.simd_cycles_per_rep,
                    100.0 * 16 * kCycPerMfma * w / both.simd_cycles_per_rep, both.ghz);
    }
    CK(hipFree(sink));
    CK(hipFree(tm));
    return 0;
}
