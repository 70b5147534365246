// fmha_merge.hip — merge of partial attention results over disjoint key sets
// (gfx950).  This build's own; the reference has no counterpart.  It is the
// merge the split-KV kernel form does in LDS, as a kernel for partials that
// come from separate launches: key chunks of one sequence, ring attention, or
// one GPU's shard of a sharded sequence.
//
// For row r and part i, O_i[r] is the part's normalised output (64 bf16) and
// LSE_i[r] its natural-log row sum (-inf when the part saw no key):
//   m = max_i LSE_i,  w_i = exp(LSE_i - m),  W = sum_i w_i
//   LSE[r] = m + log(W),  O[r] = (sum_i w_i O_i[r]) / W
// and O = 0, LSE = -inf when every part is -inf.  fp32 arithmetic, O rounded
// to bf16 (round to nearest even).
//
// HBM-bound: per row it reads n x (128 + 4) bytes and writes 128 (+4).  Eight
// lanes share a row (16 bytes = 8 head-dim values each), so one wave covers 8
// rows with 16-byte loads and stores; the 8 lanes of a row read the same LSE
// values (one cache line).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fmha_fwd.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

struct MergeArgs {
    const __bf16* o_parts;
    const float* lse_parts;
    __bf16* o;
    float* lse;
    int64_t rows;
    int64_t o_part_stride;    // elements between parts of O
    int64_t lse_part_stride;  // elements between parts of LSE
    int64_t o_row_stride;     // elements between rows of O (parts and output)
    int n_parts;
};

constexpr int kMergeBlock = 256;
constexpr int kLanesPerRow = FMHA_HEAD_DIM / 8;  // 8 lanes x 8 values
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.69314718055994530942f;

__global__ __launch_bounds__(kMergeBlock) void fmha_merge_d64_bf16_kernel(MergeArgs a) {
    const int64_t g = (int64_t)blockIdx.x * kMergeBlock + threadIdx.x;
    const int64_t r = g / kLanesPerRow;
    const int c = (int)(g % kLanesPerRow);
    if (r >= a.rows) return;
    const int64_t col = r * a.o_row_stride + 8 * c;
    float m = -__builtin_inff();
    for (int i = 0; i < a.n_parts; ++i) m = fmaxf(m, a.lse_parts[i * a.lse_part_stride + r]);
    bf16x8 out;
    if (m == -__builtin_inff()) {
        for (int e = 0; e < 8; ++e) out[e] = (__bf16)0.0f;
        *(bf16x8*)(a.o + col) = out;
        if (a.lse != nullptr && c == 0) a.lse[r] = m;
        return;
    }
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float wsum = 0.f;
    for (int i = 0; i < a.n_parts; ++i) {
        const float li = a.lse_parts[i * a.lse_part_stride + r];
        const float w = __builtin_amdgcn_exp2f((li - m) * kLog2e);  // 0 for a -inf part
        const bf16x8 v = *(const bf16x8*)(a.o_parts + i * a.o_part_stride + col);
        wsum += w;
        for (int e = 0; e < 8; ++e) acc[e] = __builtin_fmaf(w, (float)v[e], acc[e]);
    }
    const float inv = 1.0f / wsum;  // wsum >= 1: the part at the max has w = 1
    for (int e = 0; e < 8; ++e) out[e] = (__bf16)(acc[e] * inv);
    *(bf16x8*)(a.o + col) = out;
    if (a.lse != nullptr && c == 0) a.lse[r] = m + __builtin_amdgcn_logf(wsum) * kLn2;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

extern "C" hipError_t fmha_merge_d64_bf16(int n_parts, int64_t rows, const void* o_parts, int64_t o_part_stride,
                                          const float* lse_parts, int64_t lse_part_stride, int64_t o_row_stride,
                                          void* o, float* lse, hipStream_t stream) {
    if (n_parts < 1 || n_parts > FMHA_MERGE_MAX_PARTS || rows < 0) return hipErrorInvalidValue;
    if (o_parts == nullptr || lse_parts == nullptr || o == nullptr) return hipErrorInvalidValue;
    if (!aligned16(o_parts) || !aligned16(o) || (reinterpret_cast<uintptr_t>(lse_parts) & 3u) ||
        (reinterpret_cast<uintptr_t>(lse) & 3u))
        return hipErrorInvalidValue;
    if (o_row_stride < FMHA_HEAD_DIM || (o_row_stride & 7) || o_part_stride < 0 || (o_part_stride & 7) ||
        lse_part_stride < 0)
        return hipErrorInvalidValue;
    if (n_parts > 1 && (o_part_stride < rows * o_row_stride || lse_part_stride < rows)) return hipErrorInvalidValue;
    if (rows == 0) return hipSuccess;
    const int64_t threads = rows * kLanesPerRow;
    const int64_t blocks = (threads + kMergeBlock - 1) / kMergeBlock;
    if (blocks > INT32_MAX) return hipErrorInvalidValue;
    MergeArgs a{(const __bf16*)o_parts, lse_parts, (__bf16*)o, lse, rows, o_part_stride, lse_part_stride,
                o_row_stride, n_parts};
    hipLaunchKernelGGL(fmha_merge_d64_bf16_kernel, dim3((unsigned)blocks), dim3(kMergeBlock), 0, stream, a);
    return hipGetLastError();
}
