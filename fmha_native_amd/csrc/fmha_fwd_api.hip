// fmha_fwd_api.hip — C-ABI launcher for the gfx950 D64 BF16 FMHA forward.
//
// Replaces the reference's launch sites (src/bench_fmha_fwd.cpp:174-191,
// tests/test_fmha_fwd_d64.cpp:563-578): pick one of the four entries (varlen
// <=> seqstart_q set; causal flag), build the (nhead_q, ceil(seqlen_q/kM0),
// batch) grid and launch on the caller's stream.  Unlike the reference it
// validates its arguments and returns hipError_t instead of exiting.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "fmha_fwd.h"

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int kMaxGridYZ = 65535;  // largest grid y / z dimension

// Largest byte offset touched inside one (batch, head) of a tensor with `rows`
// rows must fit the 31-bit buffer offsets the kernel uses; the loaders may
// read up to one 64-key tile past the last row (zero-filled by the bound).
bool offsets_fit(int rows, int stride) {
    const int64_t max_rows = (int64_t)rows + FMHA_KN0 + FMHA_KM0;
    return max_rows * (int64_t)stride * 2 + 256 < ((int64_t)1 << 31);
}

}  // namespace

extern "C" hipError_t fmha_fwd_d64_bf16_check(const FmhaFwdParams* p, int batch, int causal) {
    if (p == nullptr) return hipErrorInvalidValue;
    if (batch < 0 || (causal != 0 && causal != 1)) return hipErrorInvalidValue;
    if (p->q == nullptr || p->k == nullptr || p->v == nullptr || p->o == nullptr) return hipErrorInvalidValue;
    if (!aligned16(p->q) || !aligned16(p->k) || !aligned16(p->v) || !aligned16(p->o)) return hipErrorInvalidValue;
    if (p->lse != nullptr && (reinterpret_cast<uintptr_t>(p->lse) & 3u)) return hipErrorInvalidValue;
    if (p->seqlen_q < 0 || p->seqlen_k < 0) return hipErrorInvalidValue;
    if (p->nhead_q <= 0 || p->nhead_k <= 0 || p->nhead_q % p->nhead_k != 0) return hipErrorInvalidValue;
    const int strides[12] = {p->stride_q, p->nhead_stride_q, p->batch_stride_q, p->stride_k, p->nhead_stride_k,
                             p->batch_stride_k, p->stride_v, p->nhead_stride_v, p->batch_stride_v, p->stride_o,
                             p->nhead_stride_o, p->batch_stride_o};
    for (int s : strides)
        if (s < 0 || (s & 7) != 0) return hipErrorInvalidValue;
    // a row must hold the 64 head-dim elements (rows never overlap)
    if (p->stride_q < FMHA_HEAD_DIM || p->stride_k < FMHA_HEAD_DIM || p->stride_v < FMHA_HEAD_DIM ||
        p->stride_o < FMHA_HEAD_DIM)
        return hipErrorInvalidValue;
    if ((p->seqstart_q == nullptr) != (p->seqstart_k == nullptr)) return hipErrorInvalidValue;
    if (!offsets_fit(p->seqlen_q, p->stride_q) || !offsets_fit(p->seqlen_k, p->stride_k) ||
        !offsets_fit(p->seqlen_k, p->stride_v) || !offsets_fit(p->seqlen_q, p->stride_o))
        return hipErrorInvalidValue;
    if (p->seqstart_q != nullptr && p->lse != nullptr && p->nhead_stride_q % p->stride_q != 0)
        return hipErrorInvalidValue;  // varlen LSE head stride is nhead_stride_q / stride_q
    // grid (nhead_q, ceil(seqlen_q / kM0), batch): y and z are at most 65535
    if ((p->seqlen_q + FMHA_KM0 - 1) / FMHA_KM0 > kMaxGridYZ || batch > kMaxGridYZ) return hipErrorInvalidValue;
    return hipSuccess;
}

namespace {

// Compute units of the current device (cached per device ordinal).
int device_cus() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

#ifndef FMHA_SPLIT_POLICY
#define FMHA_SPLIT_POLICY 2  // 0: never split, 1: always, 2: by grid size
#endif

// The split-KV entries give each M-tile twice the waves (two 4-wave groups
// per block, one block per CU), each walking half of its key range.  They pay
// off when the regular grid (two resident blocks per CU) leaves compute units
// short of work.  Measured on MI355X (256 CUs): +12-16% at 128-256 blocks,
// +2% at 626, -4% at 1024.  The pair entries are never picked automatically
// (within a few % of the regular entries either way).
int pick_variant(int blocks) {
    if (FMHA_SPLIT_POLICY == 0) return FMHA_VARIANT_REGULAR;
    if (FMHA_SPLIT_POLICY == 1) return FMHA_VARIANT_SPLITKV;
    return blocks < 3 * device_cus() ? FMHA_VARIANT_SPLITKV : FMHA_VARIANT_REGULAR;
}

}  // namespace

extern "C" hipError_t fmha_fwd_d64_bf16_variant(const FmhaFwdParams* p, int batch, int causal, int variant,
                                                hipStream_t stream) {
    const hipError_t chk = fmha_fwd_d64_bf16_check(p, batch, causal);
    if (chk != hipSuccess) return chk;
    if (variant < FMHA_VARIANT_AUTO || variant > FMHA_VARIANT_PAIR) return hipErrorInvalidValue;
    if (batch == 0 || p->seqlen_q == 0) return hipSuccess;  // nothing to compute
    const int m_tiles = (p->seqlen_q + kM0 - 1) / kM0;
    const dim3 grid(p->nhead_q, m_tiles, batch);
    const bool varlen = p->seqstart_q != nullptr;
    if (variant == FMHA_VARIANT_AUTO) variant = pick_variant(p->nhead_q * m_tiles * batch);
    if (variant == FMHA_VARIANT_PAIR) {
        const dim3 pgrid(p->nhead_q, (m_tiles + 1) / 2, batch);
        const dim3 block(FMHA_SPLIT_KBLOCK);
        if (varlen) {
            if (causal)
                hipLaunchKernelGGL(fmha_fwd_d64_bf16_pair_msk1_varlen, pgrid, block, 0, stream, *p);
            else
                hipLaunchKernelGGL(fmha_fwd_d64_bf16_pair_msk0_varlen, pgrid, block, 0, stream, *p);
        } else {
            if (causal)
                hipLaunchKernelGGL(fmha_fwd_d64_bf16_pair_msk1, pgrid, block, 0, stream, *p);
            else
                hipLaunchKernelGGL(fmha_fwd_d64_bf16_pair_msk0, pgrid, block, 0, stream, *p);
        }
        return hipGetLastError();
    }
    if (variant == FMHA_VARIANT_SPLITKV) {
        const dim3 block(FMHA_SPLIT_KBLOCK);
        if (varlen) {
            if (causal)
                hipLaunchKernelGGL(fmha_fwd_d64_bf16_splitkv_msk1_varlen, grid, block, 0, stream, *p);
            else
                hipLaunchKernelGGL(fmha_fwd_d64_bf16_splitkv_msk0_varlen, grid, block, 0, stream, *p);
        } else {
            if (causal)
                hipLaunchKernelGGL(fmha_fwd_d64_bf16_splitkv_msk1, grid, block, 0, stream, *p);
            else
                hipLaunchKernelGGL(fmha_fwd_d64_bf16_splitkv_msk0, grid, block, 0, stream, *p);
        }
        return hipGetLastError();
    }
    const dim3 block(kBlockSize);
    if (varlen) {
        if (causal)
            hipLaunchKernelGGL(fmha_fwd_d64_bf16_msk1_varlen, grid, block, 0, stream, *p);
        else
            hipLaunchKernelGGL(fmha_fwd_d64_bf16_msk0_varlen, grid, block, 0, stream, *p);
    } else {
        if (causal)
            hipLaunchKernelGGL(fmha_fwd_d64_bf16_msk1, grid, block, 0, stream, *p);
        else
            hipLaunchKernelGGL(fmha_fwd_d64_bf16_msk0, grid, block, 0, stream, *p);
    }
    return hipGetLastError();
}

extern "C" hipError_t fmha_fwd_d64_bf16(const FmhaFwdParams* p, int batch, int causal, hipStream_t stream) {
    return fmha_fwd_d64_bf16_variant(p, batch, causal, FMHA_VARIANT_AUTO, stream);
}

extern "C" void fmha_fwd_d64_bf16_tile_config(int* m0, int* n0, int* block_size, int* head_dim) {
    if (m0) *m0 = kM0;
    if (n0) *n0 = kN0;
    if (block_size) *block_size = kBlockSize;
    if (head_dim) *head_dim = kHeadDim;
}
