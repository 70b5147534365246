// fmha_fwd_kernel.hip — gfx950 (CDNA4) D64 BF16 fused MHA forward.
//
// Behaviour follows the reference's fused kernel (src/fused/kernel.cpp:55-99,
// src/fused/pipeline.hpp:98-424): per block one 128-row M-tile of one
// (batch, head); online softmax over 64-key tiles; bottom-right causal mask;
// optional natural-log LSE; dense or varlen (seqstart) addressing; GQA.
// The per-block pipeline is this build's own design for gfx950:
//
//  * Transposed scores.  Each wave owns 32 query rows and computes
//      S^T[32 keys x 32 queries] = K[32 x 64] . Q^T[64 x 32]
//    with v_mfma_f32_32x32x16_bf16.  In the MFMA D layout lane j+32h holds
//    column j (one query) and rows 8*(r/4)+4h+(r%4) (keys), so each lane
//    owns 32 scores of ONE query per 64-key tile: the softmax max/sum are
//    in-lane, plus one v_permlane32_swap to fold the two lane halves.
//  * O^T = V^T . P^T.  P^T is fed to the MFMA B operand straight from the
//    score registers (bf16-converted, no data movement): the B operand's
//    k-index for lane half h / element e is matched by reading V^T with the
//    SAME key permutation (key = 16t + 8(e/4) + 4h + e%4), which
//    ds_read_b64_tr_b16 delivers from a row-major [key][d] LDS tile.
//  * K and V tiles go HBM/L2 -> LDS directly (buffer_load_dwordx4 ... lds),
//    double-buffered with one s_barrier per tile; 16-byte chunks of each
//    128-byte row are XOR-swizzled so the b128 (K) and tr_b16 (V) reads are
//    bank-conflict free.  Out-of-range rows are zero-filled by the buffer
//    descriptor's num_records bound (never read past a tensor or sequence).
//  * Softmax in the exp2 domain with the log2(e) already folded into scale
//    (as the reference, params.hpp:38-43); the running max is only moved
//    when a tile's max exceeds it by more than 8 (log2 units), so the O^T
//    rescale is skipped on almost every tile; P <= 2^8 is exact-range safe.
//  * 4 waves x <=128 VGPRs so 4 blocks (16 waves) share a CU: MFMA of one
//    wave overlaps the exp/FMA softmax of the others on the same SIMD.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fmha_fwd.h"

namespace fmha_gfx950 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = FMHA_KBLOCK / 64;  // 4
constexpr int kRowsPerWave = 32;
constexpr int kTileM = kWaves * kRowsPerWave;  // 128
constexpr int kTileN = FMHA_KN0;               // 64 keys per tile
constexpr int kRowBytes = 128;                 // 64 bf16 per K/V row in LDS
constexpr int kTileBytes = kTileN * kRowBytes; // 8 KiB
constexpr int kStageBytes = 2 * kTileBytes;    // K + V
constexpr int kStages = 2;
constexpr int kLdsBytes = kStages * kStageBytes;  // 32 KiB
constexpr float kRescaleThreshold = 8.0f;         // log2 units
constexpr float kMaxSeed = -5000.0f;              // raw-score running max seed (pipeline.hpp:248-252)
constexpr uint32_t kBufferWord3 = 0x00020000u;    // raw dword buffer, gfx9 family

static_assert(kTileM == FMHA_KM0, "tile rows must match the grid contract");

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t num_bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)num_bytes, (int)kBufferWord3);
}

// Same descriptor as plain dwords, for the inline-asm LDS-DMA loads.
__device__ __forceinline__ i32x4 make_rsrc_words(const void* base, uint32_t num_bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    i32x4 w;
    w[0] = (int)(uint32_t)a;
    w[1] = (int)((uint32_t)(a >> 32) & 0xffffu);  // stride 0, no swizzle
    w[2] = (int)num_bytes;
    w[3] = (int)kBufferWord3;
    return w;
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// 64 lanes x 16 bytes global -> LDS, lane L lands at lds + 16*L.  Issued as
// inline asm so the compiler's waitcnt pass does not treat the in-flight
// prefetch as aliasing every LDS read (it would insert vmcnt(0) before them);
// completion is awaited explicitly with vmcnt_wait0() before the tile barrier.
__device__ __forceinline__ void lds_dma_16(const i32x4& rsrc, uint32_t lds, int voffset) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds), "v"(voffset), "s"(rsrc)
                 : "memory", "m0");
}
__device__ __forceinline__ void vmcnt_wait0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// XOR swizzle of the 16-byte chunk index inside a 128-byte K row (row & 15 is
// all it depends on).  Conflict-free ds_read_b128 for both 32- and 64-bank LDS.
__device__ __forceinline__ int k_swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }
// V rows: the tr_b16 read touches 4 consecutive rows x 4 chunks per 32 lanes.
__device__ __forceinline__ int v_swz(int row) { return (row & 3) << 1; }

__device__ __forceinline__ float wave_max_halves(float x) {
    auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float wave_sum_halves(float x) {
    auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

__device__ __forceinline__ bf16x8 pack8(const f32x16& s, int base) {
    bf16x8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = (__bf16)s[base + e];
    return r;
}

// One block = one kTileM-row M-tile of (batch b, head h).
template <bool kCausal, bool kVarlen>
__device__ __forceinline__ void fwd_mtile(const FmhaFwdParams& p, int b, int h, int mt, char* smem) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int l32 = lane & 31;
    const int hi = lane >> 5;

    // ---- sequence geometry (pipeline.hpp:115-132) ----
    int sq, sk;
    int64_t off_q = 0, off_k = 0;
    if constexpr (kVarlen) {
        off_q = p.seqstart_q[b];
        off_k = p.seqstart_k[b];
        sq = p.seqstart_q[b + 1] - (int)off_q;
        sk = p.seqstart_k[b + 1] - (int)off_k;
    } else {
        sq = p.seqlen_q;
        sk = p.seqlen_k;
    }
    const int row0 = mt * kTileM;
    if (row0 >= sq) return;  // varlen: this M-tile is past the sequence
    const int kvh = h / (p.nhead_q / p.nhead_k);

    const __bf16* qbase;
    const __bf16* kbase;
    const __bf16* vbase;
    __bf16* obase;
    if constexpr (kVarlen) {
        qbase = (const __bf16*)p.q + (int64_t)h * p.nhead_stride_q + off_q * p.stride_q;
        kbase = (const __bf16*)p.k + (int64_t)kvh * p.nhead_stride_k + off_k * p.stride_k;
        vbase = (const __bf16*)p.v + (int64_t)kvh * p.nhead_stride_v + off_k * p.stride_v;
        obase = (__bf16*)p.o + (int64_t)h * p.nhead_stride_o + off_q * p.stride_o;
    } else {
        qbase = (const __bf16*)p.q + (int64_t)b * p.batch_stride_q + (int64_t)h * p.nhead_stride_q;
        kbase = (const __bf16*)p.k + (int64_t)b * p.batch_stride_k + (int64_t)kvh * p.nhead_stride_k;
        vbase = (const __bf16*)p.v + (int64_t)b * p.batch_stride_v + (int64_t)kvh * p.nhead_stride_v;
        obase = (__bf16*)p.o + (int64_t)b * p.batch_stride_o + (int64_t)h * p.nhead_stride_o;
    }
    // num_records = end of the last valid row: rows >= seqlen read as zero
    // (loads) or are dropped (stores).
    const uint32_t qbytes = sq > 0 ? (uint32_t)((int64_t)(sq - 1) * p.stride_q * 2 + kRowBytes) : 0u;
    const uint32_t kbytes = sk > 0 ? (uint32_t)((int64_t)(sk - 1) * p.stride_k * 2 + kRowBytes) : 0u;
    const uint32_t vbytes = sk > 0 ? (uint32_t)((int64_t)(sk - 1) * p.stride_v * 2 + kRowBytes) : 0u;
    const uint32_t obytes = (uint32_t)((int64_t)(sq - 1) * p.stride_o * 2 + kRowBytes);
    const auto rq = make_rsrc(qbase, qbytes);
    const auto ro = make_rsrc(obase, obytes);

    // ---- KV range (pipeline.hpp:168-193): causal stops after the block's
    // last row's diagonal, rounded up to a whole tile ----
    const int shift = sk - sq;
    int kv_end = sk;
    if constexpr (kCausal) {
        int last = row0 + kTileM - 1;
        if (last > sq - 1) last = sq - 1;
        int e = last + shift + 1;
        kv_end = e < 0 ? 0 : (e > sk ? sk : e);
    }
    const int ntiles = (kv_end + kTileN - 1) / kTileN;

    const int wrow0 = row0 + wave * kRowsPerWave;  // first query row of this wave
    const int my_row = wrow0 + l32;                // this lane's query row

    // ---- Q^T operand (B of GEMM0): lane (q, h) holds Q[q][16t + 8h .. +7] ----
    bf16x8 qop[4];
    {
        const int qoff = my_row * p.stride_q * 2 + hi * 16;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            i32x4 raw = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff + t * 32, 0, 0);
            qop[t] = __builtin_bit_cast(bf16x8, raw);
        }
        // Retire the Q loads here, visibly to the compiler: otherwise it keeps
        // them "pending" into the loop and waits vmcnt there, which would also
        // wait for the in-flight K/V prefetch.
        asm volatile("" ::"v"(qop[0]), "v"(qop[1]), "v"(qop[2]), "v"(qop[3]));
    }

    // ---- global -> LDS tile loader: each wave moves 2 x 1 KiB of K and of V.
    // Lane L of load i writes LDS row 8*(2*wave+i) + L/8, physical chunk L%8,
    // fetched from logical chunk (L%8) ^ swz(row). ----
    const int ld_row = (2 * wave) * 8 + (lane >> 3);  // + 8 for i = 1
    const int ld_pc = lane & 7;
    const int k_ld_off0 = ld_row * p.stride_k * 2 + ((ld_pc ^ k_swz(ld_row)) << 4);
    const int k_ld_off1 = (ld_row + 8) * p.stride_k * 2 + ((ld_pc ^ k_swz(ld_row + 8)) << 4);
    const int v_ld_off0 = ld_row * p.stride_v * 2 + ((ld_pc ^ v_swz(ld_row)) << 4);
    const int v_ld_off1 = (ld_row + 8) * p.stride_v * 2 + ((ld_pc ^ v_swz(ld_row + 8)) << 4);
    const int k_tile_step = kTileN * p.stride_k * 2;
    const int v_tile_step = kTileN * p.stride_v * 2;

    const i32x4 rk_w = make_rsrc_words(kbase, kbytes);
    const i32x4 rv_w = make_rsrc_words(vbase, vbytes);
    const uint32_t lds_wave = lds_addr(smem) + (2 * wave) * 1024;
    auto issue_tile = [&](int tile, int stage) {
        const uint32_t st = lds_wave + stage * kStageBytes;
        const int kt = tile * k_tile_step;
        const int vt = tile * v_tile_step;
        lds_dma_16(rk_w, st, k_ld_off0 + kt);
        lds_dma_16(rk_w, st + 1024, k_ld_off1 + kt);
        lds_dma_16(rv_w, st + kTileBytes, v_ld_off0 + vt);
        lds_dma_16(rv_w, st + kTileBytes + 1024, v_ld_off1 + vt);
    };

    // ---- per-lane LDS read addresses ----
    // K (A of GEMM0): lane (i=l32, h) reads row kb*32 + i, logical chunk 2t + h.
    int k_rd[4];
    {
        const int f = k_swz(l32);
#pragma unroll
        for (int t = 0; t < 4; ++t) k_rd[t] = l32 * kRowBytes + (((2 * t + hi) ^ f) << 4);
    }
    // V^T (A of GEMM1) via ds_read_b64_tr_b16: in each 16-lane group, source
    // lane 4e + c supplies the address of 4 d-values (d = dbase + 4c) of key
    // row key0 + e; lane i of the group then receives V[key0 + e][dbase + i]
    // for e = 0..3.  key0 = kb*32 + 16t + 8u + 4h, dbase = 32db + 16*(g%2).
    int v_rd[2];
    {
        const int g = lane >> 4, i16 = lane & 15;
        const int e = i16 >> 2, c = i16 & 3;
        const int row = 4 * hi + e;  // + kb*32 + 16t + 8u (multiples of 8: swizzle unchanged)
#pragma unroll
        for (int db = 0; db < 2; ++db) {
            const int chunk = 4 * db + 2 * (g & 1) + (c >> 1);
            v_rd[db] = kTileBytes + row * kRowBytes + ((chunk ^ v_swz(row)) << 4) + (c & 1) * 8;
        }
    }

    // ---- online-softmax state (per lane = per query row; both lane halves
    // of a row keep identical m, partial l) ----
    const float scale = p.scale;                       // log2(e)/sqrt(D)
    const float thr_raw = kRescaleThreshold / scale;   // threshold in raw-score units
    float m_ref = kMaxSeed;
    float l_part = 0.0f;
    f32x16 oacc[2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[db][r] = 0.0f;

    // Rows this wave can see: causal limit of its last row.
    const int wave_key_limit = kCausal ? (wrow0 + kRowsPerWave - 1 + shift) : 0x7fffffff;
    const bool wave_active = wrow0 < sq;

    if (ntiles > 0) issue_tile(0, 0);

    for (int j = 0; j < ntiles; ++j) {
        const int stage = j & 1;
        // own loads of tile j complete, then make everybody's visible; the same
        // barrier also retires every wave's reads of stage (j+1)&1 (tile j-1).
        vmcnt_wait0();
        __syncthreads();
        if (j + 1 < ntiles) issue_tile(j + 1, stage ^ 1);

        const int key0 = j * kTileN;
        if (!wave_active || key0 > wave_key_limit) continue;  // wave fully masked for this tile

        const char* st = smem + stage * kStageBytes;

        // ---- GEMM0: S^T[kb] = K[kb] . Q^T ----
        f32x16 s[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            f32x16 acc = {};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const bf16x8 kop = *(const bf16x8*)(st + kb * 32 * kRowBytes + k_rd[t]);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop, qop[t], acc, 0, 0, 0);
            }
            s[kb] = acc;
        }

        // ---- mask: keys >= sk, and (causal) keys > row + shift ----
        const bool need_mask = (key0 + kTileN > sk) || (kCausal && key0 + kTileN - 1 > wrow0 + shift);
        if (need_mask) {
            const int lim = kCausal ? min(sk - 1, my_row + shift) : sk - 1;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = key0 + kb * 32 + 8 * (r >> 2) + 4 * hi + (r & 3);
                    if (key > lim) s[kb][r] = -INFINITY;
                }
        }

        // ---- row max over the tile; move the reference max only when the
        // tile exceeds it by > kRescaleThreshold (log2 units) ----
        float mx = s[0][0];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
        mx = wave_max_halves(mx);
        const bool grow = mx > m_ref + thr_raw;
        if (__builtin_amdgcn_ballot_w64(grow)) {
            const float m_new = grow ? mx : m_ref;
            const float alpha = __builtin_amdgcn_exp2f((m_ref - m_new) * scale);
            l_part *= alpha;
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
            m_ref = m_new;
        }

        // ---- P = exp2(s*scale - m_ref*scale), partial row sum, bf16 pack ----
        const float neg_ms = -m_ref * scale;
        float lsum = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][r], scale, neg_ms));
                s[kb][r] = pv;
                lsum += pv;
            }
        l_part += lsum;

        // ---- GEMM1: O^T[db] += V^T[db] . P^T ----
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const bf16x8 pop = pack8(s[kb], 8 * t);
#pragma unroll
                for (int db = 0; db < 2; ++db) {
                    const int a0 = v_rd[db] + (kb * 32 + 16 * t) * kRowBytes;
                    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(st + a0));
                    const i16x4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(st + a0 + 8 * kRowBytes));
                    i16x4 both[2] = {lo, hi4};
                    const bf16x8 vop = __builtin_bit_cast(bf16x8, both);
                    oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vop, pop, oacc[db], 0, 0, 0);
                }
            }
    }

    // ---- epilogue: O = O^T / l (rows < sq; the buffer bound drops the rest),
    // LSE = (log2(l) + scale*m) * ln2 (natural log, -inf for an empty row) ----
    const float l_tot = wave_sum_halves(l_part);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    {
        const int orow_off = my_row * p.stride_o * 2;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                bf16x2 a, c;
                a[0] = (__bf16)(oacc[db][4 * g4 + 0] * inv);
                a[1] = (__bf16)(oacc[db][4 * g4 + 1] * inv);
                c[0] = (__bf16)(oacc[db][4 * g4 + 2] * inv);
                c[1] = (__bf16)(oacc[db][4 * g4 + 3] * inv);
                i32x2 w;
                w[0] = __builtin_bit_cast(int, a);
                w[1] = __builtin_bit_cast(int, c);
                const int d0 = 32 * db + 8 * g4 + 4 * hi;
                __builtin_amdgcn_raw_buffer_store_b64(w, ro, orow_off + d0 * 2, 0, 0);
            }
    }
    if (p.lse != nullptr && hi == 0 && my_row < sq) {
        float* lse_base;
        if constexpr (kVarlen)
            lse_base = p.lse + (int64_t)h * (p.nhead_stride_q / p.stride_q) + off_q;
        else
            lse_base = p.lse + (int64_t)b * p.nhead_q * p.seqlen_q + (int64_t)h * p.seqlen_q;
        const float lse2 = __builtin_log2f(l_tot) + m_ref * scale;  // -inf when l == 0
        lse_base[my_row] = lse2 * 0.69314718055994530942f;
    }
}

}  // namespace fmha_gfx950

using namespace fmha_gfx950;

// ---- the four entries (reference src/fused/kernel.cpp:55-99).  Grid
// (nhead_q, ceil(seqlen_q/kM0), batch).  Causal entries run the heaviest
// M-tiles first (kernel.cpp:73,96). ----
#define FMHA_ENTRY_ATTRS __global__ __launch_bounds__(FMHA_KBLOCK) __attribute__((amdgpu_waves_per_eu(4, 4)))

FMHA_ENTRY_ATTRS void fmha_fwd_d64_bf16_msk0(FmhaFwdParams params) {
    __shared__ __attribute__((aligned(1024))) char smem[kLdsBytes];
    fwd_mtile<false, false>(params, blockIdx.z, blockIdx.x, blockIdx.y, smem);
}
FMHA_ENTRY_ATTRS void fmha_fwd_d64_bf16_msk1(FmhaFwdParams params) {
    __shared__ __attribute__((aligned(1024))) char smem[kLdsBytes];
    fwd_mtile<true, false>(params, blockIdx.z, blockIdx.x, gridDim.y - 1 - blockIdx.y, smem);
}
FMHA_ENTRY_ATTRS void fmha_fwd_d64_bf16_msk0_varlen(FmhaFwdParams params) {
    __shared__ __attribute__((aligned(1024))) char smem[kLdsBytes];
    fwd_mtile<false, true>(params, blockIdx.z, blockIdx.x, blockIdx.y, smem);
}
FMHA_ENTRY_ATTRS void fmha_fwd_d64_bf16_msk1_varlen(FmhaFwdParams params) {
    __shared__ __attribute__((aligned(1024))) char smem[kLdsBytes];
    fwd_mtile<true, true>(params, blockIdx.z, blockIdx.x, gridDim.y - 1 - blockIdx.y, smem);
}
