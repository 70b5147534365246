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
//  * In-wave software pipeline.  Iteration t issues the 16 MFMAs of
//    GEMM1(tile t-1) and GEMM0(tile t+1) interleaved with the softmax VALU
//    work of tile t (sched_group_barrier): the three stages have no data
//    dependence on each other inside an iteration, so one wave keeps the
//    matrix core and the VALU busy at the same time.  The first iteration
//    issues GEMM0(tile 1) only (there is no tile -1).
//  * K and V tiles go HBM/L2 -> LDS directly (buffer_load_dwordx4 ... lds)
//    in two 4-deep rings: K(t+4) and V(t+2) are fetched during iteration t,
//    i.e. both three iterations before they are read; one s_barrier per tile.
//    The loop is unrolled by the ring depth so every LDS stage offset is an
//    instruction immediate.
//    16-byte chunks of each 128-byte row are XOR-swizzled so the b128 (K)
//    and tr_b16 (V) reads are bank-conflict free.  Out-of-range rows are
//    zero-filled by the buffer descriptor's num_records bound (never read past
//    a tensor or sequence).
//  * Softmax in the exp2 domain with the log2(e) already folded into scale
//    (as the reference, params.hpp:38-43), speculative: P is computed in the
//    current reference-max frame without taking the tile's max; only when a
//    lane's tile sum of P exceeds 2^16 (so some score is far above the frame)
//    does the wave take the exact max, rescale O^T and l, and redo the tile.
//    Any frame gives the same O and LSE; this one keeps every P <= 2^16
//    (far inside fp32 and bf16 range), and a frame lasts until a row's max
//    grows by more than ~11 (log2 units) past it.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "fmha_fwd.h"
#include "fmha_internal.h"

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
constexpr int kRing = 4;                       // stages per ring (K and V)
constexpr int kLoadsPerTile = 2;                   // 1 KiB DMA per load, per wave
constexpr float kGrowSum = 65536.0f;               // tile-sum bound of the speculative softmax
// Running-max seed, in the scaled (exp2) domain: below every finite scaled
// score, so a row's first visible key always re-frames it (its P overflows
// the bound).  The reference seeds -5000 raw-score units (pipeline.hpp:248-252),
// which drops rows whose every score lies below that; its CPU checker
// (cpu_ref.cpp:124-136) has no seed at all, and neither has this kernel.
constexpr float kMaxSeed = -3.402823466e38f;       // -FLT_MAX
constexpr uint32_t kBufferWord3 = 0x00020000u;     // raw dword buffer, gfx9 family
constexpr int kPartFloatsPerWave = 34 * 64;        // balanced form: one wave's partial result (O^T, m, l)
// Cache policy of the O stores: non-temporal (NT).  No block reads O back, and
// O kept out of the caches leaves them to K/V (dense B4 H16 S2048 and causal
// B1 H16 S8192 +1 %, short form dense B128 H16 S128 +2.5 %).
constexpr int kStoreStream = 2;

// sched_group_barrier instruction classes
constexpr int kSchedVALU = 0x002;
constexpr int kSchedMFMA = 0x008;
constexpr int kSchedDSRead = 0x100;

static_assert(kTileM == FMHA_KM0, "tile rows must match the grid contract");
static_assert(kWaves * kLoadsPerTile * 1024 == kTileBytes, "one tile = one DMA round of the block");

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t num_bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)num_bytes, (int)kBufferWord3);
}

typedef __attribute__((address_space(3))) char lds_char;

// The LDS rings: every stage is its own __shared__ array, so the compiler's
// LDS alias scopes tell its waitcnt pass that a prefetch into one stage does
// not alias reads of the others (with one flat buffer it would wait for every
// in-flight prefetch before each LDS read).
struct Ring {
    lds_char* k[kRing];
    lds_char* v[kRing];
};

// 64 lanes x 16 bytes global -> LDS (buffer_load_dwordx4 ... lds); lane L
// lands at dst + 16*L.  dst must be wave-uniform.
__device__ __forceinline__ void lds_dma_16(__amdgpu_buffer_rsrc_t rsrc, lds_char* dst, int voffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)dst, 16, voffset, 0, 0, 0);
}
// The same with a wave-uniform byte offset in the scalar offset operand.
__device__ __forceinline__ void lds_dma_16(__amdgpu_buffer_rsrc_t rsrc, lds_char* dst, int voffset, int soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)dst, 16, voffset, soffset,
                                             0, 0);
}
// Own-wave DMA completion before a tile barrier (the barrier then makes every
// wave's part of the tile visible).
template <int N>
__device__ __forceinline__ void vmcnt_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// s_waitcnt immediate for vmcnt(0) alone (gfx9 encoding: vmcnt [3:0] and
// [15:14], expcnt [6:4] and lgkmcnt [11:8] at their no-wait maxima)
constexpr int kWaitVmcnt0 = 0x0F70;
// s_waitcnt immediate for lgkmcnt(0) alone (vmcnt and expcnt at their maxima)
constexpr int kWaitLgkmcnt0 = 0xC07F;
// Workgroup barrier of the K/V ring, without __syncthreads()'s memory fence:
// that fence waits vmcnt(0), i.e. also for the prefetches still in flight.
// Before the barrier each wave has waited for its own DMA of the tile about
// to be read (vmcnt_wait) and, here, for all of its own LDS reads
// (lgkmcnt(0)): right after the barrier other waves refill the stages those
// reads came from, and s_barrier itself waits for no memory operation (the
// compiler may otherwise leave a read in flight across it when it sinks the
// consuming MFMA past the barrier).  The "memory" clobber keeps the compiler
// from moving LDS accesses across it.
__device__ __forceinline__ void ring_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// A copy of a wave-uniform value in a VGPR.  A VALU operand read from an SGPR
// costs gfx950 ~4.4 issue cycles per wave64 instruction against ~2.6-3.2 for
// VGPR operands (fma, mul, sub alike), so per-element operands are kept in VGPRs.
__device__ __forceinline__ float in_vgpr(float x) {
    float v;
    asm("v_mov_b32 %0, %1" : "=v"(v) : "s"(x));
    return v;
}

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

typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
typedef __attribute__((address_space(3))) i32x4 lds_i32x4;

__device__ __forceinline__ bf16x8 lds_read_b128(const lds_char* p) { return *(const lds_bf16x8*)p; }
// 8 keys x 1 head-dim column of V for the GEMM1 A operand (two tr_b16 reads,
// rows key0..key0+3 and key0+8..key0+11).
__device__ __forceinline__ bf16x8 lds_read_vt(const lds_char* p) {
    const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p);
    const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 8 * kRowBytes));
    i16x4 both[2] = {lo, hi};
    return __builtin_bit_cast(bf16x8, both);
}

__device__ __forceinline__ f32x16 mfma(const bf16x8& a, const bf16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Schedule of one pipelined iteration: one slot per MFMA of {1 MFMA, the DS
// reads of the MFMA kDsAhead slots later, VALU}.  A full iteration has 16
// MFMAs: 0-7 GEMM1's (two tr_b16 reads each), 8-15 GEMM0's (one b128 read
// each).  The first iteration of a block has no GEMM1 (there is no tile -1)
// and the last no GEMM0 (there is no tile n): 8 slots, with twice the VALU
// each.  The reads of MFMAs 0 .. kDsAhead-1 open the iteration.  Groups are
// filled in order, respecting dependences; VALU the groups do not claim is
// placed by the scheduler, so the softmax of a tile (~115 VALU: 32 fma, 32
// exp, 32 add, 16 cvt_pk, bookkeeping) lands as 8-11 per slot over the first
// 12 slots and the last GEMM0 chain runs bare.  A rigid even spread (every
// slot fenced with sched_barrier, 7 VALU each) gives the same bits and is
// 2-3% slower on the benchmark grids.
constexpr int kValuPerSlot = 7;
constexpr int kDsAhead = 2;
template <bool kG1, bool kG0>
struct IterSchedule {
    static constexpr int kMfma = 8 * (int(kG1) + int(kG0));
    static constexpr int kValu = kMfma == 16 ? kValuPerSlot : 2 * kValuPerSlot;
    static constexpr int reads(int m) { return m >= kMfma ? 0 : (kG1 && m < 8) ? 2 : 1; }
    static constexpr int reads_before(int n) { return n <= 0 ? 0 : reads(n - 1) + reads_before(n - 1); }
    template <int I>
    static __device__ __forceinline__ void slot() {
        __builtin_amdgcn_sched_group_barrier(kSchedMFMA, 1, 0);
        if constexpr (reads(I + kDsAhead) > 0) __builtin_amdgcn_sched_group_barrier(kSchedDSRead, reads(I + kDsAhead), 0);
        __builtin_amdgcn_sched_group_barrier(kSchedVALU, kValu, 0);
    }
    template <int... Is>
    static __device__ __forceinline__ void run(std::integer_sequence<int, Is...>) {
        __builtin_amdgcn_sched_group_barrier(kSchedDSRead, reads_before(kDsAhead), 0);
        (slot<Is>(), ...);
    }
    static __device__ __forceinline__ void apply() {
        if constexpr (kMfma > 0) run(std::make_integer_sequence<int, kMfma>{});
    }
};

// Online-softmax state of one lane's query row (both lane halves of a row keep
// the same m_ref; l_part is this lane's partial sum).
struct Softmax {
    float m_ref;   // reference max, scaled: max of s * scale (exp2 domain)
    float l_part;  // partial row sum of P in the m_ref frame, tiles before the current one
    float l_tile;  // this lane's sum of P over the current tile
};

// Block forms.  Every group of kWaves waves computes 128 query rows over a
// range of key tiles; all groups of a block run the same number of
// iterations, so the block-wide barriers stay in step.
//  * kModeRegular: one group, one M-tile (the reference's entries).
//  * kModeSplitKV: two groups on the same M-tile, each walking a contiguous
//    half of its key tiles with its own half of every LDS stage; their
//    partial (O^T, m, l) are merged through LDS at the end (group 1 hands
//    over, group 0 writes O and LSE).  For grids too small to fill the GPU.
//  * kModePair: two groups on the adjacent M-tiles 2mt and 2mt+1 of one
//    (batch, head), sharing every K/V tile (loaded once, by all 8 waves).
//    The shared barrier keeps both in lockstep: two separate blocks on one
//    compute unit progress unevenly (one is served first), so the CU's last
//    block runs alone at the end; a pair has no such tail.
//  * kModeBalanced: one group, one item of a balanced causal launch: the
//    whole M-tile, or one half of its key tiles (a split M-tile), whose
//    partial result goes to a workspace slot for the merge launch.
//  * kModeBalancedPair: kModePair's two groups on one item of a balanced
//    causal launch of M-tile pairs: the pair's key tiles, or one half of
//    them, each group's partial result to its own M-tile's slot.
enum : int { kModeRegular = 0, kModeSplitKV = 1, kModePair = 2, kModeBalanced = 3, kModeBalancedPair = 4 };
// The key range of a balanced-launch item: `part` null for a whole M-tile;
// otherwise half `half` of its key tiles and the slot of its partial result.
struct Chunk {
    int half;
    float* part;
};
template <bool kCausal, bool kVarlen, int kMode>
__device__ __forceinline__ void fwd_mtile(const FmhaFwdParams& p, int b, int h, int mt, const Ring& ring,
                                          Chunk ck = Chunk{0, nullptr}) {
    constexpr int kGroups = (kMode == kModeRegular || kMode == kModeBalanced) ? 1 : 2;
    constexpr bool kSplitKV = kMode == kModeSplitKV;
    constexpr bool kPair = kMode == kModePair || kMode == kModeBalancedPair;
    constexpr bool kBalanced = kMode == kModeBalanced || kMode == kModeBalancedPair;
    constexpr int kLoads = kPair ? 1 : kLoadsPerTile;  // DMA loads per wave, tensor and tile
    const int lane = threadIdx.x & 63;
    const int wave_id = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int group = kGroups == 1 ? 0 : wave_id / kWaves;
    const int wave = kGroups == 1 ? wave_id : wave_id % kWaves;            // wave within the group
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
    const int blk_row0 = (kPair ? 2 * mt : mt) * kTileM;  // the block's first row
    if (blk_row0 >= sq) return;  // varlen: this M-tile is past the sequence
    const int row0 = blk_row0 + (kPair ? group * kTileM : 0);  // this group's M-tile
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
        int last = blk_row0 + (kPair ? 2 : 1) * kTileM - 1;
        if (last > sq - 1) last = sq - 1;
        int e = last + shift + 1;
        kv_end = e < 0 ? 0 : (e > sk ? sk : e);
    }
    const int ntiles = (kv_end + kTileN - 1) / kTileN;
    // this group's key tiles: global tiles [tile0, tile0 + ntg) (the loops
    // below count group-local tiles 0 .. ntg-1); tiles >= tile_end are dead
    int ntg = kSplitKV ? (ntiles + 1) / 2 : ntiles;
    int tile0 = kSplitKV ? group * ntg : 0;
    if constexpr (kBalanced) {
        if (ck.part != nullptr) {  // a split M-tile (pair): the first ceil(n/2) key tiles, or the rest
            const int h0 = (ntiles + 1) / 2;
            tile0 = ck.half ? h0 : 0;
            ntg = ck.half ? ntiles - h0 : h0;
        }
    }
    const int tile_end = min(ntiles, tile0 + ntg);

    const int wrow0 = row0 + wave * kRowsPerWave;  // first query row of this wave
    const int my_row = wrow0 + l32;                // this lane's query row

    // ---- Q^T operand (B of GEMM0): lane (q, h) holds Q[q][16t + 8h .. +7];
    // loaded first thing in the prologue (a block with no key tile skips it) ----
    bf16x8 qop[4];

    // ---- global -> LDS tile loaders: per tile each wave moves kLoads x 1 KiB
    // of K (or V).  Lane L of load i writes LDS row 8*(kLoads*w+i) + L/8
    // (w: the wave's index among the waves sharing the tile), physical chunk
    // L%8, fetched from logical chunk (L%8) ^ swz(row).  Tiles past the KV
    // range get an empty descriptor (zero fill, no memory traffic), so every
    // iteration issues the same number of loads. ----
    const int ld_wave = kPair ? wave_id : wave;
    const int ld_row = (kLoads * ld_wave) * 8 + (lane >> 3);
    const int ld_pc = lane & 7;
    const int k_ld_off0 = ld_row * p.stride_k * 2 + ((ld_pc ^ k_swz(ld_row)) << 4);
    const int k_ld_off1 = (ld_row + 8) * p.stride_k * 2 + ((ld_pc ^ k_swz(ld_row + 8)) << 4);
    const int v_ld_off0 = ld_row * p.stride_v * 2 + ((ld_pc ^ v_swz(ld_row)) << 4);
    const int v_ld_off1 = (ld_row + 8) * p.stride_v * 2 + ((ld_pc ^ v_swz(ld_row + 8)) << 4);
    const int k_tile_step = kTileN * p.stride_k * 2;
    const int v_tile_step = kTileN * p.stride_v * 2;
    const int goff = kSplitKV ? group * kTileBytes : 0;  // split-KV: this group's half of every stage
    const int wave_off = goff + (kLoads * ld_wave) * 1024;

    // Local tile t's K lands in K stage t % kRing, its V in V stage t % kRing.
    // The tile's own descriptor (base at the tile's first row, num_records =
    // bytes left; 0 for a dead tile) is built in scalar registers, so the
    // per-lane offsets stay loop-invariant.
    auto issue_k = [&](int tile, auto stage_c) {
        lds_char* dst = ring.k[decltype(stage_c)::value] + wave_off;
        const int gt = tile0 + tile;
        const uint32_t t0 = (uint32_t)gt * (uint32_t)k_tile_step;
        const auto r = make_rsrc((const char*)kbase + t0, gt < tile_end ? kbytes - t0 : 0u);
        lds_dma_16(r, dst, k_ld_off0);
        if constexpr (kLoads == 2) lds_dma_16(r, dst + 1024, k_ld_off1);
    };
    auto issue_v = [&](int tile, auto stage_c) {
        lds_char* dst = ring.v[decltype(stage_c)::value] + wave_off;
        const int gt = tile0 + tile;
        const uint32_t t0 = (uint32_t)gt * (uint32_t)v_tile_step;
        const auto r = make_rsrc((const char*)vbase + t0, gt < tile_end ? vbytes - t0 : 0u);
        lds_dma_16(r, dst, v_ld_off0);
        if constexpr (kLoads == 2) lds_dma_16(r, dst + 1024, v_ld_off1);
    };

    // ---- per-lane LDS read offsets inside a tile ----
    // K (A of GEMM0): lane (i=l32, h) reads row kb*32 + i, logical chunk 2t + h.
    uint32_t k_rd[4];
    {
        const int f = k_swz(l32);
#pragma unroll
        for (int t = 0; t < 4; ++t) k_rd[t] = goff + l32 * kRowBytes + (((2 * t + hi) ^ f) << 4);
    }
    // V^T (A of GEMM1) via ds_read_b64_tr_b16: in each 16-lane group, source
    // lane 4e + c supplies the address of 4 d-values (d = dbase + 4c) of key
    // row key0 + e; lane i of the group then receives V[key0 + e][dbase + i]
    // for e = 0..3.  key0 = kb*32 + 16t + 8u + 4h, dbase = 32db + 16*(g%2).
    uint32_t v_rd[2];
    {
        const int g = lane >> 4, i16 = lane & 15;
        const int e = i16 >> 2, c = i16 & 3;
        const int row = 4 * hi + e;  // + kb*32 + 16t + 8u (multiples of 8: swizzle unchanged)
#pragma unroll
        for (int db = 0; db < 2; ++db) {
            const int chunk = 4 * db + 2 * (g & 1) + (c >> 1);
            v_rd[db] = goff + row * kRowBytes + ((chunk ^ v_swz(row)) << 4) + (c & 1) * 8;
        }
    }

    const float scale = p.scale;          // log2(e)/sqrt(D)
    const float scale_v = in_vgpr(scale);  // the per-score fma's operand
    Softmax sm{kMaxSeed, 0.0f, 0.0f};
    f32x16 oacc[2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[db][r] = 0.0f;

    // ---- the three pipeline stages (stage indices are compile-time) ----
    // GEMM0 of the tile in K stage KS: S^T[kb] = K[kb] . Q^T
    auto gemm0 = [&](auto ks_c, f32x16* s) {
        const lds_char* st = ring.k[decltype(ks_c)::value];  // k_rd includes goff
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            f32x16 acc = {};
#pragma unroll
            for (int k = 0; k < 4; ++k) acc = mfma(lds_read_b128(st + k_rd[k] + kb * 32 * kRowBytes), qop[k], acc);
            s[kb] = acc;
        }
    };
    // GEMM1 of the tile in V stage VS: O^T[db] += V^T[db] . P^T
    auto gemm1 = [&](auto vs_c, const bf16x8* pp) {
        const lds_char* st = ring.v[decltype(vs_c)::value];  // v_rd includes goff
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int k = 0; k < 2; ++k)
#pragma unroll
                for (int db = 0; db < 2; ++db)
                    oacc[db] = mfma(lds_read_vt(st + v_rd[db] + (kb * 32 + 16 * k) * kRowBytes), pp[2 * kb + k],
                                    oacc[db]);
    };
    // mask of local tile t: keys >= sk, and (causal) keys > row + shift
    auto mask_tile = [&](int t, f32x16* s) {
        const int key0 = (tile0 + t) * kTileN;
        const bool need = (key0 + kTileN > sk) || (kCausal && key0 + kTileN - 1 > wrow0 + shift);
        if (need) {
            // element (kb, r) holds key key0 + 4h + c with c = 32kb + 8(r/4) + r%4;
            // it is visible iff c <= d: one compare (c is an inline constant)
            // and one select per element.
            const int lim = kCausal ? min(sk - 1, my_row + shift) : sk - 1;
            const int d = lim - (key0 + 4 * hi);
            const float ninf = in_vgpr(-__builtin_inff());
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int c = 32 * kb + 8 * (r >> 2) + (r & 3);
                    s[kb][r] = c <= d ? s[kb][r] : ninf;
                }
        }
    };
    // exact max of a score tile over the lane's row (both lane halves)
    auto tile_max = [&](const f32x16* s) {
        float mp[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) mp[i] = fmaxf(fmaxf(s[i >> 2][4 * (i & 3)], s[i >> 2][4 * (i & 3) + 1]),
                                                  fmaxf(s[i >> 2][4 * (i & 3) + 2], s[i >> 2][4 * (i & 3) + 3]));
        const float mx = fmaxf(fmaxf(fmaxf(mp[0], mp[1]), fmaxf(mp[2], mp[3])),
                               fmaxf(fmaxf(mp[4], mp[5]), fmaxf(mp[6], mp[7])));
        return wave_max_halves(mx);
    };
    // P = exp2(s*scale - m_ref), bf16-packed into the GEMM1 B operands,
    // and this lane's tile sum of P (fp32, before the bf16 rounding).
    auto exp_tile = [&](const f32x16* s, bf16x8* pp) {
        const float neg_ms = -sm.m_ref;
        float ls[4];  // 4 independent partial chains (latency)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                bf16x8 pk;
                float acc;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][8 * k + e], scale_v, neg_ms));
                    acc = e == 0 ? pv : acc + pv;
                    pk[e] = (__bf16)pv;
                }
                ls[2 * kb + k] = acc;
                pp[2 * kb + k] = pk;
            }
        sm.l_tile = (ls[0] + ls[1]) + (ls[2] + ls[3]);
    };
    // Softmax of one tile, speculatively in the current m_ref frame: no max
    // is taken on this path.  P and its sum stay exact whatever m_ref is, as
    // long as nothing overflows; settle() re-runs the tile with a new m_ref
    // when the tile sum leaves the safe range.
    auto softmax = [&](const f32x16* s, bf16x8* pp) {
        exp_tile(s, pp);
        // keep P and the tile sum computed in this block: both would otherwise
        // be sunk towards their next use, out of the interleaved region
        asm volatile("" ::"v"(pp[0]), "v"(pp[1]), "v"(pp[2]), "v"(pp[3]), "v"(sm.l_tile));
    };
    // After the interleaved block of tile t (whose GEMM1(t-1) has then been
    // issued): a lane whose tile sum exceeds kGrowSum (every P <= the sum, so
    // P <= kGrowSum otherwise) has scores well above m_ref.  Then the whole
    // wave moves m_ref to max(m_ref, tile max), rescales O^T and l, and
    // recomputes the tile's P.  The first tile's m_ref is set exactly before
    // the loop, so this path is only taken when a row's max grows by more
    // than log2(kGrowSum / 32) after its first tile.
    auto settle = [&](const f32x16* s, bf16x8* pp) {
        if (__builtin_amdgcn_ballot_w64(!(sm.l_tile <= kGrowSum))) {
            asm volatile("" ::: "memory");  // a side effect: keeps the rare path a branch, not speculated
            const float m_new = fmaxf(sm.m_ref, tile_max(s) * scale);
            const float alpha = __builtin_amdgcn_exp2f(sm.m_ref - m_new);
            sm.m_ref = m_new;
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
            sm.l_part *= alpha;
            exp_tile(s, pp);
        }
        sm.l_part += sm.l_tile;
    };
    f32x16 sacc[2][2];  // S^T of two consecutive tiles (alternating roles)
    bf16x8 pbuf[2][4];  // P^T of two consecutive tiles (alternating roles)

    // iteration t (phase J = t % kRing): GEMM1(t-1) || GEMM0(t+1) || softmax(t).
    // The first iteration has no GEMM1 (kG1 = false: there is no tile -1);
    // every iteration waits, synchronises and refills the ring the same way,
    // so all waves of a block pass the same barriers.
    auto iteration = [&](int t, auto phase_c, auto g1_c, auto g0_c) {
        constexpr int J = decltype(phase_c)::value;
        constexpr bool kG1 = decltype(g1_c)::value, kG0 = decltype(g0_c)::value;
        constexpr int cur = J & 1, nxt = cur ^ 1;
        // K(t+1) and V(t-1) were fetched three iterations ago; the loads of
        // the two previous iterations may still fly.
        vmcnt_wait<4 * kLoads>();
        ring_barrier();
        issue_k(t + kRing, std::integral_constant<int, J>{});
        issue_v(t + 2, std::integral_constant<int, (J + 2) % kRing>{});
        mask_tile(t, sacc[cur]);
        if constexpr (kG1) gemm1(std::integral_constant<int, (J + kRing - 1) % kRing>{}, pbuf[nxt]);
        if constexpr (kG0) gemm0(std::integral_constant<int, (J + 1) % kRing>{}, sacc[nxt]);
        softmax(sacc[cur], pbuf[cur]);
        IterSchedule<kG1, kG0>::apply();
        settle(sacc[cur], pbuf[cur]);
    };
    // the last GEMM1, for tile t of phase J
    auto last_gemm1 = [&](auto phase_c) {
        constexpr int J = decltype(phase_c)::value;
        vmcnt_wait<0>();  // every DMA landed (none may outlive the block)
        ring_barrier();
        gemm1(std::integral_constant<int, J>{}, pbuf[J & 1]);
    };
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    using P2 = std::integral_constant<int, 2>;
    using P3 = std::integral_constant<int, 3>;
    using Yes = std::true_type;
    using No = std::false_type;
    auto mid = [&](int t, auto phase_c) { iteration(t, phase_c, Yes{}, Yes{}); };

    // Causal: tiles past the last key this wave's rows can see hold only
    // masked scores for it (P = 0; the pair form's first group has two such
    // tiles at the end, every M-tile's first two waves one).  The wave
    // computes its live tiles only and then keeps the ring going without
    // compute: each later iteration still waits for its own loads, passes
    // the barrier and issues its share of the DMA, so every wave passes the
    // same barriers and issues the same loads as before.
    int nlive = ntg;
    if constexpr (kCausal) {
        const int last_key = min(sk - 1, wrow0 + kRowsPerWave - 1 + shift);
        const int lt = last_key < 0 ? 0 : last_key / kTileN + 1 - tile0;  // local tiles up to that key
        nlive = max(1, min(ntg, lt));
    }
    // iteration t of a wave past its live tiles (phase J): its loads, and
    // the GEMM1 of its last live tile when kG1
    auto idle = [&](int t, auto phase_c, auto g1_c) {
        constexpr int J = decltype(phase_c)::value;
        vmcnt_wait<4 * kLoads>();
        ring_barrier();
        issue_k(t + kRing, std::integral_constant<int, J>{});
        issue_v(t + 2, std::integral_constant<int, (J + 2) % kRing>{});
        if constexpr (decltype(g1_c)::value)
            gemm1(std::integral_constant<int, (J + kRing - 1) % kRing>{}, pbuf[(J & 1) ^ 1]);
    };
    // after the last live tile (phase J): the block's last GEMM1, or the
    // idle iterations up to ntg and the block's final barrier
    auto finish_live = [&](auto phase_c) {
        constexpr int J = decltype(phase_c)::value;
        if (nlive == ntg) {
            last_gemm1(phase_c);
            return;
        }
        idle(nlive, std::integral_constant<int, (J + 1) % kRing>{}, Yes{});
        for (int u = nlive + 1; u < ntg; u += kRing) {
            idle(u, std::integral_constant<int, (J + 2) % kRing>{}, No{});
            if (u + 1 >= ntg) break;
            idle(u + 1, std::integral_constant<int, (J + 3) % kRing>{}, No{});
            if (u + 2 >= ntg) break;
            idle(u + 2, std::integral_constant<int, J>{}, No{});
            if (u + 3 >= ntg) break;
            idle(u + 3, std::integral_constant<int, (J + 1) % kRing>{}, No{});
        }
        vmcnt_wait<0>();  // every DMA landed (none may outlive the block)
        ring_barrier();   // the other waves' last GEMM1 barrier
    };

    if (ntg > 0) {
        // prologue: Q, then K0 K1 V0 K2 V1 K3 in flight; GEMM0 of tile 0 once
        // Q and K0 landed
        {
            const int qoff = my_row * p.stride_q * 2 + hi * 16;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                i32x4 raw = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff + t * 32, 0, 0);
                qop[t] = __builtin_bit_cast(bf16x8, raw);
            }
        }
        issue_k(0, P0{});
        issue_k(1, P1{});
        issue_v(0, P0{});
        issue_k(2, P2{});
        issue_v(1, P1{});
        issue_k(3, P3{});
        vmcnt_wait<5 * kLoads>();  // the Q loads (issued first) and K0 have landed
        ring_barrier();
        // Retire the Q loads here, visibly to the compiler: its own wait then
        // falls where the one above already holds (Q and K0 arrive in one
        // memory latency, not two in a row), and it does not keep them
        // pending into the loop, where its wait would also cover the K/V
        // prefetch in flight.
        asm volatile("" ::"v"(qop[0]), "v"(qop[1]), "v"(qop[2]), "v"(qop[3]));
        gemm0(P0{}, sacc[0]);
        // m_ref starts at the first tile's exact (masked) row max, so the
        // speculative softmax holds from tile 0 on (rows with no visible key
        // there keep the finite seed: their P is exactly 0 until a visible
        // score overflows the bound and re-frames the row)
        mask_tile(0, sacc[0]);
        sm.m_ref = fmaxf(kMaxSeed, tile_max(sacc[0]) * scale);
        // iteration 0 has no GEMM1; iterations 1 .. ntg-1 run in groups of
        // kRing (phases 1 2 3 0) and the 0-3 left over, each with GEMM0 of
        // the next tile (for the last one a dead, zero-filled tile)
        iteration(0, P0{}, No{}, Yes{});
        int t = 1;
        for (; t + kRing <= nlive; t += kRing) {
            mid(t, P1{});
            mid(t + 1, P2{});
            mid(t + 2, P3{});
            mid(t + 3, P0{});
        }
        const int rem = nlive - t;  // 0-3 live tiles left; the last live tile's phase is rem
        if constexpr (kCausal) {
            // one shared tail after the live remainder (a copy of the
            // live/idle tail per remainder, nested as below, spills)
            if (rem >= 1) mid(t, P1{});
            if (rem >= 2) mid(t + 1, P2{});
            if (rem >= 3) mid(t + 2, P3{});
            switch (rem) {
                case 0: finish_live(P0{}); break;
                case 1: finish_live(P1{}); break;
                case 2: finish_live(P2{}); break;
                default: finish_live(P3{}); break;
            }
        } else if (rem == 0) {  // every tile live; nested (0.9 % faster than the shared tail)
            last_gemm1(P0{});
        } else {
            mid(t, P1{});
            if (rem == 1) {
                last_gemm1(P1{});
            } else {
                mid(t + 1, P2{});
                if (rem == 2) {
                    last_gemm1(P2{});
                } else {
                    mid(t + 2, P3{});
                    last_gemm1(P3{});
                }
            }
        }
    }

    if constexpr (kSplitKV) {
        // Hand-over: group 1 leaves its partial (O^T, m_ref, l_part) in LDS and
        // exits; group 0 folds it into its own.  The K stages are free: their
        // last reads (GEMM0 of the final iteration) completed before the
        // barrier in last_gemm1.  Wave w of either group owns the same 32 rows
        // and lane L the same (row, columns), so lane L meets lane L.
        typedef __attribute__((address_space(3))) float lds_float;
        // element e of lane L at x[64e + L], wave w in K stage w (a select
        // chain: a runtime-indexed table of LDS addresses cannot be emitted)
        lds_char* xs = wave == 0 ? ring.k[0] : wave == 1 ? ring.k[1] : wave == 2 ? ring.k[2] : ring.k[3];
        lds_float* x = (lds_float*)xs;
        static_assert(34 * 64 * 4 <= 2 * kTileBytes, "hand-over fits one K stage");
        if (group == 1) {
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) x[(16 * db + r) * 64 + lane] = oacc[db][r];
            x[32 * 64 + lane] = sm.m_ref;
            x[33 * 64 + lane] = sm.l_part;
        }
        __syncthreads();
        if (group == 1) return;
        const float m1 = x[32 * 64 + lane];
        const float m = fmaxf(sm.m_ref, m1);
        const float a0 = __builtin_amdgcn_exp2f(sm.m_ref - m);
        const float a1 = __builtin_amdgcn_exp2f(m1 - m);
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[db][r] = a0 * oacc[db][r] + a1 * x[(16 * db + r) * 64 + lane];
        sm.l_part = a0 * sm.l_part + a1 * x[33 * 64 + lane];
        sm.m_ref = m;
    }

    if constexpr (kBalanced) {
        // a split M-tile's half: its unnormalised O^T, reference max and partial
        // row sums, lane-major (element e of lane L of wave w at
        // part[(34w + e) * 64 + L]: every store writes 256 contiguous bytes);
        // the merge launch finishes the M-tile.  A pair's second group writes
        // the slot of M-tile 2mt+1 (two slots on: each M-tile holds its two
        // halves), unless that M-tile is past the sequence.
        if (ck.part != nullptr) {
            if (kPair && row0 >= sq) return;
            float* w = ck.part + group * (2 * kWaves * kPartFloatsPerWave) + wave * kPartFloatsPerWave;
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) w[(16 * db + r) * 64 + lane] = oacc[db][r];
            w[32 * 64 + lane] = sm.m_ref;
            w[33 * 64 + lane] = sm.l_part;
            return;
        }
    }

    // ---- epilogue: O = O^T / l (rows < sq; the buffer bound drops the rest),
    // LSE = (log2(l) + m_ref) * ln2 (natural log, -inf for an empty row) ----
    const float l_tot = wave_sum_halves(sm.l_part);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    {
        // O^T / l as bf16, transposed through 4 KiB of LDS private to the wave
        // so that every store writes whole 128-byte rows (8 lanes per row, 8
        // rows per instruction).  The K stages are idle here: their last reads
        // and DMA writes completed before the last ring barrier (and with no
        // tile at all none were issued).  Split-KV: the wave's own stage, whose
        // hand-over data it has already read.
        lds_char* const shared_stage =
            wave_id < 2 ? ring.k[0] : wave_id < 4 ? ring.k[1] : wave_id < 6 ? ring.k[2] : ring.k[3];
        lds_char* const own_stage = wave == 0 ? ring.k[0] : wave == 1 ? ring.k[1] : wave == 2 ? ring.k[2] : ring.k[3];
        lds_char* const tb = kSplitKV ? own_stage : shared_stage + (wave_id & 1) * kRowsPerWave * kRowBytes;
        static_assert(2 * kRowsPerWave * kRowBytes <= kTileBytes, "two waves' O tiles per K stage");
        // Lane (q, h) holds columns 8c + 4h .. +3 of row q, half h of 16-byte
        // chunk c = 4db + g4.  In the buffer, chunk c of row q sits at chunk
        // c ^ ((q >> 1) & 7), and odd rows swap the two 8-byte halves.  LDS
        // takes a 64-lane 8-byte write 16 lanes (128 bytes) at a time: each
        // such group (rows of both parities, so both halves) writes 128
        // distinct bank positions.  The reads take whole rows, 16 bytes a lane
        // (2 rows = 256 bytes per group), conflict free in any order; odd rows
        // swap their halves back in registers.
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                bf16x2 a, b;
                a[0] = (__bf16)(oacc[db][4 * g4 + 0] * inv);
                a[1] = (__bf16)(oacc[db][4 * g4 + 1] * inv);
                b[0] = (__bf16)(oacc[db][4 * g4 + 2] * inv);
                b[1] = (__bf16)(oacc[db][4 * g4 + 3] * inv);
                i32x2 w;
                w[0] = __builtin_bit_cast(int, a);
                w[1] = __builtin_bit_cast(int, b);
                const int c = 4 * db + g4;
                *(lds_i32x2*)(tb + l32 * kRowBytes + ((c ^ ((l32 >> 1) & 7)) << 4) + 8 * (hi ^ (l32 & 1))) = w;
            }
        // other lanes' writes must land before the reads (LDS is in order per
        // wave; the wait also keeps the compiler from reordering)
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int i = 0; i < kRowsPerWave / 8; ++i) {
            const int r = 8 * i + (lane >> 3), pc = lane & 7;  // physical chunk pc holds chunk pc ^ ((r >> 1) & 7)
            const i32x4 raw = *(const lds_i32x4*)(tb + r * kRowBytes + (pc << 4));
            const i32x4 v = (r & 1) ? i32x4{raw[2], raw[3], raw[0], raw[1]} : raw;  // odd rows: halves back in order
            const int c = pc ^ ((r >> 1) & 7);
            __builtin_amdgcn_raw_buffer_store_b128(v, ro, (wrow0 + r) * p.stride_o * 2 + c * 16, 0, kStoreStream);
        }
    }
    if (p.lse != nullptr && hi == 0 && my_row < sq) {
        float* lse_base;
        if constexpr (kVarlen)
            lse_base = p.lse + (int64_t)h * (p.nhead_stride_q / p.stride_q) + off_q;
        else
            lse_base = p.lse + (int64_t)b * p.nhead_q * p.seqlen_q + (int64_t)h * p.seqlen_q;
        const float lse2 = __builtin_log2f(l_tot) + sm.m_ref;  // -inf when l == 0
        lse_base[my_row] = lse2 * 0.69314718055994530942f;
    }
}

// ===========================================================================
// Pair stream form (this build's own; no counterpart in the reference).
//
// The pair form's 8-wave block is alone on its compute unit, so nothing
// hides its prologue (the first Q and K/V tiles from memory, GEMM0 of the
// first tile) or its epilogue (O through LDS to memory): a launch of two
// rounds of pair blocks pays both twice per CU.  Here one pair block per CU
// loops over a static list of M-tile pairs and its K/V ring runs on from one
// pair into the next: the next pair's first K/V tiles are fetched during the
// current pair's last four iterations and its Q rows arrive by LDS-DMA (in
// the current pair's second iteration) into a 4 KiB buffer per wave, read
// into the GEMM0 operand for the last iteration (whose GEMM0 is the next
// pair's first tile); the current pair's
// last GEMM1 and its epilogue run in the next pair's first iteration, the O
// tile staged through the same buffer.
//
// Items are the pair grid's blocks (head fastest, then pair, then batch).
// Dense: block i takes items i, i + G, i + 2G, ... below n_items (G =
// gridDim.x; every item has the same key tiles).  Causal: block i takes
// pair Y-1-y of its (batch, head) and then its mirror y (Y pairs per
// (batch, head); the middle pair of an odd Y alone), so the blocks' key
// tiles balance and each block's two pairs read the same K/V.  With G a
// multiple of 8 and of nhead_q a head's items all run on the XCD of its
// blocks, as in the pair grid.  Every item runs a multiple of 4 ring
// iterations (the ring stages stay compile-time), at least 8 (the
// successor's fetches in the last four never meet the predecessor's GEMM1
// in the first); the padding iterations see zero-filled, fully masked tiles.
// ===========================================================================
typedef __attribute__((address_space(4))) const FmhaStreamArgs* SArgsPtr;

// The kernarg block through a pointer the compiler cannot follow across
// calls of this function: loads through the result are issued where they
// are used instead of being held in SGPRs across the inner loop.
__device__ __forceinline__ SArgsPtr sargs_here() {
    SArgsPtr ap = (SArgsPtr)__builtin_amdgcn_kernarg_segment_ptr();
    asm volatile("" : "+s"(ap));
    return ap;
}

// Items this block runs (wave-uniform).
template <bool kCausal>
__device__ __forceinline__ int stream_items(SArgsPtr ap) {
    if constexpr (kCausal) {
        const int ny = ap->ny, half = (ny + 1) >> 1;
        const int y = (int)(blockIdx.x / ap->p.nhead_q) % half;
        return 2 * y + 1 == ny ? 1 : 2;
    } else {
        return (ap->n_items - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
    }
}

// Item k of this block: batch b, head h, pair pr (wave-uniform).
template <bool kCausal>
__device__ __forceinline__ void stream_coords(SArgsPtr ap, int k, int& b, int& h, int& pr) {
    const int nh = ap->p.nhead_q, ny = ap->ny;
    if constexpr (kCausal) {
        const int half = (ny + 1) >> 1;
        const int i = blockIdx.x;
        h = i % nh;
        const int r = i / nh;
        const int y = r % half;
        b = r / half;
        pr = k == 0 ? ny - 1 - y : y;  // the heavy pair, then its mirror
    } else {
        const int L = blockIdx.x + k * gridDim.x;
        h = L % nh;
        const int r = L / nh;
        pr = r % ny;
        b = r / ny;
    }
}

// What the K/V ring needs of an item (wave-uniform): the first K and V row
// of its (batch, KV head), the pair's first query row, its key tiles (those
// of its last row) and its ring iterations.  A dead item has no tiles (its
// loads are zero fills).
struct StreamKV {
    const char* k;
    const char* v;
    int row0;
    int ntiles;
    int npad;
};
template <bool kCausal>
__device__ __forceinline__ StreamKV stream_kv(SArgsPtr ap, int k, bool valid) {
    int b, h, pr;
    stream_coords<kCausal>(ap, valid ? k : 0, b, h, pr);
    const int sq = ap->p.seqlen_q, sk = ap->p.seqlen_k;
    int kv_end = sk;
    if constexpr (kCausal) {  // pipeline.hpp:168-193, over the pair's last row
        const int last = min(2 * pr * kTileM + 2 * kTileM - 1, sq - 1);
        const int e = last + (sk - sq) + 1;
        kv_end = e < 0 ? 0 : (e > sk ? sk : e);
    }
    StreamKV it;
    it.row0 = 2 * pr * kTileM;
    it.ntiles = valid ? (kv_end + kTileN - 1) / kTileN : 0;
    it.npad = max(2 * kRing, (it.ntiles + kRing - 1) & ~(kRing - 1));
    const int kvh = h / (ap->p.nhead_q / ap->p.nhead_k);
    it.k = (const char*)(ap->p.k + (int64_t)b * ap->p.batch_stride_k + (int64_t)kvh * ap->p.nhead_stride_k);
    it.v = (const char*)(ap->p.v + (int64_t)b * ap->p.batch_stride_v + (int64_t)kvh * ap->p.nhead_stride_v);
    return it;
}

template <bool kCausal>
__device__ __forceinline__ void fwd_pair_stream(const Ring& ring, lds_char* qbuf) {
    const int lane = threadIdx.x & 63;
    const int wave_id = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // 0-7
    const int group = wave_id / kWaves;                                    // the pair's M-tile
    const int wave = wave_id % kWaves;                                     // 32 rows of it
    const int l32 = lane & 31;
    const int hi = lane >> 5;

    // per-lane constants (VGPRs), as the pair form: each wave moves 1 KiB
    // (rows 8 * wave_id .. +7) of every K and V tile
    int k_ld_off, v_ld_off;
    // Q DMA: load i brings rows 8i + lane/8 of this wave's 32, physical chunk
    // lane%8 holding logical chunk (lane%8) ^ k_swz(8i + lane/8) =
    // (lane%8) ^ (lane/8) ^ (i&1); the offsets of even and odd i
    int q_ld_off[2];
    {
        SArgsPtr ap = sargs_here();
        const int ld_row = wave_id * 8 + (lane >> 3);
        const int ld_pc = lane & 7;
        k_ld_off = ld_row * ap->p.stride_k * 2 + ((ld_pc ^ k_swz(ld_row)) << 4);
        v_ld_off = ld_row * ap->p.stride_v * 2 + ((ld_pc ^ v_swz(ld_row)) << 4);
        const int q_row = wave * kRowsPerWave + (lane >> 3);
        const int sw = (lane & 7) ^ (lane >> 3);
        q_ld_off[0] = q_row * ap->p.stride_q * 2 + (sw << 4);
        q_ld_off[1] = q_row * ap->p.stride_q * 2 + ((sw ^ 1) << 4);
    }
    const int wave_off = wave_id * 1024;
    // this wave's 32 Q rows of the next item, swizzled as K rows (the GEMM0 B
    // operand is read with the K read pattern); also the O staging of the
    // epilogue
    lds_char* const qw = qbuf + wave_id * (kRowsPerWave * kRowBytes);

    uint32_t k_rd[4];
    {
        const int f = k_swz(l32);
#pragma unroll
        for (int t = 0; t < 4; ++t) k_rd[t] = l32 * kRowBytes + (((2 * t + hi) ^ f) << 4);
    }
    uint32_t v_rd[2];
    {
        const int g = lane >> 4, i16 = lane & 15;
        const int e = i16 >> 2, c = i16 & 3;
        const int row = 4 * hi + e;
#pragma unroll
        for (int db = 0; db < 2; ++db) {
            const int chunk = 4 * db + 2 * (g & 1) + (c >> 1);
            v_rd[db] = row * kRowBytes + ((chunk ^ v_swz(row)) << 4) + (c & 1) * 8;
        }
    }

    bf16x8 qop[4];
    f32x16 oacc[2];
    f32x16 sacc[2][2];
    bf16x8 pbuf[2][4];
    Softmax sm{kMaxSeed, 0.0f, 0.0f};
    Softmax smz{kMaxSeed, 0.0f, 0.0f};  // the previous item's, until its epilogue
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[db][r] = 0.0f;

    // the item in progress (number KX of this block, ring view X), its
    // successor (KX + 1) and its predecessor (KX - 1, whose last GEMM1 and
    // epilogue run in X's iteration 0)
    int KX = 0;
    const int n_mine = stream_items<kCausal>(sargs_here());
    StreamKV X;
    int sk, shift;
    uint32_t kbytes, vbytes;
    int k_tile_step, v_tile_step;
    float scale, scale_v;
    auto load_item = [&]() {  // X's view and the per-launch constants, reloaded per item
        SArgsPtr ap = sargs_here();
        X = stream_kv<kCausal>(ap, KX, true);
        sk = ap->p.seqlen_k;
        shift = sk - ap->p.seqlen_q;
        kbytes = sk > 0 ? (uint32_t)((int64_t)(sk - 1) * ap->p.stride_k * 2 + kRowBytes) : 0u;
        vbytes = sk > 0 ? (uint32_t)((int64_t)(sk - 1) * ap->p.stride_v * 2 + kRowBytes) : 0u;
        k_tile_step = kTileN * ap->p.stride_k * 2;
        v_tile_step = kTileN * ap->p.stride_v * 2;
        scale = ap->p.scale;
        scale_v = in_vgpr(scale);
    };

    // DMA of tile `tile` (K or V) of the item `view` into stage S
    auto issue_k = [&](const StreamKV& view, int tile, auto stage_c) {
        lds_char* dst = ring.k[decltype(stage_c)::value] + wave_off;
        const uint32_t t0 = (uint32_t)tile * (uint32_t)k_tile_step;
        lds_dma_16(make_rsrc(view.k + t0, tile < view.ntiles ? kbytes - t0 : 0u), dst, k_ld_off);
    };
    auto issue_v = [&](const StreamKV& view, int tile, auto stage_c) {
        lds_char* dst = ring.v[decltype(stage_c)::value] + wave_off;
        const uint32_t t0 = (uint32_t)tile * (uint32_t)v_tile_step;
        lds_dma_16(make_rsrc(view.v + t0, tile < view.ntiles ? vbytes - t0 : 0u), dst, v_ld_off);
    };
    // this wave's 32 Q rows of item k into its Q buffer (q_ld_off); past the
    // block's last item, zeros (an empty descriptor).  Issued on every path:
    // a branch around it would leave the compiler's wait placement with two
    // load counts to merge, and it then waits for the prefetch in flight.
    auto issue_q = [&](int k) {
        SArgsPtr ap = sargs_here();
        const bool valid = k < n_mine;
        int b, h, pr;
        stream_coords<kCausal>(ap, valid ? k : 0, b, h, pr);
        const int sq = ap->p.seqlen_q, sq_stride = ap->p.stride_q;
        const uint32_t qbytes = sq > 0 ? (uint32_t)((int64_t)(sq - 1) * sq_stride * 2 + kRowBytes) : 0u;
        const char* q = (const char*)(ap->p.q + (int64_t)b * ap->p.batch_stride_q + (int64_t)h * ap->p.nhead_stride_q);
        const uint32_t r0 = (uint32_t)(2 * pr * kTileM + group * kTileM) * (uint32_t)(sq_stride * 2);
        // wave-uniform (a saturating subtract would otherwise land in a VGPR
        // and the DMA in a loop over its lanes' values)
        const uint32_t nrec = __builtin_amdgcn_readfirstlane(valid && qbytes > r0 ? qbytes - r0 : 0u);
        const auto r = make_rsrc(q + r0, nrec);
        // the per-lane offsets are loop-invariant registers (q_ld_off), the
        // load's 8-row step a scalar: the compiler keeps a DMA's offset
        // register reserved until the DMA completes, and would wait for it
        // before reusing a temporary
#pragma unroll
        for (int i = 0; i < 4; ++i) lds_dma_16(r, qw + i * 1024, q_ld_off[i & 1], i * 8 * sq_stride * 2);
    };
    auto gemm0 = [&](auto ks_c, f32x16* s) {
        const lds_char* st = ring.k[decltype(ks_c)::value];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            f32x16 acc = {};
#pragma unroll
            for (int k = 0; k < 4; ++k) acc = mfma(lds_read_b128(st + k_rd[k] + kb * 32 * kRowBytes), qop[k], acc);
            s[kb] = acc;
        }
    };
    auto gemm1 = [&](auto vs_c, const bf16x8* pp) {
        const lds_char* st = ring.v[decltype(vs_c)::value];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int k = 0; k < 2; ++k)
#pragma unroll
                for (int db = 0; db < 2; ++db)
                    oacc[db] = mfma(lds_read_vt(st + v_rd[db] + (kb * 32 + 16 * k) * kRowBytes), pp[2 * kb + k],
                                    oacc[db]);
    };
    // X's tile t: keys >= sk, and (causal) keys > row + shift
    auto mask_tile = [&](int t, f32x16* s) {
        const int key0 = t * kTileN;
        const int wrow0 = X.row0 + group * kTileM + wave * kRowsPerWave;
        const bool need = (key0 + kTileN > sk) || (kCausal && key0 + kTileN - 1 > wrow0 + shift);
        if (need) {
            const int lim = kCausal ? min(sk - 1, wrow0 + l32 + shift) : sk - 1;
            const int d = lim - (key0 + 4 * hi);
            const float ninf = in_vgpr(-__builtin_inff());
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int c = 32 * kb + 8 * (r >> 2) + (r & 3);
                    s[kb][r] = c <= d ? s[kb][r] : ninf;
                }
        }
    };
    auto tile_max = [&](const f32x16* s) {
        float mp[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) mp[i] = fmaxf(fmaxf(s[i >> 2][4 * (i & 3)], s[i >> 2][4 * (i & 3) + 1]),
                                                  fmaxf(s[i >> 2][4 * (i & 3) + 2], s[i >> 2][4 * (i & 3) + 3]));
        const float mx = fmaxf(fmaxf(fmaxf(mp[0], mp[1]), fmaxf(mp[2], mp[3])),
                               fmaxf(fmaxf(mp[4], mp[5]), fmaxf(mp[6], mp[7])));
        return wave_max_halves(mx);
    };
    auto exp_tile = [&](const f32x16* s, bf16x8* pp) {
        const float neg_ms = -sm.m_ref;
        float ls[4];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                bf16x8 pk;
                float acc;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][8 * k + e], scale_v, neg_ms));
                    acc = e == 0 ? pv : acc + pv;
                    pk[e] = (__bf16)pv;
                }
                ls[2 * kb + k] = acc;
                pp[2 * kb + k] = pk;
            }
        sm.l_tile = (ls[0] + ls[1]) + (ls[2] + ls[3]);
    };
    auto softmax = [&](const f32x16* s, bf16x8* pp) {
        exp_tile(s, pp);
        asm volatile("" ::"v"(pp[0]), "v"(pp[1]), "v"(pp[2]), "v"(pp[3]), "v"(sm.l_tile));
    };
    auto settle = [&](const f32x16* s, bf16x8* pp) {
        if (__builtin_amdgcn_ballot_w64(!(sm.l_tile <= kGrowSum))) {
            asm volatile("" ::: "memory");
            const float m_new = fmaxf(sm.m_ref, tile_max(s) * scale);
            const float alpha = __builtin_amdgcn_exp2f(sm.m_ref - m_new);
            sm.m_ref = m_new;
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
            sm.l_part *= alpha;
            exp_tile(s, pp);
        }
        sm.l_part += sm.l_tile;
    };
    // O = O^T / l and LSE of item k (softmax state `st`), staged through this
    // wave's Q buffer as the regular form's epilogue stages through a K stage
    auto epilogue = [&](int k, const Softmax& st) {
        SArgsPtr ap = sargs_here();
        int b, h, pr;
        stream_coords<kCausal>(ap, k, b, h, pr);
        const int sq = ap->p.seqlen_q, so = ap->p.stride_o;
        const float l_tot = wave_sum_halves(st.l_part);
        const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        const uint32_t obytes = (uint32_t)((int64_t)(sq - 1) * so * 2 + kRowBytes);
        const auto ro = make_rsrc(ap->p.o + (int64_t)b * ap->p.batch_stride_o + (int64_t)h * ap->p.nhead_stride_o,
                                  obytes);
        const int wrow0 = 2 * pr * kTileM + group * kTileM + wave * kRowsPerWave;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                bf16x2 x0, x1;
                x0[0] = (__bf16)(oacc[db][4 * g4 + 0] * inv);
                x0[1] = (__bf16)(oacc[db][4 * g4 + 1] * inv);
                x1[0] = (__bf16)(oacc[db][4 * g4 + 2] * inv);
                x1[1] = (__bf16)(oacc[db][4 * g4 + 3] * inv);
                i32x2 w;
                w[0] = __builtin_bit_cast(int, x0);
                w[1] = __builtin_bit_cast(int, x1);
                const int c = 4 * db + g4;
                *(lds_i32x2*)(qw + l32 * kRowBytes + ((c ^ ((l32 >> 1) & 7)) << 4) + 8 * (hi ^ (l32 & 1))) = w;
            }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int i = 0; i < kRowsPerWave / 8; ++i) {
            const int r = 8 * i + (lane >> 3), pc = lane & 7;
            const i32x4 raw = *(const lds_i32x4*)(qw + r * kRowBytes + (pc << 4));
            const i32x4 v = (r & 1) ? i32x4{raw[2], raw[3], raw[0], raw[1]} : raw;
            const int c = pc ^ ((r >> 1) & 7);
            __builtin_amdgcn_raw_buffer_store_b128(v, ro, (wrow0 + r) * so * 2 + c * 16, 0, kStoreStream);
        }
        const int my_row = wrow0 + l32;
        float* const lse = ap->p.lse;
        if (lse != nullptr && hi == 0 && my_row < sq) {
            const float lse2 = __builtin_log2f(l_tot) + st.m_ref;  // -inf when l == 0
            lse[(int64_t)b * ap->p.nhead_q * sq + (int64_t)h * sq + my_row] = lse2 * 0.69314718055994530942f;
        }
        // the staging reads must be done before this buffer takes Q rows again
        // (the successor's Q DMA in the next iteration)
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    };

    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    using P2 = std::integral_constant<int, 2>;
    using P3 = std::integral_constant<int, 3>;

    // one ring iteration t of X (phase J = t % 4): GEMM1(t-1) || GEMM0(t+1)
    // || softmax(t); its K(t+4) and V(t+2) DMAs come from `kv`/`vv` (X's view,
    // or the successor's in the last four iterations, with the tile counted
    // from it).  The wait lets the two previous iterations' loads fly (W = 4)
    // and, in iterations 2 and 3, the successor's Q DMA issued in iteration 1
    // too (W = 8); `q_next`: iteration 1, which issues that DMA first.
    auto iteration = [&](int t, auto phase_c, const StreamKV& kv, int kt, const StreamKV& vv, int vt,
                         auto wait_c, auto q_next) {
        constexpr int J = decltype(phase_c)::value;
        constexpr int cur = J & 1, nxt = cur ^ 1;
        vmcnt_wait<decltype(wait_c)::value>();  // K(t+1) and V(t-1) landed
        ring_barrier();
        if constexpr (decltype(q_next)::value) issue_q(KX + 1);
        issue_k(kv, kt, std::integral_constant<int, J>{});
        issue_v(vv, vt, std::integral_constant<int, (J + 2) % kRing>{});
        mask_tile(t, sacc[cur]);
        gemm1(std::integral_constant<int, (J + kRing - 1) % kRing>{}, pbuf[nxt]);
        gemm0(std::integral_constant<int, (J + 1) % kRing>{}, sacc[nxt]);
        softmax(sacc[cur], pbuf[cur]);
        IterSchedule<true, true>::apply();
        settle(sacc[cur], pbuf[cur]);
    };
    using W4 = std::integral_constant<int, 4>;
    using W8 = std::integral_constant<int, 8>;
    using NoQ = std::false_type;
    auto mid = [&](int t, auto phase_c) { iteration(t, phase_c, X, t + kRing, X, t + 2, W4{}, NoQ{}); };

    // iteration 0 of X: X's frame from its first tile's exact max; GEMM1 of
    // the predecessor's last tile (kPrev), whose epilogue follows
    auto first = [&](auto prev_c) {
        constexpr bool kPrev = decltype(prev_c)::value;
        vmcnt_wait<4>();
        ring_barrier();
        issue_k(X, kRing, P0{});
        issue_v(X, 2, P2{});
        mask_tile(0, sacc[0]);
        sm.m_ref = fmaxf(kMaxSeed, tile_max(sacc[0]) * scale);
        if constexpr (kPrev) gemm1(P3{}, pbuf[1]);
        gemm0(P1{}, sacc[1]);
        softmax(sacc[0], pbuf[0]);
        IterSchedule<kPrev, true>::apply();
        sm.l_part = sm.l_tile;  // exact frame: nothing to re-frame
        if constexpr (kPrev) {
            epilogue(KX - 1, smz);
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[db][r] = 0.0f;
        }
    };
    // X's last four iterations: K(t+4) is the successor's tile t+4-npad, V(t+2)
    // too from npad-2 on; the successor's Q rows, in the Q buffer since
    // iteration 1, go into qop before the last iteration's GEMM0 (its first
    // tile); past the block's last item the successor is dead (zero tiles,
    // no Q)
    auto tail = [&]() {
        const int t = X.npad - kRing;
        const bool has_next = KX + 1 < n_mine;
        const StreamKV N = stream_kv<kCausal>(sargs_here(), KX + 1, has_next);
        // the kernarg reads above retired where the compiler's wait placement
        // sees it (see `settled`)
        __builtin_amdgcn_s_waitcnt(kWaitLgkmcnt0);
        iteration(t, P0{}, N, 0, X, t + 2, W4{}, NoQ{});
        iteration(t + 1, P1{}, N, 1, X, t + 3, W4{}, NoQ{});
        iteration(t + 2, P2{}, N, 2, N, 0, W4{}, NoQ{});
        {
            vmcnt_wait<4>();
            ring_barrier();
            issue_k(N, 3, P3{});
            issue_v(N, 1, P1{});
            // the successor's Q (zeros past the block's last item, whose
            // GEMM0 result below is then unused)
#pragma unroll
            for (int k = 0; k < 4; ++k) qop[k] = lds_read_b128(qw + k_rd[k]);
            mask_tile(t + 3, sacc[1]);
            gemm1(P2{}, pbuf[0]);
            gemm0(P0{}, sacc[0]);
            softmax(sacc[1], pbuf[1]);
            IterSchedule<true, true>::apply();
            settle(sacc[1], pbuf[1]);
        }
        return has_next;
    };

    load_item();
    // prologue of the block's first item: Q straight into registers, K0 K1
    // V0 K2 V1 K3 in flight, GEMM0 of tile 0 once Q and K0 landed
    {
        SArgsPtr ap = sargs_here();
        int b, h, pr;
        stream_coords<kCausal>(ap, 0, b, h, pr);
        const int sq = ap->p.seqlen_q;
        const uint32_t qbytes = sq > 0 ? (uint32_t)((int64_t)(sq - 1) * ap->p.stride_q * 2 + kRowBytes) : 0u;
        const auto rq = make_rsrc(ap->p.q + (int64_t)b * ap->p.batch_stride_q + (int64_t)h * ap->p.nhead_stride_q,
                                  qbytes);
        const int qoff = (X.row0 + group * kTileM + wave * kRowsPerWave + l32) * ap->p.stride_q * 2 + hi * 16;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            i32x4 raw = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff + t * 32, 0, 0);
            qop[t] = __builtin_bit_cast(bf16x8, raw);
        }
    }
    issue_k(X, 0, P0{});
    issue_k(X, 1, P1{});
    issue_v(X, 0, P0{});
    issue_k(X, 2, P2{});
    issue_v(X, 1, P1{});
    issue_k(X, 3, P3{});
    vmcnt_wait<5>();  // the Q loads (issued first) and K0 have landed
    ring_barrier();
    asm volatile("" ::"v"(qop[0]), "v"(qop[1]), "v"(qop[2]), "v"(qop[3]));
    gemm0(P0{}, sacc[0]);
    // Scalar loads (the kernarg reads of an item) and LDS reads share lgkmcnt,
    // and scalar loads return out of order: while one may be in flight the
    // compiler can only wait for an LDS operand with lgkmcnt(0), which also
    // waits for the reads issued ahead for the next MFMAs.  The ring
    // barrier's own lgkmcnt(0) is inline asm, which the compiler does not
    // see, so every item's kernarg reads are retired with the builtin before
    // the iterations: otherwise the loop header, reached with them possibly
    // in flight, puts lgkmcnt(0) before every operand of every fourth
    // iteration (2-3 % per tile).
    auto settled = [&]() { __builtin_amdgcn_s_waitcnt(kWaitLgkmcnt0); };
    bool prev = false;
    while (true) {
        settled();
        if (prev)
            first(std::true_type{});
        else
            first(std::false_type{});
        // iteration 1 issues the successor's Q DMA before its K/V loads (on
        // every path: see issue_q); the waits of iterations 2 and 3 let those
        // four loads fly too (iteration 4's wait retires them)
        iteration(1, P1{}, X, 1 + kRing, X, 1 + 2, W4{}, std::true_type{});
        iteration(2, P2{}, X, 2 + kRing, X, 2 + 2, W8{}, NoQ{});
        iteration(3, P3{}, X, 3 + kRing, X, 3 + 2, W8{}, NoQ{});
        settled();
        // iterations 4 .. npad-5 (none when npad = 8): the unrolled loop
        // starts at phase 1 like the other forms' loops, whose compiled code
        // keeps two LDS operand reads in flight in every phase (starting at
        // phase 0 the compiler stages that phase's V operands through one
        // register set and waits for each read)
        if (X.npad > 2 * kRing) {
            mid(kRing, P0{});
            for (int t = kRing + 1; t + kRing <= X.npad - 2 * kRing + 1; t += kRing) {  // t .. t+3 <= npad-8
                mid(t, P1{});
                mid(t + 1, P2{});
                mid(t + 2, P3{});
                mid(t + 3, P0{});
            }
            mid(X.npad - 2 * kRing + 1, P1{});
            mid(X.npad - 2 * kRing + 2, P2{});
            mid(X.npad - 2 * kRing + 3, P3{});
        }
        if (!tail()) break;
        smz = sm;
        ++KX;
        load_item();
        prev = true;
    }
    // drain: the last item's last GEMM1 and its epilogue
    vmcnt_wait<0>();
    ring_barrier();
    gemm1(P3{}, pbuf[1]);
    epilogue(KX, sm);
}

// ===========================================================================
// Short form (this build's own; no counterpart in the reference): the
// regular grid at four blocks per compute unit (<= 128 VGPRs and 32 KiB of
// LDS; the regular form fits two), for launches whose M-tiles see few key
// tiles.  Such blocks are bound by memory latency more than by the MFMA
// rate, so one block's loads overlap the other three's work.  K and V tiles
// stream through two-stage rings (each stage its own __shared__ array, as the
// regular form's rings), prefetched one tile ahead; each 64-key tile is taken
// as two 32-key halves (GEMM0, an online softmax with the exact running row
// max, that half's GEMM1), so a wave holds 16 scores at a time.  Any number
// of key tiles works; the launcher picks the form up to 192 keys (causal 384).
// ===========================================================================
struct ShortLds {
    lds_char* k[2];
    lds_char* v[2];
};

template <bool kCausal, bool kVarlen>
__device__ __forceinline__ void fwd_short(const FmhaFwdParams& p, int b, int h, int mt, const ShortLds& lds) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l32 = lane & 31;
    const int hi = lane >> 5;

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
    const __bf16 *qbase, *kbase, *vbase;
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
    const uint32_t qbytes = (uint32_t)((int64_t)(sq - 1) * p.stride_q * 2 + kRowBytes);
    const uint32_t kbytes = sk > 0 ? (uint32_t)((int64_t)(sk - 1) * p.stride_k * 2 + kRowBytes) : 0u;
    const uint32_t vbytes = sk > 0 ? (uint32_t)((int64_t)(sk - 1) * p.stride_v * 2 + kRowBytes) : 0u;
    const uint32_t obytes = (uint32_t)((int64_t)(sq - 1) * p.stride_o * 2 + kRowBytes);
    const int shift = sk - sq;
    int kv_end = sk;
    if constexpr (kCausal) {
        const int last = min(row0 + kTileM - 1, sq - 1);
        const int e = last + shift + 1;
        kv_end = e < 0 ? 0 : (e > sk ? sk : e);
    }
    const int ntiles = (kv_end + kTileN - 1) / kTileN;
    const int wrow0 = row0 + wave * kRowsPerWave;
    const int my_row = wrow0 + l32;
    const int ld_row = 2 * wave * 8 + (lane >> 3);
    const int ld_pc = lane & 7;
    const int fk = k_swz(l32);
    const int lim = kCausal ? min(sk - 1, my_row + shift) : sk - 1;
    // causal: the last key this wave's rows can see (uniform); a 32-key half
    // past it holds only masked scores for the wave and is skipped (P = 0)
    const int wave_last = kCausal ? min(sk - 1, wrow0 + kRowsPerWave - 1 + shift) : sk - 1;
    const float ninf = in_vgpr(-__builtin_inff());
    const float scale = p.scale;
    const float scale_v = in_vgpr(scale);
    const int g = lane >> 4, i16 = lane & 15, e4 = i16 >> 2, c4 = i16 & 3;
    float m_ref = kMaxSeed, l_part = 0.0f;  // the running max starts below every score
    f32x16 oacc[2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[db][r] = 0.0f;
    bf16x8 qop[4];
    auto load_q = [&]() {
        const auto rq = make_rsrc(qbase, qbytes);
        const int qoff = my_row * p.stride_q * 2 + hi * 16;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            i32x4 raw = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff + t * 32, 0, 0);
            qop[t] = __builtin_bit_cast(bf16x8, raw);
        }
    };
    // K (V) tile t into the LDS stage at `st`: the ring's layout and
    // swizzles, each wave 2 x 1 KiB of the tile; rows past the keys (and
    // tiles past ntiles) read as zero
    auto issue_k = [&](int t, lds_char* st) {
        const uint32_t tk = (uint32_t)t * kTileN * p.stride_k * 2;
        const auto rk = make_rsrc((const char*)kbase + tk, t < ntiles ? kbytes - tk : 0u);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row = ld_row + 8 * i;
            lds_dma_16(rk, st + (2 * wave + i) * 1024, row * p.stride_k * 2 + ((ld_pc ^ k_swz(row)) << 4));
        }
    };
    auto issue_v = [&](int t, lds_char* st) {
        const uint32_t tv = (uint32_t)t * kTileN * p.stride_v * 2;
        const auto rv = make_rsrc((const char*)vbase + tv, t < ntiles ? vbytes - tv : 0u);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row = ld_row + 8 * i;
            lds_dma_16(rv, st + (2 * wave + i) * 1024, row * p.stride_v * 2 + ((ld_pc ^ v_swz(row)) << 4));
        }
    };
    // per-lane LDS read offsets inside a tile (the regular form's): K rows
    // kb*32 + l32, logical chunk 2k + hi; V^T through ds_read_b64_tr_b16
    uint32_t k_rd[4], v_rd[2];
#pragma unroll
    for (int k = 0; k < 4; ++k) k_rd[k] = l32 * kRowBytes + (((2 * k + hi) ^ fk) << 4);
#pragma unroll
    for (int db = 0; db < 2; ++db) {
        const int row = 4 * hi + e4;
        const int chunk = 4 * db + 2 * (g & 1) + (c4 >> 1);
        v_rd[db] = row * kRowBytes + ((chunk ^ v_swz(row)) << 4) + (c4 & 1) * 8;
    }
    // GEMM0 of 32 keys (kb: which half of the LDS tile kt) into s
    auto gemm0_half = [&](const lds_char* kt, int kb, f32x16& s) {
#pragma unroll
        for (int k = 0; k < 4; ++k) s = mfma(lds_read_b128(kt + k_rd[k] + kb * 32 * kRowBytes), qop[k], s);
    };
    // GEMM1 of 32 keys (kb: which half of the LDS tile vt) with their P^T
    auto gemm1_half = [&](const lds_char* vt, int kb, const bf16x8* pp) {
#pragma unroll
        for (int k = 0; k < 2; ++k)
#pragma unroll
            for (int db = 0; db < 2; ++db)
                oacc[db] = mfma(lds_read_vt(vt + v_rd[db] + (kb * 32 + 16 * k) * kRowBytes), pp[k], oacc[db]);
    };

    // prologue: K(0), Q, V(0).  Iteration t (stage J = t % 2) waits for
    // K(t), V(t) (and Q), then prefetches tile t+1 into the other stage,
    // which tile t-1 used (every wave is past it after the barrier), and
    // computes tile t while those loads fly.
    issue_k(0, lds.k[0]);
    load_q();
    issue_v(0, lds.v[0]);
    // scores of one 32-key half: GEMM0, then the mask (keys >= sk, causal
    // keys > row + shift) where the half reaches past it
    auto scores = [&](const lds_char* kt, int t, int kb, f32x16& s) {
        s = f32x16{};
        gemm0_half(kt, kb, s);
        const int d = lim - (t * kTileN + 32 * kb + 4 * hi);
        if (__builtin_amdgcn_ballot_w64(d < 31)) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int c = 8 * (r >> 2) + (r & 3);
                s[r] = c <= d ? s[r] : ninf;
            }
        }
    };
    // exact max of the half's rows, scaled (-inf for a row with no key)
    auto half_max = [&](const f32x16& s) {
        float mx = ninf;
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[r]);
        return wave_max_halves(mx) * scale;
    };
    // P = exp2(s*scale - m_ref), bf16-packed, and this lane's sum of P
    // (fp32, before the rounding)
    auto exp_half = [&](const f32x16& s, bf16x8* pp) {
        const float neg_ms = -m_ref;
        float ls[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            bf16x8 pk;
            float acc;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(s[8 * k + e], scale_v, neg_ms));
                acc = e == 0 ? pv : acc + pv;
                pk[e] = (__bf16)pv;
            }
            ls[k] = acc;
            pp[k] = pk;
        }
        return ls[0] + ls[1];
    };
    // online softmax with the exact running row max of each half; O^T and
    // l move to a new max only where it grew (always at a row's first
    // visible keys, rarely after).  The regular form's speculative frame
    // would save the max but needs the scores and P live together on its
    // re-framing path, past 128 VGPRs.
    auto iteration = [&](int t, auto stage_c) {
        constexpr int J = decltype(stage_c)::value;
        // vmcnt(0) through the builtin, which the compiler's own wait
        // placement sees (it cannot see into inline asm): it then knows that
        // Q and tile t have landed and adds no wait of its own before tile t's
        // reads, where one would also cover the prefetch below on the path
        // that issues it
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
        ring_barrier();
        if (t + 1 < ntiles) {  // no empty prefetch after the last tile (+3.5 % at 32-64 keys)
            issue_k(t + 1, lds.k[J ^ 1]);
            issue_v(t + 1, lds.v[J ^ 1]);
        }
        lds_char* const kt = lds.k[J];
        lds_char* const vt = lds.v[J];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            // causal: this half and the next are masked for the wave (dense
            // keeps its straight-line halves: 1.2 % faster at 192 keys)
            if (kCausal && t * kTileN + 32 * kb > wave_last) break;
            __builtin_amdgcn_sched_barrier(0);
            f32x16 sacc;
            scores(kt, t, kb, sacc);
            const float m_new = fmaxf(m_ref, half_max(sacc));
            if (__builtin_amdgcn_ballot_w64(m_new > m_ref)) {
                const float alpha = __builtin_amdgcn_exp2f(m_ref - m_new);
#pragma unroll
                for (int db = 0; db < 2; ++db)
#pragma unroll
                    for (int r = 0; r < 16; ++r) oacc[db][r] *= alpha;
                l_part *= alpha;
                m_ref = m_new;
            }
            bf16x8 pp[2];
            l_part += exp_half(sacc, pp);
            __builtin_amdgcn_sched_barrier(0);
            gemm1_half(vt, kb, pp);
        }
    };
    for (int t = 0; t < ntiles; t += 2) {
        iteration(t, std::integral_constant<int, 0>{});
        if (t + 1 < ntiles) iteration(t + 1, std::integral_constant<int, 1>{});
    }

    vmcnt_wait<0>();  // a block without key tiles still has the prologue's (empty) K(0), V(0) in flight

    // epilogue: O = O^T / l through this wave's rows of the K tile area (every
    // wave's K reads are done after the barrier), LSE
    const float l_tot = wave_sum_halves(l_part);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    ring_barrier();
    lds_char* const tb = (wave < 2 ? lds.k[0] : lds.k[1]) + (wave & 1) * (kRowsPerWave * kRowBytes);
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            bf16x2 x0, x1;
            x0[0] = (__bf16)(oacc[db][4 * g4 + 0] * inv);
            x0[1] = (__bf16)(oacc[db][4 * g4 + 1] * inv);
            x1[0] = (__bf16)(oacc[db][4 * g4 + 2] * inv);
            x1[1] = (__bf16)(oacc[db][4 * g4 + 3] * inv);
            i32x2 w;
            w[0] = __builtin_bit_cast(int, x0);
            w[1] = __builtin_bit_cast(int, x1);
            const int c = 4 * db + g4;
            *(lds_i32x2*)(tb + l32 * kRowBytes + ((c ^ ((l32 >> 1) & 7)) << 4) + 8 * (hi ^ (l32 & 1))) = w;
        }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const auto ro = make_rsrc(obase, obytes);
#pragma unroll
    for (int i = 0; i < kRowsPerWave / 8; ++i) {
        const int r = 8 * i + (lane >> 3), pc = lane & 7;
        const i32x4 raw = *(const lds_i32x4*)(tb + r * kRowBytes + (pc << 4));
        const i32x4 v = (r & 1) ? i32x4{raw[2], raw[3], raw[0], raw[1]} : raw;
        const int c = pc ^ ((r >> 1) & 7);
        __builtin_amdgcn_raw_buffer_store_b128(v, ro, (wrow0 + r) * p.stride_o * 2 + c * 16, 0, kStoreStream);
    }
    if (p.lse != nullptr && hi == 0 && my_row < sq) {
        float* lse_base;
        if constexpr (kVarlen)
            lse_base = p.lse + (int64_t)h * (p.nhead_stride_q / p.stride_q) + off_q;
        else
            lse_base = p.lse + (int64_t)b * p.nhead_q * p.seqlen_q + (int64_t)h * p.seqlen_q;
        lse_base[my_row] = (__builtin_log2f(l_tot) + m_ref) * 0.69314718055994530942f;
    }
}

// ===========================================================================
// Compact causal varlen orders (this build's own; no counterpart in the
// reference).  The reference's varlen grid (nhead_q, M-tiles of the longest
// sequence, sequences) runs the sequences one after another in the caller's
// order, each heaviest M-tile first (kernel.cpp:91-99): the blocks past a
// short sequence's end are dispatched between live ones, and a long last
// sequence's heavy M-tiles start last.  On the same grid, block (h, y, z)
// here takes the item of rank r = z * gridDim.y + y (its place in the
// dispatch order) in a list of the live (sequence, M-tile) items; the ranks
// past the live items, dispatched last, exit at once.  Two lists:
//  * level order: by M-tile index, highest first, then by sequence, so every
//    sequence's heaviest M-tiles start before any lighter one (a causal
//    M-tile's key tiles grow with its index);
//  * sequence order: sequence after sequence, the sequences longest first
//    (ties: caller's order), each heaviest M-tile first, so a sequence's
//    M-tiles, which re-read its K/V, still run close together in time.
// Each wave finds its item from the sequence lengths alone: lane s < batch
// holds n_s, the M-tiles of sequence s (at most gridDim.y, as the regular
// grid computes).  Requires batch <= 64 (one lane per sequence); the results
// are wave-uniform.
// ===========================================================================
constexpr int kCompactMaxSeqs = 64;

// This lane's sequence's M-tiles (0 past the last sequence).
__device__ __forceinline__ int compact_ntiles(const FmhaFwdParams& p) {
    const int lane = threadIdx.x & 63;
    if (lane >= (int)gridDim.z) return 0;  // gridDim.z <= kCompactMaxSeqs (checked by the launcher)
    const int len = p.seqstart_q[lane + 1] - p.seqstart_q[lane];
    return min((len + kTileM - 1) / kTileM, (int)gridDim.y);
}

// Level order.  The items at level m or above number
// C(m) = sum_s max(0, n_s - m); the item of rank r sits at the highest level m
// with C(m) > r, at index r - C(m + 1) among the sequences with n_s > m.  The
// lanes evaluate C at up to 64 candidate levels at once (the n_s taken from
// their lanes one by one), narrowing [0, gridDim.y) by 64x per round: one
// round up to 64 M-tiles per sequence, two up to 4096, three beyond.
__device__ __forceinline__ bool level_item(const FmhaFwdParams& p, int rank, int& b_out, int& mt_out) {
    const int lane = threadIdx.x & 63;
    const int nseq = gridDim.z;
    const int n = compact_ntiles(p);
    // [lo, hi): the level holding `rank`; invariant C(lo) > rank (checked
    // first at lo = 0: otherwise the rank is past the live items)
    int lo = 0, hi = gridDim.y, c_next = 0;
    for (;;) {
        const int step = (hi - lo + 63) >> 6;
        const int m = lo + lane * step;  // this lane's candidate level (>= hi: none)
        int c = 0, c1 = 0;               // C(m), C(m + 1)
        for (int s = 0; s < nseq; ++s) {
            const int ns = __builtin_amdgcn_readlane(n, s);
            c += max(0, ns - m);
            c1 += max(0, ns - m - 1);
        }
        const uint64_t above = __builtin_amdgcn_ballot_w64(m < hi && c > rank);
        if (above == 0) return false;  // only at lo = 0: C(0) <= rank, a dead rank
        const int top = 63 - __builtin_clzll(above);  // C falls with m: the set lanes are a prefix
        lo = lo + top * step;
        c_next = __builtin_amdgcn_readlane(c1, top);
        if (step == 1) break;
        hi = min(hi, lo + step);
    }
    const int r = rank - c_next;  // index among the sequences with n_s > lo
    const uint64_t live = __builtin_amdgcn_ballot_w64(n > lo);
    const int before = __builtin_amdgcn_mbcnt_hi((uint32_t)(live >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)live, 0));
    const uint64_t mine = __builtin_amdgcn_ballot_w64(n > lo && before == r);
    b_out = __builtin_ctzll(mine);
    mt_out = lo;
    return true;
}

// Sequence order.  Lane s counts the items of the sequences before it
// (more M-tiles, or as many and an earlier index): its items hold ranks
// [start_s, start_s + n_s), heaviest (highest M-tile) first.
__device__ __forceinline__ bool sequence_item(const FmhaFwdParams& p, int rank, int& b_out, int& mt_out) {
    const int lane = threadIdx.x & 63;
    const int nseq = gridDim.z;
    const int n = compact_ntiles(p);
    int start = 0;
    for (int s = 0; s < nseq; ++s) {
        const int ns = __builtin_amdgcn_readlane(n, s);
        start += (ns > n || (ns == n && s < lane)) ? ns : 0;
    }
    const uint64_t mine = __builtin_amdgcn_ballot_w64(start <= rank && rank < start + n);
    if (mine == 0) return false;  // past the live items
    const int b = __builtin_ctzll(mine);
    b_out = b;
    mt_out = __builtin_amdgcn_readlane(n, b) - 1 - (rank - __builtin_amdgcn_readlane(start, b));
    return true;
}

}  // namespace fmha_gfx950

using namespace fmha_gfx950;

// ---- the four entries (reference src/fused/kernel.cpp:55-99).  Grid
// (nhead_q, ceil(seqlen_q/kM0), batch), kBlockSize threads.  Causal entries
// run the heaviest M-tiles first (kernel.cpp:73,96). ----
#define FMHA_ENTRY_ATTRS __global__ __launch_bounds__(FMHA_KBLOCK) __attribute__((amdgpu_waves_per_eu(2, 2)))
// eight distinct LDS arrays = the K and V ring stages (each `bytes` long)
#define FMHA_RING(r, bytes)                                                                                     \
    __shared__ __attribute__((aligned(1024))) char r##_k0[bytes], r##_k1[bytes], r##_k2[bytes], r##_k3[bytes],   \
        r##_v0[bytes], r##_v1[bytes], r##_v2[bytes], r##_v3[bytes];                                             \
    const Ring r{{(lds_char*)r##_k0, (lds_char*)r##_k1, (lds_char*)r##_k2, (lds_char*)r##_k3},                  \
                 {(lds_char*)r##_v0, (lds_char*)r##_v1, (lds_char*)r##_v2, (lds_char*)r##_v3}};
static_assert(kRing == 4, "FMHA_RING declares four stages per ring");

FMHA_ENTRY_ATTRS void fmha_fwd_d64_bf16_msk0(FmhaFwdParams params) {
    FMHA_RING(ring, kTileBytes)
    fwd_mtile<false, false, kModeRegular>(params, blockIdx.z, blockIdx.x, blockIdx.y, ring);
}
FMHA_ENTRY_ATTRS void fmha_fwd_d64_bf16_msk1(FmhaFwdParams params) {
    FMHA_RING(ring, kTileBytes)
    fwd_mtile<true, false, kModeRegular>(params, blockIdx.z, blockIdx.x, gridDim.y - 1 - blockIdx.y, ring);
}
FMHA_ENTRY_ATTRS void fmha_fwd_d64_bf16_msk0_varlen(FmhaFwdParams params) {
    FMHA_RING(ring, kTileBytes)
    fwd_mtile<false, true, kModeRegular>(params, blockIdx.z, blockIdx.x, blockIdx.y, ring);
}
FMHA_ENTRY_ATTRS void fmha_fwd_d64_bf16_msk1_varlen(FmhaFwdParams params) {
    FMHA_RING(ring, kTileBytes)
    fwd_mtile<true, true, kModeRegular>(params, blockIdx.z, blockIdx.x, gridDim.y - 1 - blockIdx.y, ring);
}

// ---- split-KV entries (this build's own; no counterpart in the reference):
// same grid, 2*kBlockSize threads, two key-range groups per M-tile merged in
// LDS.  For grids with too few blocks to fill the GPU, or causal grids whose
// heaviest M-tile outlasts the average load per CU. ----
#define FMHA_SPLIT_ATTRS \
    __global__ __launch_bounds__(FMHA_SPLIT_KBLOCK) __attribute__((amdgpu_waves_per_eu(2, 2)))
static_assert(FMHA_SPLIT_KBLOCK == 2 * FMHA_KBLOCK, "two groups of kBlockSize threads");

FMHA_SPLIT_ATTRS void fmha_fwd_d64_bf16_splitkv_msk0(FmhaFwdParams params) {
    FMHA_RING(ring, 2 * kTileBytes)
    fwd_mtile<false, false, kModeSplitKV>(params, blockIdx.z, blockIdx.x, blockIdx.y, ring);
}
FMHA_SPLIT_ATTRS void fmha_fwd_d64_bf16_splitkv_msk1(FmhaFwdParams params) {
    FMHA_RING(ring, 2 * kTileBytes)
    fwd_mtile<true, false, kModeSplitKV>(params, blockIdx.z, blockIdx.x, gridDim.y - 1 - blockIdx.y, ring);
}
FMHA_SPLIT_ATTRS void fmha_fwd_d64_bf16_splitkv_msk0_varlen(FmhaFwdParams params) {
    FMHA_RING(ring, 2 * kTileBytes)
    fwd_mtile<false, true, kModeSplitKV>(params, blockIdx.z, blockIdx.x, blockIdx.y, ring);
}
FMHA_SPLIT_ATTRS void fmha_fwd_d64_bf16_splitkv_msk1_varlen(FmhaFwdParams params) {
    FMHA_RING(ring, 2 * kTileBytes)
    fwd_mtile<true, true, kModeSplitKV>(params, blockIdx.z, blockIdx.x, gridDim.y - 1 - blockIdx.y, ring);
}

// ---- pair entries (this build's own; no counterpart in the reference):
// grid (nhead_q, ceil(ceil(seqlen_q/kM0)/2), batch), 2*kBlockSize threads;
// block y owns M-tiles 2y and 2y+1 (causal: heaviest pairs first). ----
FMHA_SPLIT_ATTRS void fmha_fwd_d64_bf16_pair_msk0(FmhaFwdParams params) {
    FMHA_RING(ring, kTileBytes)
    fwd_mtile<false, false, kModePair>(params, blockIdx.z, blockIdx.x, blockIdx.y, ring);
}
FMHA_SPLIT_ATTRS void fmha_fwd_d64_bf16_pair_msk1(FmhaFwdParams params) {
    FMHA_RING(ring, kTileBytes)
    fwd_mtile<true, false, kModePair>(params, blockIdx.z, blockIdx.x, gridDim.y - 1 - blockIdx.y, ring);
}
FMHA_SPLIT_ATTRS void fmha_fwd_d64_bf16_pair_msk0_varlen(FmhaFwdParams params) {
    FMHA_RING(ring, kTileBytes)
    fwd_mtile<false, true, kModePair>(params, blockIdx.z, blockIdx.x, blockIdx.y, ring);
}
FMHA_SPLIT_ATTRS void fmha_fwd_d64_bf16_pair_msk1_varlen(FmhaFwdParams params) {
    FMHA_RING(ring, kTileBytes)
    fwd_mtile<true, true, kModePair>(params, blockIdx.z, blockIdx.x, gridDim.y - 1 - blockIdx.y, ring);
}

// ---- tile-major causal entries (this build's own; no counterpart in the
// reference): the causal dense entries of the three forms on the grid
// (nhead_q, batch, tiles), tiles = the M-tiles (pairs for the pair form) of a
// (batch, head).  Blocks are dispatched x fastest, then y, then z, so every
// batch's heaviest M-tiles start before any lighter one, instead of batch
// after batch.  Each index comes straight from one grid coordinate: these
// entries never branch on the grid's shape. ----
FMHA_ENTRY_ATTRS void fmha_fwd_d64_bf16_msk1_tilemajor(FmhaFwdParams params) {
    FMHA_RING(ring, kTileBytes)
    fwd_mtile<true, false, kModeRegular>(params, blockIdx.y, blockIdx.x, gridDim.z - 1 - blockIdx.z, ring);
}
FMHA_SPLIT_ATTRS void fmha_fwd_d64_bf16_splitkv_msk1_tilemajor(FmhaFwdParams params) {
    FMHA_RING(ring, 2 * kTileBytes)
    fwd_mtile<true, false, kModeSplitKV>(params, blockIdx.y, blockIdx.x, gridDim.z - 1 - blockIdx.z, ring);
}
FMHA_SPLIT_ATTRS void fmha_fwd_d64_bf16_pair_msk1_tilemajor(FmhaFwdParams params) {
    FMHA_RING(ring, kTileBytes)
    fwd_mtile<true, false, kModePair>(params, blockIdx.y, blockIdx.x, gridDim.z - 1 - blockIdx.z, ring);
}

// ---- compact causal varlen entries (this build's own; no counterpart in the
// reference): the regular varlen grid (nhead_q, ceil(seqlen_q/kM0), batch) and
// block, batch <= 64; the block of dispatch rank z * gridDim.y + y takes the
// live (sequence, M-tile) item of that rank in the level order (highest
// M-tile index first across all sequences) or the sequence order (longest
// sequence first, each heaviest M-tile first); ranks past the live items
// exit. ----
FMHA_ENTRY_ATTRS void fmha_fwd_d64_bf16_msk1_varlen_tilemajor(FmhaFwdParams params) {
    FMHA_RING(ring, kTileBytes)
    int b, mt;
    if (!level_item(params, (int)(blockIdx.z * gridDim.y + blockIdx.y), b, mt)) return;
    fwd_mtile<true, true, kModeRegular>(params, b, blockIdx.x, mt, ring);
}
FMHA_ENTRY_ATTRS void fmha_fwd_d64_bf16_msk1_varlen_seqmajor(FmhaFwdParams params) {
    FMHA_RING(ring, kTileBytes)
    int b, mt;
    if (!sequence_item(params, (int)(blockIdx.z * gridDim.y + blockIdx.y), b, mt)) return;
    fwd_mtile<true, true, kModeRegular>(params, b, blockIdx.x, mt, ring);
}

// ---- pair stream entries (this build's own; no counterpart in the
// reference): one block of 2*kBlockSize threads per compute unit (grid
// (blocks)), each looping over M-tile pairs; 96 KiB of LDS (the K/V rings and
// a 4 KiB Q/O buffer per wave).  Launched by the C-ABI only. ----
#define FMHA_STREAM_ATTRS \
    __global__ __launch_bounds__(FMHA_SPLIT_KBLOCK) __attribute__((amdgpu_waves_per_eu(2, 2)))
constexpr int kStreamQBytes = 2 * kWaves * kRowsPerWave * kRowBytes;  // 32 KiB: 4 KiB per wave
FMHA_STREAM_ATTRS void fmha_fwd_d64_bf16_pair_stream_msk0(FmhaStreamArgs args) {
    FMHA_RING(ring, kTileBytes)
    __shared__ __attribute__((aligned(1024))) char qbuf[kStreamQBytes];
    (void)args;  // read through the kernarg segment pointer
    fwd_pair_stream<false>(ring, (lds_char*)qbuf);
}
FMHA_STREAM_ATTRS void fmha_fwd_d64_bf16_pair_stream_msk1(FmhaStreamArgs args) {
    FMHA_RING(ring, kTileBytes)
    __shared__ __attribute__((aligned(1024))) char qbuf[kStreamQBytes];
    (void)args;
    fwd_pair_stream<true>(ring, (lds_char*)qbuf);
}

// ---- balanced causal entries (this build's own; no counterpart in the
// reference): dense causal launches whose heaviest M-tiles outlast the average
// work per resident block.  Grid (nhead_q, batch, n_items); item z of every
// (batch, head) comes from the launcher's table, heaviest first: a whole
// M-tile, or one half of the key tiles of a split M-tile, whose partial result
// goes to the workspace; fmha_fwd_d64_bf16_balanced_merge then finishes the
// split M-tiles. ----
static_assert(FMHA_BALANCED_PART_BYTES == kWaves * kPartFloatsPerWave * 4, "partial slot size");
__device__ __forceinline__ Chunk balanced_chunk(const FmhaBalancedArgs& a, int b, int h, int mt, int half) {
    if (mt < a.split_from) return Chunk{0, nullptr};
    const int64_t slot = ((int64_t)(b * a.p.nhead_q + h) * a.n_split + (mt - a.split_from)) * 2 + half;
    return Chunk{half, a.part + slot * (kWaves * kPartFloatsPerWave)};
}
FMHA_ENTRY_ATTRS void fmha_fwd_d64_bf16_balanced_msk1(FmhaBalancedArgs args) {
    FMHA_RING(ring, kTileBytes)
    const int it = args.item[blockIdx.z];
    const int mt = it & 0x7fff, half = it >> 15;
    const int b = blockIdx.y, h = blockIdx.x;
    fwd_mtile<true, false, kModeBalanced>(args.p, b, h, mt, ring, balanced_chunk(args, b, h, mt, half));
}
// The same over M-tile pairs (2*kBlockSize threads): item = pair | half << 15;
// split_from is even, so a split pair's M-tiles are both split.
FMHA_SPLIT_ATTRS void fmha_fwd_d64_bf16_balanced_pair_msk1(FmhaBalancedArgs args) {
    FMHA_RING(ring, kTileBytes)
    const int it = args.item[blockIdx.z];
    const int pr = it & 0x7fff, half = it >> 15;
    const int b = blockIdx.y, h = blockIdx.x;
    fwd_mtile<true, false, kModeBalancedPair>(args.p, b, h, pr, ring, balanced_chunk(args, b, h, 2 * pr, half));
}

// Merge of the two halves of a split M-tile (grid (nhead_q, n_split, batch)):
// thread (wave, lane) holds the same O^T elements in both partials, so each
// lane merges its own: m = max(m0, m1), O^T = sum 2^(m_i - m) O^T_i, l alike;
// then the regular epilogue (O = O^T / l through LDS, LSE).
__global__ __launch_bounds__(FMHA_KBLOCK) void fmha_fwd_d64_bf16_balanced_merge(FmhaBalancedArgs args) {
    __shared__ __attribute__((aligned(1024))) char stage[kWaves * kRowsPerWave * kRowBytes];
    const FmhaFwdParams& p = args.p;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l32 = lane & 31, hi = lane >> 5;
    const int mt = args.split_from + blockIdx.y, h = blockIdx.x, b = blockIdx.z;
    const float* w0 = balanced_chunk(args, b, h, mt, 0).part + wave * kPartFloatsPerWave;
    const float* w1 = w0 + kWaves * kPartFloatsPerWave;
    const float m0 = w0[32 * 64 + lane], m1 = w1[32 * 64 + lane];
    const float m = fmaxf(m0, m1);
    const float a0 = __builtin_amdgcn_exp2f(m0 - m), a1 = __builtin_amdgcn_exp2f(m1 - m);
    f32x16 oacc[2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r)
            oacc[db][r] = a0 * w0[(16 * db + r) * 64 + lane] + a1 * w1[(16 * db + r) * 64 + lane];
    const float l_part = a0 * w0[33 * 64 + lane] + a1 * w1[33 * 64 + lane];

    const float l_tot = wave_sum_halves(l_part);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    const int sq = p.seqlen_q;
    const uint32_t obytes = (uint32_t)((int64_t)(sq - 1) * p.stride_o * 2 + kRowBytes);
    const auto ro = make_rsrc((const __bf16*)p.o + (int64_t)b * p.batch_stride_o + (int64_t)h * p.nhead_stride_o, obytes);
    const int wrow0 = mt * kTileM + wave * kRowsPerWave;
    lds_char* tb = (lds_char*)stage + wave * (kRowsPerWave * kRowBytes);
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
            bf16x2 x0, x1;
            x0[0] = (__bf16)(oacc[db][4 * g4 + 0] * inv);
            x0[1] = (__bf16)(oacc[db][4 * g4 + 1] * inv);
            x1[0] = (__bf16)(oacc[db][4 * g4 + 2] * inv);
            x1[1] = (__bf16)(oacc[db][4 * g4 + 3] * inv);
            i32x2 v;
            v[0] = __builtin_bit_cast(int, x0);
            v[1] = __builtin_bit_cast(int, x1);
            const int c = 4 * db + g4;
            *(lds_i32x2*)(tb + l32 * kRowBytes + ((c ^ ((l32 >> 1) & 7)) << 4) + 8 * (hi ^ (l32 & 1))) = v;
        }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < kRowsPerWave / 8; ++i) {
        const int r = 8 * i + (lane >> 3), pc = lane & 7;
        const i32x4 raw = *(const lds_i32x4*)(tb + r * kRowBytes + (pc << 4));
        const i32x4 v = (r & 1) ? i32x4{raw[2], raw[3], raw[0], raw[1]} : raw;
        const int c = pc ^ ((r >> 1) & 7);
        __builtin_amdgcn_raw_buffer_store_b128(v, ro, (wrow0 + r) * p.stride_o * 2 + c * 16, 0, 0);
    }
    const int my_row = wrow0 + l32;
    if (p.lse != nullptr && hi == 0 && my_row < sq) {
        const float lse2 = __builtin_log2f(l_tot) + m;  // -inf when l == 0
        p.lse[(int64_t)b * p.nhead_q * sq + (int64_t)h * sq + my_row] = lse2 * 0.69314718055994530942f;
    }
}

// ---- short entries (this build's own; no counterpart in the reference):
// the regular grid and block, <= 128 VGPRs and 32 KiB of LDS (four blocks
// per compute unit), any key count.  Causal entries run the heaviest M-tiles
// first, as the regular ones. ----
#define FMHA_SHORT_ATTRS __global__ __launch_bounds__(FMHA_KBLOCK) __attribute__((amdgpu_waves_per_eu(4, 4)))
// every K and V stage its own array
#define FMHA_SHORT_LDS                                                                                     \
    __shared__ __attribute__((aligned(1024))) char k0[kTileBytes], k1[kTileBytes], v0[kTileBytes], v1[kTileBytes]; \
    const ShortLds lds{{(lds_char*)k0, (lds_char*)k1}, {(lds_char*)v0, (lds_char*)v1}};
#define FMHA_SHORT_ENTRY(name, causal, varlen)                                                             \
    FMHA_SHORT_ATTRS void name(FmhaFwdParams params) {                                                     \
        FMHA_SHORT_LDS                                                                                      \
        fwd_short<causal, varlen>(params, blockIdx.z, blockIdx.x, causal ? gridDim.y - 1 - blockIdx.y : blockIdx.y, \
                                  lds);                                                                     \
    }
FMHA_SHORT_ENTRY(fmha_fwd_d64_bf16_short_msk0, false, false)
FMHA_SHORT_ENTRY(fmha_fwd_d64_bf16_short_msk1, true, false)
FMHA_SHORT_ENTRY(fmha_fwd_d64_bf16_short_msk0_varlen, false, true)
FMHA_SHORT_ENTRY(fmha_fwd_d64_bf16_short_msk1_varlen, true, true)
