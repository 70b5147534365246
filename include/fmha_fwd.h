/*
 * fmha_fwd.h — drop-in boundary of the MI355X (gfx950) D64 BF16 fused
 * multi-head-attention forward path.
 *
 * Two ways in, both replacing what the reference exposes:
 *
 *  1. The kernarg struct FmhaFwdParams and the four __global__ entry points
 *     fmha_fwd_d64_bf16_msk{0,1}[_varlen](FmhaFwdParams), launched by the
 *     caller exactly as the reference's callers do:
 *        hipLaunchKernelGGL(entry, dim3(nhead_q, ceil(seqlen_q / kM0), batch),
 *                           dim3(kBlockSize), 0, stream, params);
 *     Replaces: src/runner/params.hpp:18-86 (struct + tile constants) and
 *     src/fused/kernel.cpp:55-99 (the four entries).  The grid contract is kept;
 *     kM0/kBlockSize below are this build's tile sizes, and callers that read
 *     them (src/bench_fmha_fwd.cpp:174-176) keep working unchanged.
 *
 *  2. A C-ABI launcher, fmha_fwd_d64_bf16(), which validates the arguments,
 *     picks the entry (varlen <=> seqstart_q != NULL, causal flag), builds the
 *     grid itself and returns a hipError_t instead of exiting.
 *     Replaces: the launch lambda in src/bench_fmha_fwd.cpp:174-191 and the
 *     identical launch blocks in tests/test_fmha_fwd_d64.cpp:563-578.
 *
 * Semantics (identical to the reference, src/runner/params.hpp:18-64):
 *  - element (b,h,s,d) of a tensor lives at
 *      b*batch_stride + h*nhead_stride + s*stride + d     (strides in elements)
 *  - scale is PRE-MULTIPLIED by log2(e): scale = log2(e)/sqrt(64)
 *  - lse == NULL disables the LSE output.  LSE is natural-log, fp32, one value
 *    per query row.  Dense: lse[b*nhead_q*seqlen_q + h*seqlen_q + s].
 *    Varlen: lse[h*(nhead_stride_q/stride_q) + seqstart_q[b] + s]
 *    (src/fused/pipeline.hpp:408-418).
 *  - seqstart_q/seqstart_k non-NULL select varlen ("group") mode: device int32
 *    arrays of batch+1 prefix offsets; batch strides are ignored and
 *    seqlen_q/seqlen_k are upper bounds used only for the grid.
 *  - causal is bottom-right aligned: query row i attends key j iff
 *    j <= i + (seqlen_k - seqlen_q)  (per sequence in varlen mode).
 *    A query row with no visible key gets O = 0 and LSE = -inf.
 *  - GQA/MQA: nhead_q % nhead_k == 0, KV head = h / (nhead_q / nhead_k).
 *
 * Requirements checked by the launcher (the reference checks none of them):
 *  q,k,v,o non-NULL and 16-byte aligned; every stride a multiple of 8 elements
 *  (16-byte rows); seqlen_* >= 0; nhead_k > 0; nhead_q % nhead_k == 0; both or
 *  neither seqstart pointer set; every in-tensor offset of one (batch, head)
 *  fits in 31 bits; the grid fits (ceil(seqlen_q / kM0) <= 65535 and
 *  batch <= 65535); scale finite and > 0 (the running row maximum assumes
 *  that a larger score is a larger weight).  Violations return
 *  hipErrorInvalidValue and launch nothing.
 */
#ifndef FMHA_FWD_H_
#define FMHA_FWD_H_

#include <stddef.h>
#include <stdint.h>
#ifndef __HIP_PLATFORM_AMD__
#define __HIP_PLATFORM_AMD__ 1
#endif
#include <hip/hip_runtime_api.h>

#if defined(__cplusplus) && defined(__HIPCC__)
#include <hip/hip_bf16.h>
typedef __hip_bfloat16 fmha_bf16_t;
#else
typedef uint16_t fmha_bf16_t; /* bf16 bit pattern; same size and alignment */
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Kernarg block, passed by value.  Field order and offsets are the ABI and are
 * identical to the reference's struct (src/runner/params.hpp:18-64):
 * q@0 k@8 v@16 o@24 lse@32 seqlen_q@40 seqlen_k@44 nhead_q@48 nhead_k@52
 * scale@56 q-strides@60 k-strides@72 v-strides@84 o-strides@96 (pad@108)
 * seqstart_q@112 seqstart_k@120; sizeof 128, alignof 8. */
typedef struct FmhaFwdParams {
    const fmha_bf16_t *q, *k, *v;
    fmha_bf16_t* o;
    float* lse;
    int seqlen_q, seqlen_k;
    int nhead_q, nhead_k;
    float scale;
    int stride_q, nhead_stride_q, batch_stride_q;
    int stride_k, nhead_stride_k, batch_stride_k;
    int stride_v, nhead_stride_v, batch_stride_v;
    int stride_o, nhead_stride_o, batch_stride_o;
    const int32_t* seqstart_q;
    const int32_t* seqstart_k;
} FmhaFwdParams;

/* Tile geometry (same values as the reference, params.hpp:70-86).  One block
 * owns FMHA_KM0 query rows of one (batch, head): FMHA_KBLOCK/64 waves of 32
 * query rows each; keys are walked in tiles of FMHA_KN0. */
#define FMHA_KM0 128
#define FMHA_KN0 64
#define FMHA_KBLOCK 256
#define FMHA_HEAD_DIM 64
/* Threads per block of the split-KV entries (two groups of FMHA_KBLOCK, each
 * walking half of an M-tile's key range; this build's own, launched by
 * fmha_fwd_d64_bf16() when the grid is too small or too unbalanced to fill
 * the GPU). */
#define FMHA_SPLIT_KBLOCK 512

/* Launch the D64 BF16 forward pass on `stream`.
 *   params : kernarg (host memory; copied by value)
 *   batch  : number of sequences (dense batch, or number of varlen sequences)
 *   causal : 0 = no mask (reference --mask 0), 1 = bottom-right causal (--mask 1)
 * Returns hipSuccess, hipErrorInvalidValue for rejected arguments (nothing is
 * launched), or the launch error.  Asynchronous like any kernel launch; it
 * allocates nothing (its only state is a per-device cache of the compute-unit
 * count), so concurrent calls are safe.  The kernel form follows the grid
 * (see fmha_fwd_d64_bf16_variant).
 * Replaces src/bench_fmha_fwd.cpp:174-191. */
hipError_t fmha_fwd_d64_bf16(const FmhaFwdParams* params, int batch, int causal,
                             hipStream_t stream);

/* The same launch with the kernel form chosen by the caller (this build's
 * own; no counterpart in the reference):
 *   FMHA_VARIANT_AUTO     what fmha_fwd_d64_bf16() picks: short for
 *                         launches with seqlen_k <= 192 and at least
 *                         2 x CUs x 128 query rows (batch x nhead_q x
 *                         seqlen_q; varlen: the bounds), or causal with
 *                         seqlen_k <= 384 and at least 7 x CUs x 128; with
 *                         seqlen_k >= 2048,
 *                         split-KV when the regular grid has at most one
 *                         block per compute unit (causal: at most 1.5, or up
 *                         to 2 with seqlen_k >= 8192); pair when its blocks
 *                         fill whole rounds of the compute units and
 *                         seqlen_k >= 2048 (causal: exactly two rounds and
 *                         seqlen_k >= 8192, or whole rounds and >= 32768);
 *                         else the regular entries
 *   FMHA_VARIANT_REGULAR  the four reference-named entries (kBlockSize threads)
 *   FMHA_VARIANT_SPLITKV  the splitkv entries (FMHA_SPLIT_KBLOCK threads)
 *   FMHA_VARIANT_PAIR     the pair entries: one FMHA_SPLIT_KBLOCK-thread block
 *                         per two adjacent M-tiles of a (batch, head)
 *   FMHA_VARIANT_SHORT    the short entries: the regular grid at four blocks
 *                         per compute unit, K and V streamed through
 *                         two-stage LDS rings, any number of keys
 *   FMHA_VARIANT_PAIR_STREAM  not varlen: pair blocks (FMHA_SPLIT_KBLOCK
 *                         threads, 96 KiB of LDS) that each loop over
 *                         M-tile pairs, the next pair's first K/V tiles and
 *                         Q rows fetched during the current pair's last
 *                         iterations and its O stored beside the next
 *                         pair's first; dense: one block per compute unit
 *                         taking every CU-count-th pair; causal: one block
 *                         per pair of the first half of each (batch, head),
 *                         taking that pair's mirror next
 * All forms give the same results up to fp32 rounding order.  Causal dense
 * launches of more than one batch whose K/V per XCD, batch x ceil(nhead_k/8)
 * x seqlen_k x 256 bytes, is at most 8 MiB run the form's tile-major entry
 * (every batch's heaviest M-tiles first), and causal varlen launches of at
 * most 8 sequences in the regular form whose grid is at most 8 rounds of two
 * blocks per compute unit the compact entry in the sequence order (longest
 * sequence first, no block past a sequence's end between live ones), unless
 * one order flag is OR-ed into `variant`: FMHA_VARIANT_REFERENCE_ORDER (the
 * reference's order), FMHA_VARIANT_TILE_MAJOR_ORDER (tile-major, or for
 * varlen the level order: the live M-tiles of all sequences, highest M-tile
 * index first; at most 64 sequences) or FMHA_VARIANT_SEQUENCE_ORDER (varlen,
 * at most 64 sequences); the order changes no result bit.  An unknown
 * variant, or more than one order flag, returns hipErrorInvalidValue. */
#define FMHA_VARIANT_AUTO 0
#define FMHA_VARIANT_REGULAR 1
#define FMHA_VARIANT_SPLITKV 2
#define FMHA_VARIANT_PAIR 3
/* 4: retired (returns hipErrorInvalidValue) */
#define FMHA_VARIANT_BALANCED 5 /* fmha_fwd_d64_bf16_ws only: it needs a workspace */
#define FMHA_VARIANT_SHORT 6
#define FMHA_VARIANT_BALANCED_PAIR 7 /* fmha_fwd_d64_bf16_ws only: the balanced form over M-tile pairs */
#define FMHA_VARIANT_PAIR_STREAM 8   /* dense layouts (not varlen): one pair block per compute unit looping
                                        over M-tile pairs (causal: a pair, then its mirror) */
#define FMHA_VARIANT_REFERENCE_ORDER 16 /* flag: batch after batch, on the (nhead_q, tiles, batch) grid;
                                           balanced forms: the plain heaviest-first item table */
#define FMHA_VARIANT_TILE_MAJOR_ORDER 32 /* flag: causal dense batches on the tile-major entries (any K/V
                                            size); causal varlen (regular form, <= 64 sequences): level order */
#define FMHA_VARIANT_SEQUENCE_ORDER 64  /* flag: causal varlen (regular form, <= 64 sequences): sequence
                                           order; dense batches as FMHA_VARIANT_REFERENCE_ORDER */
hipError_t fmha_fwd_d64_bf16_variant(const FmhaFwdParams* params, int batch, int causal, int variant,
                                     hipStream_t stream);

/* The launch with a caller-provided workspace (this build's own; no
 * counterpart in the reference).  Dense causal launches whose heaviest M-tile
 * would outlast the average work per resident block (long sequences with few
 * heads, e.g. B1 H2 S40000) run the balanced form where it measured faster
 * (M-tiles of >= 64 key tiles on grids of at most one block per compute
 * unit, >= 128 up to 1.5 blocks per unit or on a partial second round whose
 * heaviest M-tile outlasts 1.5x the average; never at 1.5-2 blocks per
 * unit, nor for shorter M-tiles except >= 32 key tiles at up to half a block
 * per unit): the M-tiles with more key
 * tiles than half that average are split into two key halves, every item is
 * dispatched heaviest first from a table in the kernarg, each half leaves its
 * partial result in the workspace and a second launch merges the halves
 * (fp32, the same merge as the split-KV form; results equal the other forms
 * up to fp32 rounding order).
 *   variant: FMHA_VARIANT_AUTO (balanced when it applies and the workspace
 *            is large enough, else what fmha_fwd_d64_bf16 picks),
 *            FMHA_VARIANT_BALANCED (always the balanced form, with the
 *            heavy-M-tile rule applied even where the regular order would
 *            balance: causal dense only; hipErrorInvalidValue if it cannot
 *            run), FMHA_VARIANT_BALANCED_PAIR (the same over M-tile pairs in
 *            8-wave blocks, one per compute unit: pairs above 0.7 of the
 *            average work per unit are split; a group's partial goes to its
 *            own M-tile's slot, so the workspace size is the same formula),
 *            or any other variant (workspace unused, as
 *            fmha_fwd_d64_bf16_variant).  The balanced forms order their
 *            item table per group of XCDs when nhead_q * batch divides the
 *            XCD count; FMHA_VARIANT_REFERENCE_ORDER OR-ed in keeps the plain
 *            heaviest-first table (the same items: identical results).
 *   workspace: device memory, 256-byte aligned, at least
 *            fmha_fwd_d64_bf16_workspace_size() bytes, or NULL with 0 bytes
 *            (then never balanced).  Its contents need no initialisation;
 *            launches that overlap in time need workspaces of their own.
 * Allocates nothing.  Returns hipSuccess, hipErrorInvalidValue (nothing
 * launched) or the launch error. */
hipError_t fmha_fwd_d64_bf16_ws(const FmhaFwdParams* params, int batch, int causal, int variant, void* workspace,
                                int64_t workspace_bytes, hipStream_t stream);
/* Workspace bytes fmha_fwd_d64_bf16_ws needs for these arguments with
 * FMHA_VARIANT_AUTO or FMHA_VARIANT_BALANCED on the current device (0 when the
 * launch would not use one; 0 for any other variant), -1 for rejected
 * arguments.  Host only. */
int64_t fmha_fwd_d64_bf16_workspace_size(const FmhaFwdParams* params, int batch, int causal, int variant);

/* fmha_fwd_d64_bf16_ws without a workspace argument, for callers that cannot
 * allocate (code under graph capture, serving loops that forbid allocation).
 * No counterpart in the reference.  The workspace is a static device array of
 * FMHA_NOALLOC_SCRATCH_BYTES that the library holds on every GPU it runs on
 * until the process ends; a launch whose plan needs more returns
 * hipErrorInvalidValue and launches nothing (the balanced form needs
 * 2 x 34,816 bytes per split M-tile: B1 H2 S40000 causal needs 30,359,552).
 * Calls that overlap in time on one GPU share the array and race; calls in
 * stream order do not (nothing in it needs clearing).  Allocates nothing. */
#define FMHA_NOALLOC_SCRATCH_BYTES (32 << 20)
hipError_t fmha_fwd_d64_bf16_noalloc(const FmhaFwdParams* params, int batch, int causal, int variant,
                                     hipStream_t stream);

/* The balanced form's plan for these arguments on a device with
 * `compute_units` compute units and `xccs` XCDs (0 = the current device's;
 * xccs 1 gives the plain heaviest-first order that FMHA_VARIANT_REFERENCE_ORDER
 * launches; `force` 0: the automatic rule, 1: as FMHA_VARIANT_BALANCED, 2: as
 * FMHA_VARIANT_BALANCED_PAIR, whose items are M-tile pairs): writes up to
 * `capacity` items (dispatch order; M-tile (pair) | half << 15, half 0 = the
 * first ceil(n/2) key tiles) and the first split M-tile (even for pairs), and
 * returns the number of items per (batch, head); 0 when the launch would not
 * be balanced, -1 for rejected arguments.  When nhead_q * batch divides xccs
 * into g >= 2 groups of XCDs (entry z runs on group z % g), each run of g
 * consecutive entries is ordered by the first key tile its items read, so
 * that a group keeps taking items that start at the same key.  Host only
 * (this build's own; no counterpart in the reference). */
int fmha_fwd_d64_bf16_balanced_plan(const FmhaFwdParams* params, int batch, int causal, int compute_units, int xccs,
                                    int force, unsigned short* items, int capacity, int* split_from);

/* Argument checks of fmha_fwd_d64_bf16 without launching (host only, no GPU
 * needed).  Returns hipSuccess or hipErrorInvalidValue. */
hipError_t fmha_fwd_d64_bf16_check(const FmhaFwdParams* params, int batch, int causal);

/* The form FMHA_VARIANT_AUTO resolves to for these arguments on a device with
 * `compute_units` compute units (0 = the current device's count), without
 * launching (this build's own; no counterpart in the reference).  Returns
 * FMHA_VARIANT_REGULAR, _SPLITKV, _PAIR or _SHORT, or -1 for rejected
 * arguments. */
int fmha_fwd_d64_bf16_pick_variant(const FmhaFwdParams* params, int batch, int causal, int compute_units);

/* The block order of the automatic launch (FMHA_VARIANT_AUTO, no order flag)
 * with these arguments: 1 for a tile-major entry (causal dense batches) or the
 * level order of a compact varlen entry, 2 for the sequence order of a
 * compact varlen entry, 0 for the reference's order, -1 for rejected
 * arguments; host only (this build's own; no counterpart in the reference). */
int fmha_fwd_d64_bf16_tile_major(const FmhaFwdParams* params, int batch, int causal);

/* Tile constants of the linked library, so FFI callers (ctypes, cgo) need not
 * parse this header: writes kM0, kN0, kBlockSize, head dim. */
void fmha_fwd_d64_bf16_tile_config(int* m0, int* n0, int* block_size, int* head_dim);

/* Merge of partial results over disjoint key sets (this build's own; no
 * counterpart in the reference).  The LSE merge the split-KV form does in
 * LDS, for partials from separate launches of fmha_fwd_d64_bf16 (key chunks of
 * one sequence, ring attention, one GPU's shard of a sharded sequence).  For
 * each row r with parts i = 0 .. n_parts-1 (O_i: 64 bf16, normalised; LSE_i:
 * fp32 natural log, -inf for a part that saw no key):
 *   LSE[r] = log(sum_i exp(LSE_i[r])),   O[r] = sum_i exp(LSE_i[r] - LSE[r]) O_i[r]
 * and O = 0, LSE = -inf where every part is -inf (fp32 arithmetic, O rounded
 * to nearest even bf16).  Rows are flattened in LSE order (dense BHSD
 * [B][H][S], varlen [H][T]):
 *   O_i row r at  o_parts + i*o_part_stride + r*o_row_stride   (bf16 elements)
 *   LSE_i row r at lse_parts + i*lse_part_stride + r             (floats)
 *   output row r at o + r*o_row_stride, lse + r (lse may be NULL)
 * o_parts and o 16-byte aligned, strides multiples of 8 elements, o_row_stride
 * >= 64, parts not overlapping, 1 <= n_parts <= FMHA_MERGE_MAX_PARTS; o may be
 * part 0 itself (each output chunk is written after its last read).  Returns
 * hipSuccess, hipErrorInvalidValue (nothing launched) or the launch error;
 * allocates nothing. */
#define FMHA_MERGE_MAX_PARTS 64
hipError_t fmha_merge_d64_bf16(int n_parts, int64_t rows, const void* o_parts, int64_t o_part_stride,
                               const float* lse_parts, int64_t lse_part_stride, int64_t o_row_stride, void* o,
                               float* lse, hipStream_t stream);

#ifdef __cplusplus
} /* extern "C" */

static_assert(sizeof(FmhaFwdParams) == 128, "FmhaFwdParams must stay 128 bytes");
static_assert(alignof(FmhaFwdParams) == 8, "FmhaFwdParams alignment");
static_assert(offsetof(FmhaFwdParams, lse) == 32, "kernarg layout");
static_assert(offsetof(FmhaFwdParams, seqlen_q) == 40, "kernarg layout");
static_assert(offsetof(FmhaFwdParams, scale) == 56, "kernarg layout");
static_assert(offsetof(FmhaFwdParams, stride_q) == 60, "kernarg layout");
static_assert(offsetof(FmhaFwdParams, stride_k) == 72, "kernarg layout");
static_assert(offsetof(FmhaFwdParams, stride_v) == 84, "kernarg layout");
static_assert(offsetof(FmhaFwdParams, stride_o) == 96, "kernarg layout");
static_assert(offsetof(FmhaFwdParams, seqstart_q) == 112, "kernarg layout");
static_assert(offsetof(FmhaFwdParams, seqstart_k) == 120, "kernarg layout");

/* The reference's C++ tile constants, same names (src/runner/params.hpp:70-86). */
constexpr int kM0 = FMHA_KM0;
constexpr int kN0 = FMHA_KN0;
constexpr int kBlockSize = FMHA_KBLOCK;
constexpr int kHeadDim = FMHA_HEAD_DIM;
constexpr int kWarpSize = 64;
constexpr int kNumWarps = FMHA_KBLOCK / 64;

#if defined(__HIPCC__)
/* The four launchable entries (reference src/fused/kernel.cpp:55-99).  Grid
 * (nhead_q, ceil(seqlen_q/kM0), batch), block kBlockSize, no dynamic LDS. */
__global__ void fmha_fwd_d64_bf16_msk0(FmhaFwdParams params);
__global__ void fmha_fwd_d64_bf16_msk1(FmhaFwdParams params);
__global__ void fmha_fwd_d64_bf16_msk0_varlen(FmhaFwdParams params);
__global__ void fmha_fwd_d64_bf16_msk1_varlen(FmhaFwdParams params);
/* Split-KV forms of the same four (no counterpart in the reference): same
 * grid, block FMHA_SPLIT_KBLOCK, same results up to fp32 rounding order. */
__global__ void fmha_fwd_d64_bf16_splitkv_msk0(FmhaFwdParams params);
__global__ void fmha_fwd_d64_bf16_splitkv_msk1(FmhaFwdParams params);
__global__ void fmha_fwd_d64_bf16_splitkv_msk0_varlen(FmhaFwdParams params);
__global__ void fmha_fwd_d64_bf16_splitkv_msk1_varlen(FmhaFwdParams params);
/* Pair forms (no counterpart in the reference): grid (nhead_q,
 * ceil(ceil(seqlen_q/kM0)/2), batch), block FMHA_SPLIT_KBLOCK; block y
 * computes M-tiles 2y and 2y+1 with one shared K/V stream. */
__global__ void fmha_fwd_d64_bf16_pair_msk0(FmhaFwdParams params);
__global__ void fmha_fwd_d64_bf16_pair_msk1(FmhaFwdParams params);
__global__ void fmha_fwd_d64_bf16_pair_msk0_varlen(FmhaFwdParams params);
__global__ void fmha_fwd_d64_bf16_pair_msk1_varlen(FmhaFwdParams params);
/* Short forms (no counterpart in the reference): the regular grid and
 * block, four blocks per compute unit (32 KiB of LDS), any key count. */
__global__ void fmha_fwd_d64_bf16_short_msk0(FmhaFwdParams params);
__global__ void fmha_fwd_d64_bf16_short_msk1(FmhaFwdParams params);
__global__ void fmha_fwd_d64_bf16_short_msk0_varlen(FmhaFwdParams params);
__global__ void fmha_fwd_d64_bf16_short_msk1_varlen(FmhaFwdParams params);
/* Tile-major causal dense forms (no counterpart in the reference): grid
 * (nhead_q, batch, tiles), tiles = ceil(seqlen_q/kM0) (pair form: pairs of
 * them), block kBlockSize (regular) or FMHA_SPLIT_KBLOCK; block z runs M-tile
 * (pair) tiles-1-z, so all batches' heaviest M-tiles are dispatched first. */
__global__ void fmha_fwd_d64_bf16_msk1_tilemajor(FmhaFwdParams params);
__global__ void fmha_fwd_d64_bf16_splitkv_msk1_tilemajor(FmhaFwdParams params);
__global__ void fmha_fwd_d64_bf16_pair_msk1_tilemajor(FmhaFwdParams params);
/* Compact causal varlen forms (no counterpart in the reference): the grid and
 * block of fmha_fwd_d64_bf16_msk1_varlen with at most 64 sequences (batch =
 * grid z); the block of dispatch rank z * gridDim.y + y computes the live
 * (sequence, M-tile) item of that rank, the items ordered by M-tile index,
 * highest first, then by sequence (_tilemajor), or sequence after sequence,
 * longest first, each heaviest M-tile first (_seqmajor); ranks past the live
 * items do nothing.  Same results as fmha_fwd_d64_bf16_msk1_varlen, bit for
 * bit. */
__global__ void fmha_fwd_d64_bf16_msk1_varlen_tilemajor(FmhaFwdParams params);
__global__ void fmha_fwd_d64_bf16_msk1_varlen_seqmajor(FmhaFwdParams params);
#endif
#endif /* __cplusplus */

#endif /* FMHA_FWD_H_ */
