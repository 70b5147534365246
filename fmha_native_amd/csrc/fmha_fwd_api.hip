// fmha_fwd_api.hip — C-ABI launcher for the gfx950 D64 BF16 FMHA forward.
//
// Replaces the reference's launch sites (src/bench_fmha_fwd.cpp:174-191,
// tests/test_fmha_fwd_d64.cpp:563-578): pick one of the four entries (varlen
// <=> seqstart_q set; causal flag), build the (nhead_q, ceil(seqlen_q/kM0),
// batch) grid and launch on the caller's stream.  Unlike the reference it
// validates its arguments and returns hipError_t instead of exiting.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <cmath>

#include "fmha_fwd.h"
#include "fmha_internal.h"

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int kMaxGridYZ = 65535;  // largest grid y / z dimension

// Largest byte offset touched inside one (batch, head) of a tensor with `rows`
// rows must fit the 31-bit buffer offsets the kernel uses.  Row indices run
// past the last row by at most one 64-key tile (K/V loaders) or, for Q and O,
// by the rest of the block's M-tiles: up to 2*kM0 - 1 rows for the pair form's
// second M-tile.  Such rows are zero-filled or dropped by the descriptor bound,
// but their offsets are still computed in 32-bit arithmetic.
bool offsets_fit(int rows, int stride) {
    const int64_t max_rows = (int64_t)rows + FMHA_KN0 + 2 * FMHA_KM0;
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
    // the running max assumes a positive scale (a larger score is a larger
    // probability); NaN fails this comparison too
    if (!(p->scale > 0.0f) || p->scale > 3.402823466e38f) return hipErrorInvalidValue;
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

// What the launch rules read from the current device, cached per device
// ordinal: compute units, XCDs and each XCD's L2 (MI355X: 256, 8, 4 MiB,
// also the values used when a query fails).
struct DeviceShape {
    int cus, xccs, l2_bytes;
};
DeviceShape device_shape() {
    static std::atomic<int> cache[64][3];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return {256, 8, 4 << 20};
    int v[3];
    const hipDeviceAttribute_t attr[3] = {hipDeviceAttributeMultiprocessorCount, hipDeviceAttributeNumberOfXccs,
                                          hipDeviceAttributeL2CacheSize};
    const int fallback[3] = {256, 8, 4 << 20};
    for (int i = 0; i < 3; ++i) {
        v[i] = cache[dev][i].load(std::memory_order_relaxed);
        if (v[i] == 0) {
            if (hipDeviceGetAttribute(&v[i], attr[i], dev) != hipSuccess || v[i] <= 0) v[i] = fallback[i];
            cache[dev][i].store(v[i], std::memory_order_relaxed);
        }
    }
    return {v[0], v[1], v[2]};
}
int device_cus() { return device_shape().cus; }

// Form choice from the grid (measured on MI355X, 256 CUs, all forms on one
// box; blocks = regular-grid blocks, pairs = pair-grid blocks):
//  * split-KV (two 4-wave groups per M-tile, one block per CU, each group
//    walking half of the keys): when the regular grid cannot fill the GPU and
//    the M-tiles are long (seqlen_k >= 2048) — blocks <= CUs (+8-14% at
//    64-256 blocks with 4096 keys), and for causal grids, whose heaviest
//    M-tile is the critical path, below 1.5 blocks per CU (+16% at 384 = 1.5
//    per CU) or up to 2 per CU with seqlen_k >= 8192 (+6% at 512).  Elsewhere
//    it loses 2-17% to the regular form; with few key tiles the halves are
//    too short to pay for the merge (1024 keys: -2 to +1%; <= 512 keys: -4
//    to -20%, down to the two-block grid B1 H2 S128).
//  * pair (two adjacent M-tiles per 8-wave block, one block per CU): the two
//    blocks a CU holds in the regular form progress unevenly, so each CU's
//    last block runs alone; a pair block has no such tail, but pays a barrier
//    across 8 waves.  It wins when the pair blocks fill whole rounds of the
//    CUs: dense from seqlen_k >= 2048 (+1.3-5 % at 1-4 rounds, 2048-32768
//    keys; the dense B4 H16 S2048 benchmark grid +1.4-2.6 %); causal at
//    exactly two rounds from 8192 keys (+3.1-4.5 %, the causal B1 H16 S8192
//    benchmark grid +3.4-3.7 %: each CU gets one heavy and one light pair,
//    heaviest first), or at any whole number from 32768 (+1 % at four).
//    Causal at one round loses ~20 % (split-KV takes those grids), at three
//    4-5 %, at four up to 4096 keys 1-4 %; dense at 1024 keys -3.5 to +2.6 %;
//    any partial last round 8-17 %.
//  * regular: everything else.
int pick_variant(int64_t blocks, int64_t pairs, int causal, int seqlen_k, int64_t cus) {
    // blocks (up to ~2^63) is only compared, never multiplied; cus < 2^31
    if (seqlen_k >= 2048) {
        if (blocks <= cus) return FMHA_VARIANT_SPLITKV;
        if (causal && (blocks <= 3 * cus / 2 || (blocks <= 2 * cus && seqlen_k >= 8192))) return FMHA_VARIANT_SPLITKV;
    }
    const bool whole_rounds = pairs >= cus && pairs % cus == 0;
    if (!causal && whole_rounds && seqlen_k >= 2048) return FMHA_VARIANT_PAIR;
    if (causal && ((pairs == 2 * cus && seqlen_k >= 8192) || (whole_rounds && seqlen_k >= 32768)))
        return FMHA_VARIANT_PAIR;
    return FMHA_VARIANT_REGULAR;
}

// Causal dense grids of more than one batch run on the tile-major entries
// (grid (nhead_q, batch, tiles): every batch's heaviest M-tiles start first)
// instead of batch after batch, while the K/V one XCD serves stays within
// twice its L2 (MI355X: 4 MiB per XCD, 8 XCDs).  Heads go to the XCDs round
// robin, so an XCD serves batch x ceil(nhead_k / XCDs) x seqlen_k x 256 bytes
// of K/V.  Beyond that the interleaved batches push each sequence's K/V out
// of L2 before its later M-tiles run.  Measured on causal grids (regular
// form): +19% B8 H16 S1024, +8% B4 H16 S2048, +6% B16 H8 S2048, +2-6% B2 H16
// S4096/S8192, and -1 to -5% above 8 MiB.
bool use_tilemajor(const FmhaFwdParams* p, int batch, int causal) {
    if (!causal || batch < 2 || p->seqstart_q != nullptr) return false;
    const DeviceShape d = device_shape();
    // batch x heads-per-XCD x seqlen_k <= 2 x L2 / 256 B, evaluated without overflow
    const int64_t limit = 2 * (int64_t)d.l2_bytes / 256;
    const int64_t rows = (int64_t)batch * (((int64_t)p->nhead_k + d.xccs - 1) / d.xccs);  // <= 2^16 * 2^31
    return p->seqlen_k == 0 || (rows <= limit && rows * p->seqlen_k <= limit);
}

// Block order of causal launches.  Dense batches: the reference's (batch
// after batch) or the tile-major entries (use_tilemajor).  Varlen launches of
// at most 64 sequences in the regular form: the reference's order (sequence
// after sequence in the caller's order, the blocks past each short sequence's
// end dispatched between live ones) or one of the compact entries on the same
// grid, whose blocks take the live (sequence, M-tile) items in the level
// order (highest M-tile index first across all sequences) or the sequence
// order (longest sequence first, each heaviest M-tile first), the grid's
// ranks past the live items last.
enum Order : int { kOrderAuto = 0, kOrderReference = 1, kOrderTileMajor = 2, kOrderSequence = 3 };
constexpr int kOrderFlags = FMHA_VARIANT_REFERENCE_ORDER | FMHA_VARIANT_TILE_MAJOR_ORDER | FMHA_VARIANT_SEQUENCE_ORDER;
// the order a variant's flags ask for; -1 for more than one
int order_of(int variant) {
    const int f = variant & kOrderFlags;
    return f == 0                               ? kOrderAuto
           : f == FMHA_VARIANT_REFERENCE_ORDER  ? kOrderReference
           : f == FMHA_VARIANT_TILE_MAJOR_ORDER ? kOrderTileMajor
           : f == FMHA_VARIANT_SEQUENCE_ORDER   ? kOrderSequence
                                                : -1;
}
constexpr int kCompactMaxSeqs = 64;
bool compact_applies(const FmhaFwdParams* p, int batch, int causal) {
    return causal && p->seqstart_q != nullptr && batch >= 1 && batch <= kCompactMaxSeqs;
}
// The varlen order of a regular-form causal launch: kOrderReference,
// kOrderTileMajor (level order) or kOrderSequence.  Automatic: the sequence
// order for at most 8 sequences on a grid of at most 8 rounds of the resident
// blocks (2 per CU), else the reference's.  Each block of a compact entry
// finds its item in a loop over the sequences (~15 instructions each, in
// dead blocks too), which the short M-tiles of many-sequence launches do not
// repay.  Interleaved A/B in one process, H = nhead_q (reference order /
// level / sequence): cfg4's eight lengths at H4 -3.6 % / +15 %, H8 +16 % /
// +13 %, H16 -3.3 % / +2.2 %, H32 -15 % / -2.5 %; 16 lengths 100-4000 H8
// +2.6 % / +5.1 %, H16 -12 % / -2.3 %; 32 and 64 sequences of 16-2048 tokens
// H16 -17 to -29 % / -12 to -41 %; 16 x 512 H16 -1.1 % / -9.7 %.
int varlen_order(const FmhaFwdParams* p, int batch, int causal, int order) {
    if (!compact_applies(p, batch, causal) || order == kOrderReference) return kOrderReference;
    if (order != kOrderAuto) return order;
    const int64_t blocks = (int64_t)p->nhead_q * ((p->seqlen_q + kM0 - 1) / kM0) * batch;  // the grid: a bound
    return batch <= 8 && blocks <= 16 * (int64_t)device_cus() ? kOrderSequence : kOrderReference;
}
// Dense causal batches on the tile-major entries?
bool dense_tile_major(const FmhaFwdParams* p, int batch, int causal, int order) {
    if (order == kOrderReference || order == kOrderSequence) return false;
    if (order == kOrderTileMajor) return causal && batch >= 2 && p->seqstart_q == nullptr;
    return use_tilemajor(p, batch, causal);
}

// Keys up to which the automatic choice takes the short form: on every grid
// of two blocks' worth of query rows per compute unit, and causal on grids of
// eight.
constexpr int kShortKeys = 3 * FMHA_KN0, kShortKeysCausal = 6 * FMHA_KN0;

// blocks of the regular grid and of the pair grid
int64_t grid_blocks(const FmhaFwdParams* p, int batch) {
    return (int64_t)p->nhead_q * ((p->seqlen_q + kM0 - 1) / kM0) * batch;
}
int64_t pair_blocks(const FmhaFwdParams* p, int batch) {
    return (int64_t)p->nhead_q * (((p->seqlen_q + kM0 - 1) / kM0 + 1) / 2) * batch;
}

// The automatic form: the short form when its keys fit three tiles and the
// launch has at least two blocks' worth of query rows per compute unit, or,
// causal, up to 384 keys with at least eight; else the grid-shape rule above.
// For varlen launches seqlen_k and seqlen_q are the caller's bounds (the rows
// counted here are an upper bound); the short form reads each sequence's own
// lengths like the other forms, so the bounds steer the choice only.
// Kernel trace, H16, ~262,144 query rows, against the regular form: the
// short form is 12-29 % faster at 64-128 keys (dense S128 22.7 against 25.9
// us, causal S64 24.8 against 35.1 us); back to back, H16, 65,536-262,144 rows: 8-14 % faster dense at
// 160-192 keys, 3 % at 224, -6 to +1 % at 256-320, 2-8 % slower at 384;
// causal 12-21 % faster at 160-192 keys at every size, 7-11 % at 224-384
// keys from 262,144 rows, 1-9 % at 229,376-258,048 rows (7 x CUs x 128; it
// skips the key halves a wave cannot see) and -14 to +2 % below (S384 at
// 196,608 rows -7 %; S512-S640 -5 to -6 % at any size).  On smaller grids one
// block's latency sets the launch time and the regular form wins (B1 H2
// S128: 4.6 against 5.6 us).  Varlen batches of 256-2048 sequences of 16-192
// tokens, H16: 13-33 % faster.  Past a few key tiles the regular form's
// software pipeline (GEMM0 of the next tile beside the softmax of this one)
// catches up with the short form's four blocks per compute unit; causal
// grids keep the short form longer (their light M-tiles are short).
int pick_form(const FmhaFwdParams* p, int batch, int causal, int64_t cus) {
    const int64_t rows = (int64_t)batch * p->nhead_q * p->seqlen_q;
    if (p->seqlen_k <= kShortKeys && rows >= 2 * cus * kM0) return FMHA_VARIANT_SHORT;
    if (causal && p->seqlen_k <= kShortKeysCausal && rows >= 7 * cus * kM0) return FMHA_VARIANT_SHORT;
    return pick_variant(grid_blocks(p, batch), pair_blocks(p, batch), causal, p->seqlen_k, cus);
}

}  // namespace

namespace {

// Key tiles of causal M-tile mt (pipeline.hpp:168-193, as the kernel).
int causal_ntiles(const FmhaFwdParams* p, int mt) {
    const int sq = p->seqlen_q, sk = p->seqlen_k;
    const int last = std::min(mt * kM0 + kM0 - 1, sq - 1);
    const int e = last + (sk - sq) + 1;
    const int kv_end = e < 0 ? 0 : (e > sk ? sk : e);
    return (kv_end + kN0 - 1) / kN0;
}

// Plan of a balanced causal launch on `cus` compute units.  Work units are
// M-tiles (two resident blocks per CU) or, in pair mode, M-tile pairs (one
// 8-wave block per CU); the units whose key tiles exceed a fraction of the
// average work per resident block (half; pairs 0.7) are split into two key
// halves (so none outlasts the average much), and the items are ordered by
// work, heaviest first (longest processing time first; ties: later unit,
// first half).  In the automatic mode (over M-tiles) the plan is taken only
// where balanced_pays() says it measured faster.  Returns false when there is
// no plan (not causal dense, too many items for the table); fills `a` (table,
// split range in M-tiles, pair flag) when given.
//
// Modes: the automatic rule, or forced over single M-tiles
// (FMHA_VARIANT_BALANCED) or over M-tile pairs (FMHA_VARIANT_BALANCED_PAIR).
enum PlanMode : int { kPlanAuto = 0, kPlanSingle = 1, kPlanPair = 2 };
bool balanced_plan_build(const FmhaFwdParams* p, int batch, int causal, int64_t cus, int xccs, int mode,
                         FmhaBalancedArgs* a, int64_t* ws_bytes);

// The plan depends on the launch's shape only, so the last one built on a
// thread is kept: a serving loop relaunching one shape skips the sort (about
// 10 us of host time for cfg5's 531 items).
bool balanced_plan(const FmhaFwdParams* p, int batch, int causal, int64_t cus, int xccs, int mode,
                   FmhaBalancedArgs* a, int64_t* ws_bytes) {
    struct Key {
        int seqlen_q, seqlen_k, nhead_q, batch, causal, varlen, mode, xccs;
        int64_t cus;
        bool operator==(const Key& o) const {
            return seqlen_q == o.seqlen_q && seqlen_k == o.seqlen_k && nhead_q == o.nhead_q && batch == o.batch &&
                   causal == o.causal && varlen == o.varlen && mode == o.mode && xccs == o.xccs && cus == o.cus;
        }
    };
    thread_local Key last_key{-1, -1, -1, -1, -1, -1, -1, -1, -1};
    thread_local bool last_ok = false;
    thread_local int64_t last_bytes = 0;
    thread_local FmhaBalancedArgs last_plan;
    const Key key{p->seqlen_q, p->seqlen_k, p->nhead_q, batch, causal, p->seqstart_q != nullptr ? 1 : 0,
                  mode, xccs, cus};
    if (!(key == last_key)) {
        last_ok = balanced_plan_build(p, batch, causal, cus, xccs, mode, &last_plan, &last_bytes);
        last_key = key;
    }
    if (!last_ok) return false;
    if (ws_bytes) *ws_bytes = last_bytes;
    if (a) {
        a->split_from = last_plan.split_from;
        a->n_split = last_plan.n_split;
        a->n_items = last_plan.n_items;
        a->pair = last_plan.pair;
        std::copy(last_plan.item, last_plan.item + last_plan.n_items, a->item);
    }
    return true;
}

// Whether the automatic choice takes a balanced plan: where the balanced form
// measured faster than the launch without a workspace (split-KV or the
// regular form; all three on one box, causal, 256 CUs, blocks = regular-grid
// blocks, heaviest = key tiles of the last M-tile, avg = key tiles per
// resident block).  It pays for its second launch, the split M-tiles' extra
// prologues and the partials' traffic only when the M-tiles are long:
//  * at most one block per CU: heaviest >= 64 (+10-41 % at 4096-8192 keys),
//    or >= 32 at up to half a block per CU (+16 % B1 H8 S2048); shorter
//    M-tiles lose 15-50 % (B2-B16 H16 S256-S1024);
//  * up to 1.5 blocks per CU: heaviest >= 128 (+8.5 % B1 H5 S8192; 64:
//    -2.5 %);
//  * 1.5-2 blocks per CU: never (split-KV or regular are 1.4-7 % faster at
//    4096-32768 keys);
//  * more: a partial second round whose heaviest M-tile outlasts 1.5x the
//    average, with heaviest >= 128 (cfg5 B1 H2 S40000 +13 %; +0.5-15 % at
//    564-672 blocks with 8192-80000 keys; 64: -7 %; at 768 blocks, where the
//    heaviest is ~1.3x the average, -11 % to +0.7 %).
bool balanced_pays(int64_t blocks, int heaviest, double avg, int64_t cus) {
    if (heaviest <= avg) return false;  // the heaviest-first order balances already
    if (blocks <= cus) return heaviest >= 64 || (2 * blocks <= cus && heaviest >= 32);
    if (2 * blocks <= 3 * cus) return heaviest >= 128;
    if (blocks <= 2 * cus) return false;
    return heaviest >= 128 && heaviest > 1.5 * avg;
}

// Dispatch order of a plan's items (sorted heaviest first) that lets each
// XCD's L2 serve items reading the same keys.  Workgroup i of a launch runs
// on XCD i % xccs, and table entry z is block (h, b, z) of every (batch,
// head), linear id h + nhead_q * (b + batch * z); when hb = nhead_q * batch
// divides xccs into g = xccs / hb >= 2 groups, entry z runs on the XCDs of
// group z % g only.  Blocks are dispatched in order, one group after the
// other, so every run of g consecutive entries (one per group) must keep
// items of about equal work, or a group with busy slots holds back the
// dispatch of the others (a list schedule that gave each group its own run
// of heaviest items measured 20-29 % slower on B1 H1 S40000 and B1 H2
// S16384).  Within each such run the items are therefore only re-ordered by
// the first key tile they read (first halves and whole M-tiles, which start
// at key 0, to the lower groups; second halves, which start half-way, to the
// higher ones), so each group keeps taking items that start at the same key.
// Otherwise (hb not a divisor of xccs, or xccs <= 1) the order stays
// heaviest first.  Allocates nothing.
template <class Start>
void xcd_order(int n, int xccs, int64_t hb, Start start, int* order) {
    for (int i = 0; i < n; ++i) order[i] = i;
    if (xccs <= 1 || hb >= xccs || xccs % hb != 0) return;
    const int g = (int)(xccs / hb);
    for (int r = 0; r < n; r += g) {
        const int e = std::min(n, r + g);
        std::sort(order + r, order + e, [&](int x, int y) {
            const int sx = start(x), sy = start(y);
            return sx != sy ? sx < sy : x < y;
        });
    }
}

bool balanced_plan_build(const FmhaFwdParams* p, int batch, int causal, int64_t cus, int xccs, int mode,
                         FmhaBalancedArgs* a, int64_t* ws_bytes) {
    if (!causal || p->seqstart_q != nullptr || batch <= 0 || p->seqlen_q <= 0 || cus <= 0) return false;
    const int m_tiles = (p->seqlen_q + kM0 - 1) / kM0;
    if (m_tiles > FMHA_BALANCED_MAX_ITEMS) return false;
    double total = 0.0;
    for (int mt = 0; mt < m_tiles; ++mt) total += causal_ntiles(p, mt);
    total *= (double)p->nhead_q * batch;
    const int heaviest = causal_ntiles(p, m_tiles - 1);
    if (mode == kPlanAuto &&
        !balanced_pays((int64_t)m_tiles * p->nhead_q * batch, heaviest, total / (2.0 * (double)cus), cus))
        return false;
    // work units: M-tiles (two resident blocks per CU) or M-tile pairs (one
    // 8-wave block per CU), each unit's key tiles those of its last M-tile
    const bool pair = mode == kPlanPair;
    const int units = pair ? (m_tiles + 1) / 2 : m_tiles;
    auto work = [&](int u) { return causal_ntiles(p, pair ? std::min(2 * u + 1, m_tiles - 1) : u); };
    double unit_total = total;
    if (pair) {
        unit_total = 0.0;
        for (int u = 0; u < units; ++u) unit_total += work(u);
        unit_total *= (double)p->nhead_q * batch;
    }
    // key tiles per resident block (two per CU; a pair block alone on its CU)
    const double avg = unit_total / ((pair ? 1.0 : 2.0) * (double)cus);
    // units with more key tiles than this are split: half the average (pairs:
    // 0.7 of it; B1 H2 S40000 causal measured 0.6-0.7 best, 0.5 -4 %, 1.0 -25 %)
    const double limit = std::max(2.0, avg * (pair ? 0.7 : 0.5));
    int split_u = units;  // key tiles grow with the unit: the split ones are a suffix
    while (split_u > 0 && work(split_u - 1) > limit) --split_u;
    const int split_from = pair ? std::min(2 * split_u, m_tiles) : split_u;
    const int n_split = m_tiles - split_from;
    const int n_items = split_u + 2 * (units - split_u);
    if (n_items > FMHA_BALANCED_MAX_ITEMS) return false;
    if (ws_bytes) *ws_bytes = (int64_t)n_split * p->nhead_q * batch * 2 * FMHA_BALANCED_PART_BYTES;
    if (a) {
        // a fixed table and an in-place sort: the plan allocates nothing (the
        // allocation-free entry point runs it too); the order is total, so
        // std::sort needs no stability
        struct It {
            int w, u, half;
        };
        It items[FMHA_BALANCED_MAX_ITEMS];
        int n = 0;
        for (int u = 0; u < units; ++u) {
            const int kt = work(u);
            if (u < split_u) {
                items[n++] = {kt, u, 0};
            } else {
                items[n++] = {(kt + 1) / 2, u, 0};
                items[n++] = {kt / 2, u, 1};
            }
        }
        std::sort(items, items + n, [](const It& x, const It& y) {
            if (x.w != y.w) return x.w > y.w;
            if (x.u != y.u) return x.u > y.u;
            return x.half < y.half;
        });
        // the first key tile an item reads (a second half starts past the first)
        int order[FMHA_BALANCED_MAX_ITEMS];
        xcd_order(n, xccs, (int64_t)p->nhead_q * batch,
                  [&](int i) { return items[i].half ? (work(items[i].u) + 1) / 2 : 0; }, order);
        for (int i = 0; i < n_items; ++i)
            a->item[i] = (unsigned short)(items[order[i]].u | (items[order[i]].half << 15));
        a->split_from = split_from;
        a->n_split = n_split;
        a->n_items = n_items;
        a->pair = pair ? 1 : 0;
    }
    return true;
}

// The plan mode of a variant that takes a workspace, or -1 for the others.
int plan_mode(int v) {
    return v == FMHA_VARIANT_AUTO            ? kPlanAuto
           : v == FMHA_VARIANT_BALANCED      ? kPlanSingle
           : v == FMHA_VARIANT_BALANCED_PAIR ? kPlanPair
                                             : -1;
}

}  // namespace

extern "C" int fmha_fwd_d64_bf16_balanced_plan(const FmhaFwdParams* p, int batch, int causal, int compute_units,
                                               int xccs, int force, unsigned short* items, int capacity,
                                               int* split_from) {
    if (fmha_fwd_d64_bf16_check(p, batch, causal) != hipSuccess || compute_units < 0 || xccs < 0) return -1;
    if (force < kPlanAuto || force > kPlanPair) return -1;
    FmhaBalancedArgs a;
    if (!balanced_plan(p, batch, causal, compute_units > 0 ? compute_units : device_cus(),
                       xccs > 0 ? xccs : device_shape().xccs, force, &a, nullptr))
        return 0;
    if (items != nullptr)
        for (int i = 0; i < a.n_items && i < capacity; ++i) items[i] = a.item[i];
    if (split_from != nullptr) *split_from = a.split_from;
    return a.n_items;
}

extern "C" int64_t fmha_fwd_d64_bf16_workspace_size(const FmhaFwdParams* p, int batch, int causal, int variant) {
    if (fmha_fwd_d64_bf16_check(p, batch, causal) != hipSuccess) return -1;
    if (order_of(variant) < 0) return -1;
    const int mode = plan_mode(variant & ~kOrderFlags);
    if (mode < 0) return 0;
    int64_t bytes = 0;
    // the same plan (and cache entry) as the launch with this variant
    const int xccs = order_of(variant) == kOrderReference ? 1 : device_shape().xccs;
    if (!balanced_plan(p, batch, causal, device_cus(), xccs, mode, nullptr, &bytes)) return 0;
    return bytes;
}

extern "C" hipError_t fmha_fwd_d64_bf16_ws(const FmhaFwdParams* p, int batch, int causal, int variant,
                                           void* workspace, int64_t workspace_bytes, hipStream_t stream) {
    const hipError_t chk = fmha_fwd_d64_bf16_check(p, batch, causal);
    if (chk != hipSuccess) return chk;
    if (order_of(variant) < 0) return hipErrorInvalidValue;
    const int mode = plan_mode(variant & ~kOrderFlags);
    if (mode < 0) return fmha_fwd_d64_bf16_variant(p, batch, causal, variant, stream);
    if (workspace_bytes < 0 || (workspace == nullptr && workspace_bytes != 0) ||
        (reinterpret_cast<uintptr_t>(workspace) & 255u))
        return hipErrorInvalidValue;
    if (batch == 0 || p->seqlen_q == 0) return hipSuccess;
    FmhaBalancedArgs a;
    int64_t need = 0;
    // the reference-order flag keeps the plain heaviest-first table (the
    // results are the same bit for bit: the items do not change)
    const int xccs = order_of(variant) == kOrderReference ? 1 : device_shape().xccs;
    const bool plan = balanced_plan(p, batch, causal, device_cus(), xccs, mode, &a, &need);
    if (mode != kPlanAuto && (!plan || need > workspace_bytes)) return hipErrorInvalidValue;
    if (!plan || need > workspace_bytes) return fmha_fwd_d64_bf16_variant(p, batch, causal, variant, stream);
    a.p = *p;
    a.part = (float*)workspace;
    if (a.pair)
        hipLaunchKernelGGL(fmha_fwd_d64_bf16_balanced_pair_msk1, dim3(p->nhead_q, batch, a.n_items),
                           dim3(FMHA_SPLIT_KBLOCK), 0, stream, a);
    else
        hipLaunchKernelGGL(fmha_fwd_d64_bf16_balanced_msk1, dim3(p->nhead_q, batch, a.n_items), dim3(kBlockSize), 0,
                           stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.n_split == 0) return e;
    hipLaunchKernelGGL(fmha_fwd_d64_bf16_balanced_merge, dim3(p->nhead_q, a.n_split, batch), dim3(kBlockSize), 0,
                       stream, a);
    return hipGetLastError();
}

extern "C" int fmha_fwd_d64_bf16_pick_variant(const FmhaFwdParams* p, int batch, int causal, int compute_units) {
    if (fmha_fwd_d64_bf16_check(p, batch, causal) != hipSuccess || compute_units < 0) return -1;
    const int64_t cus = compute_units > 0 ? compute_units : device_cus();
    return pick_form(p, batch, causal, cus);
}

extern "C" int fmha_fwd_d64_bf16_tile_major(const FmhaFwdParams* p, int batch, int causal) {
    if (fmha_fwd_d64_bf16_check(p, batch, causal) != hipSuccess) return -1;
    if (p->seqlen_q == 0 || batch == 0) return 0;  // nothing is launched
    if (dense_tile_major(p, batch, causal, kOrderAuto)) return 1;
    // varlen: the compact orders, which only the regular form has
    if (pick_form(p, batch, causal, device_cus()) != FMHA_VARIANT_REGULAR) return 0;
    const int o = varlen_order(p, batch, causal, kOrderAuto);
    return o == kOrderTileMajor ? 1 : o == kOrderSequence ? 2 : 0;
}

extern "C" hipError_t fmha_fwd_d64_bf16_variant(const FmhaFwdParams* p, int batch, int causal, int variant,
                                                hipStream_t stream) {
    const hipError_t chk = fmha_fwd_d64_bf16_check(p, batch, causal);
    if (chk != hipSuccess) return chk;
    const int order = order_of(variant);
    if (order < 0) return hipErrorInvalidValue;  // more than one order flag
    const bool tile_major = dense_tile_major(p, batch, causal, order);
    variant &= ~kOrderFlags;
    // the balanced forms need fmha_fwd_d64_bf16_ws; 4 is a retired value
    if (!(variant == FMHA_VARIANT_AUTO || variant == FMHA_VARIANT_REGULAR || variant == FMHA_VARIANT_SPLITKV ||
          variant == FMHA_VARIANT_PAIR || variant == FMHA_VARIANT_SHORT || variant == FMHA_VARIANT_PAIR_STREAM))
        return hipErrorInvalidValue;
    const bool varlen = p->seqstart_q != nullptr;
    if (variant == FMHA_VARIANT_PAIR_STREAM && varlen) return hipErrorInvalidValue;  // dense layouts only
    if (batch == 0 || p->seqlen_q == 0) return hipSuccess;  // nothing to compute
    const int m_tiles = (p->seqlen_q + kM0 - 1) / kM0;
    const dim3 grid(p->nhead_q, m_tiles, batch);
    if (variant == FMHA_VARIANT_PAIR_STREAM) {
        // one block per compute unit over the pairs (dense), or one per pair
        // and its mirror (causal)
        const int64_t ny = (m_tiles + 1) / 2;
        const int64_t items = (int64_t)p->nhead_q * ny * batch;
        if (items >= INT32_MAX) return hipErrorInvalidValue;  // item numbers are ints
        const int64_t blocks = causal ? (int64_t)p->nhead_q * ((ny + 1) / 2) * batch
                                      : std::min<int64_t>(items, device_cus());
        FmhaStreamArgs a;
        a.p = *p;
        a.ny = (int)ny;
        a.n_items = (int)items;
        if (causal)
            hipLaunchKernelGGL(fmha_fwd_d64_bf16_pair_stream_msk1, dim3((unsigned)blocks), dim3(FMHA_SPLIT_KBLOCK), 0,
                               stream, a);
        else
            hipLaunchKernelGGL(fmha_fwd_d64_bf16_pair_stream_msk0, dim3((unsigned)blocks), dim3(FMHA_SPLIT_KBLOCK), 0,
                               stream, a);
        return hipGetLastError();
    }
    if (variant == FMHA_VARIANT_AUTO)
        variant = pick_form(p, batch, causal, device_cus());
    if (variant == FMHA_VARIANT_SHORT) {
        using Entry = void (*)(FmhaFwdParams);
        static const Entry entries[2][2] = {{fmha_fwd_d64_bf16_short_msk0, fmha_fwd_d64_bf16_short_msk0_varlen},
                                            {fmha_fwd_d64_bf16_short_msk1, fmha_fwd_d64_bf16_short_msk1_varlen}};
        hipLaunchKernelGGL(entries[causal ? 1 : 0][varlen ? 1 : 0], grid, dim3(kBlockSize), 0, stream, *p);
        return hipGetLastError();
    }
    if (tile_major) {  // causal, dense, batch > 1
        if (variant == FMHA_VARIANT_PAIR)
            hipLaunchKernelGGL(fmha_fwd_d64_bf16_pair_msk1_tilemajor, dim3(p->nhead_q, batch, (m_tiles + 1) / 2),
                               dim3(FMHA_SPLIT_KBLOCK), 0, stream, *p);
        else if (variant == FMHA_VARIANT_SPLITKV)
            hipLaunchKernelGGL(fmha_fwd_d64_bf16_splitkv_msk1_tilemajor, dim3(p->nhead_q, batch, m_tiles),
                               dim3(FMHA_SPLIT_KBLOCK), 0, stream, *p);
        else
            hipLaunchKernelGGL(fmha_fwd_d64_bf16_msk1_tilemajor, dim3(p->nhead_q, batch, m_tiles), dim3(kBlockSize),
                               0, stream, *p);
        return hipGetLastError();
    }
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
            switch (varlen_order(p, batch, causal, order)) {
                case kOrderTileMajor:
                    hipLaunchKernelGGL(fmha_fwd_d64_bf16_msk1_varlen_tilemajor, grid, block, 0, stream, *p);
                    break;
                case kOrderSequence:
                    hipLaunchKernelGGL(fmha_fwd_d64_bf16_msk1_varlen_seqmajor, grid, block, 0, stream, *p);
                    break;
                default:
                    hipLaunchKernelGGL(fmha_fwd_d64_bf16_msk1_varlen, grid, block, 0, stream, *p);
            }
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
