// fmha_internal.h — declarations shared by the kernel and launcher sources
// (not part of the C-ABI in include/).
#pragma once
#include <hip/hip_runtime.h>

#include "fmha_fwd.h"

// Persistent form: queue layout of one launch slot (see fmha_fwd_kernel.hip).
#define FMHA_PERSIST_QUEUES 8         // one queue per XCD
#define FMHA_PERSIST_QUEUE_STRIDE 32  // ints between counters (one 128-byte line each)
#define FMHA_PERSIST_QUEUE_SLOTS 64   // launch slots (launches in flight per device)

// Kernarg of the persistent entries.
struct FmhaPersistArgs {
    FmhaFwdParams p;
    int* queue;      // this launch's slot: FMHA_PERSIST_QUEUES queue heads, then a blocks-done counter
    int batch;
    int m_tiles;     // M-tiles per (batch, head)
    int n_items;     // batch * nhead_q * m_tiles
    int tile_major;  // causal: items ordered (head, batch, M-tile) instead of (head, M-tile, batch)
};

__global__ void fmha_fwd_d64_bf16_persist_msk0(FmhaPersistArgs args);
__global__ void fmha_fwd_d64_bf16_persist_msk1(FmhaPersistArgs args);

// Device address of launch slot `slot` (taken modulo FMHA_PERSIST_QUEUE_SLOTS)
// of the current device's queue counters; null if the symbol lookup fails.
extern "C" int* fmha_persist_queue_slot(unsigned slot);

// Balanced causal form (see fmha_fwd_kernel.hip): the item table of a launch
// and its workspace of partial results.
#define FMHA_BALANCED_MAX_ITEMS 1920                       // items per (batch, head): 3,840 bytes of table
#define FMHA_BALANCED_PART_BYTES (4 * 34 * 64 * 4)         // one partial result: 4 waves x 34 floats x 64 lanes

struct FmhaBalancedArgs {
    FmhaFwdParams p;
    float* part;     // workspace: 2 partial results per split M-tile of every (batch, head)
    int split_from;  // M-tiles >= split_from are split in two key halves
    int n_split;     // split M-tiles per (batch, head): m_tiles - split_from
    int n_items;     // items per (batch, head) (the grid's z)
    int pair;        // items are M-tile pairs (the pair entry, FMHA_SPLIT_KBLOCK threads)
    unsigned short item[FMHA_BALANCED_MAX_ITEMS];  // dispatch order: M-tile (pair) | half << 15
};

__global__ void fmha_fwd_d64_bf16_balanced_msk1(FmhaBalancedArgs args);
__global__ void fmha_fwd_d64_bf16_balanced_pair_msk1(FmhaBalancedArgs args);
__global__ void fmha_fwd_d64_bf16_balanced_merge(FmhaBalancedArgs args);
