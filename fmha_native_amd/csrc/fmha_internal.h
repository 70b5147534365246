// fmha_internal.h — declarations shared by the kernel and launcher sources
// (not part of the C-ABI in include/).
#pragma once
#include <hip/hip_runtime.h>

#include "fmha_fwd.h"

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

// Pair stream form (see fmha_fwd_kernel.hip): one 8-wave pair block per
// compute unit looping over a static list of M-tile pairs.
struct FmhaStreamArgs {
    FmhaFwdParams p;
    int ny;       // pairs per (batch, head): ceil(ceil(seqlen_q / kM0) / 2)
    int n_items;  // pairs of the launch: nhead_q * ny * batch
};
__global__ void fmha_fwd_d64_bf16_pair_stream_msk0(FmhaStreamArgs args);
__global__ void fmha_fwd_d64_bf16_pair_stream_msk1(FmhaStreamArgs args);
