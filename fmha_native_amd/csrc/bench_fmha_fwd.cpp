// bench_fmha_fwd — timing CLI for the gfx950 D64 BF16 FMHA forward.
//
// Same flags and the same three result lines as the reference's CLI
// (src/bench_fmha_fwd.cpp:43-117 and :231-233), so its sweep script can parse
// this one unchanged:
//   -b/--batch -h/--heads --kv-heads -s/--seq -d/--hdim --mask --lse
//   --varlen-seqs a,b,c --warmup --iters --help
// Additions (new flags only; the three result lines are untouched):
//   --seed N            input seed (reference: fixed 42)
//   --dist ref|normal   reference +-0.1 generator (default) or N(0,1)
//   --scale-inputs X    multiply N(0,1) inputs by X
//   --kv-seq N          key length (reference: always = seq)
//   --variant auto|regular|splitkv|pair|balanced|balanced_pair|short|pair_stream   kernel form (default: the launcher's choice)
//   --workspace 0|1  give the launcher a workspace (fmha_fwd_d64_bf16_ws, allocated before timing), so the
//                    automatic choice may be the balanced causal form (default 1); --variant balanced needs it
//   --order auto|reference|tilemajor|sequence   causal block order (reference: batch after batch)
// It launches through the C-ABI launcher and reports its error code instead
// of exiting silently on a bad launch.

#include <getopt.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "fmha_fwd.h"
#include "fmha_runner.h"

#define HIP_CHECK(expr)                                                                                   \
    do {                                                                                                  \
        hipError_t e_ = (expr);                                                                           \
        if (e_ != hipSuccess) {                                                                           \
            fprintf(stderr, "HIP error %d (%s) at %s:%d\n", (int)e_, hipGetErrorString(e_), __FILE__, \
                    __LINE__);                                                                            \
            exit(1);                                                                                      \
        }                                                                                                 \
    } while (0)

struct Config {
    int batch = 2, q_heads = 16, kv_heads = 0, seq_len = 4096, kv_seq_len = 0, head_dim = 64;
    int mask = 0, lse = 0, warmup = 5, iters = 20;
    unsigned seed = 42;
    std::string dist = "ref";
    int variant = FMHA_VARIANT_AUTO;
    int order_flag = 0;  // one of the FMHA_VARIANT_*_ORDER flags, or 0
    bool workspace = true;
    float scale_inputs = 1.0f;
    std::vector<int> varlen_seqs;
};

static void usage(const char* prog) {
    printf("Usage: %s [options]\n"
           "  -b  --batch N    Batch size [2]\n"
           "  -h  --heads N    Q head count [16]\n"
           "  --kv-heads N     KV head count [0 = q_heads]\n"
           "  -s  --seq N      Sequence length [4096]\n"
           "  --kv-seq N       Key/value length [0 = seq]\n"
           "  -d  --hdim N     Head dimension [64] (only 64 is supported)\n"
           "  --mask N         Causal mask 0|1 [0]\n"
           "  --lse N          LSE output enable [0]\n"
           "  --varlen-seqs L  Per-batch seq lengths (comma-separated)\n"
           "  --warmup N       Warmup iterations [5]\n"
           "  --iters N        Benchmark iterations [20]\n"
           "  --seed N         Input seed [42]\n"
           "  --dist ref|normal  Input distribution [ref]\n"
           "  --scale-inputs X Multiplier for normal inputs [1]\n"
           "  --variant V      auto|regular|splitkv|pair|balanced|balanced_pair|short|pair_stream form [auto]\n"
           "  --workspace 0|1  launch with a workspace (the balanced causal form may run) [1]\n"
           "  --order O        auto|reference|tilemajor|sequence causal block order [auto]\n",
           prog);
}

static Config parse(int argc, char** argv) {
    Config c;
    static struct option opts[] = {{"varlen-seqs", required_argument, 0, 6},
                                   {"batch", required_argument, 0, 'b'},
                                   {"heads", required_argument, 0, 'h'},
                                   {"kv-heads", required_argument, 0, 1},
                                   {"seq", required_argument, 0, 's'},
                                   {"kv-seq", required_argument, 0, 2},
                                   {"hdim", required_argument, 0, 'd'},
                                   {"mask", required_argument, 0, 'm'},
                                   {"lse", required_argument, 0, 'l'},
                                   {"warmup", required_argument, 0, 'w'},
                                   {"iters", required_argument, 0, 'i'},
                                   {"seed", required_argument, 0, 3},
                                   {"dist", required_argument, 0, 4},
                                   {"scale-inputs", required_argument, 0, 5},
                                   {"variant", required_argument, 0, 7},
                                   {"workspace", required_argument, 0, 9},
                                   {"order", required_argument, 0, 8},
                                   {"help", no_argument, 0, 0},
                                   {0, 0, 0, 0}};
    int ch, idx;
    while ((ch = getopt_long(argc, argv, "b:h:s:d:m:l:w:i:", opts, &idx)) != -1) {
        switch (ch) {
            case 6: {
                const char* s = optarg;
                while (*s) {
                    c.varlen_seqs.push_back(atoi(s));
                    while (*s && *s != ',') s++;
                    if (*s) s++;
                }
                break;
            }
            case 'b': c.batch = atoi(optarg); break;
            case 'h': c.q_heads = atoi(optarg); break;
            case 1: c.kv_heads = atoi(optarg); break;
            case 's': c.seq_len = atoi(optarg); break;
            case 2: c.kv_seq_len = atoi(optarg); break;
            case 'd': c.head_dim = atoi(optarg); break;
            case 'm': c.mask = atoi(optarg); break;
            case 'l': c.lse = atoi(optarg); break;
            case 'w': c.warmup = atoi(optarg); break;
            case 'i': c.iters = atoi(optarg); break;
            case 3: c.seed = (unsigned)strtoul(optarg, nullptr, 10); break;
            case 4: c.dist = optarg; break;
            case 5: c.scale_inputs = (float)atof(optarg); break;
            case 7:
                if (!strcmp(optarg, "auto")) c.variant = FMHA_VARIANT_AUTO;
                else if (!strcmp(optarg, "regular")) c.variant = FMHA_VARIANT_REGULAR;
                else if (!strcmp(optarg, "splitkv")) c.variant = FMHA_VARIANT_SPLITKV;
                else if (!strcmp(optarg, "pair")) c.variant = FMHA_VARIANT_PAIR;
                else if (!strcmp(optarg, "balanced")) c.variant = FMHA_VARIANT_BALANCED;
                else if (!strcmp(optarg, "balanced_pair")) c.variant = FMHA_VARIANT_BALANCED_PAIR;
                else if (!strcmp(optarg, "short")) c.variant = FMHA_VARIANT_SHORT;
                else if (!strcmp(optarg, "pair_stream")) c.variant = FMHA_VARIANT_PAIR_STREAM;
                else {
                    fprintf(stderr, "Error: --variant must be auto, regular, splitkv, pair, balanced, balanced_pair, short or pair_stream\n");
                    exit(1);
                }
                break;
            case 8:
                if (!strcmp(optarg, "auto")) c.order_flag = 0;
                else if (!strcmp(optarg, "reference")) c.order_flag = FMHA_VARIANT_REFERENCE_ORDER;
                else if (!strcmp(optarg, "tilemajor")) c.order_flag = FMHA_VARIANT_TILE_MAJOR_ORDER;
                else if (!strcmp(optarg, "sequence")) c.order_flag = FMHA_VARIANT_SEQUENCE_ORDER;
                else { fprintf(stderr, "Error: --order must be auto, reference, tilemajor or sequence\n"); exit(1); }
                break;
            case 9: c.workspace = atoi(optarg) != 0; break;
            case 0: usage(argv[0]); exit(0);
            default: usage(argv[0]); exit(1);
        }
    }
    if (c.kv_heads == 0) c.kv_heads = c.q_heads;
    if (c.q_heads <= 0 || c.kv_heads <= 0 || c.q_heads % c.kv_heads != 0) {
        fprintf(stderr, "Error: q_heads (%d) must be divisible by kv_heads (%d)\n", c.q_heads, c.kv_heads);
        exit(1);
    }
    if (c.head_dim != 64) {
        fprintf(stderr, "Error: only --hdim 64 is supported (got %d)\n", c.head_dim);
        exit(1);
    }
    if (c.dist != "ref" && c.dist != "normal") {
        fprintf(stderr, "Error: --dist must be ref or normal\n");
        exit(1);
    }
    if (!c.varlen_seqs.empty()) {
        c.batch = (int)c.varlen_seqs.size();
        int mx = 0;
        for (int s : c.varlen_seqs) mx = s > mx ? s : mx;
        c.seq_len = mx;
        c.kv_seq_len = mx;
    }
    if (c.kv_seq_len == 0) c.kv_seq_len = c.seq_len;
    return c;
}

int main(int argc, char** argv) {
    const Config c = parse(argc, argv);
    const int D = 64;
    const bool varlen = !c.varlen_seqs.empty();
    long long total = 0;
    for (int s : c.varlen_seqs) total += s;

    const size_t nq = varlen ? (size_t)c.q_heads * total * D : (size_t)c.batch * c.q_heads * c.seq_len * D;
    const size_t nk = varlen ? (size_t)c.kv_heads * total * D : (size_t)c.batch * c.kv_heads * c.kv_seq_len * D;
    const size_t nlse = nq / D;
    std::vector<uint16_t> hq(nq), hk(nk), hv(nk);
    if (c.dist == "ref") {
        fmha_runner_fill_ref(c.seed, hq.data(), nq, hk.data(), nk, hv.data(), nk);
    } else {
        fmha_runner_fill_normal(c.seed, c.scale_inputs, hq.data(), nq);
        fmha_runner_fill_normal(c.seed + 1, c.scale_inputs, hk.data(), nk);
        fmha_runner_fill_normal(c.seed + 2, c.scale_inputs, hv.data(), nk);
    }

    void *dq, *dk, *dv, *dout, *dlse = nullptr;
    int32_t* dseq = nullptr;
    HIP_CHECK(hipMalloc(&dq, nq * 2));
    HIP_CHECK(hipMalloc(&dk, nk * 2));
    HIP_CHECK(hipMalloc(&dv, nk * 2));
    HIP_CHECK(hipMalloc(&dout, nq * 2));
    if (c.lse) HIP_CHECK(hipMalloc(&dlse, nlse * 4));
    HIP_CHECK(hipMemcpy(dq, hq.data(), nq * 2, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(dk, hk.data(), nk * 2, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemcpy(dv, hv.data(), nk * 2, hipMemcpyHostToDevice));
    HIP_CHECK(hipMemset(dout, 0, nq * 2));

    FmhaFwdParams p;
    memset(&p, 0, sizeof(p));
    p.q = (const fmha_bf16_t*)dq;
    p.k = (const fmha_bf16_t*)dk;
    p.v = (const fmha_bf16_t*)dv;
    p.o = (fmha_bf16_t*)dout;
    p.lse = (float*)dlse;
    p.seqlen_q = c.seq_len;
    p.seqlen_k = c.kv_seq_len;
    p.nhead_q = c.q_heads;
    p.nhead_k = c.kv_heads;
    p.scale = 1.4426950408889634f / sqrtf((float)D);
    p.stride_q = p.stride_k = p.stride_v = p.stride_o = D;
    if (varlen) {
        std::vector<int32_t> starts(c.batch + 1, 0);
        for (int i = 0; i < c.batch; i++) starts[i + 1] = starts[i] + c.varlen_seqs[i];
        HIP_CHECK(hipMalloc(&dseq, (c.batch + 1) * 4));
        HIP_CHECK(hipMemcpy(dseq, starts.data(), (c.batch + 1) * 4, hipMemcpyHostToDevice));
        p.nhead_stride_q = p.nhead_stride_o = (int)(total * D);
        p.nhead_stride_k = p.nhead_stride_v = (int)(total * D);
        p.seqstart_q = p.seqstart_k = dseq;
    } else {
        p.nhead_stride_q = p.nhead_stride_o = c.seq_len * D;
        p.nhead_stride_k = p.nhead_stride_v = c.kv_seq_len * D;
        p.batch_stride_q = p.batch_stride_o = c.q_heads * c.seq_len * D;
        p.batch_stride_k = p.batch_stride_v = c.kv_heads * c.kv_seq_len * D;
    }

    const int variant = c.variant | c.order_flag;
    void* dws = nullptr;
    int64_t ws_bytes = 0;
    const bool use_ws = c.workspace || c.variant == FMHA_VARIANT_BALANCED || c.variant == FMHA_VARIANT_BALANCED_PAIR;
    if (use_ws) {
        ws_bytes = fmha_fwd_d64_bf16_workspace_size(&p, c.batch, c.mask, variant);
        if (ws_bytes < 0) {
            fprintf(stderr, "fmha_fwd_d64_bf16_workspace_size rejected the arguments\n");
            exit(1);
        }
        if (ws_bytes > 0) HIP_CHECK(hipMalloc(&dws, (size_t)ws_bytes));
    }
    auto launch = [&]() {
        hipError_t e = use_ws ? fmha_fwd_d64_bf16_ws(&p, c.batch, c.mask, variant, dws, ws_bytes, nullptr)
                              : fmha_fwd_d64_bf16_variant(&p, c.batch, c.mask, variant, nullptr);
        if (e != hipSuccess) {
            fprintf(stderr, "fmha_fwd_d64_bf16 failed: %d (%s)\n", (int)e, hipGetErrorString(e));
            exit(1);
        }
    };
    for (int i = 0; i < c.warmup; i++) launch();
    HIP_CHECK(hipDeviceSynchronize());

    hipEvent_t e0, e1;
    HIP_CHECK(hipEventCreate(&e0));
    HIP_CHECK(hipEventCreate(&e1));
    std::vector<float> times(c.iters > 0 ? c.iters : 1, 0.0f);
    for (int i = 0; i < c.iters; i++) {
        HIP_CHECK(hipEventRecord(e0));
        launch();
        HIP_CHECK(hipEventRecord(e1));
        HIP_CHECK(hipEventSynchronize(e1));
        HIP_CHECK(hipEventElapsedTime(&times[i], e0, e1));
    }
    // back-to-back average (launch overhead amortised), reported on an extra line
    float b2b = 0.0f;
    if (c.iters > 0) {
        HIP_CHECK(hipEventRecord(e0));
        for (int i = 0; i < c.iters; i++) launch();
        HIP_CHECK(hipEventRecord(e1));
        HIP_CHECK(hipEventSynchronize(e1));
        HIP_CHECK(hipEventElapsedTime(&b2b, e0, e1));
        b2b /= c.iters;
    }
    float tmin = times[0], tsum = 0.0f;
    for (int i = 0; i < c.iters; i++) {
        tsum += times[i];
        if (times[i] < tmin) tmin = times[i];
    }
    const float tavg = c.iters > 0 ? tsum / c.iters : 0.0f;
    // FLOP convention of the reference (src/bench_fmha_fwd.cpp:225-226)
    double flops = 4.0 * c.batch * c.q_heads * (double)c.seq_len * c.kv_seq_len * D;
    if (c.mask) flops *= 0.5;
    printf("Avg: %.3f ms\n", tavg);
    printf("min=%.3f ms\n", tmin);
    printf("TFLOPS: %.2f\n", flops / (tavg * 1e-3) / 1e12);
    printf("back-to-back avg: %.3f ms (%.2f TFLOPS)\n", b2b, b2b > 0 ? flops / (b2b * 1e-3) / 1e12 : 0.0);

    (void)hipFree(dq);
    (void)hipFree(dk);
    (void)hipFree(dv);
    (void)hipFree(dout);
    if (dlse) (void)hipFree(dlse);
    if (dseq) (void)hipFree(dseq);
    if (dws) (void)hipFree(dws);
    return 0;
}
