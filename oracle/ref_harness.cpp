// ref_harness.cpp — runs the REFERENCE's own checker on this build's kernel.
//
// TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Built by
// oracle/build_ref.sh into oracle/_ref/ref_verify from this file plus the
// reference's unmodified sources where they lie (src/runner/buffers.cpp,
// cpu_ref.cpp, gpu_ref.cpp); it links the product library only to launch it.
//
// Per invocation it follows the reference's end-to-end test
// (tests/test_fmha_fwd_d64.cpp:500-649) with this build's C-ABI launcher in
// place of the reference's kernel:
//   make_params normalisation (tests/test_params.hpp:31-61) -> FmhaBuffers ->
//   fill_random(seed) -> copy_to_device -> fmha_fwd_d64_bf16() ->
//   copy_from_device -> cpu_ref_verify() (timed) -> [LSE vs gpu_ref_fmha_fwd()]
// and prints one line "REF_VERIFY {json}" with the reference's verdict and
// statistics, the LSE comparison (|d| <= 1e-3, -inf pairs equal) and the wall
// time of cpu_ref_verify with its OpenMP thread count.
//
//   ref_verify -b B -h H [--kv-heads K] -s S [--kv-seq SK] [--mask 0|1]
//              [--lse 0|1] [--varlen-seqs a,b,...] [--seed N]
//              [--dump-inputs PATH]   also write h_Q, h_K, h_V as filled by the
//                                     reference's fill_random (raw uint16, in
//                                     that order) to PATH
//   ref_verify --stdin      one case per input line, same flags, one
//                           REF_VERIFY line per case (one process, one HIP init)
#include <omp.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "fmha_fwd.h"
#include "runner/buffers.hpp"
#include "runner/cpu_ref.hpp"
#include "runner/fmha_params.hpp"
#include "runner/gpu_ref.hpp"

static void die(const char* what, hipError_t e) {
    fprintf(stderr, "ref_verify: %s: %s\n", what, hipGetErrorString(e));
    exit(2);
}

static int run_case(const std::vector<std::string>& args) {
    int b = 1, h = 2, kvh = 0, s = 128, kvs = 0, mask = 0, lse = 0;
    unsigned seed = 42;
    std::string dump_path;
    std::vector<int> seqs;
    for (size_t i = 0; i < args.size(); ++i) {
        const std::string& a = args[i];
        const char* v = i + 1 < args.size() ? args[i + 1].c_str() : nullptr;
        if (!v) { fprintf(stderr, "ref_verify: %s needs a value\n", a.c_str()); return 2; }
        if (a == "-b") b = atoi(v);
        else if (a == "-h") h = atoi(v);
        else if (a == "--kv-heads") kvh = atoi(v);
        else if (a == "-s") s = atoi(v);
        else if (a == "--kv-seq") kvs = atoi(v);
        else if (a == "--mask") mask = atoi(v);
        else if (a == "--lse") lse = atoi(v);
        else if (a == "--seed") seed = (unsigned)strtoul(v, nullptr, 10);
        else if (a == "--dump-inputs") dump_path = v;
        else if (a == "--varlen-seqs") {
            for (const char* p = v; *p;) {
                seqs.push_back(atoi(p));
                while (*p && *p != ',') ++p;
                if (*p) ++p;
            }
        } else { fprintf(stderr, "ref_verify: unknown flag %s\n", a.c_str()); return 2; }
        ++i;
    }

    // the reference test's normalisation of a config row
    FmhaParams p;
    p.batch = b; p.q_heads = h; p.kv_heads = kvh ? kvh : h; p.gqa = 1;
    p.seq_len = s; p.kv_seq_len = kvs; p.head_dim = 64; p.hdim_padded = 64;
    p.mask = mask; p.lse = lse; p.varlen_seqs = seqs;
    if (p.q_heads != p.kv_heads) p.gqa = p.q_heads / p.kv_heads;
    if (!seqs.empty()) {
        p.batch = (int)seqs.size();
        int mx = 0;
        for (int x : seqs) mx = x > mx ? x : mx;
        p.seq_len = mx;
        if (p.kv_seq_len == 0) p.kv_seq_len = mx;
    }
    if (p.kv_seq_len == 0) p.kv_seq_len = p.seq_len;
    const bool varlen = !seqs.empty();

    FmhaBuffers bufs(p);
    bufs.fill_random(seed);
    if (!dump_path.empty()) {
        FILE* f = fopen(dump_path.c_str(), "wb");
        if (!f) { fprintf(stderr, "ref_verify: cannot write %s\n", dump_path.c_str()); return 2; }
        const std::vector<uint16_t>* parts[3] = {&bufs.h_Q, &bufs.h_K, &bufs.h_V};
        for (const auto* a : parts)
            if (fwrite(a->data(), 2, a->size(), f) != a->size()) { fclose(f); return 2; }
        fclose(f);
        printf("REF_INPUTS {\"q\": %zu, \"k\": %zu, \"v\": %zu}\n", bufs.h_Q.size(), bufs.h_K.size(),
               bufs.h_V.size());
    }
    bufs.copy_to_device();

    float* d_lse_kern = nullptr;
    hipError_t e;
    if (lse) {
        if ((e = hipMalloc(&d_lse_kern, bufs.sz_LSE * sizeof(float))) != hipSuccess) die("hipMalloc", e);
        if ((e = hipMemset(d_lse_kern, 0, bufs.sz_LSE * sizeof(float))) != hipSuccess) die("hipMemset", e);
    }

    // this build's kernarg for the reference's buffers (BHSD dense, or the
    // packed [H][T][D] varlen layout with the reference's offset tables)
    const int D = 64;
    FmhaFwdParams kp;
    memset(&kp, 0, sizeof kp);
    kp.q = (const fmha_bf16_t*)bufs.d_Q;
    kp.k = (const fmha_bf16_t*)bufs.d_K;
    kp.v = (const fmha_bf16_t*)bufs.d_V;
    kp.o = (fmha_bf16_t*)bufs.d_O;
    kp.lse = d_lse_kern;
    kp.seqlen_q = p.seq_len;
    kp.seqlen_k = p.kv_seq_len;
    kp.nhead_q = p.q_heads;
    kp.nhead_k = p.kv_heads;
    kp.scale = 1.4426950408889634f / sqrtf(64.0f);
    kp.stride_q = kp.stride_k = kp.stride_v = kp.stride_o = D;
    if (varlen) {
        const int hs = (int)bufs.total_seqlen * D;
        kp.nhead_stride_q = kp.nhead_stride_k = kp.nhead_stride_v = kp.nhead_stride_o = hs;
        kp.seqstart_q = (const int32_t*)bufs.d_qseq;
        kp.seqstart_k = (const int32_t*)bufs.d_kseq;
    } else {
        kp.nhead_stride_q = kp.nhead_stride_o = p.seq_len * D;
        kp.nhead_stride_k = kp.nhead_stride_v = p.kv_seq_len * D;
        kp.batch_stride_q = kp.batch_stride_o = p.q_heads * p.seq_len * D;
        kp.batch_stride_k = kp.batch_stride_v = p.kv_heads * p.kv_seq_len * D;
    }
    if ((e = fmha_fwd_d64_bf16(&kp, p.batch, p.mask, nullptr)) != hipSuccess) die("fmha_fwd_d64_bf16", e);
    if ((e = hipDeviceSynchronize()) != hipSuccess) die("kernel", e);
    bufs.copy_from_device();

    const auto t0 = std::chrono::steady_clock::now();
    const CpuRefResult r = cpu_ref_verify(p, bufs);
    const double secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();

    int lse_bad = -1;
    double lse_max = 0.0;
    if (lse) {
        GpuRefParams g;
        memset(&g, 0, sizeof g);
        g.d_Q = (const uint16_t*)bufs.d_Q;
        g.d_K = (const uint16_t*)bufs.d_K;
        g.d_V = (const uint16_t*)bufs.d_V;
        g.d_O = (uint16_t*)bufs.d_O;
        g.d_LSE = (float*)bufs.d_LSE;
        g.batch = p.batch; g.q_heads = p.q_heads; g.kv_heads = p.kv_heads; g.gqa = p.gqa;
        g.seq_len = p.seq_len; g.kv_seq_len = p.kv_seq_len; g.head_dim = p.head_dim;
        g.stride_q_seq = g.stride_k_seq = g.stride_v_seq = g.stride_o_seq = D;
        g.stride_q_head = g.stride_o_head = (int)(bufs.stride_q_head / 2);
        g.stride_q_batch = g.stride_o_batch = (int)(bufs.stride_q_batch / 2);
        g.stride_k_head = g.stride_v_head = (int)(bufs.stride_k_head / 2);
        g.stride_k_batch = g.stride_v_batch = (int)(bufs.stride_k_batch / 2);
        g.mask = p.mask != 0;
        g.scalar = p.scalar();
        g.d_seqstart_q = varlen ? (const uint32_t*)bufs.d_qseq : nullptr;
        g.d_seqstart_k = varlen ? (const uint32_t*)bufs.d_kseq : nullptr;
        gpu_ref_fmha_fwd(g);
        if ((e = hipDeviceSynchronize()) != hipSuccess) die("gpu_ref", e);
        std::vector<float> lk(bufs.sz_LSE), lr(bufs.sz_LSE);
        if ((e = hipMemcpy(lk.data(), d_lse_kern, lk.size() * 4, hipMemcpyDeviceToHost)) != hipSuccess) die("copy", e);
        if ((e = hipMemcpy(lr.data(), bufs.d_LSE, lr.size() * 4, hipMemcpyDeviceToHost)) != hipSuccess) die("copy", e);
        lse_bad = 0;
        for (size_t i = 0; i < lk.size(); ++i) {
            if (std::isinf(lk[i]) && std::isinf(lr[i]) && lk[i] < 0 && lr[i] < 0) continue;
            const double d = std::fabs((double)lk[i] - (double)lr[i]);
            if (!(d <= 1e-3)) ++lse_bad;
            if (d > lse_max || std::isnan(d)) lse_max = std::isnan(d) || std::isinf(d) ? 1e30 : d;
        }
        (void)hipFree(d_lse_kern);
    }

    auto fin = [](double x) { return std::isfinite(x) ? x : 1e30; };  // JSON has no inf/nan
    printf("REF_VERIFY {\"pass\": %s, \"max_abs\": %.9g, \"max_rel\": %.9g, \"min_cos\": %.12g, "
           "\"mismatch\": %zu, \"nonfinite\": %zu, \"cos_fail\": %zu, \"total\": %zu, "
           "\"lse_mismatch\": %d, \"lse_max_abs\": %.9g, \"cpu_ref_seconds\": %.6f, \"threads\": %d}\n",
           r.pass ? "true" : "false", fin(r.max_abs), fin(r.max_rel), fin(r.min_cos), r.mismatch, r.nonfinite, r.cos_fail,
           r.total_elems, lse_bad, lse_max, secs, omp_get_max_threads());
    fflush(stdout);
    return 0;
}

int main(int argc, char** argv) {
    if (argc == 2 && std::string(argv[1]) == "--stdin") {
        char line[4096];
        while (fgets(line, sizeof line, stdin)) {
            std::vector<std::string> args;
            for (char* tok = strtok(line, " \t\r\n"); tok; tok = strtok(nullptr, " \t\r\n")) args.emplace_back(tok);
            if (args.empty()) continue;
            const int rc = run_case(args);
            if (rc != 0) return rc;
        }
        return 0;
    }
    return run_case(std::vector<std::string>(argv + 1, argv + argc));
}
