"""Benchmark of the gfx950 D64 BF16 FMHA forward (one JSON line on stdout).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Metric: forward TFLOP/s (repo FLOP convention 4*B*H*Sq*Sk*D, x0.5 when
causal; reference src/bench_fmha_fwd.cpp:225-226) and its fraction of the
MI355X dense BF16 MFMA peak (2516.6 TFLOP/s).  ``value`` is measured on the
dense B4 H16 S2048 configuration; the causal B1 H16 S8192 (+LSE)
configuration is reported under ``also``.  A step is one launch of the
forward over the whole batch with Q/K/V already resident in HBM (through
fmha_fwd_d64_bf16_ws with a workspace allocated before timing, so the
launcher's automatic choice may take the balanced causal form: then a step is
its two launches), timed back to back between two HIP events on the launch
stream with synchronisations before and after, once 0.1 s of untimed
launches has brought the clock up from idle and the W warm-up steps have run;
the reference's per-launch event protocol is reported beside it
(``reference_protocol``).  Inputs are synthetic
N(0,1) bf16 (seed 42).

``roofline`` carries this run's achieved TFLOP/s and, from the committed
rocprofv3 run of the same kernel (profiles/), its HBM traffic, MFMA busy
fraction and clock.

The CPU baseline is the reference's own CPU path, cpu_ref_verify, compiled
from its sources into oracle/_ref/ref_verify and timed on this host for all
five benchmark configurations ("kind": "reference"): cfg1, cfg2 and cfg4 over
the whole workload, cfg3 over 4 of its 16 heads and cfg5 over the last 4000
of its 40000 query rows of one head, each scaled to its workload (the whole
of cfg3 and cfg5 would take its loop minutes on one thread).  Where that
harness was not built, the faithful C restatement (oracle/) on a bounded row
sample ("kind": "port").  Only this leg touches oracle/.
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.6  # 256 CU x 2.4 GHz x 4096 dense BF16 FLOP/clk/CU
HBM_PEAK_GBS = 8000.0


def _problems():
    from fmha_native_amd.problem import Problem

    cfg2 = Problem(batch=4, nhead_q=16, seqlen_q=2048, name="cfg2")
    cfg3 = Problem(batch=1, nhead_q=16, seqlen_q=8192, causal=True, lse=True, name="cfg3")
    return cfg2, cfg3


def _device_inputs(prob, torch, seed=42, mult=1.0):
    import numpy as np

    import fmha_native_amd as fmha

    nq, nk, nlse = prob.sizes()
    host = (fmha.fill_normal(seed, nq, mult), fmha.fill_normal(seed + 1, nk, mult),
            fmha.fill_normal(seed + 2, nk, mult))
    dev = [torch.from_numpy(a.view(np.int16)).to("cuda:0") for a in host]
    o = torch.empty(nq, dtype=torch.int16, device="cuda:0")
    lse = torch.empty(nlse, dtype=torch.float32, device="cuda:0") if prob.lse else None
    ss = prob.seqstart()
    seq = torch.from_numpy(ss).to("cuda:0") if ss is not None else None
    return host, dev, o, lse, seq


def _params(prob, dq, dk, dv, do, dlse, dseq=None):
    import fmha_native_amd as fmha

    p = fmha.FmhaFwdParams()
    p.q, p.k, p.v, p.o = dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), do.data_ptr()
    p.lse = dlse.data_ptr() if dlse is not None else None
    p.seqlen_q, p.seqlen_k, p.nhead_q, p.nhead_k = prob.seqlen_q, prob.seqlen_k, prob.nhead_q, prob.nhead_k
    p.scale = fmha.LOG2E / math.sqrt(64.0)
    st = prob.strides()
    for t in "qkvo":
        s, hs, bs = st[t]
        setattr(p, f"stride_{t}", s)
        setattr(p, f"nhead_stride_{t}", hs)
        setattr(p, f"batch_stride_{t}", bs)
    if dseq is not None:
        p.seqstart_q = p.seqstart_k = dseq.data_ptr()
    return p


class _HipEvents:
    """hipEventCreate/Record/Synchronize/ElapsedTime through ctypes, on the
    HIP runtime torch already loaded (one runtime per process: dlopen by its
    soname returns the loaded copy).  Recording through ctypes keeps the host
    time between an event and the launch it brackets to the launcher's own
    cost, as in the reference's C++ loop."""

    def __init__(self):
        import ctypes

        self.ct = ctypes
        self.lib = ctypes.CDLL("libamdhip64.so.7")
        vp = ctypes.c_void_p
        self.lib.hipEventCreate.argtypes = [ctypes.POINTER(vp)]
        self.lib.hipEventRecord.argtypes = [vp, vp]
        self.lib.hipEventSynchronize.argtypes = [vp]
        self.lib.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        self.lib.hipEventDestroy.argtypes = [vp]

    def create(self, n):
        evs = []
        for _ in range(n):
            e = self.ct.c_void_p()
            assert self.lib.hipEventCreate(self.ct.byref(e)) == 0, "hipEventCreate"
            evs.append(e)
        return evs

    def elapsed_ms(self, e0, e1):
        ms = self.ct.c_float()
        assert self.lib.hipEventElapsedTime(self.ct.byref(ms), e0, e1) == 0, "hipEventElapsedTime"
        return ms.value

    def destroy(self, evs):
        for e in evs:
            self.lib.hipEventDestroy(e)


RAMP_SECONDS = 0.1


def clock_ramp(launch, torch, seconds=RAMP_SECONDS):
    """Untimed launches for `seconds` of wall time before the warm-up steps.
    From an idle GPU the first ~25 ms of back-to-back cfg2 launches run up to
    2x slower while the clock ramps (MI355X, chunks of 20 launches: 179, 96,
    91, 84, 80 ... 77.3 us per launch after ~300 launches), so a short warm-up
    would put the ramp into the timed steps.  Returns the launch count."""
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(20):
            assert launch() == 0
        n += 20
        torch.cuda.synchronize()
    return n


def time_problem(prob, steps, warmup, torch, mult=1.0, variant=0):
    """Ramp the clock (clock_ramp), run `warmup` launches, then time exactly
    `steps` launches back to back on the launch stream between two HIP
    events, bracketed by synchronisations (the whole-job throughput).  Then the reference's own protocol
    (src/bench_fmha_fwd.cpp:204-210) over as many launches: events right
    before and after each launch, synchronised per launch, averaged; it adds
    the host's launch latency to every step and is reported beside it."""
    import ctypes

    import fmha_native_amd as fmha

    host, (dq, dk, dv), do, dlse, dseq = _device_inputs(prob, torch, mult=mult)
    p = _params(prob, dq, dk, dv, do, dlse, dseq)
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)
    lib = fmha.load_library()
    pp, batch, causal = ctypes.byref(p), prob.batch, int(prob.causal)
    # the launcher with a workspace (allocated before timing): the automatic
    # choice (variant 0), which takes the balanced causal form where it
    # applies, or the form a profiling run asks for
    need = fmha.workspace_size(p, batch, causal, variant)
    assert need >= 0, f"variant {variant} rejected for {prob.name}"
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device="cuda:0")
    wsp, wsn = ctypes.c_void_p(ws.data_ptr()), ctypes.c_int64(need)

    def launch():
        return lib.fmha_fwd_d64_bf16_ws(pp, batch, causal, variant, wsp, wsn, sh)

    hip = _HipEvents()
    ramp = clock_ramp(launch, torch)
    for _ in range(warmup):
        assert launch() == 0
    e0, e1 = hip.create(2)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    hip.lib.hipEventRecord(e0, sh)
    for _ in range(steps):
        launch()
    hip.lib.hipEventRecord(e1, sh)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = hip.elapsed_ms(e0, e1) / steps
    times = []
    for _ in range(steps):
        hip.lib.hipEventRecord(e0, sh)
        rc = launch()
        hip.lib.hipEventRecord(e1, sh)
        hip.lib.hipEventSynchronize(e1)
        assert rc == 0, f"launch returned {rc}"
        times.append(hip.elapsed_ms(e0, e1))
    torch.cuda.synchronize()
    ref_ms = sum(times) / steps
    hip.destroy([e0, e1])
    orders = fmha.VARIANT_REFERENCE_ORDER | fmha.VARIANT_TILE_MAJOR_ORDER | fmha.VARIANT_SEQUENCE_ORDER
    picked = (variant & ~orders) or fmha.pick_variant(p, batch, causal)
    plain = ", plain heaviest-first table" if variant & fmha.VARIANT_REFERENCE_ORDER else ""
    form = ("balanced pair" if picked == fmha.VARIANT_BALANCED_PAIR else "balanced") + plain + \
        " (two launches: items, then the merge of split M-tiles)" if need > 0 else \
        {v: k for k, v in fmha.VARIANTS.items()}.get(picked, "?")
    return {"ms": ms, "wall_ms": wall * 1e3 / steps, "tflops": prob.flops() / (ms * 1e-3) / 1e12, "ramp": ramp,
            "ref_ms": ref_ms, "ref_tflops": prob.flops() / (ref_ms * 1e-3) / 1e12, "host": host, "form": form,
            "workspace_bytes": need}


REF_VERIFY = os.path.join(ROOT, "oracle", "_ref", "ref_verify")


def _host_threads():
    """(nproc, OMP_NUM_THREADS or None, threads OpenMP will use)."""
    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:
        nproc = os.cpu_count()
    omp = os.environ.get("OMP_NUM_THREADS")
    threads = int(omp) if omp and omp.isdigit() and int(omp) > 0 else nproc
    return nproc, omp, threads


def cpu_baseline_reference(prob, heads=None, rows=None):
    """The reference's own CPU path, cpu_ref_verify (src/runner/cpu_ref.cpp:14-311,
    compiled from its sources into oracle/_ref/ref_verify), timed by the
    harness around that one call.  Its loop nest (cpu_ref.cpp:73-84) is
    OpenMP over (batch, head) rows and computes every (query, key) score,
    masked ones included, so a causal problem costs it the dense work.
    ``heads``: run that many of the workload's heads (same batch and
    sequence) and scale the time to all of them; used where the whole
    workload would take minutes and the sample keeps the loop's parallelism
    (B*H units handed out 16 at a time: both fit one chunk, one thread).
    ``rows``: run only the last ``rows`` query rows against all of the keys
    (seqlen_q = rows, seqlen_k unchanged: bottom-right alignment keeps each
    sampled row's mask) and scale by seqlen_q / rows; every row costs the
    loop the same seqlen_k dot products both ways.  None if not built."""
    import subprocess

    if not os.path.exists(REF_VERIFY):
        return None
    nh = heads or prob.nhead_q
    nrows = rows or prob.seqlen_q
    cmd = [REF_VERIFY, "-b", str(prob.batch), "-h", str(nh), "-s", str(nrows), "--kv-seq", str(prob.seqlen_k),
           "--seed", "42", "--mask", str(int(prob.causal)), "--lse", str(int(prob.lse))]
    if prob.varlen:
        cmd += ["--varlen-seqs", ",".join(str(x) for x in prob.varlen_seqs)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
    if r.returncode != 0:
        return None
    res = [json.loads(l.split(" ", 1)[1]) for l in r.stdout.splitlines() if l.startswith("REF_VERIFY ")]
    if not res:
        return None
    t_run, thr = res[0]["cpu_ref_seconds"], res[0]["threads"]
    nproc, omp, _ = _host_threads()
    units = prob.batch * prob.nhead_q
    # collapse(2) schedule(dynamic, 16) hands out the B*H (batch, head) units
    # 16 at a time: ceil(B*H / 16) chunks, so at most that many threads work
    chunks = -(-units // 16)
    if heads:
        assert -(-(prob.batch * nh) // 16) == chunks == 1, "a head sample must keep the loop's parallelism"
    t = t_run * (prob.nhead_q / nh) * (prob.seqlen_q / nrows)
    lse = f", LSE |d| max {res[0]['lse_max_abs']:.2e}" if prob.lse else ""
    seqs = f"varlen {'/'.join(str(x) for x in prob.varlen_seqs)} H{prob.nhead_q}" if prob.varlen else \
        f"B{prob.batch}H{prob.nhead_q}S{prob.seqlen_q}"
    shape = f"{seqs}{' causal' if prob.causal else ''}{' +LSE' if prob.lse else ''}"
    if rows:
        what = (f"over the last {nrows} of the {prob.seqlen_q} query rows (against all {prob.seqlen_k} keys) of "
                f"{nh} of the {prob.nhead_q} heads of the {shape} workload ({t_run:.2f} s, scaled "
                f"x{prob.seqlen_q}/{nrows} x{prob.nhead_q}/{nh} to {t:.2f} s: the loop computes every key's score "
                f"for every row, and one thread computes every head either way; the sampled rows see 90-100 % of "
                f"their keys against half on average, and only visible keys take expf, so the rate per row is "
                f"if anything understated)")
    elif heads:
        what = (f"over {nh} of the {prob.nhead_q} heads of the {shape} workload ({t_run:.2f} s, scaled "
                f"x{prob.nhead_q}/{nh} to {t:.2f} s: one thread computes every head either way, the B*H units "
                f"all fitting one chunk of 16)")
    else:
        what = f"over the full {shape} workload, {t:.2f} s"
    out = {
        "value": prob.flops() / t / 1e12,
        "unit": "TFLOP/s",
        "cores": thr,
        "kind": "reference",
        "seconds": round(t, 3),
        "seconds_measured": round(t_run, 3),
        "nproc": nproc,
        "omp_num_threads": omp,
        "effective_parallelism": min(thr, chunks),
        "sample": f"the reference's cpu_ref_verify {what} (its fill_random(42) inputs; time does not depend on "
                  f"values), on {thr} OpenMP threads, of which min({thr}, ceil(B*H/16) = {chunks}) = "
                  f"{min(thr, chunks)} have work (its loop is collapse(2) schedule(dynamic, 16) over the "
                  f"B*H = {units} (batch, head) units, cpu_ref.cpp:73-84); FLOPs by the repo convention"
                  f"{' (x0.5; the loop computes every masked score too)' if prob.causal else ''}; its check of "
                  f"this kernel's output: pass={res[0]['pass']}{lse}",
    }
    if prob.varlen:
        out["value_exact_flops"] = prob.exact_flops() / t / 1e12
    return out


def cpu_baseline(prob, host, budget_s=10.0, nthreads=None):
    """Reference-faithful oracle on rows [0, R) of every (batch, head)
    (``nthreads``: default min(host threads, B*H))."""
    import oracle

    nproc, omp, threads = _host_threads()
    if nthreads is None:
        nthreads = max(1, min(threads, prob.batch * prob.nhead_q))  # reference parallelises over (b, h)
    q, k, v = host

    def run(rows):
        t0 = time.perf_counter()
        oracle.run(prob, q, k, v, faithful=True, nthreads=nthreads, rows=(0, rows))
        return time.perf_counter() - t0

    rows = 16
    t = run(rows)
    while t < 0.5 * budget_s and rows < prob.seqlen_q:  # grow the sample to ~budget_s
        rows = int(min(prob.seqlen_q, max(rows + 1, rows * 0.9 * budget_s / max(t, 1e-3))))
        t = run(rows)
    # the loop nest computes every key of every sampled row, masked or not
    flops = 4.0 * 64 * prob.seqlen_k * rows * prob.batch * prob.nhead_q * (0.5 if prob.causal else 1.0)
    return {
        "value": flops / t / 1e12,
        "unit": "TFLOP/s",
        "cores": nthreads,
        "kind": "port",
        "seconds": round(t, 3),
        "nproc": nproc,
        "omp_num_threads": omp,
        "effective_parallelism": min(nthreads, -(-(prob.batch * prob.nhead_q) // 16)),  # dynamic,16 chunks
        "sample": f"faithful C oracle, query rows [0,{rows}) of all {prob.batch * prob.nhead_q} (b,h) of "
                  f"B{prob.batch}H{prob.nhead_q}S{prob.seqlen_q}{' causal' if prob.causal else ''} (full keys), "
                  f"{t:.1f} s on {nthreads} threads; extrapolated to the whole workload at that rate",
    }


# Query rows of cfg5 the reference's CPU loop is timed on (about 12 s on one
# thread; the whole workload would take it about four minutes).
CFG5_CPU_ROWS = 4000


def cpu_baseline_others():
    """The CPU baseline on cfg1, cfg4 and cfg5 (the reference's cpu_ref_verify
    throughout): cfg1 and cfg4 over the whole workload (cfg4: eight sequences x
    16 heads, 128 (sequence, head) units in 8 chunks of 16, so 8 threads have
    work); cfg5 (B1 H2 S40000, both units in one chunk: one thread) over the
    last CFG5_CPU_ROWS query rows of one head, scaled to the workload.  Where
    the reference harness is not built, the faithful C port on a row sample."""
    from fmha_native_amd.problem import baseline_problems

    keys = ("value", "value_exact_flops", "unit", "cores", "kind", "seconds", "effective_parallelism", "sample")
    out = {}
    probs = baseline_problems()
    for name in ("cfg1", "cfg4", "cfg5"):
        print(f"bench.py: CPU baseline {name}", file=sys.stderr, flush=True)
        prob, mult = probs[name]
        c = cpu_baseline_reference(prob, heads=1, rows=CFG5_CPU_ROWS) if name == "cfg5" else \
            cpu_baseline_reference(prob)
        if c is None:
            import fmha_native_amd as fmha

            nq, nk, _ = prob.sizes()
            host = (fmha.fill_normal(42, nq, mult), fmha.fill_normal(43, nk, mult), fmha.fill_normal(44, nk, mult))
            c = cpu_baseline(prob, host, budget_s=10.0, nthreads=None if prob.varlen else 1)
        out[name] = {k: c[k] for k in keys if k in c}
    return out


PROFILE_JSON = os.path.join(ROOT, "profiles", "roofline_fmha_fwd_d64_bf16_cfg2_cfg3.json")


def _profile(workload):
    """Counter figures for ``workload`` from the committed rocprofv3 run
    (profiles/, written by ``python -m fmha_native_amd.rocprof``), or None."""
    try:
        with open(PROFILE_JSON) as f:
            return json.load(f).get(workload)
    except (OSError, ValueError):
        return None


def _roofline(achieved, workload, ms_per_step):
    """The roofline object: ``achieved``/``frac`` from this run's HIP events;
    HBM traffic, MFMA busy and the clock from the committed rocprofv3 run of
    the same kernel (one box, one process tree), where
    frac_from_counters = mfma_busy x clock / 2.4 GHz checks the timer.  The
    kernel is cycle-bound (the same active cycles per launch on every box
    measured), so those cycles over a run's time per launch give the clock
    that box held: this run's frac over the profile run's is the ratio of the
    two clocks."""
    prof = _profile(workload)
    r = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
         "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None}
    if prof:
        active_cycles = prof["clock_ghz"] * prof["counter_dispatch_us"] * 1e3
        r.update({
            "traffic": prof["hbm_bytes_per_launch"],
            "algorithmic_bytes": prof["algorithmic_bytes"],
            "mfma_busy": prof["mfma_busy"],
            "clock_ghz": prof["clock_ghz"],
            "frac_from_counters": prof["frac_from_counters"],
            "active_cycles_per_launch": round(active_cycles),
            "clock_ghz_this_run": round(active_cycles / (ms_per_step * 1e6), 4),
            "clock_ghz_profile_run": round(active_cycles / (prof["bench_ms_per_step"] * 1e6), 4),
            "frac_profile_run": round(prof["bench_tflops"] / PEAK_BF16_TFLOPS, 4),
            "profile": {"file": os.path.relpath(PROFILE_JSON, ROOT), "kernel": prof["kernel"],
                        "trace_avg_us": prof["trace_avg_us"], "bench_ms_per_step_same_box": prof["bench_ms_per_step"],
                        "note": "traffic, mfma_busy, clock_ghz (a lower bound from the counter pass) and the "
                                "active cycles (SQ_BUSY_CYCLES per shader engine) come from that run; "
                                "frac_from_counters = mfma_busy x clock_ghz / 2.4 GHz; the active cycles over each "
                                "run's own time per launch give the clock each box held (clock_ghz_this_run, "
                                "clock_ghz_profile_run), and frac / frac_profile_run ~ their ratio"},
        })
    return r


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the cfg1/cfg4/cfg5 side measurements")
    ap.add_argument("--only", default=None,
                    help="time one workload only (profiling runs): cfg1..cfg5, or a dense shape "
                         "dense-B<b>H<h>S<s> / causal-B<b>H<h>S<s>")
    ap.add_argument("--variant", default="auto", help="with --only: the kernel form, optionally |reference, |tilemajor or |sequence "
                         "(default: the launcher's choice)")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run `steps` device-to-device copies of this many MiB (HBM counter calibration)")
    ap.add_argument("--gemm-probe", type=int, default=0,
                    help="only time `steps` bf16 N x N x N torch.matmul launches (the library GEMM beside the "
                         "kernel on one box: MFMA rate and clock under the power cap)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the path shards "
              "over independent (batch, head) units with no communication, so N GPUs = N independent runs",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import fmha_native_amd as fmha

    fmha.load_library()
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.copy_probe_mib:
        n = args.copy_probe_mib << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n, "copies": args.steps}))
        return
    if args.gemm_probe:
        n = args.gemm_probe
        g = torch.Generator(device="cuda:0").manual_seed(42)
        a = torch.randn(n, n, device="cuda:0", dtype=torch.float32, generator=g).to(torch.bfloat16)
        b = torch.randn(n, n, device="cuda:0", dtype=torch.float32, generator=g).to(torch.bfloat16)
        c = torch.empty(n, n, device="cuda:0", dtype=torch.bfloat16)
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < 0.3:  # bring the clock up, as time_problem does
            for _ in range(10):
                torch.matmul(a, b, out=c)
            torch.cuda.synchronize()
        for _ in range(args.warmup):
            torch.matmul(a, b, out=c)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(args.steps):
            torch.matmul(a, b, out=c)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / args.steps
        print(json.dumps({"gemm_n": n, "dtype": "bf16", "steps": args.steps, "ms_per_gemm": round(ms, 5),
                          "tflops": round(2.0 * n ** 3 / (ms * 1e-3) / 1e12, 1)}))
        return
    cfg2, cfg3 = _problems()
    if args.only:
        from fmha_native_amd.problem import workload

        prob, mult = {"cfg2": (cfg2, 1.0), "cfg3": (cfg3, 1.0)}.get(args.only) or workload(args.only)
        r = time_problem(prob, args.steps, args.warmup, torch, mult, fmha.variant_code(args.variant))
        # launch order, for a profiler's trace: ramp, warmup, steps timed back
        # to back, then as many under the reference's protocol
        print(json.dumps({"workload": args.only, "ms_per_step": r["ms"], "tflops": r["tflops"], "form": r["form"],
                          "reference_protocol_ms": r["ref_ms"], "ramp_launches": r["ramp"], "warmup": args.warmup,
                          "steps": args.steps}), flush=True)
        return
    r2 = time_problem(cfg2, args.steps, args.warmup, torch)
    r3 = time_problem(cfg3, max(1, args.steps // 2), max(1, args.warmup // 2), torch)
    # the other benchmark configurations, reported beside the headline
    others = {}
    if not args.no_extra:
        from fmha_native_amd.problem import baseline_problems

        for name in ("cfg1", "cfg4", "cfg5"):
            prob, mult = baseline_problems()[name]
            r = time_problem(prob, max(1, args.steps // 4), max(1, args.warmup // 2), torch, mult)
            e = {"workload": prob.name, "ms_per_step": round(r["ms"], 5), "value": round(r["tflops"], 2),
                 "pct_bf16_peak": round(100.0 * r["tflops"] / PEAK_BF16_TFLOPS, 2),
                 "reference_protocol": {"ms_per_step": round(r["ref_ms"], 5), "value": round(r["ref_tflops"], 2)},
                 "form": r["form"]}
            if prob.varlen:
                e["value_exact_flops"] = round(prob.exact_flops() / (r["ms"] * 1e-3) / 1e12, 2)
                e["note"] = ("value uses the repo FLOP convention (max S for every sequence, an overcount); "
                             "value_exact_flops counts the visible (q, k) pairs")
            if name == "cfg1":
                e["hbm_gbs"] = round(prob.io_bytes() / (r["ms"] * 1e-3) / 1e9, 1)
                e["note"] = "launch-latency bound; hbm_gbs = algorithmic bytes / time"
            others[name] = e

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_reference(cfg2) or cpu_baseline(cfg2, r2["host"])
        # the whole of cfg3 takes its loop ~80 s on one thread: 4 of its 16 heads
        c3 = cpu_baseline_reference(cfg3, heads=4) or cpu_baseline(cfg3, r3["host"])
        cpu["cfg3"] = {k: c3[k] for k in ("value", "unit", "cores", "kind", "seconds", "effective_parallelism",
                                          "sample") if k in c3}
        cpu.update(cpu_baseline_others())

    achieved = r2["tflops"]
    line = {
        "metric": "fwd TFLOP/s + % BF16 MFMA peak, d64 B4H16S2048 dense & B1H16S8192 causal",
        "value": round(achieved, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r2["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(achieved / 348.4, 3),
        "vs_baseline_note": "ratio to the reference's published MI300X figure for this config (348.4 TFLOP/s, "
                            "README.md:91); no MI355X figure is published",
        "pct_bf16_peak": round(100.0 * achieved / PEAK_BF16_TFLOPS, 2),
        "timing": "steps launched back to back on one stream between two HIP events, synchronised before and "
                  "after (whole-job throughput), after 0.1 s of untimed launches that bring the clock up from "
                  "idle and the warmup steps; reference_protocol: the reference's events around each launch, "
                  "synchronised per launch (src/bench_fmha_fwd.cpp:204-210), which adds the host's launch latency",
        "clock_ramp_launches": r2["ramp"],
        "reference_protocol": {"ms_per_step": round(r2["ref_ms"], 5), "value": round(r2["ref_tflops"], 2)},
        "form": r2["form"],
        "dtype": "bf16",
        "data": "synthetic: Q/K/V i.i.d. N(0,1) bf16, seed 42 (fill_normal)",
        "config": {"workload": "dense MHA forward B4 H16 Sq=Sk=2048 D64, no mask, no LSE, BHSD",
                   "batch": 4, "heads": 16, "seq_len": 2048, "head_dim": 64, "causal": False, "lse": False},
        "roofline": _roofline(achieved, "cfg2", r2["ms"]),
        "also": {
            "workload": "causal MHA forward B1 H16 Sq=Sk=8192 D64 with LSE (FLOPs x0.5)",
            "ms_per_step": round(r3["ms"], 5),
            "value": round(r3["tflops"], 2),
            "pct_bf16_peak": round(100.0 * r3["tflops"] / PEAK_BF16_TFLOPS, 2),
            "reference_protocol": {"ms_per_step": round(r3["ref_ms"], 5), "value": round(r3["ref_tflops"], 2)},
            "form": r3["form"],
            "roofline": _roofline(r3["tflops"], "cfg3", r3["ms"]),
            "vs_reference_mi300x": round(r3["tflops"] / 358.1, 3),
        },
        "others": others,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
