"""Performance sweep with the reference's protocol and stdout table.

    python -m fmha_native_amd.sweep [--mask 0|1] [--bench PATH] [--dist ref|normal]
    python -m fmha_native_amd.sweep --markdown profiles/NAME.md     # both masks, with ratios

Same 8 configurations, WARMUP=5, ITERS=20, 6 runs of the bench CLI per
configuration with the first dropped and runs 2-6 averaged, and the same
header and row format as the reference's scripts/run-benchmark.sh:12-21,56-99,
so tables from the two can be compared line by line.  Each run is a separate
process of ``bench_fmha_fwd`` whose ``Avg:`` / ``min=`` / ``TFLOPS:`` lines are
parsed (src/bench_fmha_fwd.cpp:231-233).
"""
import argparse
import os
import re
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
SWEEP_SIZES = [(8, 16, 1024), (4, 16, 2048), (2, 16, 4096), (1, 8, 8192), (1, 16, 8192), (1, 8, 16384),
               (1, 4, 32768), (1, 2, 40000)]
WARMUP, ITERS, NRUNS, DROP = 5, 20, 6, 1
# The reference's published sweep on MI300X (its native kernel, TFLOP/s by the
# same convention), README.md:90-97 (mask 0) and :103-110 (mask 1); the
# reference publishes no MI355X figures.
REFERENCE_MI300X = {0: [302.0, 348.4, 371.6, 335.9, 387.9, 406.5, 404.9, 335.1],
                    1: [207.8, 265.6, 305.8, 256.2, 358.1, 378.9, 395.8, 308.2]}


def parse_run(text):
    """(avg_ms, min_ms, tflops) from one bench_fmha_fwd run's stdout."""
    avg = re.search(r"^Avg:\s*([0-9.]+)", text, re.M)
    mn = re.search(r"^min=([0-9.]+)", text, re.M)
    tf = re.search(r"^TFLOPS:\s*([0-9.]+)", text, re.M)
    if not (avg and mn and tf):
        raise ValueError("bench output lacks Avg:/min=/TFLOPS: lines")
    return float(avg.group(1)), float(mn.group(1)), float(tf.group(1))


def run_config(bench, b, h, s, mask, dist, timeout=300):
    avgs, mins, tfs = [], [], []
    for run_idx in range(1, NRUNS + 1):
        cmd = [bench, "-b", str(b), "-h", str(h), "-s", str(s), "-d", "64", "--mask", str(mask), "--warmup",
               str(WARMUP), "--iters", str(ITERS), "--dist", dist]
        r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout)
        out = r.stdout + r.stderr
        if r.returncode != 0:
            m = re.search(r"(?i).*(HIP error|out of memory|error).*", out)
            return None, m.group(0) if m else f"exited {r.returncode} (run {run_idx})"
        if run_idx > DROP:
            a, mn, tf = parse_run(r.stdout)
            avgs.append(a)
            mins.append(mn)
            tfs.append(tf)
    return (sum(avgs) / len(avgs), min(mins), sum(tfs) / len(tfs)), None


def markdown(bench, dist, path):
    """Both masks' tables (the reference's stdout format) and the ratio of
    each TFLOP/s figure to the reference's published MI300X one."""
    md = ["# Reference-protocol sweep — fmha_fwd_d64_bf16 on MI355X (one GPU)", "",
          f"Command (repo root): `python -m fmha_native_amd.sweep --markdown {os.path.relpath(path)}` — the reference's "
          f"8 configs, WARMUP={WARMUP} ITERS={ITERS}, {NRUNS} runs of `bench_fmha_fwd` per config with the first "
          f"dropped (scripts/run-benchmark.sh), its {'+-0.1' if dist == 'ref' else 'N(0,1)'} inputs, the launcher's "
          "automatic kernel form (the CLI launches with a workspace, so long causal grids may take the balanced "
          "form). Each run is a fresh process timed with the reference's per-launch protocol, so it includes the "
          "GPU clock's ramp from idle. TFLOP/s use the repo convention (x0.5 when causal).", ""]
    for mask in (0, 1):
        md += ["```", f"Benchmark: {len(SWEEP_SIZES)} configs (WARMUP={WARMUP} ITERS={ITERS} RUNS={NRUNS} "
                      f"DROP={DROP} MASK={mask})", "",
               "%4s %3s %6s %4s | %10s %10s %10s" % ("B", "H", "S", "D", "Avg(ms)", "Min(ms)", "TFLOPS"),
               "---- --- ------ ---- + ---------- ---------- ----------"]
        ratios = []
        for i, (b, h, s) in enumerate(SWEEP_SIZES):
            res, err = run_config(bench, b, h, s, mask, dist)
            print(f"[sweep] mask {mask} B{b} H{h} S{s}: {res if res else err}", flush=True)
            if res is None:
                md.append("%4s %3s %6s %4s | %10s %10s %10s" % (b, h, s, 64, "ERROR", "ERROR", "ERROR"))
                ratios.append(None)
            else:
                md.append("%4s %3s %6s %4s | %10.3f %10.3f %10.2f" % (b, h, s, 64, res[0], res[1], res[2]))
                ratios.append(res[2] / REFERENCE_MI300X[mask][i])
        md += ["```", "", f"Ratio to the reference's MI300X figure (mask {mask}): "
               + ", ".join("ERROR" if r is None else f"{r:.2f}x" for r in ratios) + ".", ""]
    with open(path, "w") as f:
        f.write("\n".join(md))
    print("\n".join(md), flush=True)
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--mask", type=int, default=0, choices=[0, 1])
    ap.add_argument("--bench", default=os.path.join(PKG, "bench_fmha_fwd"))
    ap.add_argument("--dist", default="ref", choices=["ref", "normal"],
                    help="input distribution (the reference's sweep uses its +-0.1 generator)")
    ap.add_argument("--markdown", default=None, help="run both masks and write a markdown summary here")
    args = ap.parse_args(argv)
    if not os.path.exists(args.bench):
        print(f"Error: bench_fmha_fwd not found at {args.bench}.", file=sys.stderr)
        return 1
    if args.markdown:
        return markdown(args.bench, args.dist, args.markdown)
    print(f"Benchmark: {len(SWEEP_SIZES)} configs (WARMUP={WARMUP} ITERS={ITERS} RUNS={NRUNS} DROP={DROP} "
          f"MASK={args.mask})")
    if os.environ.get("HIP_VISIBLE_DEVICES"):
        print(f"GPU: HIP_VISIBLE_DEVICES={os.environ['HIP_VISIBLE_DEVICES']}")
    print("")
    print("%4s %3s %6s %4s | %10s %10s %10s" % ("B", "H", "S", "D", "Avg(ms)", "Min(ms)", "TFLOPS"))
    print("---- --- ------ ---- + ---------- ---------- ----------")
    for b, h, s in SWEEP_SIZES:
        res, err = run_config(args.bench, b, h, s, args.mask, args.dist)
        if res is None:
            avg = mn = tf = "ERROR"
        else:
            avg, mn, tf = f"{res[0]:.3f}", f"{res[1]:.3f}", f"{res[2]:.2f}"
        print("%4s %3s %6s %4s | %10s %10s %10s" % (b, h, s, 64, avg, mn, tf), flush=True)
        if err:
            print(f"  ↳ {err}")
    print("")
    return 0


if __name__ == "__main__":
    sys.exit(main())
