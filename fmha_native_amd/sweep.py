"""Performance sweep with the reference's protocol and stdout table.

    python -m fmha_native_amd.sweep [--mask 0|1] [--bench PATH] [--dist ref|normal]

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


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--mask", type=int, default=0, choices=[0, 1])
    ap.add_argument("--bench", default=os.path.join(PKG, "bench_fmha_fwd"))
    ap.add_argument("--dist", default="ref", choices=["ref", "normal"],
                    help="input distribution (the reference's sweep uses its +-0.1 generator)")
    args = ap.parse_args(argv)
    if not os.path.exists(args.bench):
        print(f"Error: bench_fmha_fwd not found at {args.bench}.", file=sys.stderr)
        return 1
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
