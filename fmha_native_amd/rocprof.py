"""rocprofv3 evidence harness for the FMHA forward kernels (run on the GPU box).

    python -m fmha_native_amd.rocprof --out gpurun_out/prof [--summary profiles/NAME.md]

The gfx950 counterpart of the reference's ATT/counter configuration
(scripts/rocprof_att.yaml:1-17).  It runs ``bench.py`` under ``rocprofv3`` in
separate passes (a counter pass never combines with tracing, and each pass
stays within one pass's hardware counter budget), each as a child process
under its own time limit, and writes a markdown summary with the exact
command of every pass:

1. kernel trace + stats for cfg2 (dense B4 H16 S2048) and cfg3 (causal
   B1 H16 S8192 + LSE): average dispatch duration, set beside bench.py's own
   HIP-event time for the same launches;
2. HBM traffic of cfg2: FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by
   what the counter reads for a device copy of known size (bench.py
   ``--copy-probe-mib``), against the algorithmic bytes;
3. utilisation of cfg2 and cfg3: clock (GRBM_GUI_ACTIVE), MFMA busy cycles,
   VALU/MFMA/LDS instruction counts, LDS bank conflicts, plus the VGPR/AGPR/
   SGPR/LDS allocation the profiler records for the dispatch.
"""
import argparse
import glob
import json
import os
import sqlite3
import subprocess
import sys
from collections import defaultdict

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PEAK_BF16_TFLOPS = 2516.6
NUM_XCD = 8
NUM_SIMD = 256 * 4

UTIL_COUNTERS = ["GRBM_GUI_ACTIVE", "SQ_WAVES", "SQ_BUSY_CYCLES", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU",
                 "SQ_INSTS_MFMA", "SQ_INSTS_LDS", "SQ_LDS_BANK_CONFLICT", "SQ_INSTS_VALU_TRANS_F32"]
WORKLOADS = {
    "cfg2": {"flops": 4.0 * 4 * 16 * 2048 * 2048 * 64, "bytes": 67108864, "desc": "dense B4 H16 S2048"},
    "cfg3": {"flops": 4.0 * 16 * 8192 * 8192 * 64 * 0.5, "bytes": 67633152, "desc": "causal B1 H16 S8192 + LSE"},
}


def _bench(*args):
    return [sys.executable, os.path.join(ROOT, "bench.py"), *args]


def _run(name, prof_args, prog, out_dir, limit):
    d = os.path.join(out_dir, name)
    cmd = ["timeout", "-s", "KILL", str(limit), "rocprofv3", *prof_args, "-d", d, "-o", "run", "--", *prog]
    print(f"[rocprof] pass {name}: {' '.join(cmd)}", flush=True)
    with open(os.path.join(out_dir, f"{name}.log"), "w") as log:
        r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=log, text=True)
    with open(os.path.join(out_dir, f"{name}.out"), "w") as f:
        f.write(r.stdout)
    dbs = glob.glob(os.path.join(d, "**", "*_results.db"), recursive=True)
    # rocprofv3 itself may end with a signal after the program finished and the
    # results were written: the program's own JSON line and the db decide
    lines = [l for l in r.stdout.splitlines() if l.startswith("{")]
    if not dbs or not lines:
        raise RuntimeError(f"pass {name} failed (rc={r.returncode}); see {name}.log")
    shown = " ".join("python3" if c == sys.executable else c for c in cmd[4:]).replace(ROOT + "/", "")
    return dbs[0], json.loads(lines[-1]), shown


def _kernel_stats(db):
    con = sqlite3.connect(db)
    # top_kernels reports durations in microseconds
    return [dict(name=n, calls=c, avg_us=a) for n, c, _t, a, _p in con.execute("select * from top_kernels")]


def _counters(db, kernel_prefix="fmha_fwd"):
    """Per-dispatch counter values (summed over the chip), averaged over dispatches."""
    con = sqlite3.connect(db)
    per = defaultdict(float)
    res = {}
    q = ("select dispatch_id, kernel_name, counter_name, value, vgpr_count, accum_vgpr_count, sgpr_count, "
         "lds_block_size from counters_collection")
    for disp, kname, cname, val, vgpr, agpr, sgpr, lds in con.execute(q):
        per[(kname, cname, disp)] += val
        res.setdefault(kname, {"vgpr": vgpr, "agpr": agpr, "sgpr": sgpr, "lds_bytes": lds})
    agg = defaultdict(list)
    for (k, c, _d), v in per.items():
        agg[(k, c)].append(v)
    out = {}
    for (k, c), v in agg.items():
        if k.startswith(kernel_prefix) or not kernel_prefix:
            out.setdefault(k, dict(res[k]))[c] = sum(v) / len(v)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default=os.path.join(ROOT, "gpurun_out", "prof"))
    ap.add_argument("--summary", default=None, help="markdown summary path (default: <out>/summary.md)")
    ap.add_argument("--traffic-json", default=None, help="also write the cfg2 traffic figures here")
    ap.add_argument("--steps", type=int, default=100)
    args = ap.parse_args()
    os.makedirs(args.out, exist_ok=True)
    md = ["# rocprofv3 summary — fmha_fwd_d64_bf16 on cfg2 (dense B4 H16 S2048) and cfg3 (causal B1 H16 "
          "S8192 + LSE)", "",
          "MI355X (gfx950), one GPU.  Made by `python -m fmha_native_amd.rocprof`, which runs the passes below "
          "from the repo root (each under `timeout -s KILL`).", ""]

    # 1. kernel trace
    md += ["## Kernel trace (average dispatch duration vs bench.py's HIP events)", "",
           "| workload | kernel | dispatches | rocprofv3 avg | bench.py HIP-event avg | TFLOP/s (trace) | % of 2516.6 |",
           "|---|---|---|---|---|---|---|"]
    cmds = []
    trace = {}
    for wl in ("cfg2", "cfg3"):
        steps = args.steps if wl == "cfg2" else args.steps // 2
        db, line, cmd = _run(f"trace_{wl}", ["--kernel-trace", "--stats"],
                             _bench("--only", wl, "--steps", str(steps), "--warmup", "10"), args.out, 300)
        cmds.append(cmd)
        k = [s for s in _kernel_stats(db) if s["name"].startswith("fmha_fwd")][0]
        tf = WORKLOADS[wl]["flops"] / (k["avg_us"] * 1e-6) / 1e12
        trace[wl] = {"avg_us": k["avg_us"], "bench_us": line["ms_per_step"] * 1e3, "tflops": tf}
        md.append(f"| {wl} | `{k['name']}` | {k['calls']} | {k['avg_us']:.2f} us | {line['ms_per_step'] * 1e3:.2f} us "
                  f"| {tf:.1f} | {100 * tf / PEAK_BF16_TFLOPS:.1f}% |")
    md += ["", "Commands:", ""] + [f"    {c}" for c in cmds] + [""]

    # 2. traffic
    cmds = []
    vals = {}
    for name, counter, prog in (("pmc_fetch", "FETCH_SIZE", _bench("--only", "cfg2", "--steps", "5", "--warmup", "1")),
                                ("pmc_write", "WRITE_SIZE", _bench("--only", "cfg2", "--steps", "5", "--warmup", "1")),
                                ("pmc_copy_fetch", "FETCH_SIZE", _bench("--copy-probe-mib", "256", "--steps", "5")),
                                ("pmc_copy_write", "WRITE_SIZE", _bench("--copy-probe-mib", "256", "--steps", "5"))):
        db, _line, cmd = _run(name, ["--pmc", counter], prog, args.out, 120)
        cmds.append(cmd)
        c = _counters(db, kernel_prefix="")
        if name.startswith("pmc_copy"):
            vals[name] = max(v[counter] for v in c.values())
        else:
            vals[name] = [v[counter] for k, v in c.items() if k.startswith("fmha_fwd")][0]
    copy_kib = 256 * 1024
    fs, ws = copy_kib / vals["pmc_copy_fetch"], copy_kib / vals["pmc_copy_write"]
    fetch_b = vals["pmc_fetch"] * fs * 1024
    write_b = vals["pmc_write"] * ws * 1024
    traffic = fetch_b + write_b
    alg = WORKLOADS["cfg2"]["bytes"]
    md += ["## HBM traffic (cfg2, per dispatch)", "",
           "| counter | kernel (KiB/dispatch) | 256 MiB copy reads (KiB) | scale | scaled bytes |", "|---|---|---|---|---|",
           f"| FETCH_SIZE | {vals['pmc_fetch']:,.0f} | {vals['pmc_copy_fetch']:,.0f} (expected 262,144) | x{fs:.3f} | "
           f"{fetch_b / 1e6:.2f} MB |",
           f"| WRITE_SIZE | {vals['pmc_write']:,.0f} | {vals['pmc_copy_write']:,.0f} (expected 262,144) | x{ws:.3f} | "
           f"{write_b / 1e6:.2f} MB |", "",
           f"Total {traffic / 1e6:.2f} MB per launch vs {alg / 1e6:.2f} MB algorithmic (Q+K+V read once, O written "
           f"once): ratio {traffic / alg:.3f}.", "", "Commands:", ""] + [f"    {c}" for c in cmds] + [""]

    # 3. utilisation
    md += ["## Utilisation counters (per dispatch, summed over the chip)", ""]
    cmds = []
    rows = []
    for wl in ("cfg2", "cfg3"):
        db, _line, cmd = _run(f"pmc_util_{wl}", ["--pmc", *UTIL_COUNTERS],
                              _bench("--only", wl, "--steps", "5", "--warmup", "1"), args.out, 120)
        cmds.append(cmd)
        k, c = list(_counters(db).items())[0]
        cycles_xcd = c["GRBM_GUI_ACTIVE"] / NUM_XCD
        ghz = cycles_xcd / (trace[wl]["avg_us"] * 1e3)  # cycles per ns
        mfma_busy = c["SQ_VALU_MFMA_BUSY_CYCLES"] / NUM_SIMD / cycles_xcd
        iters = c["SQ_INSTS_MFMA"] / 16.0  # 16 MFMA per wave per 64-key tile
        rows.append((wl, k, c, ghz, mfma_busy, iters))
    md += ["| | " + " | ".join(r[0] for r in rows) + " |", "|---|" + "---|" * len(rows)]
    md.append("| kernel | " + " | ".join(f"`{r[1]}`" for r in rows) + " |")
    md.append("| VGPR / AGPR / SGPR (rocprofv3 dispatch fields) | "
              + " | ".join(f"{r[2]['vgpr']} / {r[2]['agpr']} / {r[2]['sgpr']}" for r in rows) + " |")
    md.append("| LDS bytes per block | " + " | ".join(f"{r[2]['lds_bytes']}" for r in rows) + " |")
    md.append("| clock from GRBM_GUI_ACTIVE / 8 XCDs | " + " | ".join(f"{r[3]:.2f} GHz" for r in rows) + " |")
    md.append("| MFMA busy (per SIMD, of kernel cycles) | " + " | ".join(f"{100 * r[4]:.1f}%" for r in rows) + " |")
    for name in UTIL_COUNTERS[1:]:
        md.append(f"| {name} | " + " | ".join(f"{r[2].get(name, 0):,.0f}" for r in rows) + " |")
    md.append("| VALU instr per wave per 64-key tile (incl. 16 MFMA) | "
              + " | ".join(f"{r[2]['SQ_INSTS_VALU'] / r[5]:.1f}" for r in rows) + " |")
    md.append("| LDS instr per wave per tile | " + " | ".join(f"{r[2]['SQ_INSTS_LDS'] / r[5]:.1f}" for r in rows) + " |")
    md += ["", "The compiler reports 248-254 VGPRs used per wave for these entries (`; NumVgprs`, checked with "
           "`tests/test_codegen.py`), allocated as 256: two waves per SIMD. rocprofv3's VGPR field is consistent "
           "with the descriptor's granule count read as 4 registers per granule where gfx950 wave64 allocates "
           "8 (31 + 1 granules: 128 shown, 256 allocated).",
           "", "Commands:", ""] + [f"    {c}" for c in cmds] + [""]

    path = args.summary or os.path.join(args.out, "summary.md")
    with open(path, "w") as f:
        f.write("\n".join(md))
    print("\n".join(md), flush=True)
    if args.traffic_json:
        with open(args.traffic_json, "w") as f:
            json.dump({"kernel": "fmha_fwd_d64_bf16_msk0", "workload": "cfg2 B4 H16 S2048 D64 dense",
                       "fetch_kib_per_dispatch": vals["pmc_fetch"], "write_kib_per_dispatch": vals["pmc_write"],
                       "fetch_scale": round(fs, 4), "write_scale": round(ws, 4),
                       "hbm_bytes_per_launch": int(traffic), "algorithmic_bytes": alg,
                       "rocprof_avg_us": round(trace["cfg2"]["avg_us"], 3),
                       "made_by": "python -m fmha_native_amd.rocprof"}, f, indent=1)


if __name__ == "__main__":
    main()
