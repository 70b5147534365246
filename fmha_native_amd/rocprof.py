"""rocprofv3 evidence harness for the FMHA forward kernels (run on the GPU box).

    python -m fmha_native_amd.rocprof --out OUT_DIR --summary profiles/NAME.md --json profiles/NAME.json

The gfx950 counterpart of the reference's ATT/counter configuration
(scripts/rocprof_att.yaml:1-17).  Everything below runs in one process tree
on one GPU, so the figures describe one box at one clock.  ``bench.py`` runs
under ``rocprofv3`` in separate passes (a counter pass never combines with
tracing, and each pass stays within one pass's hardware counter budget), each
as a child process under its own time limit; the markdown summary gives the
exact command of every pass:

0. ``bench.py`` itself, unprofiled: its HIP-event time per launch on cfg2
   (dense B4 H16 S2048) and cfg3 (causal B1 H16 S8192 + LSE);
1. kernel trace + stats of cfg2 and cfg3: average dispatch duration, set
   beside bench.py's own HIP-event time for the same launches;
2. HBM traffic of cfg2 and cfg3: FETCH_SIZE and WRITE_SIZE per dispatch, each
   scaled by what the counter reads for a device copy of known size
   (bench.py ``--copy-probe-mib``), against the algorithmic bytes;
3. utilisation of cfg2 and cfg3: the cycles the shader engines had waves
   (SQ_BUSY_CYCLES over the engine count: the kernel's span in shader
   clocks), the MFMA busy fraction of those cycles, a lower bound on the clock
   (those cycles over the dispatch's duration, which also holds the launch's
   set-up and drain), VALU/MFMA/LDS instruction counts, LDS bank conflicts,
   plus the VGPR/AGPR/SGPR/LDS allocation the profiler records for the
   dispatch.  MFMA cycles per SIMD over (duration x 2.4 GHz) is the fraction
   of the 2516.6 TFLOP/s peak those dispatches reach, a check on the
   HIP-event figure that needs no timer.

The JSON (``--json``) carries the figures ``bench.py`` quotes in its
``roofline`` object (traffic, MFMA busy, clock) with the run they came from.

    python -m fmha_native_amd.rocprof --forms cfg4:auto,cfg5:auto,cfg5:regular --summary profiles/NAME.md

profiles other workloads in the kernel forms named (``auto`` = the
launcher's choice; a form the launcher did not pick, beside it, shows what
the choice gains): per workload and form, ``bench.py --only`` unprofiled, a
kernel trace of every kernel of a step (the balanced causal form is two: its
items, then the merge of its split M-tiles), the utilisation counters of
each kernel, with the clock from the same dispatches, and each kernel's HBM
traffic (FETCH_SIZE and WRITE_SIZE passes, scaled by a device copy's).

    python -m fmha_native_amd.rocprof --short --summary profiles/NAME.md

profiles the short-sequence shapes (262,144 query rows, H16, S 64-512,
dense and causal) through the bench_fmha_fwd CLI in the launcher's choice
and in the regular form, cfg1 (kernel-trace duration beside the CLI's
per-call time), and device copies of the same byte count (the HBM rate a
plain stream reaches at this size).
"""
import argparse
import glob
import json
import os
import shlex
import sqlite3
import subprocess
import sys
from collections import defaultdict

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PEAK_BF16_TFLOPS = 2516.6
NUM_XCD = 8
NUM_SIMD = 256 * 4
NUM_SE = 32  # shader engines (8 XCDs x 4); read from the profiler's agent record where present

UTIL_COUNTERS = ["GRBM_GUI_ACTIVE", "SQ_WAVES", "SQ_BUSY_CYCLES", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU",
                 "SQ_INSTS_MFMA", "SQ_INSTS_LDS", "SQ_LDS_BANK_CONFLICT", "SQ_INSTS_VALU_TRANS_F32"]
WORKLOADS = {
    "cfg2": {"flops": 4.0 * 4 * 16 * 2048 * 2048 * 64, "bytes": 67108864, "desc": "dense B4 H16 S2048"},
    "cfg3": {"flops": 4.0 * 16 * 8192 * 8192 * 64 * 0.5, "bytes": 67633152, "desc": "causal B1 H16 S8192 + LSE"},
}


def _argv():
    """This run's arguments, quoted for a shell."""
    return " ".join(shlex.quote(a) for a in sys.argv[1:])


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
    shown = " ".join("python3" if c == sys.executable else shlex.quote(c) for c in cmd[4:]).replace(ROOT + "/", "")
    return dbs[0], json.loads(lines[-1]), shown


def _kernel_stats(db):
    con = sqlite3.connect(db)
    # top_kernels reports durations in microseconds
    return [dict(name=n, calls=c, avg_us=a) for n, c, _t, a, _p in con.execute("select * from top_kernels")]


def _timed_stats(db, line):
    """Per-kernel average duration (us) of the dispatches bench.py --only
    timed back to back (after its ramp and warm-up launches; each step is one
    dispatch of every kernel of the form), from the trace's own timestamps."""
    con = sqlite3.connect(db)
    per = defaultdict(list)
    for name, t0, t1 in con.execute("select name, start, end from kernels order by start"):
        if name.startswith("fmha_fwd"):
            per[name].append((t1 - t0) / 1e3)
    first = line["ramp_launches"] + line["warmup"]
    out = {}
    for name, d in per.items():
        timed = d[first:first + line["steps"]]
        if len(timed) == line["steps"]:
            out[name] = sum(timed) / len(timed)
    return out


def _counters(db, kernel_prefix="fmha_fwd"):
    """Per-dispatch counter values (summed over the chip), averaged over the
    dispatches of each kernel after its first; also the dispatches' own
    average duration (ns) from the same pass."""
    con = sqlite3.connect(db)
    per = defaultdict(float)
    dur = {}
    res = {}
    q = ("select dispatch_id, kernel_name, counter_name, value, vgpr_count, accum_vgpr_count, sgpr_count, "
         "lds_block_size, start, end from counters_collection")
    for disp, kname, cname, val, vgpr, agpr, sgpr, lds, t0, t1 in con.execute(q):
        per[(kname, cname, disp)] += val
        dur[(kname, disp)] = t1 - t0
        res.setdefault(kname, {"vgpr": vgpr, "agpr": agpr, "sgpr": sgpr, "lds_bytes": lds})
    agg = defaultdict(list)
    for (k, c, d), v in per.items():
        agg[(k, c)].append((d, v))
    out = {}
    for (k, c), dv in agg.items():
        if k.startswith(kernel_prefix) or not kernel_prefix:
            dv.sort()
            vals = [v for _, v in (dv[1:] if len(dv) > 1 else dv)]
            e = out.setdefault(k, dict(res[k]))
            e[c] = sum(vals) / len(vals)
            ds = sorted((d, t) for (kk, d), t in dur.items() if kk == k)
            ds = ds[1:] if len(ds) > 1 else ds
            e["dispatch_ns"] = sum(t for _, t in ds) / len(ds)
            e["dispatches"] = len(ds)
    return out


def _num_se(db):
    """Shader engines of the profiled GPU (the agent record's
    num_shader_banks), else NUM_SE."""
    try:
        con = sqlite3.connect(db)
        for (ext,) in con.execute("select extdata from rocpd_info_agent where type = 'GPU'"):
            n = json.loads(ext or "{}").get("num_shader_banks")
            if n:
                return int(n)
    except sqlite3.Error:
        pass
    return NUM_SE


def _util_row(c, n_se=NUM_SE):
    """(clock lower bound in GHz, MFMA busy fraction of the cycles the
    shader engines had waves, fraction of the bf16 peak).

    SQ_BUSY_CYCLES summed over the engines, divided by their count, is the
    kernel's span in shader clocks; the dispatch duration the profiler
    records also holds the launch's set-up and drain, so cycles over duration
    bound the clock from below.  (GRBM_GUI_ACTIVE / 8 over the duration
    counts outside the waves' span and reads above the clock the kernel
    measures itself with s_memtime against s_memrealtime.)  The fraction of
    peak needs no clock: MFMA cycles per SIMD over duration x 2.4 GHz."""
    active = c["SQ_BUSY_CYCLES"] / n_se
    ghz = active / c["dispatch_ns"]
    mfma_per_simd = c["SQ_VALU_MFMA_BUSY_CYCLES"] / NUM_SIMD
    return ghz, mfma_per_simd / active, mfma_per_simd / (c["dispatch_ns"] * 2.4)


def profile_gemm(args):
    """A bf16 library GEMM (torch.matmul, N x N x N) beside cfg2 and cfg3 on
    one box: TFLOP/s from HIP events, and from one counter pass each the
    active cycles, the clock they imply, MFMA busy and busy x clock, the
    product the chip's power cap holds about constant across this kernel's
    forms."""
    n = args.gemm
    md = [f"# MFMA rate under the power cap: bf16 GEMM {n}³ beside cfg2 and cfg3 (MI355X, one GPU)", "",
          f"Every figure from one run of `python -m fmha_native_amd.rocprof {_argv()}` on one box (repo root; each "
          "pass its own process under `timeout -s KILL`). The GEMM is `torch.matmul` on bf16 operands (the "
          "library's kernel, hipBLASLt on this image); cfg2 and cfg3 run this library's automatic form.", ""]
    runs = [("gemm", _bench("--gemm-probe", str(n), "--steps", "50", "--warmup", "5"), 2.0 * n ** 3),
            ("cfg2", _bench("--only", "cfg2", "--steps", str(args.steps), "--warmup", "10"), WORKLOADS["cfg2"]["flops"]),
            ("cfg3", _bench("--only", "cfg3", "--steps", str(args.steps // 2), "--warmup", "10"),
             WORKLOADS["cfg3"]["flops"])]
    rows, cmds = [], []
    for tag, prog, flops in runs:
        print(f"[rocprof] bench: {' '.join(prog)}", flush=True)
        r = subprocess.run(["timeout", "-s", "KILL", "300", *prog], capture_output=True, text=True)
        line = json.loads([l for l in r.stdout.splitlines() if l.startswith("{")][-1])
        ms = line.get("ms_per_gemm") or line["ms_per_step"]
        cmds.append(" ".join("python3" if c == sys.executable else shlex.quote(c) for c in prog).replace(ROOT + "/", ""))
        db, _l, ucmd = _run(f"pmc_util_{tag}", ["--pmc", *UTIL_COUNTERS], prog, args.out, 180)
        cmds.append(ucmd)
        cs = _counters(db, kernel_prefix="" if tag == "gemm" else "fmha_fwd")
        # the GEMM pass also runs the operands' fill kernels: take the kernel
        # with the most time
        kname = max(cs, key=lambda k: cs[k]["dispatch_ns"] * cs[k]["dispatches"])
        c = cs[kname]
        ghz, busy, frac = _util_row(c, _num_se(db))
        rows.append((tag, kname, ms, flops / (ms * 1e-3) / 1e12, c, ghz, busy, frac))
    md += ["| workload | kernel | ms per launch (events) | TFLOP/s | % of 2516.6 | active cycles | clock ≥ | "
           "MFMA busy | busy × clock | VALU instr per MFMA |", "|---|---|---|---|---|---|---|---|---|---|"]
    for tag, kname, ms, tf, c, ghz, busy, frac in rows:
        valu = c.get("SQ_INSTS_VALU", 0) / max(1.0, c.get("SQ_INSTS_MFMA", 0))
        md.append(f"| {tag} | `{kname.split('(')[0][:60]}` | {ms:.4f} | {tf:.1f} | {100 * tf / PEAK_BF16_TFLOPS:.1f}% | "
                  f"{c['SQ_BUSY_CYCLES'] / _num_se(db) / 1e3:.1f}k | {ghz:.3f} GHz | {100 * busy:.1f}% | "
                  f"{busy * ghz:.3f} GHz | {valu:.2f} |")
    md += ["", "Active cycles = SQ_BUSY_CYCLES / shader engines; clock ≥ active cycles over the dispatch's duration "
               "in the counter pass; MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES per SIMD over the active cycles; busy × "
               "clock is the MFMA rate in GHz-equivalents of a fully busy SIMD (2.4 GHz at 100 % would be the "
               "2516.6 TFLOP/s peak). VALU instructions per MFMA count every VALU instruction the counter sees "
               "(MFMA included).", "", "Commands:", ""] + [f"    {c}" for c in cmds] + [""]
    path = args.summary or os.path.join(args.out, "gemm.md")
    with open(path, "w") as f:
        f.write("\n".join(md))
    print("\n".join(md), flush=True)


def profile_forms(args):
    """Kernel trace and utilisation counters of other workloads in the forms
    ``args.forms`` names ("cfg4:auto,cfg5:regular", ...)."""
    from fmha_native_amd.problem import workload

    md = ["# rocprofv3 summary — fmha_fwd_d64_bf16 on " + ", ".join(args.forms.split(",")), "",
          f"MI355X (gfx950), one GPU, every figure from one run of `python -m fmha_native_amd.rocprof {_argv()}` "
          "on one box (the passes below, from the repo root, each under `timeout -s KILL`). "
          "`auto` is the launcher's own choice. TFLOP/s use the repo FLOP convention "
          "(4·B·H·Sq·Sk·64, ×0.5 causal; varlen counts max(S) for every sequence, and the exact count of "
          "visible (q, k) pairs is given beside it).", ""]
    fig = {"made_by": f"python -m fmha_native_amd.rocprof {_argv()}", "forms": {}}
    # the counters' scale, from a device copy of known size (as the main run)
    copy = {}
    copy_cmds = []
    for name, counter in (("pmc_copy_fetch", "FETCH_SIZE"), ("pmc_copy_write", "WRITE_SIZE")):
        db, _l, cmd = _run(name, ["--pmc", counter], _bench("--copy-probe-mib", "256", "--steps", "5"), args.out, 120)
        copy_cmds.append(cmd)
        copy[counter] = 256 * 1024 / max(v[counter] for v in _counters(db, kernel_prefix="").values())
    md += [f"HBM traffic: FETCH_SIZE and WRITE_SIZE (KiB per dispatch, each in a pass of its own) scaled by what "
           f"each reads for a 256 MiB device copy (x{copy['FETCH_SIZE']:.3f}, x{copy['WRITE_SIZE']:.3f}), against "
           "the algorithmic bytes (Q, K, V read once, O and LSE written once):", ""]
    md += [f"    {c}" for c in copy_cmds] + [""]
    for spec in args.forms.split(","):
        wl, form = spec.split(":")
        prob, _mult = workload(wl)
        tag = f"{wl}_{form}".replace("|", "-")
        steps = str(args.steps // 4 if wl != "cfg1" else args.steps)
        # unprofiled
        cmd = _bench("--only", wl, "--variant", form, "--steps", steps, "--warmup", "5")
        print(f"[rocprof] bench: {' '.join(cmd)}", flush=True)
        r = subprocess.run(["timeout", "-s", "KILL", "300", *cmd], capture_output=True, text=True)
        line = json.loads([l for l in r.stdout.splitlines() if l.startswith("{")][-1])
        # kernel trace
        db, tline, tcmd = _run(f"trace_{tag}", ["--kernel-trace", "--stats"],
                               _bench("--only", wl, "--variant", form, "--steps", steps, "--warmup", "5"),
                               args.out, 300)
        ks = [k for k in _kernel_stats(db) if k["name"].startswith("fmha_fwd")]
        timed = _timed_stats(db, tline)
        for k in ks:
            k["avg_all_us"], k["avg_us"] = k["avg_us"], timed.get(k["name"], k["avg_us"])
        step_us = sum(k["avg_us"] for k in ks)
        # counters
        udb, _l, ucmd = _run(f"pmc_util_{tag}", ["--pmc", *UTIL_COUNTERS],
                             _bench("--only", wl, "--variant", form, "--steps", "5", "--warmup", "1"), args.out, 120)
        cs = _counters(udb)
        n_se = _num_se(udb)
        traffic, tcmds = {}, []
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            tdb, _l, c2 = _run(f"pmc_{counter.split('_')[0].lower()}_{tag}", ["--pmc", counter],
                               _bench("--only", wl, "--variant", form, "--steps", "5", "--warmup", "1"), args.out, 120)
            tcmds.append(c2)
            for kname, v in _counters(tdb).items():
                traffic.setdefault(kname, {})[counter] = v[counter] * copy[counter] * 1024
        hbm = sum(t.get("FETCH_SIZE", 0) + t.get("WRITE_SIZE", 0) for t in traffic.values())
        alg = prob.io_bytes()
        flops = prob.flops()
        md += [f"## {wl} ({prob.name}), form `{form}` → {line['form']}", "",
               f"bench.py (back-to-back HIP events): {line['ms_per_step'] * 1e3:.2f} us per step, "
               f"{line['tflops']:.1f} TFLOP/s ({100 * line['tflops'] / PEAK_BF16_TFLOPS:.1f}% of 2516.6)"
               + (f"; exact-count {prob.exact_flops() / (line['ms_per_step'] * 1e-3) / 1e12:.1f} TFLOP/s"
                  if prob.varlen else "") + ".", "",
               "| kernel | dispatches | trace avg, timed (all) | active cycles | clock ≥ | MFMA busy | "
               "fraction of peak | VGPR / AGPR / SGPR | LDS bytes |", "|---|---|---|---|---|---|---|---|---|"]
        entry = {"bench": line, "trace_step_us": round(step_us, 3),
                 "trace_tflops": round(flops / (step_us * 1e-6) / 1e12, 2), "kernels": {}}
        for k in ks:
            c = cs.get(k["name"])
            if c is None:
                continue
            ghz, busy, frac = _util_row(c, n_se)
            if c["dispatch_ns"] < 20e3:
                # a dispatch this short is mostly set-up and drain: clock and
                # busy are not meaningful for it
                md.append(f"| `{k['name']}` | {k['calls']} | {k['avg_us']:.2f} ({k['avg_all_us']:.2f}) us | — | — | — | "
                          f"— | {c['vgpr']} / {c['agpr']} / {c['sgpr']} | {c['lds_bytes']} |")
            else:
                md.append(f"| `{k['name']}` | {k['calls']} | {k['avg_us']:.2f} ({k['avg_all_us']:.2f}) us | "
                          f"{c['SQ_BUSY_CYCLES'] / n_se / 1e3:.1f}k | {ghz:.3f} GHz | "
                          f"{100 * busy:.1f}% | {100 * frac:.1f}% | {c['vgpr']} / {c['agpr']} / {c['sgpr']} | "
                          f"{c['lds_bytes']} |")
            entry["kernels"][k["name"]] = {"trace_avg_us": round(k["avg_us"], 3), "calls": k["calls"],
                                           "clock_ghz": round(ghz, 4), "mfma_busy": round(busy, 4),
                                           "frac_from_counters": round(frac, 4),
                                           **{n: c.get(n, 0) for n in UTIL_COUNTERS}}
        md += ["", "Per dispatch of the counter pass: active cycles = SQ_BUSY_CYCLES / engines (the cycles the "
                   "shader engines had waves); MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES per SIMD over those cycles; "
                   "clock ≥ those cycles over the dispatch's "
                   "duration; fraction of peak = MFMA cycles per SIMD over duration × 2.4 GHz (— for a dispatch under "
                   "20 us); VGPR as rocprofv3 records it (4 registers per granule where gfx950 wave64 allocates 8: "
                   "128 shown = 256 allocated).", "",
               f"Kernel-trace time per step (sum of the kernels' averages): {step_us:.2f} us = "
                   f"{flops / (step_us * 1e-6) / 1e12:.1f} TFLOP/s.", "",
               "HBM traffic per step: " + "; ".join(
                   f"`{k.split('(')[0]}` fetch {t.get('FETCH_SIZE', 0) / 1e6:.1f} MB, write "
                   f"{t.get('WRITE_SIZE', 0) / 1e6:.1f} MB" for k, t in sorted(traffic.items()))
               + f"; total {hbm / 1e6:.1f} MB against {alg / 1e6:.1f} MB algorithmic ({hbm / alg:.2f}x).", "",
               "Commands:", "",
               f"    python3 bench.py --only {wl} --variant {shlex.quote(form)} --steps {steps} --warmup 5",
               f"    {tcmd}", f"    {ucmd}"] + [f"    {c}" for c in tcmds] + [""]
        entry["traffic"] = {"hbm_bytes": int(hbm), "algorithmic_bytes": int(alg),
                            "kernels": {k: {c: int(v) for c, v in t.items()} for k, t in traffic.items()}}
        fig["forms"][tag] = entry
    path = args.summary or os.path.join(args.out, "forms.md")
    with open(path, "w") as f:
        f.write("\n".join(md))
    print("\n".join(md), flush=True)
    if args.json:
        with open(args.json, "w") as f:
            json.dump(fig, f, indent=1)


CLI = os.path.join(ROOT, "fmha_native_amd", "bench_fmha_fwd")
def _cli_avg(stdout, key):
    for l in stdout.splitlines():
        if l.startswith(key):
            return float(l.split()[len(key.split())])
    raise RuntimeError(f"no '{key}' line")


def profile_short(args):
    """Short sequences through the bench CLI: kernel trace per shape and form."""
    shapes = [(m, 16384 // sq, sq) for m in (0, 1) for sq in (64, 128, 192, 256, 512)]
    md = ["# Short sequences: achieved HBM bandwidth (MI355X, one GPU)", "",
          f"Every figure from one run of `python -m fmha_native_amd.rocprof {_argv()}` on one box (repo root, "
          "`TMPDIR=/tmp`); each pass is its own process under `timeout -s KILL`:", "",
          "    rocprofv3 --kernel-trace --stats -d <out>/<tag> -o run -- fmha_native_amd/bench_fmha_fwd "
          "-b <B> -h 16 -s <S> --mask <0|1> --lse 1 --dist normal --warmup 5 --iters 100 --variant <auto|regular>",
          "", "Every shape holds about 262,144 query rows (B = ⌊16,384 / S⌋, H = 16), so the algorithmic HBM "
          "traffic is about the same: Q, K, V read once and O written once, 4·B·H·S·64·2 bytes, plus the 4-byte "
          "LSE per row, 135.3 MB at B·S = 16,384 (S192: 133.7 MB). GB/s = those bytes ÷ the kernel's average "
          "dispatch duration (`top_kernels`, 205 dispatches: "
          "5 warm-up, 100 timed one by one, 100 back to back); the percentage is of MI355X's 8 TB/s. `auto` is "
          "the launcher's choice.", ""]
    # device copies of the same traffic: 2 x 67.1 MB (read + write) and a 3:1 read/write mix
    db, _l, ccmd = _run("short_copy", ["--kernel-trace", "--stats"],
                        _bench("--copy-probe-mib", "64", "--steps", "100"), args.out, 120)
    copy = [k for k in _kernel_stats(db)]
    cp = max(copy, key=lambda k: k["calls"])
    nbytes = 2 * (64 << 20)
    md += [f"Device copy of 64 MiB (134.2 MB moved, `{cp['name']}`): {cp['avg_us']:.2f} us per copy = "
           f"{nbytes / (cp['avg_us'] * 1e-6) / 1e9:,.0f} GB/s ({100 * nbytes / (cp['avg_us'] * 1e-6) / 8e12:.0f} % of "
           f"8 TB/s): the rate a plain stream of this size reaches.", "", f"    {ccmd}", "",
           "| shape | form | kernel | avg µs | GB/s | of 8 TB/s | of the copy rate | TFLOP/s |",
           "|---|---|---|---|---|---|---|---|"]
    copy_gbs = nbytes / (cp["avg_us"] * 1e-6) / 1e9
    res = {}
    for m, b, sq in shapes:
        for form in ("auto", "regular"):
            tag = f"short_m{m}_b{b}_s{sq}_{form}"
            d = os.path.join(args.out, tag)
            cmd = ["timeout", "-s", "KILL", "120", "rocprofv3", "--kernel-trace", "--stats", "-d", d, "-o", "run",
                   "--", CLI, "-b", str(b), "-h", "16", "-s", str(sq), "--mask", str(m), "--lse", "1", "--dist",
                   "normal", "--warmup", "5", "--iters", "100", "--variant", form]
            print(f"[rocprof] {tag}", flush=True)
            r = subprocess.run(cmd, capture_output=True, text=True)
            dbs = glob.glob(os.path.join(d, "**", "*_results.db"), recursive=True)
            if not dbs or "Avg:" not in r.stdout:
                raise RuntimeError(f"{tag} failed (rc={r.returncode}): {r.stderr[-500:]}")
            k = [k for k in _kernel_stats(dbs[0]) if k["name"].startswith("fmha_fwd")][0]
            rows = b * 16 * sq
            gbs = (4 * rows * 64 * 2 + 4 * rows) / (k["avg_us"] * 1e-6) / 1e9
            flops = 4.0 * b * 16 * sq * sq * 64 * (0.5 if m else 1.0)
            res[(m, sq, form)] = k["avg_us"]
            md.append(f"| {'causal' if m else 'dense'} B{b} H16 S{sq} | {form} | `{k['name']}` | {k['avg_us']:.2f} | "
                      f"{gbs:,.0f} | {100 * gbs / 8000:.0f} % | {100 * gbs / copy_gbs:.0f} % | "
                      f"{flops / (k['avg_us'] * 1e-6) / 1e12:.0f} |")
    # cfg1: the kernel's duration beside the per-call times of unprofiled runs
    md += ["", "## cfg1 (B1 H2 S128 + LSE): kernel duration and per-call time", "",
           "| form | kernel | kernel-trace avg |", "|---|---|---|"]
    cli_args = ["-b", "1", "-h", "2", "-s", "128", "--mask", "0", "--lse", "1", "--dist", "normal", "--warmup", "5",
                "--iters", "100"]
    for form in ("auto", "regular", "short"):
        tag = f"cfg1_{form}"
        d = os.path.join(args.out, tag)
        cmd = ["timeout", "-s", "KILL", "120", "rocprofv3", "--kernel-trace", "--stats", "-d", d, "-o", "run", "--",
               CLI, *cli_args, "--variant", form]
        r = subprocess.run(cmd, capture_output=True, text=True)
        dbs = glob.glob(os.path.join(d, "**", "*_results.db"), recursive=True)
        if not dbs or "Avg:" not in r.stdout:
            raise RuntimeError(f"{tag} failed (rc={r.returncode}): {r.stderr[-500:]}")
        k = [k for k in _kernel_stats(dbs[0]) if k["name"].startswith("fmha_fwd")][0]
        md.append(f"| {form} | `{k['name']}` | {k['avg_us']:.2f} us |")
    r = subprocess.run(["timeout", "-s", "KILL", "120", CLI, *cli_args], capture_output=True, text=True)
    b = subprocess.run(["timeout", "-s", "KILL", "300", *_bench("--only", "cfg1", "--steps", "2000", "--warmup", "20")],
                       capture_output=True, text=True)
    line = json.loads([l for l in b.stdout.splitlines() if l.startswith("{")][-1])
    md += ["", "Per-call time of the launcher's choice, unprofiled:", "",
           "| protocol | per call |", "|---|---|",
           f"| `bench.py --only cfg1 --steps 2000`: back to back between two events (the `bench.py` value) | "
           f"{line['ms_per_step'] * 1e3:.2f} us |",
           f"| same run, the reference's protocol: events around each launch, synchronised per launch | "
           f"{line['reference_protocol_ms'] * 1e3:.2f} us |",
           f"| the CLI, `bench_fmha_fwd {' '.join(cli_args)}`: `Avg:` (the reference's protocol, printed to "
           f"1 us) | {_cli_avg(r.stdout, 'Avg:') * 1e3:.0f} us |",
           f"| the CLI: `back-to-back avg:` | {_cli_avg(r.stdout, 'back-to-back avg:') * 1e3:.0f} us |", "",
           "The launch is latency-bound: 0.13 MB moved. Back to back the launches overlap the host's submission "
           "of the next one; the reference's protocol adds the host's launch latency to every call.", ""]
    path = args.summary or os.path.join(args.out, "short.md")
    with open(path, "w") as f:
        f.write("\n".join(md))
    print("\n".join(md), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default=os.path.join(ROOT, "rocprof_out"))
    ap.add_argument("--summary", default=None, help="markdown summary path (default: <out>/summary.md)")
    ap.add_argument("--json", default=None, help="also write the figures bench.py quotes here")
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--forms", default=None,
                    help="profile these workload:form pairs instead (e.g. cfg4:auto,cfg5:auto,cfg5:regular)")
    ap.add_argument("--short", action="store_true", help="profile the short-sequence shapes and cfg1 instead")
    ap.add_argument("--gemm", type=int, default=0,
                    help="profile a bf16 N x N x N library GEMM beside cfg2 and cfg3 instead")
    args = ap.parse_args()
    os.makedirs(args.out, exist_ok=True)
    if args.short:
        profile_short(args)
        return
    if args.gemm:
        profile_gemm(args)
        return
    if args.forms:
        profile_forms(args)
        return
    md = ["# rocprofv3 summary — fmha_fwd_d64_bf16 on cfg2 (dense B4 H16 S2048) and cfg3 (causal B1 H16 "
          "S8192 + LSE)", "",
          f"MI355X (gfx950), one GPU, every figure from one run of `python -m fmha_native_amd.rocprof {_argv()}` "
          "on one box (the passes below, from the repo root, each under `timeout -s KILL`).", ""]
    fig = {"made_by": f"python -m fmha_native_amd.rocprof {_argv()}"}

    # 0. bench.py itself, unprofiled
    cmd = [sys.executable, os.path.join(ROOT, "bench.py"), "--steps", str(args.steps), "--warmup", "20",
           "--no-cpu-baseline", "--no-extra"]
    print(f"[rocprof] bench: {' '.join(cmd)}", flush=True)
    r = subprocess.run(["timeout", "-s", "KILL", "300", *cmd], capture_output=True, text=True)
    line = json.loads([l for l in r.stdout.splitlines() if l.startswith("{")][-1])
    bench = {"cfg2": {"ms_per_step": line["ms_per_step"], "tflops": line["value"]},
             "cfg3": {"ms_per_step": line["also"]["ms_per_step"], "tflops": line["also"]["value"]}}
    fig["bench"] = {"command": f"python3 bench.py --steps {args.steps} --warmup 20 --no-cpu-baseline --no-extra",
                    **bench}
    md += ["## bench.py on this box (HIP events on the launch stream, back-to-back launches)", "",
           f"    python3 bench.py --steps {args.steps} --warmup 20 --no-cpu-baseline --no-extra", "",
           "| workload | ms per launch | TFLOP/s | % of 2516.6 |", "|---|---|---|---|"]
    for wl in ("cfg2", "cfg3"):
        b = bench[wl]
        md.append(f"| {wl} | {b['ms_per_step']:.5f} | {b['tflops']:.1f} | {100 * b['tflops'] / PEAK_BF16_TFLOPS:.1f}% |")
    md.append("")

    # 1. kernel trace
    md += ["## Kernel trace (average dispatch duration vs bench.py's HIP events in the same process)", "",
           "`timed` = the dispatches bench.py timed back to back (after its 0.1 s clock ramp and warm-up); `all` = "
           "every dispatch of the run, the ramp's included.", "",
           "| workload | kernel | dispatches | rocprofv3 avg, timed | rocprofv3 avg, all | bench.py HIP-event avg | "
           "TFLOP/s (trace, timed) | % of 2516.6 |",
           "|---|---|---|---|---|---|---|---|"]
    cmds = []
    trace = {}
    for wl in ("cfg2", "cfg3"):
        steps = args.steps if wl == "cfg2" else args.steps // 2
        db, pline, cmd = _run(f"trace_{wl}", ["--kernel-trace", "--stats"],
                              _bench("--only", wl, "--steps", str(steps), "--warmup", "10"), args.out, 300)
        cmds.append(cmd)
        k = [s for s in _kernel_stats(db) if s["name"].startswith("fmha_fwd")][0]
        timed = _timed_stats(db, pline)[k["name"]]
        tf = WORKLOADS[wl]["flops"] / (timed * 1e-6) / 1e12
        trace[wl] = {"kernel": k["name"], "avg_us": timed, "avg_all_us": k["avg_us"],
                     "bench_us": pline["ms_per_step"] * 1e3, "tflops": tf}
        md.append(f"| {wl} | `{k['name']}` | {k['calls']} | {timed:.2f} us | {k['avg_us']:.2f} us | "
                  f"{pline['ms_per_step'] * 1e3:.2f} us | {tf:.1f} | {100 * tf / PEAK_BF16_TFLOPS:.1f}% |")
    md += ["", "Commands:", ""] + [f"    {c}" for c in cmds] + [""]

    # 2. traffic
    cmds = []
    vals = {}
    passes = [("pmc_copy_fetch", "FETCH_SIZE", _bench("--copy-probe-mib", "256", "--steps", "5")),
              ("pmc_copy_write", "WRITE_SIZE", _bench("--copy-probe-mib", "256", "--steps", "5"))]
    for wl in ("cfg2", "cfg3"):
        passes += [(f"pmc_fetch_{wl}", "FETCH_SIZE", _bench("--only", wl, "--steps", "5", "--warmup", "1")),
                   (f"pmc_write_{wl}", "WRITE_SIZE", _bench("--only", wl, "--steps", "5", "--warmup", "1"))]
    for name, counter, prog in passes:
        db, _line, cmd = _run(name, ["--pmc", counter], prog, args.out, 120)
        cmds.append(cmd)
        c = _counters(db, kernel_prefix="")
        if name.startswith("pmc_copy"):
            vals[name] = max(v[counter] for v in c.values())
        else:
            vals[name] = [v[counter] for k, v in c.items() if k.startswith("fmha_fwd")][0]
    copy_kib = 256 * 1024
    fs, ws = copy_kib / vals["pmc_copy_fetch"], copy_kib / vals["pmc_copy_write"]
    md += ["## HBM traffic (per dispatch)", "",
           f"FETCH_SIZE and WRITE_SIZE (KiB per dispatch) are scaled by what each reads for a 256 MiB device copy "
           f"(expected 262,144 KiB each way): FETCH_SIZE read {vals['pmc_copy_fetch']:,.0f} KiB (x{fs:.3f}), "
           f"WRITE_SIZE {vals['pmc_copy_write']:,.0f} KiB (x{ws:.3f}).", "",
           "| workload | FETCH_SIZE (KiB) | WRITE_SIZE (KiB) | scaled bytes | algorithmic bytes | ratio |",
           "|---|---|---|---|---|---|"]
    traffic = {}
    for wl in ("cfg2", "cfg3"):
        t = vals[f"pmc_fetch_{wl}"] * fs * 1024 + vals[f"pmc_write_{wl}"] * ws * 1024
        alg = WORKLOADS[wl]["bytes"]
        traffic[wl] = {"fetch_kib": vals[f"pmc_fetch_{wl}"], "write_kib": vals[f"pmc_write_{wl}"],
                       "hbm_bytes": int(t), "algorithmic_bytes": alg}
        md.append(f"| {wl} | {vals[f'pmc_fetch_{wl}']:,.0f} | {vals[f'pmc_write_{wl}']:,.0f} | {t / 1e6:.2f} MB | "
                  f"{alg / 1e6:.2f} MB | {t / alg:.3f} |")
    md += ["", "Algorithmic bytes: Q+K+V read once, O (and LSE) written once.", "", "Commands:", ""]
    md += [f"    {c}" for c in cmds] + [""]

    # 3. utilisation, with the clock from each dispatch's own duration
    md += ["## Utilisation counters (per dispatch, summed over the chip)", "",
           "Active cycles = SQ_BUSY_CYCLES / shader engines: the kernel's span in shader clocks (waves present). MFMA "
           "busy = SQ_VALU_MFMA_BUSY_CYCLES / 1024 SIMDs over the active cycles. Clock ≥ active cycles over the "
           "dispatch's duration in this pass (the duration also holds the launch's set-up and drain). Fraction of "
           "peak = MFMA cycles per SIMD over duration × 2.4 GHz (the clock the 2516.6 TFLOP/s figure assumes), "
           "which needs no clock estimate. GRBM_GUI_ACTIVE / 8 over the duration is not used: it counts outside the "
           "waves' span and reads above the clock the kernel measures itself.",
           ""]
    cmds = []
    rows = []
    for wl in ("cfg2", "cfg3"):
        db, _line, cmd = _run(f"pmc_util_{wl}", ["--pmc", *UTIL_COUNTERS],
                              _bench("--only", wl, "--steps", "10", "--warmup", "1"), args.out, 120)
        cmds.append(cmd)
        k, c = list(_counters(db).items())[0]
        n_se = _num_se(db)
        ghz, mfma_busy, frac = _util_row(c, n_se)
        iters = c["SQ_INSTS_MFMA"] / 16.0  # 16 MFMA per wave per 64-key tile
        rows.append((wl, k, c, ghz, mfma_busy, iters, frac, c["SQ_BUSY_CYCLES"] / n_se))
    md += ["| | " + " | ".join(r[0] for r in rows) + " |", "|---|" + "---|" * len(rows)]
    md.append("| kernel | " + " | ".join(f"`{r[1]}`" for r in rows) + " |")
    md.append("| VGPR / AGPR / SGPR (rocprofv3 dispatch fields) | "
              + " | ".join(f"{r[2]['vgpr']} / {r[2]['agpr']} / {r[2]['sgpr']}" for r in rows) + " |")
    md.append("| LDS bytes per block | " + " | ".join(f"{r[2]['lds_bytes']}" for r in rows) + " |")
    md.append("| dispatch duration in this pass | " + " | ".join(f"{r[2]['dispatch_ns'] / 1e3:.2f} us" for r in rows)
              + " |")
    md.append("| active cycles (SQ_BUSY_CYCLES / shader engines) | "
              + " | ".join(f"{r[7]:,.0f}" for r in rows) + " |")
    md.append("| clock ≥ (active cycles / duration) | " + " | ".join(f"{r[3]:.3f} GHz" for r in rows) + " |")
    md.append("| MFMA busy (per SIMD, of active cycles) | " + " | ".join(f"{100 * r[4]:.1f}%" for r in rows) + " |")
    md.append("| fraction of peak (MFMA cycles per SIMD / (duration x 2.4 GHz)) | "
              + " | ".join(f"{100 * r[6]:.1f}%" for r in rows) + " |")
    for name in UTIL_COUNTERS[1:]:
        md.append(f"| {name} | " + " | ".join(f"{r[2].get(name, 0):,.0f}" for r in rows) + " |")
    md.append("| VALU instr per wave per 64-key tile (incl. 16 MFMA) | "
              + " | ".join(f"{r[2]['SQ_INSTS_VALU'] / r[5]:.1f}" for r in rows) + " |")
    md.append("| LDS instr per wave per tile | " + " | ".join(f"{r[2]['SQ_INSTS_LDS'] / r[5]:.1f}" for r in rows) + " |")
    md += ["", "rocprofv3's VGPR field reads the descriptor's granule count as 4 registers per granule where gfx950 "
           "wave64 allocates 8 (so 128 shown = 256 allocated: two waves per SIMD); `tests/test_codegen.py` checks "
           "the compiler's own counts.", "", "Commands:", ""] + [f"    {c}" for c in cmds] + [""]

    for wl, k, c, ghz, busy, _it, frac, _active in rows:
        fig[wl] = {
            "kernel": k,
            "workload": WORKLOADS[wl]["desc"],
            "bench_ms_per_step": bench[wl]["ms_per_step"],
            "bench_tflops": bench[wl]["tflops"],
            "trace_avg_us": round(trace[wl]["avg_us"], 3),
            "trace_avg_all_dispatches_us": round(trace[wl]["avg_all_us"], 3),
            "trace_tflops": round(trace[wl]["tflops"], 2),
            "trace_bench_us": round(trace[wl]["bench_us"], 3),
            "counter_dispatch_us": round(c["dispatch_ns"] / 1e3, 3),
            "clock_ghz": round(ghz, 4),
            "mfma_busy": round(busy, 4),
            "frac_from_counters": round(frac, 4),
            "hbm_bytes_per_launch": traffic[wl]["hbm_bytes"],
            "algorithmic_bytes": traffic[wl]["algorithmic_bytes"],
            "fetch_kib_per_dispatch": traffic[wl]["fetch_kib"],
            "write_kib_per_dispatch": traffic[wl]["write_kib"],
        }
    fig["fetch_scale"], fig["write_scale"] = round(fs, 4), round(ws, 4)

    path = args.summary or os.path.join(args.out, "summary.md")
    with open(path, "w") as f:
        f.write("\n".join(md))
    print("\n".join(md), flush=True)
    if args.json:
        with open(args.json, "w") as f:
            json.dump(fig, f, indent=1)


if __name__ == "__main__":
    main()
