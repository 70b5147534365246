"""Interleaved A/B timing of kernel forms and block orders on one GPU.

    python -m fmha_native_amd.abtest SPEC.json [--md OUT.md] [--title TITLE]

SPEC is a JSON list of cases::

    [{"label": "cfg2", "problem": {"batch": 4, "nhead_q": 16, "seqlen_q": 2048},
      "variants": ["pair", "pair_stream", "regular|reference"], "mult": 1.0}, ...]

``problem`` takes the fields of :class:`fmha_native_amd.problem.Problem`
(``varlen_seqs`` as a list); a variant is a form name of
``fmha_native_amd.VARIANTS`` optionally followed by ``|reference``,
``|tilemajor`` or ``|sequence`` (the block-order flags), or an integer.

Per case, in one process: inputs are N(0,1)·mult bf16 (seed 42) resident on
the GPU; the first variant runs 0.3 s of untimed launches (from an idle GPU
the clock needs ~25 ms of back-to-back launches to come up); then for each
of ``reps`` rounds every variant runs 5 untimed launches and a timed chunk of
launches (about 60 ms) back to back between two events on the launch
stream, the variants taking turns, so that slow drifts of the clock touch
them alike.  The best chunk of each variant is reported, as microseconds per
launch and as the gain over the first variant.  Every launch goes through
``fmha_fwd_d64_bf16_ws`` with the workspace its variant needs.  One JSON
line per case on stdout; ``--md`` also writes a markdown table.
"""
import argparse
import ctypes
import json
import shlex
import sys
import time

import numpy as np


def parse_variant(v):
    import fmha_native_amd as fmha

    return fmha.variant_code(v)


def run_case(case, torch, reps=5, target_ms=60.0, ramp_s=0.3):
    import fmha_native_amd as fmha
    from fmha_native_amd.problem import Problem

    kw = dict(case["problem"])
    if "varlen_seqs" in kw:
        kw["varlen_seqs"] = tuple(kw["varlen_seqs"])
    prob = Problem(**kw)
    mult = float(case.get("mult", 1.0))
    names = [str(v) for v in case["variants"]]
    codes = [parse_variant(v) for v in case["variants"]]
    nq, nk, nlse = prob.sizes()
    dev = [torch.from_numpy(fmha.fill_normal(42 + i, n, mult).view(np.int16)).to("cuda:0")
           for i, n in enumerate((nq, nk, nk))]
    o = torch.empty(nq, dtype=torch.int16, device="cuda:0")
    lse = torch.empty(nlse, dtype=torch.float32, device="cuda:0") if prob.lse else None
    ss = prob.seqstart()
    seq = torch.from_numpy(ss).to("cuda:0") if ss is not None else None
    p = fmha.FmhaFwdParams()
    p.q, p.k, p.v, p.o = dev[0].data_ptr(), dev[1].data_ptr(), dev[2].data_ptr(), o.data_ptr()
    p.lse = lse.data_ptr() if lse is not None else None
    p.seqlen_q, p.seqlen_k, p.nhead_q, p.nhead_k = prob.seqlen_q, prob.seqlen_k, prob.nhead_q, prob.nhead_k
    p.scale = fmha.LOG2E / 8.0
    for t, (s, hs, bs) in prob.strides().items():
        setattr(p, f"stride_{t}", s)
        setattr(p, f"nhead_stride_{t}", hs)
        setattr(p, f"batch_stride_{t}", bs)
    if seq is not None:
        p.seqstart_q = p.seqstart_k = seq.data_ptr()
    lib = fmha.load_library()
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)
    pp, b, c = ctypes.byref(p), prob.batch, int(prob.causal)
    ws = {}
    for code in codes:
        need = fmha.workspace_size(p, b, c, code)
        if need < 0:
            raise ValueError(f"variant {code} rejected for {case.get('label')}")
        buf = torch.empty(max(need, 256), dtype=torch.uint8, device="cuda:0")
        ws[code] = (buf, ctypes.c_void_p(buf.data_ptr()), ctypes.c_int64(need))

    def launch(code):
        rc = lib.fmha_fwd_d64_bf16_ws(pp, b, c, code, ws[code][1], ws[code][2], sh)
        if rc != 0:
            raise fmha.FmhaError(rc, "fmha_fwd_d64_bf16_ws")

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < ramp_s:
        for _ in range(20):
            launch(codes[0])
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(20):
        launch(codes[0])
    e1.record(stream)
    torch.cuda.synchronize()
    n = max(20, int(target_ms / (e0.elapsed_time(e1) / 20)))
    best = {code: float("inf") for code in codes}
    for _ in range(reps):
        for code in codes:
            for _ in range(5):
                launch(code)
            e0.record(stream)
            for _ in range(n):
                launch(code)
            e1.record(stream)
            torch.cuda.synchronize()
            best[code] = min(best[code], e0.elapsed_time(e1) / n)
    base = best[codes[0]]
    out = {"label": case.get("label", prob.name), "launches_per_chunk": n, "reps": reps,
           "us": {nm: round(best[cd] * 1e3, 2) for nm, cd in zip(names, codes)},
           "gain_vs_first": {nm: round(base / best[cd] - 1.0, 4) for nm, cd in zip(names, codes)}}
    if prob.causal or prob.varlen:
        out["exact_tflops"] = {nm: round(prob.exact_flops() / (best[cd] * 1e-3) / 1e12, 1) for nm, cd in zip(names, codes)}
    else:
        out["tflops"] = {nm: round(prob.flops() / (best[cd] * 1e-3) / 1e12, 1) for nm, cd in zip(names, codes)}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("spec", help="JSON file with the list of cases")
    ap.add_argument("--md", default=None, help="also write a markdown table here")
    ap.add_argument("--title", default="Interleaved A/B")
    ap.add_argument("--reps", type=int, default=5)
    args = ap.parse_args()
    import torch

    assert torch.cuda.is_available(), "abtest needs a GPU"
    with open(args.spec) as f:
        cases = json.load(f)
    rows = []
    for case in cases:
        r = run_case(case, torch, reps=args.reps)
        print(json.dumps(r), flush=True)
        rows.append(r)
    if args.md:
        md = [f"# {args.title}", "", "MI355X (gfx950), one GPU, one process, one run of", "",
              f"    python -m fmha_native_amd.abtest {' '.join(shlex.quote(a) for a in sys.argv[1:])}", "",
              "Inputs N(0,1) bf16 resident on the GPU; per case the clock is brought up with 0.3 s of launches, then "
              "the variants take turns over several rounds, each timing a chunk of back-to-back launches between "
              "two events; the best chunk per variant is given (µs per launch) with its gain over the case's first "
              "variant. Causal and varlen rates count the visible (q, k) pairs.", "",
              "| case | variant | µs per launch | gain over first | TFLOP/s |", "|---|---|---|---|---|"]
        for r in rows:
            rate = r.get("exact_tflops") or r.get("tflops")
            for nm in r["us"]:
                cell = nm.replace("|", "\\|")  # a pipe inside a table cell must be escaped
                md.append(f"| {r['label']} | `{cell}` | {r['us'][nm]:.2f} | {100 * r['gain_vs_first'][nm]:+.1f} % | "
                          f"{rate[nm]:.1f} |")
        with open(args.md, "w") as f:
            f.write("\n".join(md) + "\n")


if __name__ == "__main__":
    main()
