"""GPU checks against the committed golden fixtures and the reference's own
checker.

* The kernel on config 1 (reference inputs, fill_random(42)) and on the CK
  known-answer inputs, through the C-ABI, against tests/golden/ (no oracle run
  needed at test time).
* oracle/_ref/ref_verify — the reference's src/runner/cpu_ref.cpp and
  gpu_ref.cpp compiled from its own sources (oracle/build_ref.sh) — run on this
  build's kernel over the reference's 63-row kAllFull matrix, exactly its
  MatchesGpuRef suite (tests/test_fmha_fwd_d64.cpp:500-651): the reference's
  pass rule on O and |dLSE| <= 1e-3 against its GPU oracle.  Skipped when the
  harness was not built (the reference tree is only present where it was built).
"""
import json
import os
import subprocess

import numpy as np
import pytest

import fmha_native_amd as fmha
from configs import K_ALL_FULL, problem_from_row
from fmha_native_amd.problem import Problem
from harness import make_inputs, run_kernel
from oracle import verify

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
REF_VERIFY = os.path.join(ROOT, "oracle", "_ref", "ref_verify")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    fmha.load_library()


@pytest.mark.parametrize("args,geom", [
    (["-b", "1", "-h", "2", "-s", "128", "--seed", "42"], None),   # cfg1: the golden fixture's inputs
    (["-b", "2", "-h", "4", "--kv-heads", "2", "-s", "200", "--kv-seq", "333", "--seed", "7"], (2 * 4 * 200, 2 * 2 * 333)),
    (["-h", "4", "--kv-heads", "1", "--varlen-seqs", "100,257,64", "--seed", "123"], (4 * 421, 1 * 421)),
])
def test_reference_fill_random_equals_oracle_generator(tmp_path, args, geom):
    """The reference's own fill_random (src/runner/buffers.cpp:99-127, compiled
    into oracle/_ref/ref_verify) writes, bit for bit, the inputs the oracle's
    generator (oracle_fill_ref) and the product's (fmha.fill_ref) write; for
    config 1 they also hash to the committed golden digests."""
    import hashlib

    import oracle

    if not os.path.exists(REF_VERIFY):
        pytest.skip("oracle/_ref/ref_verify not built (no reference tree where this was built)")
    path = tmp_path / "inputs.bin"
    r = subprocess.run([REF_VERIFY, *args, "--dump-inputs", str(path)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    sizes = json.loads([l for l in r.stdout.splitlines() if l.startswith("REF_INPUTS ")][0].split(" ", 1)[1])
    raw = np.fromfile(path, dtype=np.uint16)
    nq, nk, nv = sizes["q"], sizes["k"], sizes["v"]
    assert raw.size == nq + nk + nv
    ref = raw[:nq], raw[nq:nq + nk], raw[nq + nk:]
    if geom is not None:
        assert (nq, nk) == (geom[0] * 64, geom[1] * 64)
    seed = int(args[args.index("--seed") + 1])
    for mine in (oracle.fill_ref(seed, nq, nk, nv), fmha.fill_ref(seed, nq, nk, nv)):
        for a, b in zip(ref, mine):
            assert np.array_equal(a, b)
    if geom is None:
        g = np.load(os.path.join(GOLDEN, "cfg1_ref42.npz"))
        for name, a in zip("qkv", ref):
            assert hashlib.sha256(a.tobytes()).hexdigest() == str(g[f"{name}_sha"])


def test_kernel_matches_golden_cfg1():
    g = np.load(os.path.join(GOLDEN, "cfg1_ref42.npz"))
    prob = Problem(batch=1, nhead_q=2, seqlen_q=128, lse=True, name="cfg1")
    q, k, v = make_inputs(prob, dist="ref", seed=42)
    o_bits, lse = run_kernel(prob, q, k, v)
    o = verify.bf16_bits_to_f32(o_bits)
    ref = verify.reference_rule(g["o"], o)
    base = verify.baseline_rule(g["o_exact"], o)
    lr = verify.lse_rule(g["lse_exact"], lse)
    print("cfg1 golden:", ref, base, lr, flush=True)
    assert ref["pass"] and base["pass"] and lr["pass"]


def test_kernel_matches_golden_ck_known_answer():
    g = np.load(os.path.join(GOLDEN, "ck_known_answer.npz"))
    D = 64
    for sq, sk in ((64, 64), (17, 33)):
        prob = Problem(batch=1, nhead_q=1, seqlen_q=sq, seqlen_k=sk, name=f"ck_{sq}x{sk}")
        iq, ik = np.arange(sq * D), np.arange(sk * D)
        trunc = lambda x: (np.asarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)  # noqa: E731
        q = trunc((iq % 256) / np.float32(256.0))
        k = trunc(((ik + 64) % 256) / np.float32(256.0))
        v = trunc((ik % 256) / np.float32(256.0) + np.float32(1.0))
        o_bits, _ = run_kernel(prob, q, k, v)
        o = verify.bf16_bits_to_f32(o_bits)
        base = verify.baseline_rule(g[f"o_exact_{sq}x{sk}"], o)
        print(f"ck {sq}x{sk}:", base, flush=True)
        assert base["pass"], base


def _row_flags(row):
    prob = problem_from_row(row)
    f = ["-b", str(prob.batch), "-h", str(prob.nhead_q), "--kv-heads", str(prob.nhead_k), "-s", str(prob.seqlen_q),
         "--kv-seq", str(prob.seqlen_k), "--mask", str(int(prob.causal)), "--lse", str(int(prob.lse)), "--seed", "42"]
    if prob.varlen:
        f += ["--varlen-seqs", ",".join(str(s) for s in prob.varlen_seqs)]
    return " ".join(f)


@pytest.fixture(scope="module")
def reference_checker_results():
    if not os.path.exists(REF_VERIFY):
        pytest.skip("oracle/_ref/ref_verify not built (needs the reference tree at build time)")
    cases = "\n".join(_row_flags(r) for r in K_ALL_FULL) + "\n"
    print(f"running {REF_VERIFY} on {len(K_ALL_FULL)} kAllFull cases", flush=True)
    r = subprocess.run([REF_VERIFY, "--stdin"], input=cases, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [json.loads(line.split(" ", 1)[1]) for line in r.stdout.splitlines() if line.startswith("REF_VERIFY ")]
    assert len(lines) == len(K_ALL_FULL)
    return dict(zip([row[0] for row in K_ALL_FULL], lines))


@pytest.mark.parametrize("row", K_ALL_FULL, ids=[r[0] for r in K_ALL_FULL])
def test_reference_checker(reference_checker_results, row):
    res = reference_checker_results[row[0]]
    print(row[0], res, flush=True)
    assert res["pass"], res
    if res["lse_mismatch"] >= 0:
        assert res["lse_mismatch"] == 0, res
