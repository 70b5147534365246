"""The bench_fmha_fwd CLI: the reference's flags and output contract.

The reference's sweep parses three lines of its CLI's stdout,
``Avg: <ms> ms``, ``min=<ms> ms`` and ``TFLOPS: <x>``
(src/bench_fmha_fwd.cpp:231-233, scripts/run-benchmark.sh:56-99), and the
CLI exits 1 on arguments it cannot run (src/bench_fmha_fwd.cpp:43-117).
The GPU tests run the built binary on a dense, a causal+LSE and a varlen
problem and parse its output with the sweep's own parser; the argument
errors are checked on the CPU (they exit before any HIP call).
"""
import os
import subprocess

import pytest

from fmha_native_amd import sweep

BENCH = os.path.join(os.path.dirname(sweep.__file__), "bench_fmha_fwd")


def _run(*args, timeout=120):
    if not os.path.exists(BENCH):
        pytest.skip("bench_fmha_fwd not built")
    print("CLI:", " ".join(args), flush=True)
    return subprocess.run([BENCH, *args], capture_output=True, text=True, timeout=timeout)


@pytest.mark.parametrize("args,msg", [
    (["-b", "1", "-h", "4", "-s", "128", "--hdim", "128"], "only --hdim 64"),
    (["-b", "1", "-h", "16", "--kv-heads", "3", "-s", "128"], "divisible by kv_heads"),
    (["-b", "1", "-h", "4", "-s", "128", "--variant", "fast"], "--variant must be"),
    (["-b", "1", "-h", "4", "-s", "128", "--dist", "uniform"], "--dist must be"),
    (["--no-such-flag"], "Usage"),
])
def test_cli_rejects(args, msg):
    r = _run(*args)
    assert r.returncode == 1, (r.returncode, r.stdout, r.stderr)
    assert msg in r.stdout + r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("args,flops", [
    # dense, no mask: 4*B*H*S*S*64
    (["-b", "2", "-h", "4", "-s", "512", "--mask", "0"], 4.0 * 2 * 4 * 512 * 512 * 64),
    # causal + LSE with GQA: halved (src/bench_fmha_fwd.cpp:225-226)
    (["-b", "1", "-h", "4", "--kv-heads", "2", "-s", "700", "--mask", "1", "--lse", "1"],
     0.5 * 4.0 * 1 * 4 * 700 * 700 * 64),
    # varlen causal + LSE: the repo convention counts max(S) for every sequence
    (["-h", "4", "--varlen-seqs", "100,257,64", "--mask", "1", "--lse", "1"], 0.5 * 4.0 * 3 * 4 * 257 * 257 * 64),
])
def test_cli_runs_and_prints_the_contract(args, flops):
    r = _run(*args, "--warmup", "2", "--iters", "5")
    assert r.returncode == 0, (r.stdout, r.stderr)
    avg, mn, tf = sweep.parse_run(r.stdout)
    print(r.stdout, flush=True)
    assert 0.0 < mn <= avg * (1 + 1e-3) + 1e-3
    # TFLOPS is the convention's FLOPs over the average time; Avg is printed to
    # 0.001 ms, so the printed TFLOPS lies between the values at avg +- 0.0005
    hi = flops / (max(avg - 0.0005, 1e-6) * 1e-3) / 1e12
    lo = flops / ((avg + 0.0005) * 1e-3) / 1e12
    assert lo - 0.01 <= tf <= hi + 0.01, (lo, tf, hi)
    assert "back-to-back avg:" in r.stdout
