"""Host-side logic without a GPU: input generators, problem geometry, FLOP
conventions and the configuration tables."""
import numpy as np
import pytest

import fmha_native_amd as fmha
import oracle
from configs import K_ALL_FULL, all_full, baseline_problems
from fmha_native_amd.problem import Problem, bhsd_to_bshd, bshd_to_bhsd


@pytest.mark.parametrize("seed,n", [(42, 4096), (7, 1000), (123456, 33)])
def test_fill_ref_two_implementations_agree(seed, n):
    """The product's generator (C++, runner.cpp) and the oracle's (C) restate
    the reference's fill_random (src/runner/buffers.cpp:99-127) separately."""
    a = fmha.fill_ref(seed, n, n + 5, n + 7)
    b = oracle.fill_ref(seed, n, n + 5, n + 7)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_fill_ref_value_set():
    """bf16((r % 1000 - 500) / 5000): |x| <= 0.1 and 1000 distinct fp32 sources."""
    q, _, _ = fmha.fill_ref(42, 200000, 0, 0)
    f = (q.astype(np.uint32) << 16).view(np.float32)
    assert np.abs(f).max() <= 0.1
    assert f.min() == np.float32(-0.1) or f.min() < -0.099
    src = np.arange(-500, 500, dtype=np.float32) / np.float32(5000.0)
    allowed = np.unique((src.view(np.uint32) >> 16).astype(np.uint16))
    assert np.isin(q, allowed).all()


def test_fill_normal_properties():
    a = fmha.fill_normal(42, 1 << 20)
    b = fmha.fill_normal(42, 1 << 20)
    c = fmha.fill_normal(43, 1 << 20)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    f = (a.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    assert abs(f.mean()) < 5e-3 and abs(f.std() - 1.0) < 5e-3
    # prefix-stable (counter-based): the first n values do not depend on the length
    assert np.array_equal(fmha.fill_normal(42, 1000), a[:1000])
    # scaling by 2 is exact in bf16
    d = fmha.fill_normal(42, 1 << 16, 2.0)
    fd = (d.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(fd, 2 * f[: 1 << 16].astype(np.float32))


def test_varlen_lengths():
    a = fmha.varlen_lengths(42, 8, 128, 4096)
    assert a == fmha.varlen_lengths(42, 8, 128, 4096)
    assert a != fmha.varlen_lengths(43, 8, 128, 4096)
    assert all(128 <= s <= 4096 for s in a)
    assert sum(s % 64 != 0 for s in a) >= 4
    with pytest.raises(ValueError):
        fmha.varlen_lengths(1, 4, 10, 5)


def test_problem_geometry():
    p = Problem(batch=2, nhead_q=8, nhead_k=2, seqlen_q=100, seqlen_k=300, causal=True, lse=True)
    assert p.sizes() == (2 * 8 * 100 * 64, 2 * 2 * 300 * 64, 2 * 8 * 100)
    assert p.strides()["q"] == (64, 100 * 64, 8 * 100 * 64)
    assert p.strides()["k"] == (64, 300 * 64, 2 * 300 * 64)
    b = Problem(batch=2, nhead_q=8, nhead_k=2, seqlen_q=100, seqlen_k=300, layout="bshd")
    assert b.strides()["q"] == (8 * 64, 64, 100 * 8 * 64)
    v = Problem(batch=0, nhead_q=4, seqlen_q=0, varlen_seqs=(5, 70, 33))
    assert v.batch == 3 and v.seqlen_q == 70 and v.seqlen_k == 70
    assert v.seqstart().tolist() == [0, 5, 75, 108]
    assert v.strides()["q"] == (64, 108 * 64, 0)
    with pytest.raises(ValueError):
        Problem(batch=1, nhead_q=6, nhead_k=4, seqlen_q=8)


def test_layout_roundtrip():
    a = np.arange(2 * 3 * 5 * 64, dtype=np.uint16)
    assert np.array_equal(bshd_to_bhsd(bhsd_to_bshd(a, 2, 3, 5), 2, 3, 5), a)
    t = bhsd_to_bshd(a, 2, 3, 5).reshape(2, 5, 3, 64)
    assert np.array_equal(t[1, 4, 2], a.reshape(2, 3, 5, 64)[1, 2, 4])


def test_flop_conventions():
    """src/bench_fmha_fwd.cpp:225-226: 4*B*H*Sq*Sk*D, x0.5 causal."""
    cfg = {k: v[0] for k, v in baseline_problems().items()}
    assert cfg["cfg1"].flops() == 8388608
    assert cfg["cfg2"].flops() == 68719476736
    assert cfg["cfg3"].flops() == 137438953472  # 4*16*8192^2*64 * 0.5
    assert cfg["cfg5"].flops() == 409600000000  # 4*2*40000^2*64 * 0.5
    # exact causal count: sum over rows of the visible keys
    p = Problem(batch=1, nhead_q=1, seqlen_q=4, seqlen_k=6, causal=True)
    assert p.exact_flops() == 4 * 64 * (3 + 4 + 5 + 6)
    assert Problem(batch=1, nhead_q=2, seqlen_q=8).exact_flops() == Problem(batch=1, nhead_q=2, seqlen_q=8).flops()


def test_io_bytes():
    cfg = {k: v[0] for k, v in baseline_problems().items()}
    assert cfg["cfg1"].io_bytes() == 132096
    assert cfg["cfg2"].io_bytes() == 67108864
    assert cfg["cfg3"].io_bytes() == 67633152
    assert cfg["cfg5"].io_bytes() == 41280000


def test_config_tables():
    assert len(K_ALL_FULL) == 63
    names = [r[0] for r in K_ALL_FULL]
    assert len(set(names)) == len(names)
    probs = all_full()
    assert all(p.nhead_q % p.nhead_k == 0 for p in probs)
    cfg4 = baseline_problems()["cfg4"][0]
    assert cfg4.batch == 8 and cfg4.causal and cfg4.lse
    assert baseline_problems()["cfg5"][1] == 2.0


def test_sweep_protocol_and_table(tmp_path, capsys):
    """fmha_native_amd.sweep: 6 runs per config, first dropped, the reference's
    table format (scripts/run-benchmark.sh:56-99)."""
    from fmha_native_amd import sweep

    counter = tmp_path / "n"
    fake = tmp_path / "bench"
    # run k of each config reports Avg = k ms (the dropped first run is 1 ms)
    fake.write_text("#!/bin/bash\nn=$(cat %s 2>/dev/null || echo 0); n=$((n %% 6 + 1)); echo $n > %s\n"
                    "echo \"Avg: $n.000 ms\"; echo \"min=0.$n ms\"; echo \"TFLOPS: ${n}0.00\"\n" % (counter, counter))
    fake.chmod(0o755)
    assert sweep.main(["--bench", str(fake), "--mask", "1"]) == 0
    out = capsys.readouterr().out.splitlines()
    assert out[0] == "Benchmark: 8 configs (WARMUP=5 ITERS=20 RUNS=6 DROP=1 MASK=1)"
    rows = [l for l in out if "|" in l][1:]
    assert len(rows) == 8
    assert rows[1] == "   4  16   2048   64 |      4.000      0.200      40.00"
    bad = tmp_path / "bad"
    bad.write_text("#!/bin/bash\necho 'HIP error 98 (invalid device function)'; exit 1\n")
    bad.chmod(0o755)
    sweep.main(["--bench", str(bad)])
    out = capsys.readouterr().out
    assert "ERROR" in out and "HIP error 98" in out


# ---------------------------------------------------------------- torch tensor checks

def _bf16(*shape):
    import torch

    return torch.zeros(shape, dtype=torch.bfloat16)


@pytest.mark.parametrize("case,match", [
    ("dtype", "bfloat16"),
    ("rank", "dimensions"),
    ("head_dim", "last dimension of 64"),
    ("inner_stride", "last dimension of 64"),
    ("o_shape", "q's shape"),
    ("kv_shape", "same shape"),
    ("batch", "batch sizes differ"),
    ("lse", "lse must be"),
    ("seqstart_dtype", "int32"),
    ("seqstart_k_only", "seqstart_k without"),
    ("cpu", "same GPU"),
    ("varlen_lse_head_stride", "head stride"),
    ("stride_wraps", "32-bit int"),
    ("varlen_head_stride_wraps", "32-bit int"),
])
def test_params_from_tensors_rejects(case, match):
    """Tensors the kernel cannot take are refused before any pointer is used
    (a host tensor's address would be read by the GPU)."""
    import torch

    q, k, v, o = _bf16(2, 4, 100, 64), _bf16(2, 2, 120, 64), _bf16(2, 2, 120, 64), _bf16(2, 4, 100, 64)
    kw = {}
    if case == "dtype":
        q = q.float()
    elif case == "rank":
        q, o = q[0], o[0]
    elif case == "head_dim":
        q, o = _bf16(2, 4, 100, 32), _bf16(2, 4, 100, 32)
    elif case == "inner_stride":
        q = _bf16(2, 4, 100, 128)[..., ::2]
    elif case == "o_shape":
        o = _bf16(2, 4, 99, 64)
    elif case == "kv_shape":
        v = _bf16(2, 2, 121, 64)
    elif case == "batch":
        k, v = _bf16(3, 2, 120, 64), _bf16(3, 2, 120, 64)
    elif case == "lse":
        kw["lse"] = torch.zeros((2, 4, 99), dtype=torch.float32)
    elif case == "seqstart_dtype":
        q, k, v, o = _bf16(4, 300, 64), _bf16(2, 300, 64), _bf16(2, 300, 64), _bf16(4, 300, 64)
        ss = torch.tensor([0, 100, 300], dtype=torch.int64)
        kw.update(seqstart_q=ss, seqstart_k=ss, max_seqlen_q=200)
    elif case == "seqstart_k_only":
        kw["seqstart_k"] = torch.tensor([0, 100], dtype=torch.int32)
    elif case == "varlen_lse_head_stride":
        # q/o are token slices [4, 300 of 400, 64]: LSE rows of heads >= 1 would land past [4, 300]
        q, o = _bf16(4, 400, 64)[:, :300], _bf16(4, 400, 64)[:, :300]
        k, v = _bf16(2, 300, 64), _bf16(2, 300, 64)
        ss = torch.tensor([0, 100, 300], dtype=torch.int32)
        kw.update(seqstart_q=ss, seqstart_k=ss, max_seqlen_q=200, lse=torch.zeros((4, 300), dtype=torch.float32))
    elif case == "stride_wraps":
        # batch stride 2^32 would read back as 0 from a C int (meta tensors: no memory)
        big = lambda: torch.empty_strided((2, 256, 262144, 64), (2**32, 2**24, 64, 1), dtype=torch.bfloat16,
                                          device="meta")
        q, k, v, o = big(), big(), big(), big()
    elif case == "varlen_head_stride_wraps":
        T = 2**25  # head stride T * 64 = 2^31
        mk = lambda h: torch.empty_strided((h, T, 64), (T * 64, 64, 1), dtype=torch.bfloat16, device="meta")
        q, k, v, o = mk(2), mk(1), mk(1), mk(2)
        ss = torch.tensor([0, T], dtype=torch.int32)
        kw.update(seqstart_q=ss, seqstart_k=ss, max_seqlen_q=T)
    with pytest.raises(ValueError, match=match):
        fmha.params_from_tensors(q, k, v, o, **kw)


@pytest.mark.parametrize("case,match", [
    ("parts_disagree", "must be \\[n"),
    ("o_dtype", "bfloat16"),
    ("lse_dtype", "float32"),
    ("head_dim", "must be \\[n"),
    ("noncontiguous", "contiguous"),
    ("o_shape", "o must be"),
    ("lse_shape", "lse must be"),
    ("cpu", "same GPU"),
])
def test_merge_partials_rejects(case, match):
    """merge_partials refuses arguments the merge kernel would read or write
    out of bounds, before any pointer is used."""
    import torch

    o_parts, lse_parts = _bf16(3, 10, 64), torch.zeros((3, 10), dtype=torch.float32)
    kw = {}
    if case == "parts_disagree":
        lse_parts = torch.zeros((4, 10), dtype=torch.float32)   # 4 LSE parts for 3 O parts
    elif case == "o_dtype":
        o_parts = o_parts.float()
    elif case == "lse_dtype":
        lse_parts = lse_parts.double()
    elif case == "head_dim":
        o_parts = _bf16(3, 10, 32)
    elif case == "noncontiguous":
        o_parts = _bf16(3, 20, 64)[:, ::2]
    elif case == "o_shape":
        kw["o"] = _bf16(9, 64)
    elif case == "lse_shape":
        kw["lse"] = torch.zeros(11, dtype=torch.float32)
    with pytest.raises(ValueError, match=match):
        fmha.merge_partials(o_parts, lse_parts, **kw)


def test_abtest_variants_and_specs():
    """The A/B tool's variant names resolve to the launcher's codes (a form,
    optionally with one block-order flag), and every committed spec names
    known forms and valid problems."""
    import glob
    import os
    import json

    from fmha_native_amd import abtest
    from fmha_native_amd.problem import Problem

    assert abtest.parse_variant("pair") == fmha.VARIANT_PAIR
    assert abtest.parse_variant("regular|reference") == fmha.VARIANT_REGULAR | fmha.VARIANT_REFERENCE_ORDER
    assert abtest.parse_variant("regular|tilemajor") == fmha.VARIANT_REGULAR | fmha.VARIANT_TILE_MAJOR_ORDER
    assert abtest.parse_variant("regular|sequence") == fmha.VARIANT_REGULAR | fmha.VARIANT_SEQUENCE_ORDER
    assert abtest.parse_variant("pair_stream") == fmha.VARIANT_PAIR_STREAM
    assert abtest.parse_variant(3) == 3
    specs = glob.glob(os.path.join(os.path.dirname(fmha.__file__), "abspecs", "*.json"))
    assert specs
    for path in specs:
        with open(path) as f:
            for case in json.load(f):
                kw = dict(case["problem"])
                if "varlen_seqs" in kw:
                    kw["varlen_seqs"] = tuple(kw["varlen_seqs"])
                Problem(**kw)
                for v in case["variants"]:
                    abtest.parse_variant(v)


def test_workload_names():
    """bench.py --only and rocprof --forms take the five configurations or a
    dense shape by name; anything else is refused."""
    from fmha_native_amd.problem import workload

    assert workload("cfg5")[1] == 2.0 and workload("cfg5")[0].seqlen_q == 40000
    p, mult = workload("causal-B2H16S8192")
    assert (p.batch, p.nhead_q, p.seqlen_q, p.causal, p.lse, mult) == (2, 16, 8192, True, True, 1.0)
    p, _ = workload("dense-B1H16S4096")
    assert (p.batch, p.nhead_q, p.seqlen_q, p.causal, p.lse) == (1, 16, 4096, False, False)
    for bad in ("cfg6", "dense-B1H16", "causal-b1h2s3", ""):
        with pytest.raises(ValueError):
            workload(bad)
