"""Host-side pieces of the rocprofv3 evidence harness (fmha_native_amd/rocprof.py):
which trace dispatches are the timed ones, the clock/MFMA-busy arithmetic and
the CLI output parser.  The passes themselves run on the GPU box."""
import sqlite3

import pytest

from fmha_native_amd import rocprof


def _db(tmp_path, rows):
    path = tmp_path / "t.db"
    con = sqlite3.connect(path)
    con.execute("create table kernels (name text, start integer, end integer)")
    con.executemany("insert into kernels values (?, ?, ?)", rows)
    con.commit()
    con.close()
    return str(path)


def test_timed_stats_takes_the_back_to_back_window(tmp_path):
    # bench.py --only launch order: ramp R, warmup W, K timed back to back,
    # then K under the reference's protocol; durations encode the phase
    R, W, K = 7, 3, 5
    rows, t = [], 0
    for phase, n, dur in (("ramp", R, 9000), ("warm", W, 8000), ("timed", K, 1000), ("ref", K, 5000)):
        for _ in range(n):
            rows.append(("fmha_fwd_d64_bf16_msk0(FmhaFwdParams)", t, t + dur))
            rows.append(("other_kernel", t + dur, t + dur + 10))  # not ours
            t += dur + 100
    got = rocprof._timed_stats(_db(tmp_path, rows), {"ramp_launches": R, "warmup": W, "steps": K})
    assert got == {"fmha_fwd_d64_bf16_msk0(FmhaFwdParams)": pytest.approx(1.0)}  # us


def test_timed_stats_two_kernels_per_step(tmp_path):
    # the balanced form: every step is one dispatch of each kernel
    rows, t = [], 0
    for i in range(2 + 1 + 4 + 4):
        timed = 3 <= i < 7
        rows.append(("fmha_fwd_d64_bf16_balanced_msk1(FmhaBalancedArgs)", t, t + (2000 if timed else 6000)))
        rows.append(("fmha_fwd_d64_bf16_balanced_merge(FmhaBalancedArgs)", t + 7000, t + 7000 + (300 if timed else 900)))
        t += 10000
    got = rocprof._timed_stats(_db(tmp_path, rows), {"ramp_launches": 2, "warmup": 1, "steps": 4})
    assert got["fmha_fwd_d64_bf16_balanced_msk1(FmhaBalancedArgs)"] == pytest.approx(2.0)
    assert got["fmha_fwd_d64_bf16_balanced_merge(FmhaBalancedArgs)"] == pytest.approx(0.3)


def test_timed_stats_drops_a_kernel_with_too_few_dispatches(tmp_path):
    rows = [("fmha_fwd_x", i * 10, i * 10 + 5) for i in range(4)]
    assert rocprof._timed_stats(_db(tmp_path, rows), {"ramp_launches": 2, "warmup": 1, "steps": 4}) == {}


def test_util_row():
    # 32 engines x 2e5 busy cycles -> a 2e5-cycle span; over a 100 us dispatch
    # the clock is at least 2.0 GHz; 1024 SIMDs each busy 1e5 MFMA cycles ->
    # 50 % of the span; of the peak: 1e5 / (1e5 ns x 2.4 GHz)
    c = {"SQ_BUSY_CYCLES": 32 * 2.0e5, "dispatch_ns": 1.0e5, "SQ_VALU_MFMA_BUSY_CYCLES": 1024 * 1.0e5,
         "GRBM_GUI_ACTIVE": 8 * 2.5e5}
    ghz, busy, frac = rocprof._util_row(c, 32)
    assert ghz == pytest.approx(2.0)
    assert busy == pytest.approx(0.5)
    assert frac == pytest.approx(1.0e5 / (1.0e5 * 2.4))
    assert frac == pytest.approx(busy * ghz / 2.4)  # the identity the roofline line quotes


def test_num_se_from_agent_record(tmp_path):
    import json

    path = tmp_path / "a.db"
    con = sqlite3.connect(path)
    con.execute("create table rocpd_info_agent (type text, extdata text)")
    con.execute("insert into rocpd_info_agent values ('CPU', '{}')")
    con.execute("insert into rocpd_info_agent values ('GPU', ?)", (json.dumps({"num_shader_banks": 16}),))
    con.commit()
    con.close()
    assert rocprof._num_se(str(path)) == 16
    assert rocprof._num_se(_db(tmp_path, [])) == rocprof.NUM_SE  # no agent table


def test_cli_avg_parser():
    out = "Avg: 0.082 ms\nmin=0.078 ms\nTFLOPS: 842.44\nback-to-back avg: 0.077 ms (892.10 TFLOPS)\n"
    assert rocprof._cli_avg(out, "Avg:") == pytest.approx(0.082)
    assert rocprof._cli_avg(out, "back-to-back avg:") == pytest.approx(0.077)
    with pytest.raises(RuntimeError):
        rocprof._cli_avg("nothing", "Avg:")
