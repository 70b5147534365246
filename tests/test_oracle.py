"""Pins of the CPU oracle (no GPU): golden fixtures, an independent float64
evaluation, closed forms, invariants, and planted mistakes that must fail.

The oracle restates src/runner/cpu_ref.cpp:86-153 (O) and
src/runner/gpu_ref.cpp:116-117 (LSE).  Each check below would catch a
plausible restatement error:
  * faithful vs fast forms, bit for bit      -> a divergence between the two loop nests
  * float64 numpy (tests/np_ref.py)          -> a dropped term, wrong scale, index or mask
  * golden fixtures (tests/golden/)          -> any drift of the oracle or its inputs
  * closed forms (Q=0, S=1, causal row 0, constant V, one-hot, fully masked)
  * invariants (BSHD==BHSD, GQA==replicated MHA, varlen==per-sequence dense,
    head permutation)
  * planted mistakes in the numpy evaluation fail the comparison.
"""
import hashlib
import os

import numpy as np
import pytest

import np_ref
import oracle
from fmha_native_amd.problem import Problem, bhsd_to_bshd
from oracle import verify

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def ref_inputs(prob, seed=42):
    nq, nk, _ = prob.sizes()
    q, k, v = oracle.fill_ref(seed, nq, nk, nk)
    if prob.layout == "bshd":
        q = bhsd_to_bshd(q, prob.batch, prob.nhead_q, prob.seqlen_q)
        k = bhsd_to_bshd(k, prob.batch, prob.nhead_k, prob.seqlen_k)
        v = bhsd_to_bshd(v, prob.batch, prob.nhead_k, prob.seqlen_k)
    return q, k, v


def bf16(x):
    """float -> bf16 bits by truncation (src/runner/bf16_utils.hpp:18-22)."""
    return (np.asarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


PROBLEMS = [
    Problem(batch=1, nhead_q=2, seqlen_q=128, lse=True, name="cfg1"),
    Problem(batch=2, nhead_q=2, seqlen_q=77, causal=True, lse=True, name="causal_ragged"),
    Problem(batch=1, nhead_q=2, seqlen_q=40, seqlen_k=100, causal=True, lse=True, name="causal_sq_lt_sk"),
    Problem(batch=1, nhead_q=2, seqlen_q=100, seqlen_k=40, causal=True, lse=True, name="causal_sq_gt_sk"),
    Problem(batch=1, nhead_q=4, nhead_k=2, seqlen_q=65, causal=True, lse=True, name="gqa"),
    Problem(batch=1, nhead_q=4, nhead_k=1, seqlen_q=33, lse=True, name="mqa"),
    Problem(batch=0, nhead_q=2, seqlen_q=0, causal=True, lse=True, varlen_seqs=(17, 64, 130), name="varlen"),
    Problem(batch=2, nhead_q=2, seqlen_q=70, causal=True, lse=True, layout="bshd", name="bshd"),
    Problem(batch=1, nhead_q=1, seqlen_q=1, lse=True, name="s1"),
]
IDS = [p.name for p in PROBLEMS]


# ---------------------------------------------------------------- golden fixtures

def test_golden_cfg1_inputs():
    g = np.load(os.path.join(GOLDEN, "cfg1_ref42.npz"))
    prob = PROBLEMS[0]
    q, k, v = ref_inputs(prob)
    for name, a in (("q", q), ("k", k), ("v", v)):
        assert hashlib.sha256(a.tobytes()).hexdigest() == str(g[f"{name}_sha"])


@pytest.mark.parametrize("faithful", [True, False])
def test_golden_cfg1_oracle_bitwise(faithful):
    g = np.load(os.path.join(GOLDEN, "cfg1_ref42.npz"))
    prob = PROBLEMS[0]
    q, k, v = ref_inputs(prob)
    o, lse = oracle.run(prob, q, k, v, faithful=faithful)
    assert np.array_equal(o.view(np.uint32), g["o"].view(np.uint32))
    assert np.array_equal(lse.view(np.uint32), g["lse"].view(np.uint32))


def test_golden_cfg1_exact():
    """The fixture's float64 outputs are reproduced by the numpy evaluation and
    sit within the reference's own tolerance of the oracle."""
    g = np.load(os.path.join(GOLDEN, "cfg1_ref42.npz"))
    prob = PROBLEMS[0]
    q, k, v = ref_inputs(prob)
    o64, lse64 = np_ref.attention(prob, q, k, v)
    assert np.abs(o64 - g["o_exact"]).max() < 1e-7
    assert np.abs(lse64 - g["lse_exact"]).max() < 1e-6
    assert verify.reference_rule(g["o_exact"], g["o"])["pass"]


def test_golden_ck_known_answer():
    g = np.load(os.path.join(GOLDEN, "ck_known_answer.npz"))
    D = 64
    for sq, sk in ((64, 64), (17, 33)):
        prob = Problem(batch=1, nhead_q=1, seqlen_q=sq, seqlen_k=sk)
        iq, ik = np.arange(sq * D), np.arange(sk * D)
        q = bf16((iq % 256) / np.float32(256.0))
        k = bf16(((ik + 64) % 256) / np.float32(256.0))
        v = bf16((ik % 256) / np.float32(256.0) + np.float32(1.0))
        o, _ = oracle.run(prob, q, k, v)
        assert np.array_equal(o.view(np.uint32), g[f"o_{sq}x{sk}"].view(np.uint32))
        o64, _ = np_ref.attention(prob, q, k, v)
        assert np.abs(o64 - g[f"o_exact_{sq}x{sk}"]).max() < 1e-6
        # V in [1, 2): the reference's bf16 P truncation makes sum(P) <= 1
        assert verify.baseline_rule(o64, o)["pass"]


# ---------------------------------------------------------------- two forms, float64

@pytest.mark.parametrize("prob", PROBLEMS, ids=IDS)
def test_faithful_equals_fast(prob):
    q, k, v = ref_inputs(prob)
    o1, l1 = oracle.run(prob, q, k, v, faithful=True)
    o2, l2 = oracle.run(prob, q, k, v, faithful=False)
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))
    assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32))


@pytest.mark.parametrize("prob", PROBLEMS, ids=IDS)
def test_oracle_vs_float64(prob):
    q, k, v = ref_inputs(prob)
    o64, l64 = np_ref.attention(prob, q, k, v)
    # the C float64 brute force agrees with numpy to rounding
    c64, cl64 = oracle.run_f64(prob, q, k, v)
    assert np.allclose(c64, o64, rtol=0, atol=1e-12)
    assert np.array_equal(np.isneginf(cl64), np.isneginf(l64))
    fin = np.isfinite(l64)
    assert np.abs(cl64[fin] - l64[fin]).max() < 1e-12
    # fp32 oracle without the P truncation: fp32 rounding only
    o, lse = oracle.run(prob, q, k, v, p_trunc=False)
    assert np.abs(o - o64).max() < 2e-6
    assert np.array_equal(np.isneginf(lse), np.isneginf(l64))
    assert np.abs(lse[fin] - l64[fin]).max() < 2e-6
    # with it: within the reference's own pass rule
    o, lse = oracle.run(prob, q, k, v)
    assert verify.reference_rule(o64, o)["pass"]
    assert verify.lse_rule(l64, lse)["pass"]


# ---------------------------------------------------------------- closed forms

def test_q_zero_uniform_attention():
    """Q = 0: every visible key gets P = 1/n, O = mean of the visible V rows,
    LSE = ln(n)."""
    prob = Problem(batch=1, nhead_q=1, seqlen_q=96, seqlen_k=128, causal=True, lse=True)
    q, k, v = ref_inputs(prob)
    q = np.zeros_like(q)
    o, lse = oracle.run(prob, q, k, v, p_trunc=False)
    vf = np_ref.bits_to_f64(v).reshape(128, 64)
    shift = 128 - 96
    for i in (0, 1, 50, 95):
        n = i + shift + 1
        assert np.abs(o.reshape(96, 64)[i] - vf[:n].mean(0)).max() < 1e-6
        assert abs(lse[i] - np.log(n)) < 1e-6
    # non-causal over a power-of-two key count: 1/n is exact in bf16, so the
    # truncating form gives the mean too
    prob = Problem(batch=1, nhead_q=1, seqlen_q=8, seqlen_k=64, lse=True)
    q, k, v = ref_inputs(prob)
    o, lse = oracle.run(prob, np.zeros_like(q), k, v)
    vf = np_ref.bits_to_f64(v).reshape(64, 64)
    assert np.abs(o.reshape(8, 64) - vf.mean(0)).max() < 1e-6
    assert np.abs(lse - np.log(64)).max() < 1e-6


def test_single_key():
    """S = 1: P = 1 exactly, O = V0, LSE = q.k / 8."""
    prob = PROBLEMS[-1]
    q, k, v = ref_inputs(prob)
    o, lse = oracle.run(prob, q, k, v)
    assert np.array_equal(o, np_ref.bits_to_f64(v).astype(np.float32))
    s = np.dot(np_ref.bits_to_f64(q), np_ref.bits_to_f64(k)) / 8
    assert abs(lse[0] - s) < 1e-6


def test_causal_first_row():
    """Causal with Sq = Sk: row 0 sees only key 0, so O[0] = V[0] exactly."""
    prob = Problem(batch=1, nhead_q=2, seqlen_q=50, causal=True, lse=True)
    q, k, v = ref_inputs(prob)
    o, lse = oracle.run(prob, q, k, v)
    O = o.reshape(2, 50, 64)
    V = np_ref.bits_to_f64(v).reshape(2, 50, 64)
    Q = np_ref.bits_to_f64(q).reshape(2, 50, 64)
    K = np_ref.bits_to_f64(k).reshape(2, 50, 64)
    for h in range(2):
        assert np.array_equal(O[h, 0], V[h, 0].astype(np.float32))
        assert abs(lse.reshape(2, 50)[h, 0] - Q[h, 0] @ K[h, 0] / 8) < 1e-6


def test_constant_v():
    """V = c: O = c * sum(P); sum(P) = 1 untruncated, in [1 - 2^-7, 1] truncated
    (the reference's PROBE_V_CONST, src/runner/buffers.cpp:130-141)."""
    prob = Problem(batch=1, nhead_q=2, seqlen_q=70, causal=True)
    q, k, v = ref_inputs(prob)
    c = 0.75
    v = np.full_like(v, bf16(np.float32(c)))
    o, _ = oracle.run(prob, q, k, v, p_trunc=False)
    assert np.abs(o - c).max() < 1e-6
    o, _ = oracle.run(prob, q, k, v)
    assert (o <= c + 1e-7).all() and (o >= c * (1 - 2.0 ** -7)).all()


def test_one_hot_peak():
    """A single key with a dominant score takes all the weight: O = V[j*]."""
    prob = Problem(batch=1, nhead_q=1, seqlen_q=4, seqlen_k=96, lse=True)
    q, k, v = ref_inputs(prob)
    q = np.zeros_like(q).reshape(4, 64)
    k = np.zeros_like(k).reshape(96, 64)
    q[:, 0] = bf16(np.float32(100.0))
    jstar = 57
    k[jstar, 0] = bf16(np.float32(100.0))
    o, lse = oracle.run(prob, q.reshape(-1), k.reshape(-1), v)
    V = np_ref.bits_to_f64(v).reshape(96, 64)
    for i in range(4):
        assert np.array_equal(o.reshape(4, 64)[i], V[jstar].astype(np.float32))
    assert np.abs(lse - 100.0 * 100.0 / 8).max() < 1e-3


def test_fully_masked_rows():
    """Causal with Sq > Sk: rows i < Sq - Sk see no key -> O = 0, LSE = -inf
    (src/runner/cpu_ref.cpp:124-129, gpu_ref.cpp:116-117)."""
    prob = PROBLEMS[3]
    q, k, v = ref_inputs(prob)
    o, lse = oracle.run(prob, q, k, v)
    n_dead = prob.seqlen_q - prob.seqlen_k
    O = o.reshape(prob.nhead_q, prob.seqlen_q, 64)
    L = lse.reshape(prob.nhead_q, prob.seqlen_q)
    assert (O[:, :n_dead] == 0).all() and np.isneginf(L[:, :n_dead]).all()
    assert np.isfinite(L[:, n_dead:]).all()


def test_no_keys():
    prob = Problem(batch=1, nhead_q=1, seqlen_q=5, lse=True, varlen_seqs=(0, 5))
    q, k, v = ref_inputs(prob)
    o, lse = oracle.run(prob, q, k, v)
    assert np.isfinite(o).all()


# ---------------------------------------------------------------- invariants

def test_bshd_equals_bhsd():
    p1 = Problem(batch=2, nhead_q=3, seqlen_q=45, seqlen_k=70, causal=True, lse=True)
    p2 = Problem(batch=2, nhead_q=3, seqlen_q=45, seqlen_k=70, causal=True, lse=True, layout="bshd")
    q, k, v = ref_inputs(p1)
    o1, l1 = oracle.run(p1, q, k, v)
    o2, l2 = oracle.run(p2, bhsd_to_bshd(q, 2, 3, 45), bhsd_to_bshd(k, 2, 3, 70), bhsd_to_bshd(v, 2, 3, 70))
    assert np.array_equal(bhsd_to_bshd(o1, 2, 3, 45).view(np.uint32), o2.view(np.uint32))
    assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32))


def test_gqa_equals_replicated_mha():
    g = Problem(batch=1, nhead_q=6, nhead_k=2, seqlen_q=33, causal=True, lse=True)
    m = Problem(batch=1, nhead_q=6, seqlen_q=33, causal=True, lse=True)
    q, k, v = ref_inputs(g)
    rep = lambda a: np.repeat(a.reshape(2, 33 * 64), 3, axis=0).reshape(-1)  # noqa: E731
    o1, l1 = oracle.run(g, q, k, v)
    o2, l2 = oracle.run(m, q, rep(k), rep(v))
    assert np.array_equal(o1.view(np.uint32), o2.view(np.uint32))
    assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32))


def test_varlen_equals_per_sequence_dense():
    seqs = (17, 64, 130)
    pv = Problem(batch=0, nhead_q=2, seqlen_q=0, causal=True, lse=True, varlen_seqs=seqs)
    q, k, v = ref_inputs(pv)
    ov, lv = oracle.run(pv, q, k, v)
    T = sum(seqs)
    Q, K, V = (a.reshape(2, T, 64) for a in (q, k, v))
    OV, LV = ov.reshape(2, T, 64), lv.reshape(2, T)
    off = 0
    for s in seqs:
        pd = Problem(batch=1, nhead_q=2, seqlen_q=s, causal=True, lse=True)
        sl = slice(off, off + s)
        od, ld = oracle.run(pd, *(np.ascontiguousarray(X[:, sl]).reshape(-1) for X in (Q, K, V)))
        assert np.array_equal(od.view(np.uint32), np.ascontiguousarray(OV[:, sl]).reshape(-1).view(np.uint32))
        assert np.array_equal(ld.view(np.uint32), np.ascontiguousarray(LV[:, sl]).reshape(-1).view(np.uint32))
        off += s


def test_head_permutation_commutes():
    prob = Problem(batch=1, nhead_q=4, seqlen_q=40, causal=True, lse=True)
    q, k, v = ref_inputs(prob)
    perm = np.array([2, 0, 3, 1])
    P = lambda a: np.ascontiguousarray(a.reshape(4, -1)[perm]).reshape(-1)  # noqa: E731
    o1, l1 = oracle.run(prob, q, k, v)
    o2, l2 = oracle.run(prob, P(q), P(k), P(v))
    assert np.array_equal(P(o1).view(np.uint32), o2.view(np.uint32))
    assert np.array_equal(P(l1).view(np.uint32), l2.view(np.uint32))


# ---------------------------------------------------------------- planted mistakes

@pytest.mark.parametrize("mutation,prob", [
    ("causal_off_by_one", Problem(batch=1, nhead_q=2, seqlen_q=64, causal=True, lse=True)),
    ("no_scale", Problem(batch=1, nhead_q=2, seqlen_q=64, lse=True)),
    ("gqa_modulo", Problem(batch=1, nhead_q=4, nhead_k=2, seqlen_q=64, lse=True)),
    ("swap_kv", Problem(batch=1, nhead_q=2, seqlen_q=64, lse=True)),
    ("transpose_v", Problem(batch=1, nhead_q=1, seqlen_q=64, lse=True)),
])
def test_planted_mistake_is_caught(mutation, prob):
    """A wrong restatement fails the same comparison the real one passes."""
    q, k, v = ref_inputs(prob)
    o, lse = oracle.run(prob, q, k, v)
    good, good_lse = np_ref.attention(prob, q, k, v)
    assert verify.reference_rule(good, o)["pass"] and verify.lse_rule(good_lse, lse)["pass"]
    bad, bad_lse = np_ref.attention(prob, q, k, v, mutate=mutation)
    assert not (verify.reference_rule(bad, o)["pass"] and verify.lse_rule(bad_lse, lse)["pass"])


# ---------------------------------------------------------------- pass rules

def test_rules():
    ref = np.array([0.5, -0.25, 1.0, 0.0], dtype=np.float32)
    assert verify.baseline_rule(ref, ref + 0.009)["pass"]
    assert not verify.baseline_rule(ref, ref + 0.03)["pass"]
    assert not verify.baseline_rule(ref, np.array([0.5, np.nan, 1.0, 0.0], dtype=np.float32))["pass"]
    inf = np.float32(-np.inf)
    assert verify.lse_rule(np.array([1.0, inf]), np.array([1.0005, inf]))["pass"]
    assert not verify.lse_rule(np.array([1.0, inf]), np.array([1.0, 0.0]))["pass"]
    assert not verify.lse_rule(np.array([1.0]), np.array([np.nan]))["pass"]
    r = np.linspace(-1, 1, 128, dtype=np.float32)
    assert verify.reference_rule(r, r + 5e-4)["pass"]
    assert not verify.reference_rule(r, r + 2e-3)["pass"]
