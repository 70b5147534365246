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


def test_scores_far_below_zero():
    """Q = 10, K = -10 in every dimension (exact in bf16): every score is -6400
    raw, -800 after the 1/8 scale.  The softmax is still uniform: O = mean of
    the visible V rows and LSE = ln(n) - 800 (cpu_ref.cpp:124-136 subtracts the
    true row max; no fixed seed can drop such a row)."""
    prob = Problem(batch=1, nhead_q=1, seqlen_q=96, seqlen_k=128, causal=True, lse=True)
    q, k, v = ref_inputs(prob)
    q = np.full_like(q, 0x4120)   # bf16 10.0
    k = np.full_like(k, 0xC120)   # bf16 -10.0
    o, lse = oracle.run(prob, q, k, v, p_trunc=False)
    vf = np_ref.bits_to_f64(v).reshape(128, 64)
    for i in (0, 1, 50, 95):
        n = i + 32 + 1
        assert np.abs(o.reshape(96, 64)[i] - vf[:n].mean(0)).max() < 1e-6
        assert abs(lse[i] - (np.log(n) - 800.0)) < 1e-4  # fp32 LSE near -800: ulp 6e-5


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


# ---------------------------------------------------------------- partial-result merge

def bf16_rne(x):
    """float -> bf16 bits, round to nearest even."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _random_parts(n, rows, seed):
    rng = np.random.default_rng(seed)
    o = bf16_rne(rng.standard_normal((n, rows * 64)))
    lse = (rng.standard_normal((n, rows)) * 3).astype(np.float32)
    return o, lse


def test_merge_one_part_is_identity():
    o, lse = _random_parts(1, 37, 1)
    mo, ml = oracle.merge(o, lse)
    assert np.array_equal(mo, o[0]) and np.array_equal(ml, lse[0])


def test_merge_equal_lse_averages():
    o, lse = _random_parts(3, 29, 2)
    lse[:] = lse[0]
    mo, ml = oracle.merge(o, lse)
    mean = np.mean(verify.bf16_bits_to_f32(o).reshape(3, -1).astype(np.float64), axis=0)
    assert np.array_equal(mo, bf16_rne(mean))
    np.testing.assert_allclose(ml, lse[0] + np.log(3.0), rtol=1e-6, atol=1e-6)


def test_merge_minus_inf_parts_drop_out():
    o, lse = _random_parts(3, 41, 3)
    lse[2, :] = -np.inf
    lse[1, :5] = -np.inf
    mo, ml = oracle.merge(o, lse)
    mo2, ml2 = oracle.merge(o[:2], lse[:2])
    assert np.array_equal(mo, mo2) and np.array_equal(ml, ml2)
    lse[:, 7] = -np.inf  # every part empty for row 7: O = 0, LSE = -inf
    mo, ml = oracle.merge(o, lse)
    assert np.all(mo.reshape(41, 64)[7] == 0) and np.isneginf(ml[7])


def _numpy_merge(o_parts, lse_parts, mistake=None):
    o = verify.bf16_bits_to_f32(o_parts).reshape(lse_parts.shape + (64,)).astype(np.float64)
    l = lse_parts.astype(np.float64)
    m = l.max(axis=0)
    w = np.exp(m - l) if mistake == "sign" else np.exp(l - m)
    out = (w[..., None] * o).sum(axis=0)
    if mistake != "no_renorm":
        out /= w.sum(axis=0)[..., None]
    return out.reshape(-1), m + np.log(w.sum(axis=0))


def _chunked_f64(prob, q, k, v, cuts):
    """float64 attention of each key chunk [c0, c1): (O bits bf16 RNE, LSE float32) per chunk."""
    B, Hk, Sk = prob.batch, prob.nhead_k, prob.seqlen_k
    k4, v4 = k.reshape(B, Hk, Sk, 64), v.reshape(B, Hk, Sk, 64)
    o_parts, l_parts = [], []
    for c0, c1 in zip(cuts[:-1], cuts[1:]):
        pc = Problem(batch=B, nhead_q=prob.nhead_q, nhead_k=Hk, seqlen_q=prob.seqlen_q, seqlen_k=c1 - c0, lse=True)
        oc, lc = oracle.run_f64(pc, q, np.ascontiguousarray(k4[:, :, c0:c1]).reshape(-1),
                                np.ascontiguousarray(v4[:, :, c0:c1]).reshape(-1))
        o_parts.append(bf16_rne(oc.astype(np.float32)))
        l_parts.append(lc.astype(np.float32))
    return np.stack(o_parts), np.stack(l_parts)


def test_merge_of_key_chunks_is_full_attention():
    """Merging the attention of disjoint key chunks gives the attention of all
    keys (O within the bf16 rounding of the parts, LSE to float32); the merge
    with a wrong exponent sign or without renormalisation does not."""
    prob = Problem(batch=2, nhead_q=4, nhead_k=2, seqlen_q=37, seqlen_k=150, lse=True)
    rng = np.random.default_rng(5)
    nq, nk, _ = prob.sizes()
    q, k, v = (bf16_rne(rng.standard_normal(n)) for n in (nq, nk, nk))
    o_full, l_full = oracle.run_f64(prob, q, k, v)
    o_parts, l_parts = _chunked_f64(prob, q, k, v, [0, 40, 41, 110, 150])
    mo, ml = oracle.merge(o_parts, l_parts)
    got = verify.bf16_bits_to_f32(mo).astype(np.float64)
    # each part carries its own bf16 rounding (<= 2^-9 |O_i|), weighted by
    # exp(LSE_i - LSE); the merged value adds one more rounding
    w = np.exp(l_parts.astype(np.float64) - l_full[None, :])[..., None]
    o_abs = np.abs(verify.bf16_bits_to_f32(o_parts).reshape(w.shape[:2] + (64,)).astype(np.float64))
    tol = 2.0 ** -8 * ((w * o_abs).sum(axis=0).reshape(-1) + np.abs(o_full)) + 1e-7
    assert np.all(np.abs(got - o_full) <= tol)
    np.testing.assert_allclose(ml, l_full, rtol=0, atol=1e-5)
    on, ln = _numpy_merge(o_parts, l_parts)
    assert np.all(np.abs(on - o_full) <= tol)
    for mistake in ("sign", "no_renorm"):
        bad, _ = _numpy_merge(o_parts, l_parts, mistake)
        assert not np.all(np.abs(bad - o_full) <= tol), mistake
