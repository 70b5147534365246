"""Write the golden fixtures under tests/golden/ (run from the repo root):

    python tests/golden/make_golden.py

The reference ships no golden vectors (its CK dumps under /tmp are not in the
tree, tests/test_fmha_fwd_d64.cpp:787-795), so the fixtures pin this build's
oracle on the reference's own inputs, cross-checked at generation time by an
independent float64 numpy evaluation (tests/np_ref.py):

* ``cfg1_ref42.npz`` — config 1 (B1 H2 S128, D64, non-causal, LSE) on the
  reference generator ``fill_random(42)`` (src/runner/buffers.cpp:99-127):
  SHA-256 of the Q/K/V bf16 bit patterns, the oracle's fp32 O and LSE
  (bit-exact targets for the oracle) and the float64 O and LSE (stored
  rounded to float32: ``o_exact``, ``lse_exact``).
* ``ck_known_answer.npz`` — the reference's CK known-answer inputs
  (tests/test_fmha_fwd_d64.cpp:690-695: Q = (i%256)/256, K = ((i+64)%256)/256,
  V = (i%256)/256 + 1, bf16-truncated, B1 H1) at Sq x Sk = 64x64 and 17x33:
  oracle O and the float64 O (rounded to float32).

Regenerating must reproduce the committed files exactly (tests check the
oracle against them bit for bit).
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import oracle  # noqa: E402
import np_ref  # noqa: E402
from fmha_native_amd.problem import Problem  # noqa: E402


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def f32_to_bf16_trunc(x):
    return (np.asarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def cfg1():
    prob = Problem(batch=1, nhead_q=2, seqlen_q=128, lse=True, name="cfg1")
    nq, nk, _ = prob.sizes()
    q, k, v = oracle.fill_ref(42, nq, nk, nk)
    o, lse = oracle.run(prob, q, k, v, faithful=True, nthreads=1)
    o64, lse64 = np_ref.attention(prob, q, k, v)
    return prob, (q, k, v), dict(q_sha=sha(q), k_sha=sha(k), v_sha=sha(v), o=o, lse=lse,
                                 o_exact=o64.astype(np.float32), lse_exact=lse64.astype(np.float32))


def ck_inputs(sq, sk):
    D = 64
    iq = np.arange(sq * D)
    ik = np.arange(sk * D)
    q = f32_to_bf16_trunc((iq % 256) / np.float32(256.0))
    k = f32_to_bf16_trunc(((ik + 64) % 256) / np.float32(256.0))
    v = f32_to_bf16_trunc((ik % 256) / np.float32(256.0) + np.float32(1.0))
    return q, k, v


def ck_case(sq, sk):
    prob = Problem(batch=1, nhead_q=1, seqlen_q=sq, seqlen_k=sk, name=f"ck_{sq}x{sk}")
    q, k, v = ck_inputs(sq, sk)
    o, _ = oracle.run(prob, q, k, v, faithful=True, nthreads=1)
    o64, _ = np_ref.attention(prob, q, k, v)
    return o, o64


def main():
    prob, _, d = cfg1()
    # generation-time cross-check: oracle (with its bf16 P truncation) vs float64
    err = np.abs(d["o"] - d["o_exact"]).max()
    lerr = np.abs(d["lse"] - d["lse_exact"]).max()
    assert err < 2e-3 and lerr < 1e-5, (err, lerr)
    np.savez_compressed(os.path.join(HERE, "cfg1_ref42.npz"), **d)
    out = {}
    for sq, sk in ((64, 64), (17, 33)):
        o, o64 = ck_case(sq, sk)
        assert np.abs(o - o64).max() < 2e-2
        out[f"o_{sq}x{sk}"] = o
        out[f"o_exact_{sq}x{sk}"] = o64.astype(np.float32)
    np.savez_compressed(os.path.join(HERE, "ck_known_answer.npz"), **out)
    print("wrote cfg1_ref42.npz, ck_known_answer.npz; cfg1 oracle-vs-f64 max |dO| =", err, "|dLSE| =", lerr)


if __name__ == "__main__":
    main()
