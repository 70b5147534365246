"""GPU parity of the partial-result merge (fmha_merge_d64_bf16, through the C-ABI).

(1) Against the float64 merge oracle on random partials: 1, 2 and 5 parts,
rows where some or all parts are empty (LSE = -inf), and the in-place form
(output = part 0).  (2) End to end: the attention kernel run on disjoint key
chunks of a sequence and merged on the GPU reproduces the attention of all
keys (against the oracle, with the benchmark rule, and against the kernel's
own single launch).
"""
import numpy as np
import pytest

import fmha_native_amd as fmha
import oracle
from fmha_native_amd.problem import Problem
from harness import build_params, make_inputs, to_device
from oracle import verify

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    fmha.load_library()


def _bf16_rne(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


@pytest.mark.parametrize("n,inplace", [(1, False), (2, False), (5, False), (5, True)])
def test_merge_matches_oracle(n, inplace):
    import torch

    rows = 3001
    rng = np.random.default_rng(40 + n)
    o_parts = _bf16_rne(rng.standard_normal((n, rows * 64)))
    lse_parts = (rng.standard_normal((n, rows)) * 4).astype(np.float32)
    lse_parts[rng.random((n, rows)) < 0.2] = -np.inf  # parts that saw no key
    lse_parts[:, 17] = -np.inf                         # a row no part saw
    o_ref, l_ref = oracle.merge(o_parts, lse_parts)

    d_o = torch.from_numpy(o_parts.view(np.int16)).cuda().reshape(n, rows, 64)
    d_l = torch.from_numpy(lse_parts).cuda()
    if inplace:
        out_o, out_l = fmha.merge_partials(d_o, d_l, o=d_o[0], lse=torch.empty(rows, device="cuda"))
    else:
        out_o, out_l = fmha.merge_partials(d_o, d_l)
    torch.cuda.synchronize()
    got = out_o.cpu().numpy().reshape(-1).view(np.uint16)
    g, r = verify.bf16_bits_to_f32(got), verify.bf16_bits_to_f32(o_ref)
    # fp32 on the GPU vs float64 in the oracle: one bf16 step (<= 2^-7 |O|)
    # plus fp32 accumulation error on the weighted parts (matters only where
    # the parts cancel)
    lref = np.where(np.isfinite(l_ref), l_ref, 0.0).astype(np.float64)
    w = np.exp(lse_parts.astype(np.float64) - lref[None, :])[..., None]
    parts = np.abs(verify.bf16_bits_to_f32(o_parts).reshape(n, rows, 64))
    scale = (w * parts).sum(axis=0).reshape(-1)
    assert np.all(np.abs(g - r) <= 2.0 ** -7 * np.abs(r) + 2.0 ** -20 * scale)
    assert np.mean(got == o_ref) > 0.99
    lg = out_l.cpu().numpy()
    assert np.array_equal(np.isneginf(lg), np.isneginf(l_ref))
    fin = np.isfinite(l_ref)
    np.testing.assert_allclose(lg[fin], l_ref[fin], rtol=1e-6, atol=2e-6)
    assert np.all(got.reshape(rows, 64)[17] == 0)


def test_merge_rejects_bad_arguments():
    import torch

    x = torch.zeros((2, 8, 64), dtype=torch.int16, device="cuda")
    l = torch.zeros((2, 8), dtype=torch.float32, device="cuda")
    ok = (2, 8, x.data_ptr(), 8 * 64, l.data_ptr(), 8, 64, x[0].data_ptr(), None)
    fmha.fmha_merge_d64_bf16(*ok)
    torch.cuda.synchronize()
    for bad in [(0,) + ok[1:], (65,) + ok[1:], ok[:2] + (x.data_ptr() + 2,) + ok[3:],
                ok[:6] + (60,) + ok[7:], ok[:3] + (4 * 64,) + ok[4:]]:
        with pytest.raises(fmha.FmhaError):
            fmha.fmha_merge_d64_bf16(*bad)


@pytest.mark.parametrize("cuts", [(0, 700, 1400, 2000), (0, 64, 1999, 2000)])
def test_key_chunks_merged_equal_full_attention(cuts):
    import torch

    prob = Problem(batch=2, nhead_q=4, nhead_k=2, seqlen_q=1000, seqlen_k=2000, lse=True)
    q, k, v = make_inputs(prob, "normal", 77)
    nq, nk, nlse = prob.sizes()
    dq, dk, dv = to_device(q, torch), to_device(k, torch), to_device(v, torch)
    n = len(cuts) - 1
    o_parts = torch.zeros((n, nq), dtype=torch.int16, device="cuda")
    l_parts = torch.zeros((n, nlse), dtype=torch.float32, device="cuda")
    for i, (c0, c1) in enumerate(zip(cuts[:-1], cuts[1:])):
        p = build_params(prob, dq, dk, dv, o_parts[i], l_parts[i], None)
        p.k = dk.data_ptr() + c0 * p.stride_k * 2  # rows c0 .. c1-1 of every (batch, head)
        p.v = dv.data_ptr() + c0 * p.stride_v * 2
        p.seqlen_k = c1 - c0
        fmha.fmha_fwd_d64_bf16(p, prob.batch, 0, torch.cuda.current_stream().cuda_stream)
    o_m, l_m = fmha.merge_partials(o_parts.reshape(n, -1, 64), l_parts)
    torch.cuda.synchronize()
    o_merged = verify.bf16_bits_to_f32(o_m.cpu().numpy().reshape(-1).view(np.uint16))

    o_ref, lse_ref = oracle.run(prob, q, k, v, p_trunc=False)
    assert verify.baseline_rule(o_ref, o_merged)["pass"]
    assert verify.lse_rule(lse_ref, l_m.cpu().numpy())["pass"]

    from harness import run_kernel

    o_one, l_one = run_kernel(prob, q, k, v)
    assert verify.baseline_rule(verify.bf16_bits_to_f32(o_one), o_merged)["pass"]
    np.testing.assert_allclose(l_m.cpu().numpy(), l_one, rtol=0, atol=1e-4)
