"""GPU tests of the balanced causal form, through fmha_fwd_d64_bf16_ws.

A split M-tile's two key halves are the split-KV form's two halves (the first
ceil(n/2) key tiles and the rest) merged with the same fp32 arithmetic, and a
whole M-tile runs the regular form's code path; so every M-tile's rows of O
and LSE must equal, bit for bit, the split-KV form's (split M-tiles) or the
regular form's (the others).  The results also meet the benchmark rule
against the oracle, the automatic choice takes the balanced form on the
B1 H2 S40000 configuration when given a workspace, and a workspace can be
reused without clearing it.
"""
import numpy as np
import pytest

import fmha_native_amd as fmha
import oracle
from fmha_native_amd.problem import Problem
from harness import build_params, make_inputs, run_kernel, to_device
from oracle import verify

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    fmha.load_library()


def _split_from(prob):
    import torch

    nq, nk, nlse = prob.sizes()
    host = [torch.empty(n, dtype=torch.int16) for n in (nq, nk, nk, nq)]
    p = build_params(prob, *host, torch.empty(max(nlse, 1), dtype=torch.float32) if prob.lse else None, None)
    items, sf = fmha.balanced_plan(p, prob.batch, 1, 0, force=True)
    assert items, "the forced plan must exist for a causal dense problem"
    return sf


@pytest.mark.parametrize("b,h,hk,sq,sk,lse,mult", [
    (1, 2, 2, 40000, 40000, True, 2.0),   # the benchmark configuration (heavy M-tiles split)
    (1, 2, 1, 5000, 5000, True, 1.0),
    (2, 4, 2, 3000, 3500, True, 1.0),     # Sk > Sq, GQA, two batches
    (1, 3, 1, 2000, 1500, False, 1.0),    # Sq > Sk: the first rows see no key
    (3, 2, 2, 700, 700, True, 1.0),
])
def test_balanced_equals_splitkv_and_regular_per_mtile(b, h, hk, sq, sk, lse, mult):
    prob = Problem(batch=b, nhead_q=h, nhead_k=hk, seqlen_q=sq, seqlen_k=sk, causal=True, lse=lse)
    sf = _split_from(prob)
    q, k, v = make_inputs(prob, "normal", 61, mult)
    ob, lb = run_kernel(prob, q, k, v, variant=fmha.VARIANT_BALANCED)
    os_, ls = run_kernel(prob, q, k, v, variant=fmha.VARIANT_SPLITKV)
    orr, lr = run_kernel(prob, q, k, v, variant=fmha.VARIANT_REGULAR)
    rows = np.arange(sq)
    split = (rows // 128) >= sf
    print(f"split_from {sf}: {split.sum()} of {sq} rows in split M-tiles", flush=True)
    o3 = [x.reshape(b, h, sq, 64) for x in (ob, os_, orr)]
    assert np.array_equal(o3[0][:, :, split], o3[1][:, :, split])
    assert np.array_equal(o3[0][:, :, ~split], o3[2][:, :, ~split])
    if lse:
        l3 = [x.reshape(b, h, sq) for x in (lb, ls, lr)]
        assert np.array_equal(l3[0][:, :, split], l3[1][:, :, split])
        assert np.array_equal(l3[0][:, :, ~split], l3[2][:, :, ~split])
    o_ref, l_ref = oracle.run(prob, q, k, v, p_trunc=False)
    assert verify.baseline_rule(o_ref, verify.bf16_bits_to_f32(ob))["pass"]
    if lse:
        assert verify.lse_rule(l_ref, lb)["pass"]


@pytest.mark.parametrize("b,h,hk,sq,sk,lse,mult", [
    (1, 2, 2, 40000, 40000, True, 2.0),   # the benchmark configuration: 313 M-tiles, an odd last pair
    (1, 2, 1, 5000, 5000, True, 1.0),
    (2, 4, 2, 3000, 3500, True, 1.0),     # Sk > Sq, GQA, two batches
    (1, 3, 1, 2000, 1500, False, 1.0),    # Sq > Sk: the first rows see no key
    (3, 2, 2, 700, 700, True, 1.0),
    (1, 2, 2, 8192, 8192, True, 1.0),     # an even M-tile count
])
def test_balanced_pair_equals_pair_and_splitkv_per_mtile(b, h, hk, sq, sk, lse, mult):
    """The balanced form over M-tile pairs: a whole pair runs the pair form's
    code path (bits equal the pair form's); a split pair's second M-tile has
    the pair's key tiles, so its two halves are the split-KV form's (bits
    equal); its first M-tile's halves differ from the split-KV form's (the
    pair's two extra, masked, key tiles shift the cut), so those rows meet the
    rule against the oracle, as every row does."""
    import torch

    prob = Problem(batch=b, nhead_q=h, nhead_k=hk, seqlen_q=sq, seqlen_k=sk, causal=True, lse=lse)
    nq, nk, nlse = prob.sizes()
    host = [torch.empty(n, dtype=torch.int16) for n in (nq, nk, nk, nq)]
    p = build_params(prob, *host, torch.empty(max(nlse, 1), dtype=torch.float32) if lse else None, None)
    items, sf = fmha.balanced_plan(p, prob.batch, 1, 0, force="pair")
    assert items
    q, k, v = make_inputs(prob, "normal", 64, mult)
    ob, lb = run_kernel(prob, q, k, v, variant=fmha.VARIANT_BALANCED_PAIR)
    op, lp = run_kernel(prob, q, k, v, variant=fmha.VARIANT_PAIR)
    os_, ls = run_kernel(prob, q, k, v, variant=fmha.VARIANT_SPLITKV)
    mt = np.arange(sq) // 128
    split = mt >= sf
    odd = split & (mt % 2 == 1)
    print(f"split_from {sf}: {split.sum()} of {sq} rows in split M-tiles", flush=True)
    o3 = [x.reshape(b, h, sq, 64) for x in (ob, op, os_)]
    assert np.array_equal(o3[0][:, :, ~split], o3[1][:, :, ~split])
    assert np.array_equal(o3[0][:, :, odd], o3[2][:, :, odd])
    if lse:
        l3 = [x.reshape(b, h, sq) for x in (lb, lp, ls)]
        assert np.array_equal(l3[0][:, :, ~split], l3[1][:, :, ~split])
        assert np.array_equal(l3[0][:, :, odd], l3[2][:, :, odd])
    o_ref, l_ref = oracle.run(prob, q, k, v, p_trunc=False)
    assert verify.baseline_rule(o_ref, verify.bf16_bits_to_f32(ob))["pass"]
    if lse:
        assert verify.lse_rule(l_ref, lb)["pass"]


@pytest.mark.parametrize("form", ["balanced", "balanced_pair"])
@pytest.mark.parametrize("b,h,sq,mult", [
    (1, 2, 40000, 2.0),   # the benchmark configuration: 4 XCD groups per (batch, head)
    (1, 1, 20000, 1.0),   # 8 groups
    (1, 4, 16384, 1.0),   # 2 groups
    (2, 1, 12000, 1.0),   # 4 groups, two batches
])
def test_xcd_ordered_table_equals_plain_order_bitwise(form, b, h, sq, mult):
    """The default table orders each run of XCD groups by first key;
    FMHA_VARIANT_REFERENCE_ORDER launches the plain heaviest-first table.
    Both hold the same items, so O and LSE are equal bit for bit."""
    import torch

    prob = Problem(batch=b, nhead_q=h, seqlen_q=sq, causal=True, lse=True)
    nq, nk, nlse = prob.sizes()
    host = [torch.empty(n, dtype=torch.int16) for n in (nq, nk, nk, nq)]
    p = build_params(prob, *host, torch.empty(nlse, dtype=torch.float32), None)
    force = "pair" if form == "balanced_pair" else True
    table, _ = fmha.balanced_plan(p, b, 1, 0, force=force)
    plain, _ = fmha.balanced_plan(p, b, 1, 0, force=force, xccs=1)
    print(f"{prob.name} {form}: {sum(x != y for x, y in zip(table, plain))} of {len(plain)} entries moved", flush=True)
    assert table != plain and sorted(table) == sorted(plain)  # the device's 8 XCDs group this shape
    v = fmha.VARIANTS[form]
    q, k, vv = make_inputs(prob, "normal", 71, mult)
    og, lg = run_kernel(prob, q, k, vv, variant=v)
    op, lp = run_kernel(prob, q, k, vv, variant=v | fmha.VARIANT_REFERENCE_ORDER)
    assert np.array_equal(og, op)
    assert np.array_equal(lg, lp)


def test_auto_takes_balanced_with_a_workspace_and_reuses_it():
    """B1 H2 S40000 causal: the automatic choice with a workspace is the
    balanced form (its bits equal the forced balanced launch's); a second
    launch into the same, now dirty, workspace gives the same bits; without a
    workspace the launch falls back to the regular form's bits."""
    import torch

    prob = Problem(batch=1, nhead_q=2, seqlen_q=40000, causal=True, lse=True)
    q, k, v = make_inputs(prob, "normal", 62, 2.0)
    nq, nk, nlse = prob.sizes()
    dq, dk, dv = to_device(q, torch), to_device(k, torch), to_device(v, torch)
    do = torch.zeros(nq, dtype=torch.int16, device="cuda:0")
    dl = torch.zeros(nlse, dtype=torch.float32, device="cuda:0")
    p = build_params(prob, dq, dk, dv, do, dl, None)
    need = fmha.workspace_size(p, 1, 1)
    assert need > 0 and need == fmha.workspace_size(p, 1, 1, fmha.VARIANT_BALANCED)
    ws = torch.full((need,), 0x7F, dtype=torch.uint8, device="cuda:0")  # garbage: needs no clearing
    outs = []
    for variant in (fmha.VARIANT_AUTO, fmha.VARIANT_AUTO, fmha.VARIANT_BALANCED):
        do.zero_()
        fmha.fmha_fwd_d64_bf16_ws(p, 1, 1, ws.data_ptr(), need, None, variant)
        torch.cuda.synchronize()
        outs.append((do.clone(), dl.clone()))
    for o, l in outs[1:]:
        assert torch.equal(o, outs[0][0]) and torch.equal(l, outs[0][1])
    ob, lb = run_kernel(prob, q, k, v, variant=fmha.VARIANT_BALANCED)
    assert np.array_equal(outs[0][0].cpu().numpy().view(np.uint16), ob)
    do.zero_()
    fmha.fmha_fwd_d64_bf16_ws(p, 1, 1, None, 0, None)  # no workspace: the regular form
    torch.cuda.synchronize()
    orr, _ = run_kernel(prob, q, k, v, variant=fmha.VARIANT_REGULAR)
    assert np.array_equal(do.cpu().numpy().view(np.uint16), orr)


def test_fmha_fwd_wrapper_uses_the_workspace_path():
    """The torch wrapper allocates the workspace itself: its output equals
    the balanced launch's."""
    import torch

    prob = Problem(batch=1, nhead_q=2, seqlen_q=40000, causal=True, lse=True)
    q, k, v = make_inputs(prob, "normal", 63)
    t = lambda a, hh: torch.from_numpy(a.view(np.int16)).cuda().view(torch.bfloat16).view(1, hh, 40000, 64)
    o, lse = fmha.fmha_fwd(t(q, 2), t(k, 2), t(v, 2), causal=True, return_lse=True)
    torch.cuda.synchronize()
    ob, lb = run_kernel(prob, q, k, v, variant=fmha.VARIANT_BALANCED)
    assert np.array_equal(o.view(torch.int16).cpu().numpy().reshape(-1).view(np.uint16), ob)
    assert np.array_equal(lse.cpu().numpy().reshape(-1), lb)
