"""Shared helpers: seeded inputs, one kernel run through the C-ABI, oracle checks.

The reference's full-kernel test does: make_params -> FmhaBuffers ->
fill_random(42) -> copy_to_device -> launch -> copy_from_device ->
cpu_ref_verify, plus LSE vs its GPU oracle (tests/test_fmha_fwd_d64.cpp:500-649).
``check_problem`` is that sequence with this build's oracle.
"""
import ctypes

import numpy as np

import fmha_native_amd as fmha
import oracle
from fmha_native_amd.problem import bhsd_to_bshd
from oracle import verify

O_SENTINEL = 0x7FC1  # bf16 NaN pattern pre-filled into O: any row left unwritten fails


def make_inputs(prob, dist="ref", seed=42, mult=1.0):
    """Host Q, K, V (uint16 bf16 bits) in ``prob``'s storage layout."""
    nq, nk, _ = prob.sizes()
    if dist == "ref":
        # reference order: Q, K, V from one srand(seed) stream, generated BHSD
        q, k, v = fmha.fill_ref(seed, nq, nk, nk)
        if prob.layout == "bshd":
            q = bhsd_to_bshd(q, prob.batch, prob.nhead_q, prob.seqlen_q)
            k = bhsd_to_bshd(k, prob.batch, prob.nhead_k, prob.seqlen_k)
            v = bhsd_to_bshd(v, prob.batch, prob.nhead_k, prob.seqlen_k)
    elif dist == "normal":
        q = fmha.fill_normal(seed, nq, mult)
        k = fmha.fill_normal(seed + 1, nk, mult)
        v = fmha.fill_normal(seed + 2, nk, mult)
    else:
        raise ValueError(dist)
    return q, k, v


def to_device(a, torch):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to("cuda:0")


def build_params(prob, dq, dk, dv, do, dlse, dseq):
    p = fmha.FmhaFwdParams()
    p.q, p.k, p.v, p.o = dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), do.data_ptr()
    p.lse = dlse.data_ptr() if dlse is not None else None
    p.seqlen_q, p.seqlen_k = prob.seqlen_q, prob.seqlen_k
    p.nhead_q, p.nhead_k = prob.nhead_q, prob.nhead_k
    p.scale = np.float32(fmha.LOG2E / np.sqrt(64.0))
    st = prob.strides()
    for t in "qkvo":
        s, hs, bs = st[t]
        setattr(p, f"stride_{t}", s)
        setattr(p, f"nhead_stride_{t}", hs)
        setattr(p, f"batch_stride_{t}", bs)
    if dseq is not None:
        p.seqstart_q = p.seqstart_k = dseq.data_ptr()
    return p


def run_kernel(prob, q, k, v, stream=None, variant=0):
    """One launch through the C-ABI; returns (O bits uint16, LSE float32 or None)."""
    import torch

    nq, nk, nlse = prob.sizes()
    dq, dk, dv = to_device(q, torch), to_device(k, torch), to_device(v, torch)
    do = torch.full((nq,), O_SENTINEL, dtype=torch.int16, device="cuda:0")
    dlse = torch.full((nlse,), float("nan"), dtype=torch.float32, device="cuda:0") if prob.lse else None
    ss = prob.seqstart()
    dseq = torch.from_numpy(ss).to("cuda:0") if ss is not None else None
    p = build_params(prob, dq, dk, dv, do, dlse, dseq)
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    orders = fmha.VARIANT_REFERENCE_ORDER | fmha.VARIANT_TILE_MAJOR_ORDER | fmha.VARIANT_SEQUENCE_ORDER
    if variant & ~orders in (fmha.VARIANT_BALANCED, fmha.VARIANT_BALANCED_PAIR):
        # the balanced form runs through the workspace entry point
        need = fmha.workspace_size(p, prob.batch, int(prob.causal), variant)
        ws = torch.empty(max(need, 256), dtype=torch.uint8, device="cuda:0")
        fmha.fmha_fwd_d64_bf16_ws(p, prob.batch, int(prob.causal), ws.data_ptr(), need, stream, variant)
    else:
        fmha.fmha_fwd_d64_bf16(p, prob.batch, int(prob.causal), stream, variant)
    torch.cuda.synchronize()
    o = do.cpu().numpy().view(np.uint16)
    lse = dlse.cpu().numpy() if dlse is not None else None
    return o, lse


def check_problem(prob, dist="ref", seed=42, mult=1.0, rule="reference", variant=0):
    """Kernel vs oracle on seeded inputs.  Returns a dict of results."""
    q, k, v = make_inputs(prob, dist, seed, mult)
    o_bits, lse = run_kernel(prob, q, k, v, variant=variant)
    o_ref, lse_ref = oracle.run(prob, q, k, v)
    o_k = verify.bf16_bits_to_f32(o_bits)
    res = {"name": prob.name}
    if rule == "reference":
        res["o"] = verify.reference_rule(o_ref, o_k)
    else:
        res["o"] = verify.baseline_rule(o_ref, o_k)
    res["pass"] = res["o"]["pass"]
    if prob.lse:
        res["lse"] = verify.lse_rule(lse_ref, lse)
        res["pass"] = res["pass"] and res["lse"]["pass"]
    return res


# Recorded parity of the benchmark configurations against the plain rule
# (|O - O_ref| <= 1e-2 + 1e-2|O_ref|, O_ref the reference-faithful oracle):
# (most violating elements, largest excess over the bound among them), per
# configuration and kernel form.  cfg5 (inputs x2, a peaked softmax) is where
# the oracle's own bf16 truncation of P (cpu_ref.cpp:137-144) reaches the
# tolerance; its counts are those of the kernels as built (MI355X, one run of
# each form; the results are deterministic) and a change that adds violations
# fails.  Every other configuration passes the plain rule outright.
CONTRACT_BOUNDS = {
    "cfg5": {"auto": (15, 0.0059), "regular": (15, 0.0059), "pair": (15, 0.0059), "splitkv": (14, 0.0030),
             "balanced": (15, 0.0059), "balanced_pair": (16, 0.0059), "short": (3, 0.0011),
             "pair_stream": (15, 0.0059)},
}


def contract_bound(cfg, form):
    """(violations, excess) allowed for ``cfg`` in ``form`` (0, 0.0: none)."""
    return CONTRACT_BOUNDS.get(cfg, {}).get(form, (0, 0.0))


def contract_ok(res, bound):
    """Whether a check_baseline result stays within a recorded bound: no more
    plain-rule violations, no larger excess, and every violation explained by
    the oracle's own P truncation (``o_unexplained == 0``)."""
    n, excess = bound
    return (res["o_plain"]["violations"] <= n and res["o_plain"]["max_excess"] <= excess
            and res["o_unexplained"] == 0)


def contract_counts(o_t, o_u, o_k):
    """Plain rule against the faithful oracle ``o_t`` and the count of
    violations not covered by that oracle's truncation error |o_t - o_u|."""
    err = np.abs(o_k - o_t)
    tol = 1e-2 + 1e-2 * np.abs(o_t) + np.abs(o_t - o_u)
    return verify.baseline_rule(o_t, o_k), int(np.count_nonzero(~(err <= tol)))


def check_baseline(prob, mult=1.0, seed=42, variant=0):
    """Benchmark-configuration check (N(0,1)*mult inputs).

    O must be within 1e-2 + 1e-2|O| of (a) the oracle without the reference's
    bf16 truncation of P, everywhere, and (b) the reference-faithful oracle,
    where any excess must be covered by that oracle's own truncation error
    |O_trunc - O_untrunc| at the element.  The plain count against (b) is
    reported as ``o_plain``.  LSE within 1e-3 of the oracle.
    """
    q, k, v = make_inputs(prob, "normal", seed, mult)
    o_bits, lse = run_kernel(prob, q, k, v, variant=variant)
    o_t, lse_t = oracle.run(prob, q, k, v)
    o_u, _ = oracle.run(prob, q, k, v, p_trunc=False)
    o_k = verify.bf16_bits_to_f32(o_bits)
    res = {"name": prob.name}
    res["o_plain"], res["o_unexplained"] = contract_counts(o_t, o_u, o_k)
    res["o_vs_untruncated"] = verify.baseline_rule(o_u, o_k)
    res["pass"] = res["o_vs_untruncated"]["pass"] and res["o_unexplained"] == 0
    if prob.lse:
        res["lse"] = verify.lse_rule(lse_t, lse)
        res["pass"] = res["pass"] and res["lse"]["pass"]
    return res
