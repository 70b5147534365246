"""The allocation-free entry point, through the C-ABI: fmha_fwd_d64_bf16_noalloc
must give the bits of fmha_fwd_d64_bf16_ws with a workspace of its own, call
after call in one process (the static array keeps the previous call's
contents), and refuse plans larger than its array without launching.
"""
import ctypes

import numpy as np
import pytest

import fmha_native_amd as fmha
from fmha_native_amd.problem import Problem
from harness import build_params, make_inputs, to_device

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20  # FMHA_NOALLOC_SCRATCH_BYTES


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    fmha.load_library()


def _launch(prob, q, k, v, noalloc, variant=fmha.VARIANT_AUTO):
    import torch

    nq, nk, nlse = prob.sizes()
    dq, dk, dv = to_device(q, torch), to_device(k, torch), to_device(v, torch)
    do = torch.full((nq,), 0x7FC1, dtype=torch.int16, device="cuda:0")
    dl = torch.full((nlse,), float("nan"), dtype=torch.float32, device="cuda:0")
    p = build_params(prob, dq, dk, dv, do, dl, None)
    lib = fmha.load_library()
    if noalloc:
        rc = lib.fmha_fwd_d64_bf16_noalloc(ctypes.byref(p), prob.batch, 1, variant, None)
    else:
        need = fmha.workspace_size(p, prob.batch, 1, variant)
        ws = torch.empty(max(need, 256), dtype=torch.uint8, device="cuda:0")
        rc = lib.fmha_fwd_d64_bf16_ws(ctypes.byref(p), prob.batch, 1, variant, ws.data_ptr(), need, None)
    assert rc == 0, rc
    torch.cuda.synchronize()
    return do.cpu().numpy().view(np.uint16), dl.cpu().numpy()


@pytest.mark.parametrize("variant", [fmha.VARIANT_AUTO, fmha.VARIANT_BALANCED_PAIR])
def test_no_alloc_equals_workspace_entry_on_two_calls(variant):
    """Two calls in a row, the second on a smaller problem: the balanced form
    (30.4 MB of partials, then 2.3 MB; over M-tile pairs 24.9 MB, then less)
    from the static array gives the bits the workspace entry gives."""
    for seq, heads, mult in ((40000, 2, 2.0), (16384, 2, 1.0)):
        prob = Problem(batch=1, nhead_q=heads, seqlen_q=seq, causal=True, lse=True)
        q, k, v = make_inputs(prob, "normal", 70 + heads, mult)
        print(f"noalloc vs ws (variant {variant}): B1 H{heads} S{seq} causal", flush=True)
        o_ws, l_ws = _launch(prob, q, k, v, noalloc=False, variant=variant)
        o_na, l_na = _launch(prob, q, k, v, noalloc=True, variant=variant)
        assert np.array_equal(o_na, o_ws)
        assert np.array_equal(l_na, l_ws)


def test_no_alloc_refuses_plans_beyond_its_array():
    """B1 H16 S8192 with the balanced form forced needs 35.7 MB of partials,
    more than the 32 MiB array: refused, nothing launched, the output left
    as it was."""
    import torch

    prob = Problem(batch=1, nhead_q=16, seqlen_q=8192, causal=True, lse=True)
    nq, nk, nlse = prob.sizes()
    t = [torch.zeros(n, dtype=torch.int16, device="cuda:0") for n in (nq, nk, nk)]
    do = torch.full((nq,), 0x7FC1, dtype=torch.int16, device="cuda:0")
    p = build_params(prob, *t, do, torch.zeros(nlse, dtype=torch.float32, device="cuda:0"), None)
    assert fmha.workspace_size(p, 1, 1, fmha.VARIANT_BALANCED) > SCRATCH_BYTES
    lib = fmha.load_library()
    assert lib.fmha_fwd_d64_bf16_noalloc(ctypes.byref(p), 1, 1, fmha.VARIANT_BALANCED, None) == fmha.HIP_ERROR_INVALID_VALUE
    torch.cuda.synchronize()
    assert bool((do == 0x7FC1).all())
