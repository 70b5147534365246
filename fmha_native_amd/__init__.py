"""fmha_native_amd — MI355X (gfx950) D64 BF16 fused multi-head attention forward.

Host-side mirror of the reference's interface for this path:

* ``FmhaFwdParams`` — the kernarg struct, field for field and byte for byte
  (reference ``src/runner/params.hpp:18-64``; C declaration in
  ``include/fmha_fwd.h``).
* ``fmha_fwd_d64_bf16(params, batch, causal, stream)`` — the C-ABI launcher
  that replaces the reference's launch sites (``src/bench_fmha_fwd.cpp:174-191``).
  Errors raise :class:`FmhaError` carrying the ``hipError_t`` code.
* ``fill_ref`` / ``fill_normal`` / ``varlen_lengths`` — the seeded input
  generators (reference ``src/runner/buffers.cpp:99-127`` plus N(0,1)).
* ``fmha_fwd(q, k, v, ...)`` — convenience wrapper over torch device tensors
  (torch is used only for device memory and the stream).

The compiled library ``libfmha_native_amd.so`` is required: there is no CPU or
PyTorch fallback for the attention itself, and a missing library raises.
"""
import ctypes
import math
import os

import numpy as np

__all__ = [
    "FmhaError", "FmhaFwdParams", "LIB_PATH", "load_library", "fmha_fwd_d64_bf16", "check_params",
    "tile_config", "pick_variant", "tile_major", "fill_ref", "fill_normal", "varlen_lengths", "params_from_tensors", "fmha_fwd",
    "fmha_merge_d64_bf16", "merge_partials", "MERGE_MAX_PARTS",
    "LOG2E", "HIP_ERROR_INVALID_VALUE", "VARIANT_AUTO", "VARIANT_REGULAR", "VARIANT_SPLITKV", "VARIANT_PAIR",
    "VARIANT_BALANCED", "VARIANT_SHORT", "VARIANT_BALANCED_PAIR", "VARIANT_PAIR_STREAM", "fmha_fwd_d64_bf16_ws", "workspace_size", "balanced_plan",
    "VARIANT_REFERENCE_ORDER", "VARIANT_TILE_MAJOR_ORDER", "VARIANT_SEQUENCE_ORDER", "VARIANTS",
    "ORDERS", "variant_code",
]

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libfmha_native_amd.so")
LOG2E = 1.4426950408889634
HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1
HEAD_DIM = 64
MERGE_MAX_PARTS = 64
INT32_MAX = 2**31 - 1


class FmhaError(RuntimeError):
    """A non-zero hipError_t returned by the library."""

    def __init__(self, code, what="fmha_fwd_d64_bf16"):
        super().__init__(f"{what} returned hipError_t {code}")
        self.code = code


class FmhaFwdParams(ctypes.Structure):
    """Kernarg block; identical layout to the C struct (128 bytes, align 8)."""

    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p), ("lse", ctypes.c_void_p),
        ("seqlen_q", ctypes.c_int), ("seqlen_k", ctypes.c_int),
        ("nhead_q", ctypes.c_int), ("nhead_k", ctypes.c_int),
        ("scale", ctypes.c_float),
        ("stride_q", ctypes.c_int), ("nhead_stride_q", ctypes.c_int), ("batch_stride_q", ctypes.c_int),
        ("stride_k", ctypes.c_int), ("nhead_stride_k", ctypes.c_int), ("batch_stride_k", ctypes.c_int),
        ("stride_v", ctypes.c_int), ("nhead_stride_v", ctypes.c_int), ("batch_stride_v", ctypes.c_int),
        ("stride_o", ctypes.c_int), ("nhead_stride_o", ctypes.c_int), ("batch_stride_o", ctypes.c_int),
        ("seqstart_q", ctypes.c_void_p), ("seqstart_k", ctypes.c_void_p),
    ]


_lib = None


def load_library(path=LIB_PATH):
    """Load the HIP library (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is missing: build it with `python -m fmha_native_amd.build` "
            "(there is no fallback implementation)")
    lib = ctypes.CDLL(path)
    P = ctypes.POINTER(FmhaFwdParams)
    lib.fmha_fwd_d64_bf16.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.fmha_fwd_d64_bf16.restype = ctypes.c_int
    lib.fmha_fwd_d64_bf16_variant.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.fmha_fwd_d64_bf16_variant.restype = ctypes.c_int
    lib.fmha_fwd_d64_bf16_check.argtypes = [P, ctypes.c_int, ctypes.c_int]
    lib.fmha_fwd_d64_bf16_check.restype = ctypes.c_int
    lib.fmha_fwd_d64_bf16_pick_variant.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.fmha_fwd_d64_bf16_pick_variant.restype = ctypes.c_int
    lib.fmha_fwd_d64_bf16_tile_major.argtypes = [P, ctypes.c_int, ctypes.c_int]
    lib.fmha_fwd_d64_bf16_tile_major.restype = ctypes.c_int
    lib.fmha_fwd_d64_bf16_ws.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64,
                                         ctypes.c_void_p]
    lib.fmha_fwd_d64_bf16_ws.restype = ctypes.c_int
    lib.fmha_fwd_d64_bf16_noalloc.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.fmha_fwd_d64_bf16_noalloc.restype = ctypes.c_int
    lib.fmha_fwd_d64_bf16_workspace_size.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.fmha_fwd_d64_bf16_workspace_size.restype = ctypes.c_int64
    lib.fmha_fwd_d64_bf16_balanced_plan.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                    ctypes.c_int, ctypes.POINTER(ctypes.c_uint16), ctypes.c_int,
                                                    ctypes.POINTER(ctypes.c_int)]
    lib.fmha_fwd_d64_bf16_balanced_plan.restype = ctypes.c_int
    ip = ctypes.POINTER(ctypes.c_int)
    lib.fmha_fwd_d64_bf16_tile_config.argtypes = [ip, ip, ip, ip]
    lib.fmha_fwd_d64_bf16_tile_config.restype = None
    i64, vp = ctypes.c_int64, ctypes.c_void_p
    lib.fmha_merge_d64_bf16.argtypes = [ctypes.c_int, i64, vp, i64, vp, i64, i64, vp, vp, vp]
    lib.fmha_merge_d64_bf16.restype = ctypes.c_int
    u16p = ctypes.POINTER(ctypes.c_uint16)
    lib.fmha_runner_fill_ref.argtypes = [ctypes.c_uint, u16p, ctypes.c_size_t, u16p, ctypes.c_size_t, u16p,
                                         ctypes.c_size_t]
    lib.fmha_runner_fill_ref.restype = None
    lib.fmha_runner_fill_normal.argtypes = [ctypes.c_uint64, ctypes.c_float, u16p, ctypes.c_size_t]
    lib.fmha_runner_fill_normal.restype = None
    lib.fmha_runner_varlen_lengths.argtypes = [ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ip]
    lib.fmha_runner_varlen_lengths.restype = ctypes.c_int
    _lib = lib
    return lib


VARIANT_AUTO, VARIANT_REGULAR, VARIANT_SPLITKV, VARIANT_PAIR, VARIANT_BALANCED = 0, 1, 2, 3, 5
VARIANT_SHORT = 6
VARIANT_BALANCED_PAIR = 7  # the balanced form over M-tile pairs (a workspace, like VARIANT_BALANCED)
VARIANT_PAIR_STREAM = 8  # pair blocks looping over M-tile pairs (dense layouts only)
# flag OR-ed into a variant: causal dense batches run batch after batch on the
# reference's grid, never on the tile-major entries (results are identical)
VARIANT_REFERENCE_ORDER = 16
# flags: tile-major entries / the level order of causal varlen launches, and
# the sequence order of causal varlen launches (longest sequence first)
VARIANT_TILE_MAJOR_ORDER = 32
VARIANT_SEQUENCE_ORDER = 64
VARIANTS = {"auto": VARIANT_AUTO, "regular": VARIANT_REGULAR, "splitkv": VARIANT_SPLITKV, "pair": VARIANT_PAIR,
            "balanced": VARIANT_BALANCED, "short": VARIANT_SHORT,
            "balanced_pair": VARIANT_BALANCED_PAIR, "pair_stream": VARIANT_PAIR_STREAM}
ORDERS = {"reference": VARIANT_REFERENCE_ORDER, "tilemajor": VARIANT_TILE_MAJOR_ORDER,
          "sequence": VARIANT_SEQUENCE_ORDER}


def variant_code(v):
    """Launcher code of a variant name: a form of ``VARIANTS`` optionally
    followed by ``|reference``, ``|tilemajor`` or ``|sequence`` (one block-order
    flag), e.g. ``"regular|sequence"``; an integer or digit string is taken
    as the code itself."""
    if isinstance(v, int):
        return v
    name, _, order = str(v).partition("|")
    code = int(name) if name.isdigit() else VARIANTS[name]
    return code | (ORDERS[order] if order else 0)


def fmha_fwd_d64_bf16(params, batch, causal, stream=None, variant=VARIANT_AUTO):
    """Launch on ``stream`` (a hipStream_t as int, or None for the null stream).

    ``variant``: VARIANT_AUTO (the launcher's choice), VARIANT_REGULAR (the
    reference-named entries), VARIANT_SPLITKV (the split-KV entries),
    VARIANT_PAIR (the pair entries) or VARIANT_SHORT (the short entries),
    each optionally OR-ed with
    VARIANT_REFERENCE_ORDER (keep the reference's batch-after-batch block order
    for causal dense batches)."""
    lib = load_library()
    if variant == VARIANT_AUTO:
        rc = lib.fmha_fwd_d64_bf16(ctypes.byref(params), int(batch), int(causal), stream)
    else:
        rc = lib.fmha_fwd_d64_bf16_variant(ctypes.byref(params), int(batch), int(causal), int(variant), stream)
    if rc != HIP_SUCCESS:
        raise FmhaError(rc)


def fmha_fwd_d64_bf16_ws(params, batch, causal, workspace=None, workspace_bytes=0, stream=None,
                         variant=VARIANT_AUTO):
    """The launch with a workspace (device pointer as int, 256-byte aligned,
    at least :func:`workspace_size` bytes; None with 0 bytes allowed), which
    lets dense causal launches with few heavy M-tiles run the balanced form.
    ``variant``: VARIANT_AUTO, VARIANT_BALANCED, VARIANT_BALANCED_PAIR or any
    other (workspace unused).  Raises :class:`FmhaError` on a non-zero hipError_t."""
    rc = load_library().fmha_fwd_d64_bf16_ws(ctypes.byref(params), int(batch), int(causal), int(variant), workspace,
                                             int(workspace_bytes), stream)
    if rc != HIP_SUCCESS:
        raise FmhaError(rc, "fmha_fwd_d64_bf16_ws")


def workspace_size(params, batch, causal, variant=VARIANT_AUTO):
    """Workspace bytes :func:`fmha_fwd_d64_bf16_ws` needs (0: none; -1:
    rejected arguments).  Host only."""
    return load_library().fmha_fwd_d64_bf16_workspace_size(ctypes.byref(params), int(batch), int(causal),
                                                           int(variant))


def balanced_plan(params, batch, causal, compute_units=0, force=False, xccs=0):
    """(items, split_from) of the balanced form's plan: items per (batch,
    head) in dispatch order as (unit, half) pairs, half None for a whole
    unit; ([], None) when the launch would not be balanced.  ``force``: False
    (the automatic rule), True (over M-tiles, as VARIANT_BALANCED) or "pair"
    (over M-tile pairs, as VARIANT_BALANCED_PAIR: unit u is M-tiles 2u and
    2u+1).  ``xccs``: XCD count of the dispatch order (0: the current
    device's, 8 without one; 1: plain heaviest first, as launched with
    VARIANT_REFERENCE_ORDER).  split_from counts M-tiles.  Host only."""
    pair = force == "pair"
    cap = 4096
    buf = (ctypes.c_uint16 * cap)()
    sf = ctypes.c_int(-1)
    n = load_library().fmha_fwd_d64_bf16_balanced_plan(ctypes.byref(params), int(batch), int(causal),
                                                       int(compute_units), int(xccs), 2 if pair else int(bool(force)),
                                                       buf, cap,
                                                       ctypes.byref(sf))
    if n < 0:
        raise FmhaError(HIP_ERROR_INVALID_VALUE, "fmha_fwd_d64_bf16_balanced_plan")
    if n == 0:
        return [], None
    first = 2 if pair else 1  # M-tiles per unit
    items = [(v & 0x7FFF, (v >> 15) if first * (v & 0x7FFF) >= sf.value else None) for v in buf[:n]]
    return items, sf.value


def check_params(params, batch, causal):
    """Host-only argument check; returns the hipError_t code (0 = accepted)."""
    return load_library().fmha_fwd_d64_bf16_check(ctypes.byref(params), int(batch), int(causal))


def pick_variant(params, batch, causal, compute_units=0):
    """The form VARIANT_AUTO resolves to on a device with ``compute_units``
    CUs (0 = the current device's); -1 for rejected arguments.  Host only."""
    return load_library().fmha_fwd_d64_bf16_pick_variant(ctypes.byref(params), int(batch), int(causal),
                                                          int(compute_units))


def tile_major(params, batch, causal):
    """Block order of the automatic launch: 1 for a tile-major causal entry
    (every batch's heaviest M-tiles first) or the level order of a compact
    causal varlen entry (the live M-tiles of all sequences, highest M-tile
    index first), 2 for the sequence order of a compact varlen entry (longest
    sequence first), 0 for the reference's batch-after-batch order, -1 for
    rejected arguments.  Host only."""
    return load_library().fmha_fwd_d64_bf16_tile_major(ctypes.byref(params), int(batch), int(causal))


def tile_config():
    vals = [ctypes.c_int() for _ in range(4)]
    load_library().fmha_fwd_d64_bf16_tile_config(*[ctypes.byref(v) for v in vals])
    return {"kM0": vals[0].value, "kN0": vals[1].value, "kBlockSize": vals[2].value, "kHeadDim": vals[3].value}


def _u16ptr(a):
    assert a.dtype == np.uint16 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))


def fill_ref(seed, nq, nk, nv):
    """The reference generator: srand(seed) then Q, K, V (uint16 bf16 bits)."""
    q, k, v = (np.empty(n, dtype=np.uint16) for n in (nq, nk, nv))
    load_library().fmha_runner_fill_ref(seed, _u16ptr(q), nq, _u16ptr(k), nk, _u16ptr(v), nv)
    return q, k, v


def fill_normal(seed, n, mult=1.0):
    """i.i.d. N(0,1)*mult as bf16 bits (stream ``seed``)."""
    out = np.empty(n, dtype=np.uint16)
    load_library().fmha_runner_fill_normal(seed, mult, _u16ptr(out), n)
    return out


def varlen_lengths(seed, n, lo, hi):
    out = (ctypes.c_int * n)()
    rc = load_library().fmha_runner_varlen_lengths(seed, n, lo, hi, out)
    if rc != 0:
        raise ValueError("bad varlen length request")
    return list(out)


def _check_kernarg_ints(q, k, v, o, max_seqlen_q, max_seqlen_k):
    """Every kernarg integer is a C int: reject a value that would wrap instead
    of letting ctypes truncate it silently (a wrapped stride can come out
    positive, pass every check and alias another batch or head)."""
    ints = {"max_seqlen_q": max_seqlen_q, "max_seqlen_k": max_seqlen_k}
    for name, t in (("q", q), ("k", k), ("v", v), ("o", o)):
        ints[f"{name}.shape"] = max(t.shape)
        ints.update({f"{name}.stride({d})": t.stride(d) for d in range(t.dim())})
    for name, val in ints.items():
        if val is not None and not 0 <= int(val) <= INT32_MAX:
            raise ValueError(f"{name} = {val} does not fit the kernarg's 32-bit int")


def _check_tensors(q, k, v, o, lse, seqstart_q, seqstart_k, max_seqlen_q, max_seqlen_k=None):
    import torch

    varlen = seqstart_q is not None
    rank = 3 if varlen else 4
    for name, t in (("q", q), ("k", k), ("v", v), ("o", o)):
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bfloat16, got {t.dtype}")
        if t.dim() != rank:
            raise ValueError(f"{name} must have {rank} dimensions ({'[H, T, 64]' if varlen else '[B, H, S, 64]'} "
                             f"view), got {tuple(t.shape)}")
        if t.shape[-1] != HEAD_DIM or t.stride(-1) != 1:
            raise ValueError(f"{name} needs a contiguous last dimension of {HEAD_DIM}")
    if tuple(o.shape) != tuple(q.shape):
        raise ValueError(f"o {tuple(o.shape)} must have q's shape {tuple(q.shape)}")
    if tuple(k.shape) != tuple(v.shape):
        raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} must have the same shape")
    if varlen:
        if seqstart_k is None or max_seqlen_q is None:
            raise ValueError("varlen needs seqstart_q, seqstart_k and max_seqlen_q")
        for name, t in (("seqstart_q", seqstart_q), ("seqstart_k", seqstart_k)):
            if t.dtype != torch.int32 or t.dim() != 1 or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous 1-D int32 tensor")
        if seqstart_q.numel() != seqstart_k.numel() or seqstart_q.numel() < 1:
            raise ValueError("seqstart_q and seqstart_k need the same batch + 1 entries")
    elif seqstart_k is not None:
        raise ValueError("seqstart_k without seqstart_q")
    elif q.shape[0] != k.shape[0]:
        raise ValueError(f"q and k batch sizes differ ({q.shape[0]} vs {k.shape[0]})")
    if lse is not None:
        if lse.dtype != torch.float32 or tuple(lse.shape) != tuple(q.shape[:-1]) or not lse.is_contiguous():
            raise ValueError(f"lse must be a contiguous float32 tensor of shape {tuple(q.shape[:-1])}")
        if varlen and q.stride(0) != q.shape[1] * q.stride(1):
            # the kernel addresses varlen LSE rows as h * (nhead_stride_q / stride_q) + token
            # (include/fmha_fwd.h), so q's head stride must be exactly T rows
            raise ValueError("varlen LSE needs q's head stride to be T rows (q.stride(0) == q.shape[1] * q.stride(1))")
    _check_kernarg_ints(q, k, v, o, max_seqlen_q, max_seqlen_k)
    tensors = [q, k, v, o] + [t for t in (lse, seqstart_q, seqstart_k) if t is not None]
    if not all(t.is_cuda for t in tensors) or len({t.device for t in tensors}) != 1:
        raise ValueError("all tensors must be on the same GPU")


def params_from_tensors(q, k, v, o, lse=None, seqstart_q=None, seqstart_k=None, max_seqlen_q=None,
                        max_seqlen_k=None, scale=None):
    """Build FmhaFwdParams from device tensors.

    Dense: q/o are [B, Hq, Sq, 64] and k/v [B, Hk, Sk, 64] *views* with any
    strides (BHSD, or BSHD permuted to that order).  Varlen: q/o are
    [Hq, T, 64], k/v [Hk, T, 64], with int32 ``seqstart_*`` of batch+1 entries.
    ``lse``: float32, [B, Hq, Sq] (dense) or [Hq, T] (varlen), contiguous.
    Raises ValueError for tensors the kernel cannot take (dtype, rank, head
    dim, inner stride, mismatched shapes, a varlen q whose head stride is not
    T rows while LSE is written, a size or stride outside the kernarg's 32-bit
    ints, or memory that is not on one GPU).
    """
    _check_tensors(q, k, v, o, lse, seqstart_q, seqstart_k, max_seqlen_q, max_seqlen_k)
    varlen = seqstart_q is not None
    p = FmhaFwdParams()
    p.q, p.k, p.v, p.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()
    p.lse = lse.data_ptr() if lse is not None else None
    p.scale = LOG2E / math.sqrt(HEAD_DIM) if scale is None else float(scale)
    if varlen:
        p.nhead_q, p.nhead_k = q.shape[0], k.shape[0]
        p.seqlen_q = int(max_seqlen_q)
        p.seqlen_k = int(max_seqlen_k if max_seqlen_k is not None else max_seqlen_q)
        for name, t in (("q", q), ("k", k), ("v", v), ("o", o)):
            setattr(p, f"stride_{name}", t.stride(1))
            setattr(p, f"nhead_stride_{name}", t.stride(0))
            setattr(p, f"batch_stride_{name}", 0)
        p.seqstart_q, p.seqstart_k = seqstart_q.data_ptr(), seqstart_k.data_ptr()
    else:
        p.nhead_q, p.nhead_k = q.shape[1], k.shape[1]
        p.seqlen_q, p.seqlen_k = q.shape[2], k.shape[2]
        for name, t in (("q", q), ("k", k), ("v", v), ("o", o)):
            setattr(p, f"batch_stride_{name}", t.stride(0))
            setattr(p, f"nhead_stride_{name}", t.stride(1))
            setattr(p, f"stride_{name}", t.stride(2))
        p.seqstart_q = p.seqstart_k = None
    return p


def fmha_fwd(q, k, v, causal=False, return_lse=False, seqstart_q=None, seqstart_k=None, max_seqlen_q=None,
             max_seqlen_k=None, stream=None):
    """Attention forward on torch bf16 device tensors; returns (o, lse or None).

    Layouts as in :func:`params_from_tensors`; ``o`` is allocated with q's
    shape (contiguous).  Runs on ``stream`` (default: torch's current stream).
    """
    import torch

    o = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = None
    if return_lse:
        lse = torch.empty(q.shape[:-1], dtype=torch.float32, device=q.device)
    p = params_from_tensors(q, k, v, o, lse, seqstart_q, seqstart_k, max_seqlen_q, max_seqlen_k)
    batch = (seqstart_q.numel() - 1) if seqstart_q is not None else q.shape[0]
    if stream is None:
        stream = torch.cuda.current_stream(q.device).cuda_stream
    causal = 1 if causal else 0
    need = workspace_size(p, batch, causal)
    if need > 0:  # the balanced form: a workspace from torch's allocator, freed after this stream's work
        ws = torch.empty(need, dtype=torch.uint8, device=q.device)
        fmha_fwd_d64_bf16_ws(p, batch, causal, ws.data_ptr(), need, stream)
    else:
        fmha_fwd_d64_bf16(p, batch, causal, stream)
    return o, lse


def fmha_merge_d64_bf16(n_parts, rows, o_parts, o_part_stride, lse_parts, lse_part_stride, o_row_stride, o, lse,
                        stream=None):
    """The C-ABI merge of partial (O, LSE) results (device pointers as ints;
    strides in elements).  Raises :class:`FmhaError` on a non-zero hipError_t."""
    rc = load_library().fmha_merge_d64_bf16(int(n_parts), int(rows), o_parts, int(o_part_stride), lse_parts,
                                            int(lse_part_stride), int(o_row_stride), o, lse, stream)
    if rc != HIP_SUCCESS:
        raise FmhaError(rc, "fmha_merge_d64_bf16")


def merge_partials(o_parts, lse_parts, o=None, lse=None, stream=None):
    """Merge partial results over disjoint key sets on torch device tensors.

    ``o_parts``: bf16 [n, ..., 64] and ``lse_parts``: float32 [n, ...] with the
    same ``...`` (rows in LSE order, e.g. [B, H, S] or [H, T]), both contiguous.
    Returns (o, lse) with shapes [..., 64] and [...]; ``o``/``lse`` may be given.
    """
    import torch

    if o_parts.dtype not in (torch.bfloat16, torch.int16) or lse_parts.dtype != torch.float32:
        raise ValueError("o_parts must be bfloat16 (or int16 bf16 bits) and lse_parts float32")
    if o_parts.dim() < 2 or o_parts.shape[-1] != HEAD_DIM or tuple(o_parts.shape[:-1]) != tuple(lse_parts.shape):
        raise ValueError(f"o_parts {tuple(o_parts.shape)} must be [n, ..., {HEAD_DIM}] over lse_parts "
                         f"{tuple(lse_parts.shape)} = [n, ...]")
    if not (o_parts.is_contiguous() and lse_parts.is_contiguous()):
        raise ValueError("o_parts and lse_parts must be contiguous")
    n = o_parts.shape[0]
    rows = lse_parts[0].numel()
    if o is None:
        o = torch.empty(o_parts.shape[1:], dtype=o_parts.dtype, device=o_parts.device)
    elif o.dtype != o_parts.dtype or tuple(o.shape) != tuple(o_parts.shape[1:]) or not o.is_contiguous():
        raise ValueError(f"o must be a contiguous {o_parts.dtype} tensor of shape {tuple(o_parts.shape[1:])}")
    if lse is None:
        lse = torch.empty(lse_parts.shape[1:], dtype=torch.float32, device=lse_parts.device)
    elif lse.dtype != torch.float32 or tuple(lse.shape) != tuple(lse_parts.shape[1:]) or not lse.is_contiguous():
        raise ValueError(f"lse must be a contiguous float32 tensor of shape {tuple(lse_parts.shape[1:])}")
    tensors = (o_parts, lse_parts, o, lse)
    if not all(t.is_cuda for t in tensors) or len({t.device for t in tensors}) != 1:
        raise ValueError("all tensors must be on the same GPU")
    if stream is None:
        stream = torch.cuda.current_stream(o_parts.device).cuda_stream
    fmha_merge_d64_bf16(n, rows, o_parts.data_ptr(), rows * HEAD_DIM, lse_parts.data_ptr(), rows, HEAD_DIM,
                        o.data_ptr(), lse.data_ptr(), stream)
    return o, lse
