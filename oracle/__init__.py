"""CPU oracle for the D64 BF16 FMHA forward — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker / the timed CPU
baseline.  The product (``fmha_native_amd``) never imports it.

``liboracle.so`` is built from ``fmha_oracle.c`` (a C restatement of the
reference's ``src/runner/cpu_ref.cpp:73-153`` plus the LSE of
``src/runner/gpu_ref.cpp:116-117``); ``verify`` restates the reference's pass
rule.  Parity pins for each function are listed in ``fmha_oracle.c``'s header
and exercised by ``tests/test_oracle.py``.
"""
import ctypes
import os

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_DIR, "liboracle.so")


class OracleParams(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p), ("lse", ctypes.c_void_p),
        ("seqlen_q", ctypes.c_int), ("seqlen_k", ctypes.c_int),
        ("nhead_q", ctypes.c_int), ("nhead_k", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("softmax_scale", ctypes.c_float),
        ("stride_q", ctypes.c_int), ("nhead_stride_q", ctypes.c_int), ("batch_stride_q", ctypes.c_int),
        ("stride_k", ctypes.c_int), ("nhead_stride_k", ctypes.c_int), ("batch_stride_k", ctypes.c_int),
        ("stride_v", ctypes.c_int), ("nhead_stride_v", ctypes.c_int), ("batch_stride_v", ctypes.c_int),
        ("stride_o", ctypes.c_int), ("nhead_stride_o", ctypes.c_int), ("batch_stride_o", ctypes.c_int),
        ("seqstart_q", ctypes.c_void_p), ("seqstart_k", ctypes.c_void_p),
    ]


_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            from fmha_native_amd.build import build_oracle
            build_oracle()
        lib = ctypes.CDLL(LIB_PATH)
        P = ctypes.POINTER(OracleParams)
        lib.oracle_fmha_fwd.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.oracle_fmha_fwd.restype = ctypes.c_int
        lib.oracle_fmha_fwd_ex.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.oracle_fmha_fwd_ex.restype = ctypes.c_int
        lib.oracle_fmha_fwd_faithful.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                 ctypes.c_int]
        lib.oracle_fmha_fwd_faithful.restype = ctypes.c_int
        lib.oracle_fmha_fwd_f64.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        lib.oracle_fmha_fwd_f64.restype = ctypes.c_int
        u16p = ctypes.POINTER(ctypes.c_uint16)
        lib.oracle_fill_ref.argtypes = [ctypes.c_uint, u16p, ctypes.c_size_t, u16p, ctypes.c_size_t, u16p,
                                        ctypes.c_size_t]
        lib.oracle_fill_ref.restype = None
        i64, vp = ctypes.c_int64, ctypes.c_void_p
        lib.oracle_merge_d64.argtypes = [ctypes.c_int, i64, vp, i64, vp, i64, i64, vp, vp]
        lib.oracle_merge_d64.restype = None
        _lib = lib
    return _lib


def _ptr(a):
    return a.ctypes.data if a is not None else None


def _params(prob, q, k, v, o, lse):
    st = prob.strides()
    p = OracleParams()
    p.q, p.k, p.v, p.o, p.lse = _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse)
    p.seqlen_q, p.seqlen_k = prob.seqlen_q, prob.seqlen_k
    p.nhead_q, p.nhead_k = prob.nhead_q, prob.nhead_k
    p.head_dim = 64
    p.softmax_scale = np.float32(1.0 / np.sqrt(np.float32(64)))  # FmhaParams::scalar(), fmha_params.hpp:40
    for t in "qkvo":
        s, hs, bs = st[t]
        setattr(p, f"stride_{t}", s)
        setattr(p, f"nhead_stride_{t}", hs)
        setattr(p, f"batch_stride_{t}", bs)
    ss = prob.seqstart()
    if ss is not None:
        p.seqstart_q = p.seqstart_k = ss.ctypes.data
    return p, ss


NO_P_TRUNC = 1
P_RNE_UNNORM = 2
P_TRUNC_UNNORM = 4  # the kernel model with P truncated: a mistake tests plant in it


def run(prob, q, k, v, *, faithful=False, nthreads=0, rows=None, p_trunc=True, kernel_model=False):
    """Oracle O (fp32, q's layout) and LSE (fp32, the kernel's LSE indexing).

    ``faithful``: the reference loop nest (slow); ``rows=(lo, hi)`` restricts
    it to those query rows of every (batch, head) (rows outside stay NaN).
    ``p_trunc=False``: skip the reference's bf16 truncation of P (fast form only).
    ``kernel_model=True``: not the reference but a model of this build's
    kernel's P rounding (nearest-even bf16 of the unnormalised P, fp32 row
    sum), for tests that plant mistakes in it (fast form only).
    """
    nq, _, nlse = prob.sizes()
    o = np.full(nq, np.nan, dtype=np.float32)
    lse = np.full(nlse, np.nan, dtype=np.float32)
    p, _keep = _params(prob, q, k, v, o, lse)
    lib = load()
    if faithful:
        lo, hi = rows if rows is not None else (-1, -1)
        assert p_trunc
        rc = lib.oracle_fmha_fwd_faithful(ctypes.byref(p), prob.batch, int(prob.causal), nthreads, lo, hi)
    else:
        assert rows is None
        flags = P_RNE_UNNORM if kernel_model else (0 if p_trunc else NO_P_TRUNC)
        rc = lib.oracle_fmha_fwd_ex(ctypes.byref(p), prob.batch, int(prob.causal), nthreads, flags)
    if rc != 0:
        raise RuntimeError(f"oracle failed ({rc})")
    return o, lse


def run_f64(prob, q, k, v):
    """float64 brute force (exact softmax, no bf16 P): an independent check."""
    nq, _, nlse = prob.sizes()
    o = np.full(nq, np.nan, dtype=np.float64)
    lse = np.full(nlse, np.nan, dtype=np.float64)
    o32 = np.empty(1, dtype=np.float32)
    p, _keep = _params(prob, q, k, v, o32, None)
    rc = load().oracle_fmha_fwd_f64(ctypes.byref(p), prob.batch, int(prob.causal), o.ctypes.data, lse.ctypes.data)
    if rc != 0:
        raise RuntimeError(f"f64 oracle failed ({rc})")
    return o, lse


def fill_ref(seed, nq, nk, nv):
    q, k, v = (np.empty(n, dtype=np.uint16) for n in (nq, nk, nv))
    u16p = ctypes.POINTER(ctypes.c_uint16)
    load().oracle_fill_ref(seed, q.ctypes.data_as(u16p), nq, k.ctypes.data_as(u16p), nk, v.ctypes.data_as(u16p), nv)
    return q, k, v


def merge(o_parts, lse_parts):
    """float64 merge of partial results: ``o_parts`` uint16 bf16 bits [n, rows*64],
    ``lse_parts`` float32 [n, rows].  Returns (O bits uint16 [rows*64], LSE [rows])."""
    o_parts = np.ascontiguousarray(o_parts, dtype=np.uint16)
    lse_parts = np.ascontiguousarray(lse_parts, dtype=np.float32)
    n, rows = lse_parts.shape
    assert o_parts.shape == (n, rows * 64)
    o = np.empty(rows * 64, dtype=np.uint16)
    lse = np.empty(rows, dtype=np.float32)
    load().oracle_merge_d64(n, rows, o_parts.ctypes.data, rows * 64, lse_parts.ctypes.data, rows, 64, o.ctypes.data,
                            lse.ctypes.data)
    return o, lse
