"""Problem geometry of the FMHA forward harness (host side).

The counterpart of the reference's ``FmhaParams`` normalisation
(``tests/test_params.hpp:31-61``, ``src/bench_fmha_fwd.cpp:101-115``) and of
``FmhaBuffers``' sizes and layouts (``src/runner/buffers.cpp:22-56``):

* dense BHSD: Q/O ``[B, Hq, Sq, 64]``, K/V ``[B, Hk, Sk, 64]``, contiguous;
* dense BSHD: the same logical tensors stored ``[B, S, H, 64]``
  (``tests/test_fmha_fwd_d64.cpp:198-346``);
* varlen: Q/O ``[Hq, T, 64]``, K/V ``[Hk, T, 64]`` with ``seqstart`` = prefix
  sums of the per-sequence lengths, identical for q and k
  (``src/runner/buffers.cpp:70-84``).
LSE is ``[B, Hq, Sq]`` (dense) or ``[Hq, T]`` (varlen).
"""
from dataclasses import dataclass, field

import numpy as np

HEAD_DIM = 64


@dataclass
class Problem:
    batch: int
    nhead_q: int
    seqlen_q: int
    nhead_k: int = 0
    seqlen_k: int = 0
    causal: bool = False
    lse: bool = False
    varlen_seqs: tuple = field(default_factory=tuple)
    layout: str = "bhsd"
    name: str = ""

    def __post_init__(self):
        # make_params normalisation (tests/test_params.hpp:43-58)
        if self.nhead_k == 0:
            self.nhead_k = self.nhead_q
        if self.nhead_q % self.nhead_k:
            raise ValueError("nhead_q must be a multiple of nhead_k")
        self.varlen_seqs = tuple(int(s) for s in self.varlen_seqs)
        if self.varlen_seqs:
            self.batch = len(self.varlen_seqs)
            mx = max(self.varlen_seqs)
            self.seqlen_q = mx
            if self.seqlen_k == 0:
                self.seqlen_k = mx
            if self.layout != "bhsd":
                raise ValueError("varlen uses the packed [H, T, D] layout")
        if self.seqlen_k == 0:
            self.seqlen_k = self.seqlen_q
        if self.layout not in ("bhsd", "bshd"):
            raise ValueError(self.layout)

    @property
    def varlen(self):
        return bool(self.varlen_seqs)

    @property
    def total(self):
        return sum(self.varlen_seqs)

    def sizes(self):
        """Element counts (nq == no, nk == nv, nlse)."""
        if self.varlen:
            t = self.total
            return self.nhead_q * t * HEAD_DIM, self.nhead_k * t * HEAD_DIM, self.nhead_q * t
        nq = self.batch * self.nhead_q * self.seqlen_q * HEAD_DIM
        nk = self.batch * self.nhead_k * self.seqlen_k * HEAD_DIM
        return nq, nk, self.batch * self.nhead_q * self.seqlen_q

    def strides(self):
        """(stride, nhead_stride, batch_stride) in elements for q, k, v, o."""
        D = HEAD_DIM
        if self.varlen:
            t = self.total
            q = (D, t * D, 0)
            k = (D, t * D, 0)
        elif self.layout == "bhsd":
            q = (D, self.seqlen_q * D, self.nhead_q * self.seqlen_q * D)
            k = (D, self.seqlen_k * D, self.nhead_k * self.seqlen_k * D)
        else:  # bshd
            q = (self.nhead_q * D, D, self.seqlen_q * self.nhead_q * D)
            k = (self.nhead_k * D, D, self.seqlen_k * self.nhead_k * D)
        return {"q": q, "k": k, "v": k, "o": q}

    def seqstart(self):
        if not self.varlen:
            return None
        return np.concatenate([[0], np.cumsum(self.varlen_seqs)]).astype(np.int32)

    def seq_lengths(self):
        if self.varlen:
            return list(self.varlen_seqs), list(self.varlen_seqs)
        return [self.seqlen_q] * self.batch, [self.seqlen_k] * self.batch

    def flops(self):
        """Repo FLOP convention: 4*B*H*Sq*Sk*D, x0.5 when causal
        (src/bench_fmha_fwd.cpp:225-226; varlen uses max S for every sequence)."""
        f = 4.0 * self.batch * self.nhead_q * self.seqlen_q * self.seqlen_k * HEAD_DIM
        return f * 0.5 if self.causal else f

    def exact_flops(self):
        """4*D*(number of visible (q,k) pairs) summed over sequences and heads."""
        sqs, sks = self.seq_lengths()
        pairs = 0
        for sq, sk in zip(sqs, sks):
            if self.causal:
                shift = sk - sq
                lim = np.clip(np.arange(sq) + shift + 1, 0, sk)
                pairs += int(lim.sum())
            else:
                pairs += sq * sk
        return 4.0 * HEAD_DIM * pairs * self.nhead_q

    def io_bytes(self):
        """Algorithmic HBM bytes: Q, K, V read once, O (and LSE) written once."""
        nq, nk, nlse = self.sizes()
        return 2 * (nq + 2 * nk + nq) + (4 * nlse if self.lse else 0)


def bhsd_to_bshd(a, b, h, s, d=HEAD_DIM):
    """Rearrange a flat BHSD array to BSHD storage (test_fmha_fwd_d64.cpp:217-231)."""
    return np.ascontiguousarray(np.asarray(a).reshape(b, h, s, d).transpose(0, 2, 1, 3)).reshape(-1)


def bshd_to_bhsd(a, b, h, s, d=HEAD_DIM):
    return np.ascontiguousarray(np.asarray(a).reshape(b, s, h, d).transpose(0, 2, 1, 3)).reshape(-1)


def baseline_problems(varlen_seed=42):
    """The five benchmark configurations as {name: (Problem, input multiplier)}:
    cfg1 B1 H2 S128 (+LSE), cfg2 B4 H16 S2048 dense, cfg3 B1 H16 S8192 causal
    (+LSE), cfg4 eight varlen sequences U[128, 4096] causal (+LSE), cfg5 B1 H2
    S40000 causal (+LSE) with inputs x2.  Inputs are N(0,1) (seed 42)."""
    from fmha_native_amd import varlen_lengths

    lens = varlen_lengths(varlen_seed, 8, 128, 4096)
    return {
        "cfg1": (Problem(batch=1, nhead_q=2, seqlen_q=128, lse=True, name="cfg1_B1H2S128"), 1.0),
        "cfg2": (Problem(batch=4, nhead_q=16, seqlen_q=2048, name="cfg2_B4H16S2048"), 1.0),
        "cfg3": (Problem(batch=1, nhead_q=16, seqlen_q=8192, causal=True, lse=True, name="cfg3_B1H16S8192_causal"),
                 1.0),
        "cfg4": (Problem(batch=8, nhead_q=16, seqlen_q=0, causal=True, lse=True, varlen_seqs=tuple(lens),
                         name="cfg4_varlen8_causal"), 1.0),
        "cfg5": (Problem(batch=1, nhead_q=2, seqlen_q=40000, causal=True, lse=True,
                         name="cfg5_B1H2S40000_causal_x2"), 2.0),
    }


def workload(spec):
    """(Problem, input multiplier) of a workload name: one of the five
    benchmark configurations ("cfg1" .. "cfg5"), or a dense shape written
    "dense-B<b>H<h>S<s>" / "causal-B<b>H<h>S<s>" (causal with LSE; N(0,1)
    inputs)."""
    import re

    probs = baseline_problems()
    if spec in probs:
        return probs[spec]
    m = re.fullmatch(r"(dense|causal)-B(\d+)H(\d+)S(\d+)", spec)
    if not m:
        raise ValueError(f"unknown workload {spec!r}: cfg1..cfg5, dense-B<b>H<h>S<s> or causal-B<b>H<h>S<s>")
    causal = m.group(1) == "causal"
    b, h, sq = (int(m.group(i)) for i in (2, 3, 4))
    return Problem(batch=b, nhead_q=h, seqlen_q=sq, causal=causal, lse=causal, name=spec), 1.0

