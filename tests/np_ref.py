"""Independent float64 attention in numpy — a second, separately written check.

Test infrastructure.  It shares no code with the C oracle (``oracle/``): it
starts from the bf16 bit patterns, widens them to float64 and evaluates
softmax(Q K^T / sqrt(64) + mask) V with numpy's own reductions, per (batch,
head) in the storage layouts of :class:`fmha_native_amd.problem.Problem`.
The bottom-right causal rule and GQA head mapping follow the reference's CPU
reference (``src/runner/cpu_ref.cpp:88-120``); the natural-log LSE follows
``src/runner/gpu_ref.cpp:116-117`` (-inf for a row with no visible key).

``mutate`` plants one named mistake, so tests can show that each check would
catch it: "causal_off_by_one", "no_scale", "gqa_modulo", "swap_kv",
"transpose_v".
"""
import numpy as np

SCALE = 0.125  # float32(1/sqrt(64)) is exactly 1/8


def bits_to_f64(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _views(prob, q, k, v):
    """Per (b, h) 2-D float64 views: yields (b, h, hk, Qbh, Kbh, Vbh, out_index, lse_index)."""
    D = 64
    qf, kf, vf = bits_to_f64(q), bits_to_f64(k), bits_to_f64(v)
    ratio = prob.nhead_q // prob.nhead_k
    if prob.varlen:
        t = prob.total
        Q = qf.reshape(prob.nhead_q, t, D)
        K = kf.reshape(prob.nhead_k, t, D)
        V = vf.reshape(prob.nhead_k, t, D)
        off = 0
        for b, s in enumerate(prob.varlen_seqs):
            for h in range(prob.nhead_q):
                yield b, h, h // ratio, Q[h, off:off + s], K[h // ratio, off:off + s], V[h // ratio, off:off + s], \
                    ("varlen", h, off, s)
            off += s
        return
    if prob.layout == "bhsd":
        Q = qf.reshape(prob.batch, prob.nhead_q, prob.seqlen_q, D)
        K = kf.reshape(prob.batch, prob.nhead_k, prob.seqlen_k, D)
        V = vf.reshape(prob.batch, prob.nhead_k, prob.seqlen_k, D)
    else:
        Q = qf.reshape(prob.batch, prob.seqlen_q, prob.nhead_q, D).transpose(0, 2, 1, 3)
        K = kf.reshape(prob.batch, prob.seqlen_k, prob.nhead_k, D).transpose(0, 2, 1, 3)
        V = vf.reshape(prob.batch, prob.seqlen_k, prob.nhead_k, D).transpose(0, 2, 1, 3)
    for b in range(prob.batch):
        for h in range(prob.nhead_q):
            yield b, h, h // ratio, Q[b, h], K[b, h // ratio], V[b, h // ratio], ("dense", b, h)


def attention(prob, q, k, v, mutate=None):
    """(O float64 in q's layout, LSE float64 in the kernel's LSE indexing)."""
    D = 64
    nq, _, nlse = prob.sizes()
    out = np.full(nq, np.nan)
    lse = np.full(nlse, np.nan)
    if prob.varlen:
        O = out.reshape(prob.nhead_q, prob.total, D)
        L = lse.reshape(prob.nhead_q, prob.total)
    elif prob.layout == "bhsd":
        O = out.reshape(prob.batch, prob.nhead_q, prob.seqlen_q, D)
        L = lse.reshape(prob.batch, prob.nhead_q, prob.seqlen_q)
    else:
        O = out.reshape(prob.batch, prob.seqlen_q, prob.nhead_q, D).transpose(0, 2, 1, 3)
        L = lse.reshape(prob.batch, prob.nhead_q, prob.seqlen_q)
    views = _views(prob, q, k, v)
    for b, h, hk, Qb, Kb, Vb, idx in views:
        if mutate == "gqa_modulo" and prob.nhead_q != prob.nhead_k:
            # wrong head mapping h % Hk instead of h // (Hq / Hk)
            alt = list(_views(prob, q, k, v))
            hk2 = h % prob.nhead_k
            for bb, hh, hkk, _, Kx, Vx, _ in alt:
                if bb == b and hkk == hk2:
                    Kb, Vb = Kx, Vx
                    break
        if mutate == "swap_kv":
            Kb, Vb = Vb, Kb
        if mutate == "transpose_v" and Vb.shape[0] == D:
            Vb = Vb.T
        sq, sk = Qb.shape[0], Kb.shape[0]
        s = Qb @ Kb.T * (1.0 if mutate == "no_scale" else SCALE)
        if prob.causal:
            shift = sk - sq + (1 if mutate == "causal_off_by_one" else 0)
            i = np.arange(sq)[:, None]
            j = np.arange(sk)[None, :]
            s = np.where(j > i + shift, -np.inf, s)
        m = s.max(axis=1, keepdims=True) if sk else np.full((sq, 1), -np.inf)
        finite = np.isfinite(m)
        p = np.where(finite, np.exp(s - np.where(finite, m, 0.0)), 0.0)
        denom = p.sum(axis=1, keepdims=True)
        o = np.where(denom > 0, (p @ Vb) / np.where(denom > 0, denom, 1.0), 0.0)
        row_lse = np.where(denom[:, 0] > 0, np.log(np.where(denom[:, 0] > 0, denom[:, 0], 1.0)) + m[:, 0], -np.inf)
        if idx[0] == "varlen":
            _, hh, off, n = idx
            O[hh, off:off + n] = o
            L[hh, off:off + n] = row_lse
        else:
            _, bb, hh = idx
            O[bb, hh] = o
            L[bb, hh] = row_lse
    return out, lse
