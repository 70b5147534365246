"""GPU tests at the launcher's limits, through the C-ABI.

* the longest key sequence the 31-bit buffer-offset check accepts for 64-wide
  rows (16,776,000 keys: (rows + 320) * 128 bytes + 256 < 2^31), dense and
  bottom-right causal, in the automatic form and the reference-named entries;
* the largest grid y: 65,535 M-tiles (seqlen_q = 65,535 * 128);
* the largest grid z: 65,535 batches, and the tile-major grid with the most
  batches in y that its 8 MiB rule allows (32,768);
* thousands of varlen sequences, some of them empty.

Each is checked against a float64 numpy evaluation of sampled rows
(O within 1e-2 + 1e-2 |O|, LSE within 1e-3, rows with no visible key O = 0
and LSE = -inf); the inputs are N(0, 1) bf16 drawn on the device.  The one
other limit, nhead_q, is the grid x dimension (2^31 - 1) and is not tested
at its maximum.
"""
import numpy as np
import pytest

import fmha_native_amd as fmha

pytestmark = pytest.mark.gpu

SCALE = 0.125
MAX_KEYS = 16_776_000  # largest multiple of 1000 below the offset limit (16,776,893 rows)


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    fmha.load_library()


def _f64(t):
    import torch

    return t.float().cpu().numpy().astype(np.float64) if t.dtype == torch.bfloat16 else t.cpu().numpy()


def _check_rows(o_rows, lse_rows, q_rows, k, v, ends, tag):
    """float64 attention of ``q_rows`` (n, 64) over keys [0, ends[i]) of k, v
    (host float32 arrays, any length); O and LSE of the kernel for those rows."""
    n = q_rows.shape[0]
    chunk = 1 << 20
    s_all = []
    for c0 in range(0, k.shape[0], chunk):
        s_all.append(k[c0:c0 + chunk].astype(np.float64) @ q_rows.T * SCALE)  # (c, n)
    s = np.concatenate(s_all, axis=0) if s_all else np.zeros((0, n))
    keys = np.arange(s.shape[0])[:, None]
    s = np.where(keys < np.asarray(ends)[None, :], s, -np.inf)
    m = s.max(axis=0) if s.shape[0] else np.full(n, -np.inf)
    o_ref = np.zeros((n, 64))
    l_ref = np.zeros(n)
    finite = np.isfinite(m)
    for c0 in range(0, s.shape[0], chunk):
        p = np.exp(s[c0:c0 + chunk] - np.where(finite, m, 0.0)[None, :])  # masked -> 0
        l_ref += p.sum(axis=0)
        o_ref += p.T @ v[c0:c0 + chunk].astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        o_ref = np.where(l_ref[:, None] > 0, o_ref / l_ref[:, None], 0.0)
        lse_ref = np.where(l_ref > 0, np.log(l_ref) + m, -np.inf)
    err = np.abs(o_rows - o_ref)
    bound = 1e-2 + 1e-2 * np.abs(o_ref)
    assert np.all(err <= bound), f"{tag}: O max err {err.max():.3g}"
    if lse_rows is not None:
        empty = ~np.isfinite(lse_ref)
        assert np.all(np.isneginf(lse_rows[empty])), f"{tag}: LSE of rows without keys"
        assert np.all(o_rows[empty] == 0), f"{tag}: O of rows without keys"
        d = np.abs(lse_rows[~empty] - lse_ref[~empty])
        assert d.size == 0 or d.max() <= 1e-3, f"{tag}: LSE max err {d.max():.3g}"


def _run(q, k, v, causal, form, lse=True, **kw):
    import torch

    o = torch.empty_like(q)
    ls = torch.empty(q.shape[:-1], dtype=torch.float32, device=q.device) if lse else None
    p = fmha.params_from_tensors(q, k, v, o, ls, **kw)
    batch = (kw["seqstart_q"].numel() - 1) if kw.get("seqstart_q") is not None else q.shape[0]
    print(f"launch: q{tuple(q.shape)} k{tuple(k.shape)} causal={causal} form={form}", flush=True)
    fmha.fmha_fwd_d64_bf16(p, batch, int(causal), torch.cuda.current_stream().cuda_stream, form)
    torch.cuda.synchronize()
    return o, ls


@pytest.mark.parametrize("causal", [False, True])
def test_longest_key_sequence(causal):
    import torch

    sq, sk = 256, MAX_KEYS
    g = torch.Generator(device="cuda").manual_seed(11)
    q = torch.randn((1, 1, sq, 64), generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    k = torch.randn((1, 1, sk, 64), generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    v = torch.randn((1, 1, sk, 64), generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    p = fmha.params_from_tensors(q, k, v, q, None)
    assert fmha.check_params(p, 1, int(causal)) == 0  # inside the accepted range
    rows = np.array([0, 1, 63, 127, 128, 200, 255])
    ends = [sk if not causal else r + (sk - sq) + 1 for r in rows]
    outs = [_run(q, k, v, causal, form) for form in (fmha.VARIANT_AUTO, fmha.VARIANT_REGULAR)]
    kf, vf = k[0, 0].float().cpu().numpy(), v[0, 0].float().cpu().numpy()
    qf = _f64(q[0, 0])[rows]
    for form, (o, ls) in zip(("auto", "regular"), outs):
        _check_rows(_f64(o[0, 0])[rows], _f64(ls[0, 0])[rows], qf, kf, vf, ends, f"causal={causal} form={form}")


@pytest.mark.parametrize("causal", [False, True])
def test_largest_grid_y(causal):
    import torch

    sq, sk = 65535 * 128, 100
    g = torch.Generator(device="cuda").manual_seed(12)
    q = torch.randn((1, 1, sq, 64), generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    k = torch.randn((1, 1, sk, 64), generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    v = torch.randn((1, 1, sk, 64), generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    o, ls = _run(q, k, v, causal, fmha.VARIANT_AUTO)
    rng = np.random.default_rng(3)
    rows = np.unique(np.concatenate([rng.integers(0, sq, 2000), np.arange(sq - 300, sq), np.arange(0, 130),
                                     [sq - sk - 1, sq - sk, sq - sk + 1]]))
    ends = [sk if not causal else max(0, min(sk, r + (sk - sq) + 1)) for r in rows]
    idx = torch.from_numpy(rows).cuda()
    _check_rows(_f64(o[0, 0][idx]), _f64(ls[0, 0][idx]), _f64(q[0, 0][idx]), _f64(k[0, 0]), _f64(v[0, 0]), ends,
                f"grid y 65535 causal={causal}")


@pytest.mark.parametrize("causal", [False, True])
def test_largest_grid_z(causal):
    _many_batches(65535, 3, causal, tile_major=0)


@pytest.mark.parametrize("b,s", [(32768, 1), (10922, 3)])
def test_largest_tile_major_grid(b, s):
    """Causal batches at the tile-major rule's limit (b x s K/V rows of one
    head per XCD = 32,768 or 32,766, i.e. 8 MiB): grid (2, b, tiles)."""
    _many_batches(b, s, True, tile_major=1)


def _many_batches(b, s, causal, tile_major):
    import torch

    hq, hk = 2, 1
    g = torch.Generator(device="cuda").manual_seed(13)
    q = torch.randn((b, hq, s, 64), generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    k = torch.randn((b, hk, s, 64), generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    v = torch.randn((b, hk, s, 64), generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    o = torch.empty_like(q)
    ls = torch.empty(q.shape[:-1], dtype=torch.float32, device=q.device)
    assert fmha.tile_major(fmha.params_from_tensors(q, k, v, o, ls), b, int(causal)) == tile_major
    o, ls = _run(q, k, v, causal, fmha.VARIANT_AUTO)
    qf, kf, vf = _f64(q), _f64(k)[:, [0, 0]], _f64(v)[:, [0, 0]]  # GQA: both q heads read kv head 0
    sc = np.einsum("bhid,bhjd->bhij", qf, kf) * SCALE
    if causal:
        sc = np.where(np.tril(np.ones((s, s), bool))[None, None], sc, -np.inf)
    m = sc.max(-1, keepdims=True)
    pr = np.exp(sc - m)
    l_ref = pr.sum(-1)
    o_ref = np.einsum("bhij,bhjd->bhid", pr, vf) / l_ref[..., None]
    err = np.abs(_f64(o) - o_ref)
    assert np.all(err <= 1e-2 + 1e-2 * np.abs(o_ref)), err.max()
    assert np.abs(_f64(ls) - (np.log(l_ref) + m[..., 0])).max() <= 1e-3


@pytest.mark.parametrize("causal", [False, True])
def test_many_varlen_sequences_with_empty_ones(causal):
    import torch

    rng = np.random.default_rng(14)
    lens = rng.integers(0, 301, 3000)
    lens[[0, 1, 1500, 2998, 2999]] = [0, 0, 0, 0, 0]
    lens[[2, 3]] = [1, 300]
    starts = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    t, hq, hk = int(starts[-1]), 4, 2
    g = torch.Generator(device="cuda").manual_seed(15)
    q = torch.randn((hq, t, 64), generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    k = torch.randn((hk, t, 64), generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    v = torch.randn((hk, t, 64), generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    ss = torch.from_numpy(starts).cuda()
    o, ls = _run(q, k, v, causal, fmha.VARIANT_AUTO, seqstart_q=ss, seqstart_k=ss, max_seqlen_q=int(lens.max()))
    of, lf, qf, kf, vf = _f64(o), _f64(ls), _f64(q), _f64(k), _f64(v)
    picks = sorted(set([0, 1, 2, 3, 4, 1499, 1500, 1501, 2997, 2998, 2999]) | set(rng.integers(0, 3000, 150)))
    for bi in picks:
        a, n = int(starts[bi]), int(lens[bi])
        if n == 0:
            continue
        for h in range(hq):
            ends = [(i + 1) if causal else n for i in range(n)]
            _check_rows(of[h, a:a + n], lf[h, a:a + n], qf[h, a:a + n], kf[h // 2, a:a + n], vf[h // 2, a:a + n],
                        ends, f"seq {bi} len {n} head {h}")
