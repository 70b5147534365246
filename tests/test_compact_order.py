"""CPU models of the compact causal varlen orders (``level_item`` and
``sequence_item`` in fmha_fwd_kernel.hip): the dispatch rank of a block on
the regular varlen grid (nhead_q, M-tile bound, sequences) maps to the live
(sequence, M-tile) items, ordered by M-tile index, highest first, then by
sequence (level order), or sequence after sequence, longest first, each
highest M-tile first (sequence order); ranks past the live items are dead.
The kernel finds a level-order item with 64 candidate levels per round (one
lane each) and a sequence-order item from per-lane prefix counts; these
models run the same steps on numpy arrays and are checked against the sorted
lists themselves, for the grid bounds the kernel sees (up to 64 sequences,
M-tile bounds that take one, two and three rounds).  The GPU tests check the
kernel's bits against the reference order.
"""
import numpy as np
import pytest


def level_item_model(n, mtiles, rank):
    """The kernel's rounds; ``n``: M-tiles per sequence (already capped at
    ``mtiles``).  Returns (sequence, M-tile) or None for a dead rank."""
    n = np.asarray(n, dtype=np.int64)
    lo, hi, c_next = 0, mtiles, 0
    while True:
        step = (hi - lo + 63) >> 6
        m = lo + np.arange(64) * step
        c = np.maximum(0, n[None, :] - m[:, None]).sum(1)
        c1 = np.maximum(0, n[None, :] - m[:, None] - 1).sum(1)
        above = (m < hi) & (c > rank)
        if not above.any():
            assert lo == 0
            return None
        top = int(np.nonzero(above)[0].max())
        assert above[:top + 1].all()  # the set lanes are a prefix
        lo = lo + top * step
        c_next = int(c1[top])
        if step == 1:
            break
        hi = min(hi, lo + step)
    r = rank - c_next
    live = np.nonzero(n > lo)[0]
    assert 0 <= r < len(live)
    return int(live[r]), lo


def sequence_item_model(n, rank):
    """The kernel's sequence order: lane s counts the items of the sequences
    before it (more M-tiles, or as many and a lower index)."""
    n = np.asarray(n, dtype=np.int64)
    idx = np.arange(len(n))
    before = (n[None, :] > n[:, None]) | ((n[None, :] == n[:, None]) & (idx[None, :] < idx[:, None]))
    start = (before * n[None, :]).sum(1)
    mine = np.nonzero((start <= rank) & (rank < start + n))[0]
    if len(mine) == 0:
        return None
    assert len(mine) == 1
    s = int(mine[0])
    return s, int(n[s] - 1 - (rank - start[s]))


def expected_sequence_order(n):
    seqs = sorted(range(len(n)), key=lambda s: (-n[s], s))
    return [(s, mt) for s in seqs for mt in reversed(range(n[s]))]


def expected_order(n):
    items = [(s, mt) for s in range(len(n)) for mt in range(n[s])]
    return sorted(items, key=lambda x: (-x[1], x[0]))


@pytest.mark.parametrize("seed", range(40))
def test_model_matches_sorted_items(seed):
    rng = np.random.default_rng(seed)
    nseq = int(rng.integers(1, 65))
    mtiles = int(rng.choice([1, 2, 7, 31, 64, 65, 100, 4096, 4097, 20000]))
    lens = rng.integers(0, mtiles * 128 + 1, size=nseq)
    if seed % 5 == 0:
        lens[rng.integers(0, nseq)] = 0  # empty sequences have no item
    n = np.minimum((lens + 127) // 128, mtiles)
    order = expected_order(n)
    total = nseq * mtiles
    ranks = range(total) if total <= 3000 else list(rng.integers(0, total, size=2000)) + [len(order) - 1, len(order)]
    seq_order = expected_sequence_order(n)
    for r in ranks:
        got = level_item_model(n, mtiles, int(r))
        want = order[r] if r < len(order) else None
        assert got == want, (r, got, want)
        got = sequence_item_model(n, int(r))
        want = seq_order[r] if r < len(seq_order) else None
        assert got == want, (r, got, want)


def test_cfg4_order_is_heaviest_first():
    """cfg4's eight sequences (lengths from seed 42): 147 live M-tiles of the
    248 grid ranks, M-tile index never rising along the dispatch order."""
    lens = [2323, 2446, 1908, 2056, 691, 1943, 2905, 3964]
    n = [(x + 127) // 128 for x in lens]
    got = [level_item_model(n, 31, r) for r in range(8 * 31)]
    live = [g for g in got if g is not None]
    assert len(live) == sum(n) == 147 and got[147:] == [None] * (248 - 147)
    assert all(a[1] >= b[1] for a, b in zip(live, live[1:]))
    assert sorted(live) == sorted((s, mt) for s in range(8) for mt in range(n[s]))


def test_cfg4_sequence_order():
    """cfg4 in the sequence order: the 3964-token sequence's 31 M-tiles first
    (heaviest first), the 691-token sequence's 6 last."""
    lens = [2323, 2446, 1908, 2056, 691, 1943, 2905, 3964]
    n = [(x + 127) // 128 for x in lens]
    got = [sequence_item_model(n, r) for r in range(8 * 31)]
    assert got[:31] == [(7, mt) for mt in range(30, -1, -1)]
    assert got[141:147] == [(4, mt) for mt in range(5, -1, -1)] and got[147:] == [None] * (248 - 147)
