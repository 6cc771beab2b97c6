"""Pins the oracle's protected-sinks decode (sdpa_decode over
[0, sink) U [max(sink, pos - W), pos], openspec/changes/archive/
2026-08-28-agent-runtime-optimizations/design.md:211-216).

  * a window at least as long as the sequence, and W = 0, reduce to the
    reference sdpa_decode (forward_cpu.rs:424-510), bit for bit;
  * attention over the window equals plain sdpa_decode over a dense copy of
    exactly the attended token rows (softmax over a set: order kept), bit for
    bit, with the set built from the spec's wording (sinks = the first
    K_sink tokens, window = the last W + 1 positions);
  * a huge value planted in a K row of the gap leaves the output unchanged,
    one planted in the window does not.
"""
import numpy as np
import pytest

from oracle import orc


def setup(rng, lens, bt, n_kv, hd, n_head):
    need = [(int(l) + bt - 1) // bt for l in lens]
    stride = max(max(need), 1)
    nb = sum(need) + 2
    perm = rng.permutation(nb).astype(np.uint32)
    tab = np.full((len(lens), stride), 0xFFFFFFFF, np.uint32)
    p = 0
    for b, c in enumerate(need):
        tab[b, :c] = perm[p:p + c]
        p += c
    pool = rng.standard_normal(nb * bt * 2 * n_kv * hd).astype(np.float32)
    q = rng.standard_normal((len(lens), n_head, hd)).astype(np.float32)
    return tab, pool, q


def attended(n, sink, window):
    """Spec wording: the first `sink` tokens, and positions pos-W .. pos."""
    if window == 0:
        return list(range(n))
    pos = n - 1
    keep = set(range(min(sink, n)))
    keep |= set(range(max(0, pos - window), pos + 1))
    return sorted(keep)


@pytest.mark.parametrize("sink,window", [(0, 0), (4, 0), (4, 10 ** 6), (0, 5000)])
def test_reduces_to_sdpa(sink, window):
    rng = np.random.default_rng(1)
    lens = np.array([1, 17, 300, 2049], np.uint32)
    tab, pool, q = setup(rng, lens, 16, 2, 64, 6)
    a = orc.sdpa_decode_window_batched(pool, tab, lens, 16, q, 6, 2, 64, sink, window)
    b = orc.sdpa_decode_batched(pool, tab, lens, 16, q, 6, 2, 64)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("sink,window", [(4, 1), (4, 16), (4, 100), (0, 7), (20, 33), (64, 10)])
def test_equals_dense_subset(sink, window):
    rng = np.random.default_rng(2 + sink + window)
    n_kv, hd, n_head, bt = 2, 64, 6, 16
    lens = np.array([1, 3, 5, 20, 64, 65, 300, 1000], np.uint32)
    tab, pool, q = setup(rng, lens, bt, n_kv, hd, n_head)
    got = orc.sdpa_decode_window_batched(pool, tab, lens, bt, q, n_head, n_kv, hd, sink, window)
    rows = pool.reshape(-1, bt, 2 * n_kv * hd)
    for b, n in enumerate(lens):
        keep = attended(int(n), sink, window)
        sub = np.stack([rows[tab[b, t // bt], t % bt] for t in keep]).reshape(-1)
        ident = np.zeros((1, 1), np.uint32)
        want = orc.sdpa_decode_batched(sub, ident, np.array([len(keep)], np.uint32), len(keep),
                                       q[b:b + 1], n_head, n_kv, hd)
        assert np.array_equal(got[b:b + 1].view(np.uint32), want.view(np.uint32)), (b, n)


def test_gap_tokens_do_not_count():
    rng = np.random.default_rng(9)
    n_kv, hd, n_head, bt = 1, 32, 2, 16
    lens = np.array([200], np.uint32)
    tab, pool, q = setup(rng, lens, bt, n_kv, hd, n_head)
    base = orc.sdpa_decode_window_batched(pool, tab, lens, bt, q, n_head, n_kv, hd, 4, 50)
    rows = pool.reshape(-1, bt, 2, n_kv * hd)
    gap_t, win_t = 100, 180            # window is 149..199, sinks 0..3
    p2 = rows.copy()
    p2[tab[0, gap_t // bt], gap_t % bt, :] = 1e4
    same = orc.sdpa_decode_window_batched(p2.reshape(-1), tab, lens, bt, q, n_head, n_kv, hd, 4, 50)
    assert np.array_equal(same, base)
    p3 = rows.copy()
    p3[tab[0, win_t // bt], win_t % bt, 1, :] = 1e4     # its V row
    moved = orc.sdpa_decode_window_batched(p3.reshape(-1), tab, lens, bt, q, n_head, n_kv, hd, 4, 50)
    assert not np.array_equal(moved, base)


def test_attention_mass_invariants():
    """Per-page attention mass (the H2O score of record_attention_mass,
    streaming.rs:135-141): each sequence's pages receive n_head in total (each
    head's weights sum to 1); with q = 0 every attended token weighs 1/|set|,
    so a page receives n_head * (its attended tokens) / |set|."""
    rng = np.random.default_rng(4)
    n_kv, hd, n_head, bt = 2, 64, 6, 16
    lens = np.array([1, 20, 300, 77], np.uint32)
    tab, pool, q = setup(rng, lens, bt, n_kv, hd, n_head)
    nb = int(tab[tab != 0xFFFFFFFF].max()) + 3
    for sink, window in ((0, 0), (4, 30)):
        _, mass = orc.sdpa_decode_window_batched(pool, tab, lens, bt, q, n_head, n_kv, hd, sink,
                                                 window, n_blocks=nb)
        assert abs(mass.sum() - n_head * len(lens)) < 1e-9
        for b, n in enumerate(lens):
            pages = set(int(p) for p in tab[b, :(int(n) + bt - 1) // bt])
            assert abs(sum(mass[p] for p in pages) - n_head) < 1e-9
        _, m0 = orc.sdpa_decode_window_batched(pool, tab, lens, bt, np.zeros_like(q), n_head, n_kv,
                                               hd, sink, window, n_blocks=nb)
        want = np.zeros(nb)
        for b, n in enumerate(lens):
            keep = attended(int(n), sink, window)
            for t in keep:
                want[tab[b, t // bt]] += n_head / len(keep)
        assert np.allclose(m0, want, rtol=1e-12, atol=1e-12)
