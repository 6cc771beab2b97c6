"""Product CoW / radix / streaming bookkeeping (include/kv_share.h) against the
reference's own tests and, on random schedules, against the oracle.

Known answers: cow_fork_test.rs:4-44, radix_cache_test.rs:4-95,
streaming.rs:148-174.  Differential: identical random operation sequences
drive titan_amd.share and oracle.orc and must agree on every observable
(ids, sharing flags, ref counts, matches, eviction victims, prune output).
Eviction order is compared under both sides' logical clocks; prune under
distinct scores (ties are unspecified in the reference).
"""
import numpy as np
import pytest

from oracle import orc
from titan_amd.share import (CowBlockTable, RadixTree, StreamingKvConfig,
                             StreamingKvManager)


# ---------------------------------------------------------------- CoW
def test_cow_fork_and_mutate():
    # cow_fork_test.rs:4-44
    parent = CowBlockTable()
    parent.append_block(10)
    parent.append_block(20)
    assert len(parent) == 2 and parent.physical_block_ids() == [10, 20]
    assert not parent.is_shared(0) and not parent.is_shared(1)
    child = parent.fork()
    assert len(child) == 2 and child.physical_block_ids() == [10, 20]
    assert all(t.is_shared(i) for t in (parent, child) for i in (0, 1))
    assert parent.tail_needs_cow() and child.tail_needs_cow()
    child.perform_tail_cow(99)
    assert child.physical_block_ids() == [10, 99]
    assert parent.physical_block_ids() == [10, 20]
    assert parent.is_shared(0) and not parent.is_shared(1)
    assert child.is_shared(0) and not child.is_shared(1)
    assert child.is_dirty(1) and not child.is_dirty(0)
    child.append_block(100)
    assert child.physical_block_ids() == [10, 99, 100]
    assert parent.physical_block_ids() == [10, 20]


def test_cow_refcounts_follow_drops():
    a = CowBlockTable()
    a.append_block(7)
    kids = [a.fork() for _ in range(5)]
    assert a.ref_count(0) == 6
    del kids[:3]
    assert a.ref_count(0) == 3
    kids[0].perform_tail_cow(8)
    assert a.ref_count(0) == 2 and kids[0].ref_count(0) == 1
    assert a.ref_count(5) == 0 and not a.is_shared(5)
    e = CowBlockTable()
    assert not e.tail_needs_cow() and e.is_empty()
    e.perform_tail_cow(3)   # no-op on an empty table
    assert e.physical_block_ids() == []


def test_cow_random_schedule_matches_oracle():
    rng = np.random.default_rng(42)
    prod, ref = [CowBlockTable()], [orc.Cow()]
    next_id = 0
    for _ in range(3000):
        op = rng.integers(0, 5)
        k = int(rng.integers(0, len(prod)))
        if op == 0 and len(prod) < 40:
            prod.append(prod[k].fork())
            ref.append(ref[k].fork())
        elif op == 1:
            prod[k].append_block(next_id)
            ref[k].append_block(next_id)
            next_id += 1
        elif op == 2:
            prod[k].perform_tail_cow(next_id)
            ref[k].perform_tail_cow(next_id)
            next_id += 1
        elif op == 3 and len(prod) > 1:
            del prod[k]
            del ref[k]
            continue
        for p, r in zip(prod, ref):
            assert p.physical_block_ids() == r.physical_block_ids()
            assert p.tail_needs_cow() == r.tail_needs_cow()
        p, r = prod[k], ref[k]
        for i in range(len(p)):
            assert p.is_shared(i) == r.is_shared(i)
            assert p.ref_count(i) == r.refcount(i)
            assert p.is_dirty(i) == r.is_dirty(i)


# ---------------------------------------------------------------- radix
def test_radix_basic_match_and_insert():
    # radix_cache_test.rs:4-40
    t = RadixTree(16)
    r = t.match_prefix([1, 2, 3, 4])
    assert r.matched_tokens == 0 and r.matched_blocks == []
    sys_tok = list(range(1, 33))
    t.insert(sys_tok, [101, 102], True)
    r = t.match_prefix(sys_tok)
    assert (r.matched_tokens, r.matched_blocks) == (32, [101, 102])
    user = sys_tok + list(range(33, 41))
    r = t.match_prefix(user)
    assert (r.matched_tokens, r.matched_blocks) == (32, [101, 102])
    t.insert(user, [101, 102, 103], False)
    r = t.match_prefix(user)
    assert (r.matched_tokens, r.matched_blocks) == (40, [101, 102, 103])


def test_radix_branching_and_split():
    # radix_cache_test.rs:42-71
    t = RadixTree(16)
    pre = list(range(1, 17))
    t.insert(pre + [17, 18, 19, 20], [1, 2], False)
    t.insert(pre + [100, 101, 102, 103], [1, 3], False)
    assert t.match_prefix(pre + [17, 18, 19, 20]).matched_blocks == [1, 2]
    assert t.match_prefix(pre + [100, 101, 102, 103]).matched_blocks == [1, 3]
    r = t.match_prefix(pre)
    assert (r.matched_tokens, r.matched_blocks) == (16, [1])


def test_radix_lru_eviction_with_pinned_protection():
    # radix_cache_test.rs:73-95
    t = RadixTree(16)
    t.insert([1, 2, 3, 4], [999], True)
    t.insert([1, 2, 3, 4, 10, 20], [999, 100], False)
    t.insert([1, 2, 3, 4, 30, 40], [999, 200], False)
    freed = t.evict_lru(1)
    assert freed and 999 not in freed
    assert freed == [100]          # older of the two unpinned leaves (logical clock)
    r = t.match_prefix([1, 2, 3, 4])
    assert (r.matched_tokens, r.matched_blocks) == (4, [999])
    assert t.evict_lru(10) == [200]
    assert t.total_cached_blocks() == 1


def test_radix_zero_block_tokens_rejected():
    with pytest.raises(ValueError):
        RadixTree(0)


def _rand_seq(rng, alphabet, lo, hi):
    return [int(x) for x in rng.integers(0, alphabet, size=int(rng.integers(lo, hi)))]


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_radix_random_schedule_matches_oracle(seed):
    rng = np.random.default_rng(seed)
    bt = int(rng.choice([1, 2, 4, 16]))
    prod, ref = RadixTree(bt), orc.Radix(bt)
    seqs = []
    next_blk = 0
    for _ in range(600):
        op = rng.integers(0, 10)
        if op < 4 or not seqs:
            base = seqs[int(rng.integers(0, len(seqs)))] if seqs and rng.random() < 0.6 else []
            s = base[: int(rng.integers(0, len(base) + 1))] + _rand_seq(rng, 6, 1, 40)
            nb = len(s) // bt + int(rng.integers(-1, 2))
            blocks = list(range(next_blk, next_blk + max(nb, 0)))
            next_blk += max(nb, 0)
            pinned = bool(rng.random() < 0.1)
            prod.insert(s, blocks, pinned)
            ref.insert(s, blocks, pinned)
            seqs.append(s)
        elif op < 7:
            s = seqs[int(rng.integers(0, len(seqs)))]
            s = s[: int(rng.integers(0, len(s) + 1))] + _rand_seq(rng, 6, 0, 5)
            pm = prod.match_prefix(s)
            rm = ref.match_prefix(s)
            assert (pm.matched_tokens, pm.matched_blocks) == (rm[0], rm[1])
        elif op < 8:
            k = int(rng.integers(0, 6))
            assert prod.evict_lru(k) == ref.evict_lru(k)
        elif op < 9:
            victims = [int(x) for x in rng.integers(0, max(next_blk, 1), size=3)]
            prod.invalidate_physical_blocks(victims)
            ref.invalidate_physical_blocks(victims)
        else:
            s = seqs[int(rng.integers(0, len(seqs)))]
            rc = int(rng.integers(0, 2))
            assert prod.set_ref_count(s, rc) == (ref.set_ref_count(s, rc) == 0)
        assert prod.total_cached_blocks() == ref.total_cached_blocks()
    # drain: the full eviction order must agree
    assert prod.evict_lru(1 << 30) == ref.evict_lru(1 << 30)


# ---------------------------------------------------------------- streaming
def test_streaming_prune_preserves_sink_and_recent():
    # streaming.rs:148-174
    m = StreamingKvManager(StreamingKvConfig(16, 32, 64, 16))
    table = list(range(100, 108))
    kept, ev = m.prune_blocks(table)
    assert len(kept) == 4 and kept[0] == 100 and 106 in kept and 107 in kept
    assert len(ev) == 4


def test_streaming_config_clamps_and_default():
    c = StreamingKvConfig(0, 1, 0, 0)
    assert (c.sink_tokens, c.recent_window_tokens, c.max_budget_tokens, c.block_tokens) == (1, 1, 2, 1)
    d = StreamingKvConfig.default()
    assert (d.sink_tokens, d.recent_window_tokens, d.max_budget_tokens, d.block_tokens) == (4, 256, 512, 16)
    assert (d.sink_blocks(), d.recent_blocks(), d.max_active_blocks()) == (1, 16, 32)
    m = StreamingKvManager(d)
    assert len(m.block_scores) == 128
    m.record_attention_mass(200, 1.5)
    assert len(m.block_scores) == 264 and m.block_scores[200] == 1.5


@pytest.mark.parametrize("seed", range(6))
def test_streaming_random_matches_oracle(seed):
    rng = np.random.default_rng(100 + seed)
    args = [int(x) for x in rng.integers(1, 200, size=4)]
    args[3] = int(rng.choice([1, 4, 16, 32]))
    prod = StreamingKvManager(StreamingKvConfig(*args))
    ref = orc.Streaming(*args)
    for b in rng.permutation(300)[:200]:
        mass = float(rng.random())              # distinct with probability 1
        prod.record_attention_mass(int(b), mass)
        ref.record_attention_mass(int(b), mass)
    assert len(prod.block_scores) == ref.scores_len()
    for n in (0, 1, 5, 17, 60, 250):
        table = [int(x) for x in rng.permutation(400)[:n]]
        assert prod.prune_blocks(table) == ref.prune_blocks(table)


def test_streaming_bulk_record_equals_per_block():
    """record_attention_masses(array) == record_attention_mass(i, a[i]) for the
    non-zero entries, as seen through prune_blocks and the scores."""
    rng = np.random.default_rng(3)
    cfg = StreamingKvConfig(4, 32, 96, 16)
    a, b = StreamingKvManager(cfg), StreamingKvManager(cfg)
    masses = np.where(rng.random(300) < 0.4, rng.random(300), 0.0).astype(np.float32)
    for _ in range(2):
        a.record_attention_masses(masses)
        for i, m in enumerate(masses):
            if m != 0.0:
                b.record_attention_mass(i, float(m))
    sa, sb = a.block_scores, b.block_scores
    n = max(len(sa), len(sb))
    assert np.array_equal(np.pad(sa, (0, n - len(sa))), np.pad(sb, (0, n - len(sb))))
    table = rng.permutation(300)[:40]
    assert a.prune_blocks(table) == b.prune_blocks(table)
