"""Pins the oracle's conversions, CowBlockTable, RadixTree and StreamingKvManager
restatements against the reference's own tests (engine-kvcache/tests/*.rs,
streaming.rs:148-174) and independent models."""
import numpy as np
import pytest
import torch

from oracle import orc


def test_f16_widening_all_patterns():
    # forward_cpu.rs:74-92: exact for every finite pattern; exponent 31 -> +inf.
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_bits_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.all(got[~finite] == np.inf)


def test_f16_bf16_narrowing_round_to_nearest_even():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(4000).astype(np.float32) * 10,
                        np.float32([0.0, -0.0, 65504.0, 65520.0, 1e-8, 6.1e-5, 2.0 ** -24,
                                    1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, np.inf, -np.inf])])
    with np.errstate(over="ignore"):
        ref16 = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(orc.f32_to_f16_bits(x), ref16)
    ref_bf16 = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.f32_to_bf16_bits(x), ref_bf16)
    assert np.array_equal(orc.bf16_bits_to_f32(ref_bf16),
                          torch.from_numpy(ref_bf16.view(np.int16)).view(torch.bfloat16)
                          .float().numpy())


def test_cow_fork_and_mutate():
    # engine-kvcache/tests/cow_fork_test.rs:4-44
    parent = orc.Cow()
    parent.append_block(10)
    parent.append_block(20)
    assert len(parent) == 2 and parent.physical_block_ids() == [10, 20]
    assert not parent.is_shared(0) and not parent.is_shared(1)
    child = parent.fork()
    assert child.physical_block_ids() == [10, 20]
    assert parent.is_shared(0) and parent.is_shared(1)
    assert child.is_shared(0) and child.is_shared(1)
    assert parent.tail_needs_cow() and child.tail_needs_cow()
    child.perform_tail_cow(99)
    assert child.physical_block_ids() == [10, 99] and parent.physical_block_ids() == [10, 20]
    assert parent.is_shared(0) and not parent.is_shared(1)
    assert child.is_shared(0) and not child.is_shared(1)
    assert child.is_dirty(1) and not parent.is_dirty(1)
    child.append_block(100)
    assert child.physical_block_ids() == [10, 99, 100]
    # refcount = number of tables holding the block (Arc::strong_count)
    third = child.fork()
    assert third.refcount(0) == 3 and third.refcount(1) == 2 and parent.refcount(1) == 1
    del third
    assert child.refcount(0) == 2


def test_cow_empty_table():
    t = orc.Cow()
    assert not t.tail_needs_cow() and not t.is_shared(0)
    t.perform_tail_cow(5)        # no-op on an empty table (cow.rs:74)
    assert t.physical_block_ids() == []


def test_radix_basic_match_and_insert():
    # engine-kvcache/tests/radix_cache_test.rs:4-39
    tree = orc.Radix(16)
    assert tree.match_prefix([1, 2, 3, 4]) == (0, [])
    system = list(range(1, 33))
    tree.insert(system, [101, 102], True)
    assert tree.match_prefix(system) == (32, [101, 102])
    user = system + list(range(33, 41))
    assert tree.match_prefix(user) == (32, [101, 102])
    tree.insert(user, [101, 102, 103], False)
    assert tree.match_prefix(user) == (40, [101, 102, 103])


def test_radix_branching_and_split():
    # radix_cache_test.rs:41-71
    tree = orc.Radix(16)
    prefix = list(range(1, 17))
    a = prefix + [17, 18, 19, 20]
    b = prefix + [100, 101, 102, 103]
    tree.insert(a, [1, 2], False)
    tree.insert(b, [1, 3], False)
    assert tree.match_prefix(a) == (20, [1, 2])
    assert tree.match_prefix(b) == (20, [1, 3])
    assert tree.match_prefix(prefix) == (16, [1])


def test_radix_lru_eviction_with_pinned_protection():
    # radix_cache_test.rs:73-95, with the victim now determined by the logical clock
    tree = orc.Radix(16)
    tree.insert([1, 2, 3, 4], [999], True)
    tree.insert([1, 2, 3, 4, 10, 20], [999, 100], False)
    tree.insert([1, 2, 3, 4, 30, 40], [999, 200], False)
    freed = tree.evict_lru(1)
    assert freed == [100]          # session A is the oldest unpinned leaf
    assert 999 not in freed
    assert tree.match_prefix([1, 2, 3, 4]) == (4, [999])
    # touching B makes it newer; the next victim is B only once nothing older remains
    tree.insert([1, 2, 3, 4, 50, 60], [999, 300], False)
    tree.match_prefix([1, 2, 3, 4, 30, 40])
    assert tree.evict_lru(1) == [300]
    assert tree.evict_lru(5) == [200]      # nothing else is evictable
    assert tree.total_cached_blocks() == 1


def test_radix_partial_edge_match_and_invalidate():
    tree = orc.Radix(4)
    tree.insert(list(range(10)), [7, 8], False)      # 10 tokens, only 2 full blocks recorded
    assert tree.match_prefix(list(range(6)) + [99]) == (6, [7])   # 6//4 = 1 full block
    assert tree.match_prefix(list(range(9))) == (9, [7, 8])
    tree.invalidate_physical_blocks([8])
    assert tree.match_prefix(list(range(10))) == (0, [])
    assert tree.total_cached_blocks() == 0


def test_radix_lru_order_matches_touch_order():
    # Brute-force model of the LRU rule (radix.rs:224-253): with all candidates
    # siblings under one pinned node, eviction order is the touch order.
    rng = np.random.default_rng(5)
    tree = orc.Radix(2)
    tree.insert([0, 0], [1000], True)
    leaves = {}
    for i in range(12):
        toks = [0, 0, 100 + i, 7]
        tree.insert(toks, [1000, i], False)
        leaves[i] = toks
    touch = list(range(12))
    for _ in range(20):
        i = int(rng.integers(12))
        tree.match_prefix(leaves[i])
        touch.remove(i)
        touch.append(i)
    got = [tree.evict_lru(1)[0] for _ in range(12)]
    assert got == touch


def test_streaming_prune_preserves_sink_and_recent():
    # streaming.rs:148-174
    m = orc.Streaming(16, 32, 64, 16)
    assert (m.sink_blocks(), m.recent_blocks(), m.max_active_blocks()) == (1, 2, 4)
    kept, evicted = m.prune_blocks([100, 101, 102, 103, 104, 105, 106, 107])
    assert len(kept) == 4 and kept[0] == 100 and 106 in kept and 107 in kept
    assert len(evicted) == 4


def test_streaming_config_clamps_and_scores():
    d = orc.Streaming()
    assert (d.cfg.sink_tokens, d.cfg.recent_window_tokens, d.cfg.max_budget_tokens,
            d.cfg.block_tokens) == (4, 256, 512, 16)
    c = orc.Streaming(0, 3, 5, 0)     # streaming.rs:38-41 clamps
    assert (c.cfg.block_tokens, c.cfg.sink_tokens, c.cfg.recent_window_tokens,
            c.cfg.max_budget_tokens) == (1, 1, 3, 5)
    m = orc.Streaming(16, 32, 96, 16)          # 1 sink, 2 recent, 6 active -> 3 middle slots
    assert m.scores_len() == 24
    for blk, s in ((11, 5.0), (12, 1.0), (13, 9.0), (14, 3.0), (15, 7.0)):
        m.record_attention_mass(blk, s)
    m.record_attention_mass(200, 2.5)          # grows to 200 + 64 (streaming.rs:137-139)
    assert m.scores_len() == 264
    kept, evicted = m.prune_blocks([10, 11, 12, 13, 14, 15, 16, 17, 18])
    # middle [11..16] ranked by score desc: 13 (9), 15 (7), 11 (5) kept; 14, 12, 16 evicted
    assert kept == [10, 13, 15, 11, 17, 18]
    assert evicted == [14, 12, 16]
    assert m.prune_blocks([1, 2, 3]) == ([1, 2, 3], [])
