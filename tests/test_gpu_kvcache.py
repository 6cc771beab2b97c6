"""PagedKvCache with its pool in HBM (titan_amd.kvcache) against the oracle's
restatement of engine-kvcache/src/cache.rs.

1. The reference's own known-answer tests (cache.rs:258-472) on the product
   surface: exact floats, reads across non-adjacent pages, exhaustion with no
   partial state, free then reuse, the budget bound -- and after each one the
   device pool equals orc.Cache's pool byte for byte.
2. All-or-nothing appends: a failed launch rolls the reservation back; a batch
   that exhausts the pool mid-way changes no sequence.
3. Real paging in a decode loop (the ForwardDriver path, forward_driver.rs:
   613-723, whose reference runs one page per sequence and feeds RadixTree a
   dummy &[0] at :1240): a PagedKvCache on a shuffled free list serves a
   ragged prompt append and 20 fused decode steps for 24 sequences; one
   sequence is freed mid-run and a new one reuses its pages; the step's
   tables come from eh_kvcache_export_tables; every step's pool bytes,
   tables and attention output are compared with orc.Cache +
   orc.sdpa_decode_batched; each sequence's real page ids go into a
   RadixTree and match back; a final reserve hits PoolExhausted.
"""
import numpy as np
import pytest
import torch

from oracle import orc
from titan_amd import KvDataType, PagedAttention
from titan_amd.errors import KvCacheError
from titan_amd.kvcache import PagedKvCache, PagedKvCacheConfig
from titan_amd.share import RadixTree

import parity

pytestmark = pytest.mark.gpu

NP = {KvDataType.F32: np.float32, KvDataType.F16: np.float16}


def pair(n_blocks, block_tokens, heads, head_dim, dtype=KvDataType.F32):
    cfg = PagedKvCacheConfig(n_blocks, block_tokens, heads, head_dim)
    return (PagedKvCache(cfg, dtype), orc.Cache(n_blocks, block_tokens, heads, head_dim,
                                                dtype=NP[dtype]))


def same_pool(c, o):
    torch.cuda.synchronize()
    got = c.pool.cpu().numpy().view(np.uint8)
    assert np.array_equal(got, o.buffer().view(np.uint8))


def both_append(c, o, seq, k, v):
    c.append(seq, np.asarray(k, np.float32), np.asarray(v, np.float32))
    o.append(seq, np.asarray(k, np.float32), np.asarray(v, np.float32))


def test_create_pool_reports_blocks_total(dev):
    # cache.rs:262-275
    c, _ = pair(8, 16, 4, 6)
    assert c.blocks_total() == 8 and c.blocks_used() == 0
    assert c.config().floats_per_token() == 2 * 4 * 6
    assert c.config().floats_per_block() == 16 * 48
    assert torch.count_nonzero(c.pool).item() == 0           # zero-filled (cache.rs:78-79)


def test_append_single_token_reads_back_exact_floats(dev):
    # cache.rs:277-302
    c, o = pair(8, 16, 2, 3)
    s = c.new_sequence()
    assert o.new_sequence() == s
    key, value = [1.5, -2.25, 0.5, 3.0, -4.0, 6.0], [4.0, 8.0, -16.0, 1.0, 2.0, 3.0]
    both_append(c, o, s, key, value)
    assert c.read_key(s, 0).cpu().tolist() == key
    assert c.read_value(s, 0).cpu().tolist() == value
    same_pool(c, o)


def test_append_spanning_scattered_blocks(dev):
    # cache.rs:304-370: sequence A on non-adjacent physical pages
    c, o = pair(4, 4, 1, 2)
    a, b = c.new_sequence(), c.new_sequence()
    o.new_sequence(), o.new_sequence()
    for k in range(4):
        both_append(c, o, a, [k, k * 10.0], [0.0, 0.0])
    for x in (9.0, 8.0, 7.0, 6.0):
        both_append(c, o, b, [x, x], [x, x])
    for t in range(4, 8):
        both_append(c, o, a, [t, t * 10.0], [0.0, 0.0])
    assert c.token_count(a) == 8
    # (the reference's comment expects pages 0 and 3 for A, but B's 4 tokens
    # fit one 4-token page, so A continues on page 2; its test checks data only)
    assert c.seq_block_table(a) == o.seq_block_table(a).tolist() == [0, 2]
    assert c.seq_block_table(b) == o.seq_block_table(b).tolist() == [1]
    keys = c.read_keys(a).cpu().numpy().reshape(8, 2)
    assert keys.tolist() == [[t, t * 10.0] for t in range(8)]
    same_pool(c, o)


def test_pool_exhaustion_returns_typed_error(dev):
    # cache.rs:372-405
    c, o = pair(1, 2, 1, 2)
    s = c.new_sequence()
    o.new_sequence()
    both_append(c, o, s, [0.5, 1.5], [0.5, 1.5])
    both_append(c, o, s, [0.5, 1.5], [0.5, 1.5])
    with pytest.raises(KvCacheError) as e:
        c.append(s, np.array([0.5, 1.5], np.float32), np.array([0.5, 1.5], np.float32))
    assert e.value.kind == "PoolExhausted"
    assert (e.value.blocks_used, e.value.blocks_total) == (1, 1)
    assert c.blocks_used() == 1 and c.token_count(s) == 2     # no partial state
    same_pool(c, o)


def test_free_then_realloc_succeeds(dev):
    # cache.rs:407-444
    c, o = pair(2, 2, 1, 2)
    s = c.new_sequence()
    o.new_sequence()
    for _ in range(4):
        both_append(c, o, s, [1.0, 2.0], [1.0, 2.0])
    with pytest.raises(KvCacheError) as e:
        c.append(s, np.array([1.0, 2.0], np.float32), np.array([1.0, 2.0], np.float32))
    assert e.value.kind == "PoolExhausted"
    c.free_sequence(s)
    o.free_sequence(s)
    assert c.blocks_used() == 0 and c.token_count(s) == 0
    for i in range(3):
        both_append(c, o, s, [3.0 + i, -1.0 - i], [0.25 * i, 7.0])
    assert c.token_count(s) == 3 and c.blocks_used() == 2
    assert c.seq_block_table(s) == o.seq_block_table(s).tolist() == [0, 1]
    assert c.read_keys(s).cpu().numpy().reshape(3, 2).tolist() == \
        [[3.0 + i, -1.0 - i] for i in range(3)]                  # fresh rows, not stale ones
    same_pool(c, o)


def test_budget_capacity_matches_config_total(dev):
    # cache.rs:446-472
    c, _ = pair(3, 4, 2, 3)
    a, b = c.new_sequence(), c.new_sequence()
    row = np.full(6, 0.1, np.float32)
    while c.blocks_used() < c.blocks_total():
        c.append(a, row, row)
        assert c.blocks_used() <= c.blocks_total()
    with pytest.raises(KvCacheError) as e:
        c.append(b, row, row)
    assert e.value.kind == "PoolExhausted"


def test_invalid_append_and_read(dev):
    c, _ = pair(4, 4, 1, 2)
    s = c.new_sequence()
    with pytest.raises(KvCacheError) as e:
        c.append(s, np.zeros(3, np.float32), np.zeros(2, np.float32))
    assert e.value.msg == "key/value length must equal heads * head_dim"
    with pytest.raises(KvCacheError) as e:
        c.append(5, np.zeros(2, np.float32), np.zeros(2, np.float32))
    assert e.value.msg == "unknown sequence id"
    with pytest.raises(KvCacheError) as e:
        c.read_key(s, 0)
    assert e.value.msg == "token out of range"
    assert c.token_count(s) == 0 and c.blocks_used() == 0


def test_failed_launch_rolls_back_reservation(dev, monkeypatch):
    c, o = pair(6, 2, 1, 2, KvDataType.F16)
    s, t = c.new_sequence(), c.new_sequence()
    o.new_sequence(), o.new_sequence()
    for i in range(4):                                    # pages 0, 1 full
        both_append(c, o, s, [i, i], [i, -i])

    def boom(*a, **k):
        raise RuntimeError("launch failed")
    monkeypatch.setattr(c._kv, "append_kv", boom)
    with pytest.raises(RuntimeError):
        c.append(s, np.ones(2, np.float32), np.ones(2, np.float32))
    assert c.token_count(s) == 4 and c.seq_block_table(s) == [0, 1] and c.blocks_used() == 2
    monkeypatch.setattr(c._kv, "append_kv_batched", boom)
    with pytest.raises(RuntimeError):
        c.append_batch([s, t], torch.ones((2, 2), dtype=torch.float16, device=dev),
                       torch.ones((2, 2), dtype=torch.float16, device=dev))
    assert c.token_count(s) == 4 and c.token_count(t) == 0 and c.blocks_used() == 2
    monkeypatch.undo()
    # the next pops are the pages the rolled-back calls had taken, in order
    both_append(c, o, s, [5, 5], [5, 5])
    both_append(c, o, t, [6, 6], [6, 6])
    assert c.seq_block_table(s) == o.seq_block_table(s).tolist()
    assert c.seq_block_table(t) == o.seq_block_table(t).tolist()
    same_pool(c, o)


def test_batch_exhaustion_mid_batch_changes_nothing(dev):
    c, o = pair(5, 4, 1, 2, KvDataType.F16)
    seqs = [c.new_sequence() for _ in range(3)]
    for _ in range(3):
        o.new_sequence()
    rows = torch.arange(2 * 3 * 4, dtype=torch.float16, device=dev).reshape(12, 2)
    c.extend_batch(seqs, [4, 3, 5], rows, -rows)          # pages: 1 + 1 + 2 = 4 of 5
    r = rows.cpu().numpy().astype(np.float32)
    at = 0
    for s, n in zip(seqs, [4, 3, 5]):
        for i in range(n):
            o.append(s, r[at + i], -r[at + i])
        at += n
    same_pool(c, o)
    before = [(c.seq_block_table(s), c.token_count(s)) for s in seqs]
    # 4 -> 5, 3 -> 5 and 5 -> 9 tokens each need a fresh page: 3 needed, 1 free
    one = torch.ones((3, 2), dtype=torch.float16, device=dev)
    with pytest.raises(KvCacheError) as e:
        c.extend_batch(seqs, [1, 2, 4], torch.ones((7, 2), dtype=torch.float16, device=dev),
                       torch.ones((7, 2), dtype=torch.float16, device=dev))
    assert e.value.kind == "PoolExhausted" and (e.value.blocks_used, e.value.blocks_total) == (4, 5)
    assert [(c.seq_block_table(s), c.token_count(s)) for s in seqs] == before
    assert c.blocks_used() == 4
    # shapes and counts are checked before any page moves
    with pytest.raises(KvCacheError):
        c.append_batch(seqs, one[:2], one)
    with pytest.raises(KvCacheError) as e:
        c.extend_batch(seqs, [2, -1, 2], one, one)
    assert e.value.msg == "token counts must not be negative"
    assert [(c.seq_block_table(s), c.token_count(s)) for s in seqs] == before
    same_pool(c, o)


def test_allocator_driven_batched_decode(dev):
    rng = np.random.default_rng(2024)
    n_head, n_kv, hd, bt = 12, 2, 128, 16
    rl = n_kv * hd
    B, steps = 24, 20
    prompts = rng.integers(1, 300, size=B)
    prompts[3], prompts[7] = 16, 1                        # a full page, a single token
    need = sum((int(p) + steps + 40 + bt - 1) // bt for p in prompts) + 8
    nb = int(need * 1.1)
    c, o = pair(nb, bt, n_kv, hd, KvDataType.F16)
    order = rng.permutation(nb).astype(np.uint32)
    c.seed_free_list(order)
    o.seed_free_list(order)
    seqs = [c.new_sequence() for _ in range(B)]
    for _ in range(B):
        o.new_sequence()
    for s in seqs:
        assert c.seq_block_table(s) == []

    def rows(n):
        k = rng.standard_normal((n, rl)).astype(np.float16)
        v = rng.standard_normal((n, rl)).astype(np.float16)
        return k, v

    def o_append(s, k, v):
        for i in range(k.shape[0]):
            o.append(s, k[i], v[i])

    # ragged prompt append: one launch for the whole batch
    pk, pv = rows(int(prompts.sum()))
    c.extend_batch(seqs, prompts, torch.from_numpy(pk).to(dev), torch.from_numpy(pv).to(dev))
    at = 0
    for s, n in zip(seqs, prompts):
        o_append(s, pk[at:at + n], pv[at:at + n])
        at += int(n)
    same_pool(c, o)

    plan = PagedAttention.plan(B, n_head, n_kv, hd, bt, 4096)
    ws = PagedAttention.workspace(plan)
    pa = PagedAttention(0)
    radix = RadixTree(bt)
    tokens = {}
    freed = replacement = None
    stride = (300 + steps + 40 + bt - 1) // bt
    for step in range(steps):
        if step == 8:
            # retire one sequence mid-run; a new one takes its pages (free list order)
            freed = seqs[5]
            pages = c.seq_block_table(freed)
            c.free_sequence(freed)
            o.free_sequence(freed)
            replacement = c.new_sequence()
            assert o.new_sequence() == replacement
            n_new = 37
            k, v = rows(n_new)
            c.extend_batch([replacement], [n_new], torch.from_numpy(k).to(dev),
                           torch.from_numpy(v).to(dev))
            o_append(replacement, k, v)
            assert c.seq_block_table(replacement) == pages[:(n_new + bt - 1) // bt]
            seqs[5] = replacement
        # the step reserves one slot per sequence, all or nothing
        starts = c.reserve_batch(seqs, [1] * B)
        tables, lens = c.block_tables(seqs, stride)
        assert np.array_equal(lens.cpu().numpy(), starts + 1)
        host_tab = tables.cpu().numpy().view(np.uint32)
        for i, s in enumerate(seqs):
            t = c.seq_block_table(s)
            assert host_tab[i, :len(t)].tolist() == t
            assert (host_tab[i, len(t):] == 0xFFFFFFFF).all()
        k, v = rows(B)
        q = rng.standard_normal((B, n_head, hd)).astype(np.float32)
        out = torch.empty((B, n_head, hd), device=dev)
        pos = torch.from_numpy(starts.astype(np.int32)).to(dev)
        pa.append_decode_batched(None, c.layout, c.pool, torch.from_numpy(k).to(dev),
                                 torch.from_numpy(v).to(dev), tables, pos,
                                 torch.from_numpy(q).to(dev), out, n_head, hd, plan, ws)
        for i, s in enumerate(seqs):
            o.append(s, k[i], v[i])
        assert [o.token_count(s) for s in seqs] == [c.token_count(s) for s in seqs]
        for s in seqs:
            assert o.seq_block_table(s).tolist() == c.seq_block_table(s)
        same_pool(c, o)
        ref = orc.sdpa_decode_batched(o.buffer().astype(np.float32), host_tab,
                                      (starts + 1).astype(np.uint32), bt, q, n_head, n_kv, hd)
        parity.check_close(out.cpu().numpy(), ref, what=f"step {step}")
    # real page ids into the radix index, matched back
    for i, s in enumerate(seqs):
        n = c.token_count(s)
        tokens[s] = [100_000 * (i + 1) + t for t in range(n)]
        radix.insert(tokens[s], c.seq_block_table(s), False)
    for s in seqs:
        r = radix.match_prefix(tokens[s])
        full = c.token_count(s) // bt
        assert r.matched_tokens == c.token_count(s)
        assert r.matched_blocks[:full] == c.seq_block_table(s)[:full]
    # the pool runs out on a final oversized reserve; nothing changes
    used = c.blocks_used()
    state = [(c.seq_block_table(s), c.token_count(s)) for s in seqs]
    with pytest.raises(KvCacheError) as e:
        c.reserve_batch(seqs, [bt * nb] * B)
    assert e.value.kind == "PoolExhausted" and e.value.blocks_used == used
    assert [(c.seq_block_table(s), c.token_count(s)) for s in seqs] == state
