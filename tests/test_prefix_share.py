"""Benchmark config 4: prefix-shared KV with copy-on-write, LRU eviction and
gather-compaction (titan_amd.prefix_share).

CPU: the flow driven by the product bookkeeping (titan_amd.share) and by the
oracle's restatement (orc.Cow / orc.Radix, cow.rs / radix.rs) must agree on
every block table, CoW pair, eviction victim and strong count.
GPU: the page moves (batched append, CoW page copies, compaction copies,
table remap, reference recount) must leave the device bit-exact with the host
model, and every surviving sequence must gather back exactly the rows that
were appended for it.
"""
import numpy as np
import pytest

from oracle import orc
from titan_amd.prefix_share import PrefixShareScenario, model_pool, run_on_gpu


def _plan(seed, backend, **kw):
    if backend == "oracle":
        scn = PrefixShareScenario(seed, cow_cls=orc.Cow, radix_cls=orc.Radix,
                                  compaction_plan=orc.compaction_plan, **kw)
    else:
        scn = PrefixShareScenario(seed, **kw)
    return scn, scn.plan()


def _assert_same_plan(a, b):
    assert a.n_blocks == b.n_blocks
    assert a.cow_pairs == b.cow_pairs and a.cow_pairs > 0
    assert a.victims == b.victims
    assert a.evicted_seqs == b.evicted_seqs
    assert a.tables == b.tables and a.compacted == b.compacted
    assert a.strong_counts == b.strong_counts
    assert np.array_equal(a.remap, b.remap)
    assert np.array_equal(a.compaction.src, b.compaction.src)
    assert np.array_equal(a.compaction.dst, b.compaction.dst)


@pytest.mark.parametrize("seed", [0, 1])
def test_config4_bookkeeping_matches_oracle(seed):
    kw = dict(n_seqs=64, head_dim=8, n_kv=1)    # full config-4 page counts, tiny rows
    _, a = _plan(seed, "product", **kw)
    _, b = _plan(seed, "oracle", **kw)
    _assert_same_plan(a, b)
    # >= 25 % of the live pages were freed, pinned prefix pages never
    assert len(a.victims) >= 0.25 * a.live_before_evict
    prefix_pages = set(next(iter(a.tables.values()))[:64])
    assert not prefix_pages.intersection(a.victims)
    # compaction: live pages occupy exactly the lowest ids
    live = sorted({p for t in a.compacted.values() for p in t})
    assert live == list(range(len(live)))
    # refcounts: prefix pages are held by every survivor, private pages once
    for p, c in a.strong_counts.items():
        assert c == (len(a.tables) if p in {a.remap[q] for q in prefix_pages} else 1)


def test_config4_plan_independent_of_row_size():
    # the eviction touch order has its own generator: the bookkeeping of the
    # full-size rows equals that of the tiny rows the CPU test compares
    _, a = _plan(3, "product", n_seqs=16, head_dim=8, n_kv=1)
    _, b = _plan(3, "product", n_seqs=16, head_dim=32, n_kv=2)
    _assert_same_plan(a, b)


def test_oracle_compaction_plan_matches_product():
    from titan_amd.share import compaction_plan
    rng = np.random.default_rng(5)
    for _ in range(20):
        nb = int(rng.integers(1, 200))
        B = int(rng.integers(1, 8))
        stride = int(rng.integers(1, 30))
        tab = rng.integers(0, nb, size=(B, stride)).astype(np.uint32)
        used = rng.integers(0, stride + 1, size=B).astype(np.uint32)
        a, b = compaction_plan(tab, used, nb), orc.compaction_plan(tab, used, nb)
        for x, y in zip(a, b):
            assert np.array_equal(x, y)


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [0, 1])
def test_config4_page_moves_bit_exact(dev, seed):
    import torch

    from titan_amd import PagedKvGpu
    scn, plan = _plan(seed, "product")
    # config 4 at its real size (64 sequences, 8 kv heads, hd 128): the plan
    # the GPU executes equals the one the oracle's CoW / radix restatements
    # and compaction rule produce on the same seed
    _, oplan = _plan(seed, "oracle", n_seqs=64, head_dim=128, n_kv=8)
    _assert_same_plan(plan, oplan)
    print(f"config4 seed {seed}: {len(plan.victims)} victims of {plan.live_before_evict} live "
          f"pages, {plan.cow_pairs} CoW copies, {len(plan.compaction.src)} compaction moves",
          flush=True)
    pool, tables, counts, layout = run_on_gpu(scn, plan)
    # block tables after remap
    got = tables.cpu().numpy().view(np.uint32)
    for i, s in enumerate(scn.survivors):
        n = len(plan.compacted[s])
        assert got[i, :n].tolist() == plan.compacted[s]
    # device reference counts == CoW strong counts on live pages, 0 elsewhere
    cnt = counts.cpu().numpy()
    exp = np.zeros(plan.n_blocks, np.int64)
    for p, c in plan.strong_counts.items():
        exp[p] = c
    assert np.array_equal(cnt, exp)
    # page bytes of every live page
    model = model_pool(scn, plan)
    dev_pool = pool.cpu().numpy().reshape(model.shape)
    live = np.nonzero(exp)[0]
    assert np.array_equal(dev_pool[live].view(np.uint16), model[live].view(np.uint16))
    # every survivor gathers back its own rows
    kv = PagedKvGpu(0)
    for i, s in enumerate(scn.survivors):
        n_tok = plan.tokens[s]
        for is_value in (0, 1):
            out = torch.empty((n_tok, scn.row_len), dtype=torch.float16, device=pool.device)
            fn = kv.read_values if is_value else kv.read_keys
            fn(None, layout, pool, tables[i], out, 0, n_tok)
            torch.cuda.synchronize()
            assert np.array_equal(out.cpu().numpy().view(np.uint16),
                                  plan.rows[s][is_value].view(np.uint16)), (s, is_value)
