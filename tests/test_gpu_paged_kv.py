"""GPU parity of append / gather / page copy / table kernels against the oracle.

Bit-exact throughout: every check compares raw bytes (pool pages, gathered
rows, block tables, reference counts).  Mirrors
engine-cuda/tests/paged_kv_gpu.rs and paged_kv_parity.rs, extended to f16 /
bf16 pools, ragged batched append, pos_ptr, copy-on-write and compaction.
"""
import numpy as np
import pytest
import torch

from oracle import orc
from titan_amd import HipError, KvDataType, PagedKvGpu, PagedKvLayout

pytestmark = pytest.mark.gpu

NP = {KvDataType.F32: np.float32, KvDataType.F16: np.float16, KvDataType.BF16: np.uint16,
      KvDataType.FP8: np.uint8}
TD = {KvDataType.F32: torch.float32, KvDataType.F16: torch.float16,
      KvDataType.BF16: torch.int16, KvDataType.FP8: torch.uint8}


def to_dev(a, dev):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint32:
        a = a.view(np.int32)
    elif a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to(dev)


def raw(t):
    return t.cpu().contiguous().view(torch.uint8).numpy()


def test_append_and_gather_roundtrip_scattered(dev):
    # paged_kv_gpu.rs:45-141: 12 tokens over pages [1, 2, 0], rows t + h/8, -t - h/2.
    layout = PagedKvLayout(3, 4, 6)
    kv = PagedKvGpu(0)
    pool = torch.zeros(layout.floats_total(), dtype=torch.float32, device=dev)
    t = np.arange(12, dtype=np.float32)[:, None]
    h = np.arange(6, dtype=np.float32)[None, :]
    keys = (t + h * 0.125).astype(np.float32)
    vals = (-t - h * 0.5).astype(np.float32)
    bt = to_dev(np.array([1, 2, 0], np.uint32), dev)
    kv.append_kv(None, layout, pool, to_dev(keys, dev), to_dev(vals, dev), bt, 0, 12)
    ok = torch.empty(12 * 6, device=dev)
    ov = torch.empty(12 * 6, device=dev)
    kv.read_keys(None, layout, pool, bt, ok, 0, 12)
    kv.read_values(None, layout, pool, bt, ov, 0, 12)
    torch.cuda.synchronize()
    assert np.array_equal(ok.cpu().numpy(), keys.ravel())
    assert np.array_equal(ov.cpu().numpy(), vals.ravel())


@pytest.mark.parametrize("dtype", [KvDataType.F32, KvDataType.F16, KvDataType.BF16])
def test_append_matches_oracle_pool_bytes(dev, dtype):
    """paged_kv_parity.rs:68-225 scenario: seq_a takes 5 pages, seq_b (the
    target) spans pages 5..8; pool bytes and gathers must match the oracle."""
    heads, hd, bt, nb = 2, 8, 6, 9
    rl = heads * hd
    c = orc.Cache(nb, bt, heads, hd, dtype=NP[dtype])
    a, b = c.new_sequence(), c.new_sequence()
    ka, va = orc.generate_rows_b(0xDEADBEEF, 5 * bt, rl)
    kb, vb = orc.generate_rows_b(0x12345678, 3 * bt + 4, rl)
    if dtype == KvDataType.F16:
        ka, va, kb, vb = (x.astype(np.float16) for x in (ka, va, kb, vb))
    elif dtype == KvDataType.BF16:
        ka, va, kb, vb = (orc.f32_to_bf16_bits(x) for x in (ka, va, kb, vb))
    for t in range(5 * bt):
        c.append(a, ka[t * rl:(t + 1) * rl], va[t * rl:(t + 1) * rl])
    nb_tok = 3 * bt + 4
    for t in range(nb_tok):
        c.append(b, kb[t * rl:(t + 1) * rl], vb[t * rl:(t + 1) * rl])

    layout = PagedKvLayout(nb, bt, rl, dtype)
    kv = PagedKvGpu(0)
    pool = torch.zeros(layout.floats_total(), dtype=TD[dtype], device=dev)
    for seq, k, v, n in ((a, ka, va, 5 * bt), (b, kb, vb, nb_tok)):
        table = to_dev(c.seq_block_table(seq), dev)
        # append in two uneven calls to cross a page boundary mid-call
        cut = 7
        kv.append_kv(None, layout, pool, to_dev(k[:cut * rl], dev), to_dev(v[:cut * rl], dev),
                     table, 0, cut)
        kv.append_kv(None, layout, pool, to_dev(k[cut * rl:], dev), to_dev(v[cut * rl:], dev),
                     table, cut, n - cut)
    torch.cuda.synchronize()
    assert np.array_equal(raw(pool), c.buffer().view(np.uint8))
    table_b = to_dev(c.seq_block_table(b), dev)
    outk = torch.empty(nb_tok * rl, dtype=TD[dtype], device=dev)
    kv.read_keys(None, layout, pool, table_b, outk, 0, nb_tok)
    outv = torch.empty(nb_tok * rl, dtype=TD[dtype], device=dev)
    kv.read_values(None, layout, pool, table_b, outv, 0, nb_tok)
    # gather from a middle start, crossing pages
    outm = torch.empty(9 * rl, dtype=TD[dtype], device=dev)
    kv.read_values(None, layout, pool, table_b, outm, 5, 9)
    torch.cuda.synchronize()
    assert np.array_equal(raw(outk), c.read_keys(b).view(np.uint8))
    assert np.array_equal(raw(outv), c.read_values(b).view(np.uint8))
    assert np.array_equal(raw(outm), c.read_values(b)[5 * rl:14 * rl].view(np.uint8))


def test_append_with_pos_ptr_and_zero_tokens(dev):
    layout = PagedKvLayout(4, 4, 8)
    kv = PagedKvGpu(0)
    pool = torch.zeros(layout.floats_total(), device=dev)
    bt = to_dev(np.array([2, 0, 3, 1], np.uint32), dev)
    k = torch.arange(8, dtype=torch.float32, device=dev) + 100
    v = -k
    pos = torch.tensor([9], dtype=torch.int32, device=dev)
    kv.append_kv_with_pos_ptr(None, layout, pool, k, v, bt, 0, 1, pos)
    kv.append_kv(None, layout, pool, k, v, bt, 0, 0)  # n_tokens == 0 is Ok
    torch.cuda.synchronize()
    p = pool.cpu().numpy().reshape(4, 4, 2, 8)
    assert np.array_equal(p[3, 1, 0], np.arange(8) + 100)     # pos 9 -> page idx 2 -> phys 3, slot 1
    assert np.array_equal(p[3, 1, 1], -(np.arange(8) + 100))
    assert np.count_nonzero(p) == 16


def test_invalid_sizes_match_reference_rules(dev):
    layout = PagedKvLayout(2, 4, 8)
    kv = PagedKvGpu(0)
    pool = torch.zeros(layout.floats_total(), device=dev)
    k = torch.zeros(16, device=dev)
    bt = to_dev(np.array([0, 1], np.uint32), dev)
    small_pool = torch.zeros(layout.floats_total() - 1, device=dev)
    with pytest.raises(HipError) as e:
        kv.append_kv(None, layout, small_pool, k, k, bt, 0, 2)
    assert e.value.kind == "InvalidSize" and e.value.expected == layout.bytes_total()
    with pytest.raises(HipError) as e:
        kv.append_kv(None, layout, pool, k, k, bt, 0, 3)
    assert (e.value.expected, e.value.actual) == (3 * 8 * 4, 64)
    with pytest.raises(HipError) as e:
        kv.append_kv(None, layout, pool, k, k, torch.zeros(0, dtype=torch.int32, device=dev), 0, 1)
    assert (e.value.expected, e.value.actual) == (4, 0)
    # added check: the table must cover start + n
    with pytest.raises(HipError) as e:
        kv.append_kv(None, layout, pool, k, k, bt, 7, 2)
    assert e.value.kind == "InvalidSize"
    out = torch.zeros(8, device=dev)
    with pytest.raises(HipError):
        kv.read_keys(None, layout, pool, bt, out, 0, 2)


@pytest.mark.parametrize("dtype", [KvDataType.F16, KvDataType.F32])
def test_batched_ragged_append_matches_oracle(dev, dtype):
    rng = np.random.default_rng(11)
    heads, hd, bt = 2, 16, 4
    rl = heads * hd
    lens0 = [0, 3, 9, 4, 1]          # tokens already cached
    new = [5, 1, 0, 7, 12]           # tokens appended now (ragged, one sequence empty)
    nb = 40
    c = orc.Cache(nb, bt, heads, hd, dtype=NP[dtype])
    c.seed_free_list(rng.permutation(nb))
    seqs = [c.new_sequence() for _ in lens0]
    rows = {}
    for s, n in zip(seqs, lens0):
        rows[s] = rng.standard_normal((n, 2, rl)).astype(NP[dtype])
        for t in range(n):
            c.append(s, rows[s][t, 0], rows[s][t, 1])
    base = c.buffer()
    layout = PagedKvLayout(nb, bt, rl, dtype)
    kv = PagedKvGpu(0)
    pool = to_dev(base.copy(), dev)
    newk, newv = [], []
    for s, n in zip(seqs, new):
        r = rng.standard_normal((n, 2, rl)).astype(NP[dtype])
        for t in range(n):
            c.append(s, r[t, 0], r[t, 1])
        newk.append(r[:, 0]); newv.append(r[:, 1])
    stride = max(len(c.seq_block_table(s)) for s in seqs)
    tab = np.full((len(seqs), stride), 0xFFFFFFFF, np.uint32)
    for i, s in enumerate(seqs):
        t = c.seq_block_table(s)
        tab[i, :len(t)] = t
    cu = np.concatenate([[0], np.cumsum(new)]).astype(np.uint32)
    kv.append_kv_batched(None, layout, pool, to_dev(np.concatenate(newk), dev),
                         to_dev(np.concatenate(newv), dev), to_dev(tab, dev), to_dev(cu, dev),
                         to_dev(np.array(lens0, np.uint32), dev), int(cu[-1]))
    torch.cuda.synchronize()
    assert np.array_equal(raw(pool), c.buffer().view(np.uint8))


def test_copy_pages_remap_and_refcounts(dev):
    rng = np.random.default_rng(5)
    layout = PagedKvLayout(16, 4, 32, KvDataType.F16)
    kv = PagedKvGpu(0)
    host = rng.standard_normal(layout.floats_total()).astype(np.float16)
    pool = to_dev(host, dev)
    src = np.array([3, 9, 12], np.uint32)
    dst = np.array([0, 1, 2], np.uint32)
    kv.copy_pages(None, layout, pool, to_dev(src, dev), to_dev(dst, dev))
    tables = np.array([[3, 9, 5, 0xFFFFFFFF], [3, 12, 9, 7]], np.uint32)
    n_used = np.array([3, 4], np.uint32)
    remap = np.arange(16, dtype=np.uint32)
    remap[src] = dst
    dt = to_dev(tables, dev)
    kv.remap_block_tables(None, dt, to_dev(remap, dev))
    counts = torch.full((16,), 77, dtype=torch.int32, device=dev)
    kv.page_refcounts(None, dt, to_dev(n_used, dev), counts)
    torch.cuda.synchronize()
    exp = host.reshape(16, -1).copy()
    exp[dst] = exp[src]
    assert np.array_equal(raw(pool), exp.view(np.uint8).ravel())
    exp_tab = tables.copy()
    mask = exp_tab < 16
    exp_tab[mask] = remap[exp_tab[mask]]
    assert np.array_equal(dt.cpu().numpy().view(np.uint32), exp_tab)
    exp_counts = np.zeros(16, np.int64)
    for r, n in zip(exp_tab, n_used):
        for p in r[:n]:
            exp_counts[p] += 1
    assert np.array_equal(counts.cpu().numpy(), exp_counts)


@pytest.mark.parametrize("n_kv,hd,dtype", [(2, 128, KvDataType.F16), (8, 128, KvDataType.F16),
                                           (4, 64, KvDataType.F32), (1, 128, KvDataType.BF16)],
                         ids=["2x128-f16", "8x128-f16", "4x64-f32", "1x128-bf16"])
def test_stream_pages_fold_every_listed_word(dev, n_kv, hd, dtype):
    """The read-ceiling aids fold every word of the listed pages into their
    per-wave xors exactly once: the xor over all waves equals the xor of
    the listed pages' words on the host, for whole pages (eh_stream_pages,
    depth 1 and 2, where pages are a multiple of 16 KiB) and for the
    per-kv-head pattern of the decode (eh_stream_pages_heads), on grids
    smaller and larger than the page count; an id past the pool is skipped."""
    bt, nb = 16, 37
    rl = n_kv * hd
    layout = PagedKvLayout(nb, bt, rl, dtype)
    rng = np.random.default_rng(77 + n_kv + hd)
    words = rng.integers(0, 2**32, size=layout.bytes_total() // 4, dtype=np.uint32)
    pool = to_dev(words, dev)
    listed = rng.permutation(nb)[:29].astype(np.uint32)
    ids = np.insert(listed, 11, nb + 5)                      # past the pool: skipped
    dids = to_dev(ids, dev)
    pw = layout.page_bytes() // 4
    want = np.bitwise_xor.reduce(np.concatenate([words[p * pw:(p + 1) * pw] for p in listed]))
    kv = PagedKvGpu(0)
    for grid in (1, 3, 64):
        out = torch.zeros(grid * 8, dtype=torch.int32, device=dev)
        kv.stream_pages_heads(None, layout, pool, dids, out, hd, grid)
        torch.cuda.synchronize()
        got = np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32))
        assert got == want, ("heads", grid)
        if layout.page_bytes() % 16384 == 0:
            for depth in (1, 2):
                out.zero_()
                kv.stream_pages(None, layout, pool, dids, out, depth, grid)
                torch.cuda.synchronize()
                got = np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32))
                assert got == want, ("whole", depth, grid)
