"""GPU parity of decode over the protected-sinks range (attention sinks +
rolling window, openspec/specs/protected-kv-sinks/spec.md:9-15) against the
oracle's windowed sdpa_decode (pinned in tests/test_oracle_window.py).

Tolerance: max-abs <= 2e-3 and
|gpu - ref| <= 2e-3 + 1e-3*|ref| (tests/parity.py) (16-bit and E4M3 pages).  The
cases cover sinks that end mid-tile, windows shorter than one tile, windows
that start mid-tile, gaps of many tiles, sinks covering the whole sequence,
runs that cross sequences whose walked tiles skip a gap, graph replay as the
device lengths grow, and window 0 (which
must equal the plain decode bit for bit).
"""
import numpy as np
import pytest
import torch

from oracle import orc
from titan_amd import KvDataType, PagedAttention

import parity
from e4m3_data import gauss_codes

pytestmark = pytest.mark.gpu

TD = {KvDataType.F16: torch.float16, KvDataType.BF16: torch.bfloat16}


def i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(dev)


def make_tables(rng, lens, bt):
    need = [(int(l) + bt - 1) // bt for l in lens]
    stride = max(max(need), 1)
    nb = sum(need) + 2
    perm = rng.permutation(nb).astype(np.uint32)
    tab = np.full((len(lens), stride), 0xFFFFFFFF, np.uint32)
    p = 0
    for b, c in enumerate(need):
        tab[b, :c] = perm[p:p + c]
        p += c
    return tab, nb


def check_close(gpu, ref, what="window"):
    parity.check_close(gpu, ref, what=what)


LENS = np.array([0, 1, 3, 4, 5, 16, 17, 33, 300, 2049, 3000, 100, 7], np.int64)


def run(dev, dtype, shape, sink, window, seed, grid=None, lens=LENS):
    n_head, n_kv, hd, bt = shape
    rng = np.random.default_rng(seed)
    tab, nb = make_tables(rng, lens, bt)
    n = nb * bt * 2 * n_kv * hd
    q = rng.standard_normal((len(lens), n_head, hd)).astype(np.float32)
    ks = vs = None
    if dtype == KvDataType.FP8:  # quantised N(0,1) K/V, scales max|x| / 448
        codes, ksn, vsn = gauss_codes(rng, nb, bt, n_kv, hd)
        f = orc.e4m3_to_f32(codes).reshape(nb, bt, 2, n_kv, hd)
        f[:, :, 0] *= ksn[None, None, :, None]
        f[:, :, 1] *= vsn[None, None, :, None]
        pool_f32 = f.reshape(-1)
        pool = torch.from_numpy(codes).to(dev)
        ks, vs = torch.from_numpy(ksn).to(dev), torch.from_numpy(vsn).to(dev)
    else:
        host = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(TD[dtype])
        pool, pool_f32 = host.to(dev), host.float().numpy()
    plan = PagedAttention.plan(len(lens), n_head, n_kv, hd, bt, int(max(lens)), 0, dtype)
    assert plan[0] == 0
    if grid is not None:
        plan = PagedAttention.with_grid(plan, grid, len(lens), n_head)
    out = torch.full((len(lens), n_head, hd), float("nan"), device=dev)
    PagedAttention(0).decode_batched_window(None, torch.from_numpy(q).to(dev), pool, i32(tab, dev),
                                            i32(lens, dev), out, n_head, n_kv, hd, bt, dtype, sink,
                                            window, plan, PagedAttention.workspace(plan), ks, vs)
    torch.cuda.synchronize()
    ref = orc.sdpa_decode_window_batched(pool_f32, tab, lens.astype(np.uint32), bt, q, n_head,
                                         n_kv, hd, sink, window)
    return out.cpu().numpy(), ref, (q, pool, tab, plan)


@pytest.mark.parametrize("dtype", [KvDataType.F16, KvDataType.BF16, KvDataType.FP8],
                         ids=lambda d: d.name)
@pytest.mark.parametrize("sink,window", [(4, 1), (4, 15), (4, 16), (4, 100), (0, 40), (20, 1000),
                                         (40, 3)])
def test_window_matches_oracle(dev, dtype, sink, window):
    out, ref, _ = run(dev, dtype, (12, 2, 128, 16), sink, window, 7 + sink + window)
    check_close(out, ref)


@pytest.mark.parametrize("shape", [(32, 8, 128, 16), (8, 1, 128, 32), (16, 4, 128, 64)],
                         ids=lambda s: "x".join(map(str, s)))
def test_window_shapes(dev, shape):
    out, ref, _ = run(dev, KvDataType.F16, shape, 4, 200, 11 + sum(shape))
    check_close(out, ref)


@pytest.mark.parametrize("grid", [1, 2, 5, 64])
def test_window_small_grids(dev, grid):
    """Runs that walk several sequences across their sink/window gaps."""
    out, ref, _ = run(dev, KvDataType.F16, (12, 2, 128, 16), 4, 50, 20 + grid, grid)
    check_close(out, ref)


def test_window_zero_equals_plain_decode(dev):
    out, _, (q, pool, tab, plan) = run(dev, KvDataType.F16, (12, 2, 128, 16), 4, 0, 3)
    plain = torch.full(out.shape, float("nan"), device=dev)
    PagedAttention(0).decode_batched(None, torch.from_numpy(q).to(dev), pool, i32(tab, dev),
                                     i32(LENS, dev), plain, 12, 2, 128, 16, KvDataType.F16, plan,
                                     PagedAttention.workspace(plan))
    torch.cuda.synchronize()
    assert np.array_equal(out.view(np.uint32), plain.cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("dtype,shape,sink,window,grid", [
    (KvDataType.F16, (12, 2, 128, 16), 0, 0, None),
    (KvDataType.F16, (12, 2, 128, 16), 4, 100, None),
    (KvDataType.F16, (12, 2, 128, 16), 4, 100, 3),
    (KvDataType.BF16, (8, 1, 128, 32), 4, 40, None),      # two tiles per page
    (KvDataType.FP8, (32, 8, 128, 16), 0, 0, None),
    (KvDataType.F16, (16, 4, 128, 64), 20, 500, 7),
], ids=lambda v: str(v))
def test_block_mass_matches_oracle(dev, dtype, shape, sink, window, grid):
    """block_mass[page] += the page's attention mass summed over q heads (the
    H2O score of record_attention_mass), against the oracle's f64 weights;
    each sequence's pages receive n_head in total."""
    n_head, n_kv, hd, bt = shape
    rng = np.random.default_rng(5 + sink + window)
    tab, nb = make_tables(rng, LENS, bt)
    n = nb * bt * 2 * n_kv * hd
    q = rng.standard_normal((len(LENS), n_head, hd)).astype(np.float32)
    ks = vs = None
    if dtype == KvDataType.FP8:  # quantised N(0,1) K/V, scales max|x| / 448
        codes, ksn, vsn = gauss_codes(rng, nb, bt, n_kv, hd)
        f = orc.e4m3_to_f32(codes).reshape(nb, bt, 2, n_kv, hd)
        f[:, :, 0] *= ksn[None, None, :, None]
        f[:, :, 1] *= vsn[None, None, :, None]
        pool_f32, pool = f.astype(np.float32).reshape(-1), torch.from_numpy(codes).to(dev)
        ks, vs = torch.from_numpy(ksn).to(dev), torch.from_numpy(vsn).to(dev)
    else:
        host = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(TD[dtype])
        pool, pool_f32 = host.to(dev), host.float().numpy()
    plan = PagedAttention.plan(len(LENS), n_head, n_kv, hd, bt, int(max(LENS)), 0, dtype)
    if grid is not None:
        plan = PagedAttention.with_grid(plan, grid, len(LENS), n_head)
    extra = PagedAttention.mass_workspace_bytes(len(LENS), tab.shape[1], bt, n_head)
    ws = torch.zeros((plan[2] + extra + 3) // 4, device=dev)
    mass = torch.full((nb,), 0.5, device=dev)
    out = torch.full((len(LENS), n_head, hd), float("nan"), device=dev)
    PagedAttention(0).decode_batched_window(None, torch.from_numpy(q).to(dev), pool, i32(tab, dev),
                                            i32(LENS, dev), out, n_head, n_kv, hd, bt, dtype, sink,
                                            window, plan, ws, ks, vs, block_mass=mass)
    torch.cuda.synchronize()
    ref, ref_mass = orc.sdpa_decode_window_batched(pool_f32, tab, LENS.astype(np.uint32), bt, q,
                                                   n_head, n_kv, hd, sink, window, n_blocks=nb)
    check_close(out.cpu().numpy(), ref)
    got = mass.cpu().numpy().astype(np.float64) - 0.5
    bad = np.abs(got - ref_mass) > 2e-4 * n_head + 1e-3 * ref_mass
    assert not bad.any(), (np.argwhere(bad)[:4], got[bad][:4], ref_mass[bad][:4])
    for b, L in enumerate(LENS):
        if L:
            pages = [int(p) for p in tab[b, :(int(L) + bt - 1) // bt]]
            assert abs(got[pages].sum() - n_head) < 1e-3 * n_head


def test_h2o_scores_drive_prune_like_oracle(dev):
    """End to end: three decode steps accumulate block_mass on the device; the
    host StreamingKvManager records it and prunes.  Pages whose keys align with
    the queries are heavy hitters; the retained and evicted pages equal the
    oracle manager's fed with the oracle's f64 masses."""
    from titan_amd.share import StreamingKvConfig, StreamingKvManager
    n_head, n_kv, hd, bt = 8, 1, 128, 16
    rng = np.random.default_rng(17)
    lens = np.array([1000, 900], np.int64)
    tab, nb = make_tables(rng, lens, bt)
    pool_f32 = (rng.standard_normal((nb, bt, 2, n_kv, hd)) * 0.3).astype(np.float32)
    q = rng.standard_normal((2, n_head, hd)).astype(np.float32)
    heavy = {0: [10, 25, 40], 1: [7, 30, 44]}   # page indices within each sequence
    for b, pages in heavy.items():
        for k, j in enumerate(pages):            # distinct strengths: distinct masses
            pool_f32[tab[b, j], :, 0, 0] = q[b].mean(axis=0) * (0.4 + 0.1 * k)
    host = torch.from_numpy(pool_f32.reshape(-1)).half()
    pool, pool_f32 = host.to(dev), host.float().numpy()
    plan = PagedAttention.plan(2, n_head, n_kv, hd, bt, 1000, 0, KvDataType.F16)
    ws = torch.zeros((plan[2] + PagedAttention.mass_workspace_bytes(2, tab.shape[1], bt, n_head)
                      + 3) // 4, device=dev)
    mass = torch.zeros(nb, device=dev)
    out = torch.empty((2, n_head, hd), device=dev)
    ref_mass = np.zeros(nb)
    for step in range(3):
        L = lens - 2 + step
        PagedAttention(0).decode_batched_window(None, torch.from_numpy(q).to(dev), pool,
                                                i32(tab, dev), i32(L, dev), out, n_head, n_kv, hd,
                                                bt, KvDataType.F16, 0, 0, plan, ws, block_mass=mass)
        _, m = orc.sdpa_decode_window_batched(pool_f32, tab, L.astype(np.uint32), bt, q, n_head,
                                              n_kv, hd, 0, 0, n_blocks=nb)
        ref_mass += m
    torch.cuda.synchronize()
    got = mass.cpu().numpy()
    assert np.allclose(got, ref_mass, rtol=1e-3, atol=2e-4 * n_head)
    cfg = StreamingKvConfig(4 * bt, 8 * bt, 15 * bt, bt)   # 4 sink + 8 recent + 3 middle pages
    mgr, ref = StreamingKvManager(cfg), orc.Streaming(4 * bt, 8 * bt, 15 * bt, bt)
    mgr.record_attention_masses(got)
    for i, v in enumerate(ref_mass.astype(np.float32)):
        if v != 0.0:
            ref.record_attention_mass(i, float(v))
    for b in range(2):
        row = tab[b, :(int(lens[b]) + bt - 1) // bt]
        kept, evicted = mgr.prune_blocks(row)
        rkept, revicted = ref.prune_blocks(row)
        assert kept == rkept                      # sinks, heavy hitters by score, recent
        assert sorted(evicted) == sorted(revicted)
        assert sorted(kept[4:7]) == sorted(int(tab[b, j]) for j in heavy[b])


def test_window_mass_buffer_checks(dev):
    """block_mass shorter than the pool's pages, or a workspace without the
    mass scratch, is rejected; without block_mass the plan's workspace suffices."""
    from titan_amd import HipError
    n_head, n_kv, hd, bt = 12, 2, 128, 16
    rng = np.random.default_rng(1)
    lens = np.array([40, 7], np.int64)
    tab, nb = make_tables(rng, lens, bt)
    pool = torch.zeros(nb * bt * 2 * n_kv * hd, dtype=torch.float16, device=dev)
    q = torch.zeros((2, n_head, hd), device=dev)
    out = torch.empty_like(q)
    plan = PagedAttention.plan(2, n_head, n_kv, hd, bt, 64, 0, KvDataType.F16)
    pa = PagedAttention(0)
    args = (None, q, pool, i32(tab, dev), i32(lens, dev), out, n_head, n_kv, hd, bt,
            KvDataType.F16, 4, 16, plan)
    with pytest.raises(HipError):
        pa.decode_batched_window(*args, PagedAttention.workspace(plan),
                                 block_mass=torch.zeros(nb - 1, device=dev))
    with pytest.raises(HipError):
        pa.decode_batched_window(*args, PagedAttention.workspace(plan),
                                 block_mass=torch.zeros(nb, device=dev))
    pa.decode_batched_window(*args, PagedAttention.workspace(plan))
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()


def test_window_graph_replay_growing_lengths(dev):
    """The windowed decode with H2O mass captured once in a graph and replayed
    as the device lengths grow across tile, page and window edges (the
    walked tiles and cut tiles follow the lengths each replay): output and
    per-page mass equal the oracle at every replay, with eager work and
    synchronisations between the replays."""
    n_head, n_kv, hd, bt = 12, 2, 128, 16
    sink, window = 4, 40
    rng = np.random.default_rng(23)
    start = np.array([1, 14, 44, 300, 47, 0], np.int64)
    steps = 6
    B = len(start)
    tab, nb = make_tables(rng, start + 3 * steps, bt)
    host = torch.from_numpy(rng.standard_normal(nb * bt * 2 * n_kv * hd).astype(np.float32)).half()
    pool, pool_f32 = host.to(dev), host.float().numpy()
    plan = PagedAttention.plan(B, n_head, n_kv, hd, bt, int(start.max()) + 3 * steps)
    extra = PagedAttention.mass_workspace_bytes(B, tab.shape[1], bt, n_head)
    ws = torch.zeros((plan[2] + extra + 3) // 4, device=dev)
    mass = torch.zeros((nb,), device=dev)
    lens = i32(start, dev)
    q = torch.empty((B, n_head, hd), device=dev)
    out = torch.empty((B, n_head, hd), device=dev)
    dtab = i32(tab, dev)
    pa = PagedAttention(0)

    def call(st):
        pa.decode_batched_window(st, q, pool, dtab, lens, out, n_head, n_kv, hd, bt,
                                 KvDataType.F16, sink, window, plan, ws, block_mass=mass)
    call(None)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call(s)
    torch.cuda.synchronize()
    for step in range(steps):
        cur = start + 3 * step
        qn = rng.standard_normal((B, n_head, hd)).astype(np.float32)
        q.copy_(torch.from_numpy(qn))
        lens.copy_(i32(cur, dev))
        mass.zero_()
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ref, ref_mass = orc.sdpa_decode_window_batched(pool_f32, tab, cur.astype(np.uint32), bt, qn,
                                                       n_head, n_kv, hd, sink, window,
                                                       n_blocks=nb)
        check_close(out.cpu().numpy(), ref, what=f"window graph replay {step}")
        got = mass.cpu().numpy().astype(np.float64)
        bad = np.abs(got - ref_mass) > 2e-4 * n_head + 1e-3 * ref_mass
        assert not bad.any(), (step, np.argwhere(bad)[:4])
