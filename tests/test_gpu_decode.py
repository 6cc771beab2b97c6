"""GPU parity of paged decode attention against the oracle's sdpa_decode.

Tolerances (stated by the benchmark contract): f32 KV max-abs 1e-5; f16/bf16
KV with f32 accumulation max-abs <= 2e-3 and
|gpu - ref| <= 2e-3 + 1e-3*|ref| (tests/parity.py).  The oracle runs
on the exactly widened f32 pool.  Shapes follow the reference's own tests
(engine-cuda/tests/paged_attention_gpu.rs, paged_attention_parity.rs,
graph_dynamic_params_test.rs) plus the five benchmark configurations.
"""
import numpy as np
import pytest
import torch

from oracle import orc
from titan_amd import HipError, KvDataType, PagedAttention, PagedKvGpu, PagedKvLayout
from titan_amd import synth

import parity

pytestmark = pytest.mark.gpu

TD = {KvDataType.F32: torch.float32, KvDataType.F16: torch.float16,
      KvDataType.BF16: torch.bfloat16}


def i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(dev)


def check_close(gpu, ref, dtype, what=""):
    parity.check_close(gpu, ref, f32=dtype == KvDataType.F32, what=what or KvDataType(dtype).name)


def cosine(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return a @ b / (np.linalg.norm(a) * np.linalg.norm(b))


def make_pool(rng, n_blocks, bt, n_kv, hd, dtype, dev):
    host = rng.standard_normal(n_blocks * bt * 2 * n_kv * hd).astype(np.float32)
    t = torch.from_numpy(host).to(TD[dtype])
    return t.to(dev), t.to(torch.float32).numpy()


@pytest.mark.parametrize("method", ["launch", "launch_flash_decoding"])
@pytest.mark.parametrize("cfg", [(4, 1, 64, 16), (8, 2, 32, 16), (4, 4, 16, 8), (2, 1, 8, 4)])
def test_gqa_multiconfig_matches_sdpa(dev, cfg, method):
    # paged_attention_gpu.rs:144-183 (pages [3,0,2,1], xorshift seed 0xABCD)
    n_head, n_kv, hd, bt = cfg
    pa = PagedAttention(0)
    table = np.array([3, 0, 2, 1], np.uint32)
    for n in (1, bt * 3 + 3):
        pool = np.zeros(4 * bt * 2 * n_kv * hd, np.float32)
        orc.fill_pool_paged(pool, table, bt, n_kv, hd, 0xABCD, n)
        q = orc.xorshift_a(0xABCD ^ 0xF00D, n_head * hd)
        ref = orc.sdpa_decode(pool, table, bt, n, q, n_head, n_kv, hd, False, n)
        out = torch.empty(n_head * hd, device=dev)
        getattr(pa, method)(None, torch.from_numpy(q).to(dev), torch.from_numpy(pool).to(dev),
                            i32(table, dev), out, n_head, n_kv, hd, bt, n, n, False)
        torch.cuda.synchronize()
        check_close(out.cpu().numpy(), ref, KvDataType.F32)


def test_single_token_returns_value_row(dev):
    # paged_attention_gpu.rs:106-142
    pa = PagedAttention(0)
    table = np.array([3, 0, 2, 1], np.uint32)
    pool = np.zeros(4 * 4 * 2 * 4, np.float32)
    orc.fill_pool_paged(pool, table, 4, 1, 4, 0x1234, 1)
    q = orc.xorshift_a(0x1234 ^ 0xF00D, 8)
    out = torch.empty(8, device=dev)
    pa.launch(None, torch.from_numpy(q).to(dev), torch.from_numpy(pool).to(dev), i32(table, dev),
              out, 2, 1, 4, 4, 1, 1, False)
    torch.cuda.synchronize()
    vrow = pool[3 * 32 + 4: 3 * 32 + 8]
    assert np.array_equal(out.cpu().numpy(), np.concatenate([vrow, vrow]))


def test_causal_decode_matches_sdpa(dev):
    # paged_attention_gpu.rs:185-221 (causal, query_pos inside the context)
    pa = PagedAttention(0)
    bt, n_head, n_kv, hd = 4, 4, 2, 16
    table = np.array([3, 0, 2, 1], np.uint32)
    n, qp = 3 * bt + 2, 2 * bt + 1
    pool = np.zeros(4 * bt * 2 * n_kv * hd, np.float32)
    orc.fill_pool_paged(pool, table, bt, n_kv, hd, 0xCAFE, n)
    q = orc.xorshift_a(0xCAFE ^ 0xF00D, n_head * hd)
    ref = orc.sdpa_decode(pool, table, bt, n, q, n_head, n_kv, hd, True, qp)
    for fn in (pa.launch, pa.launch_flash_decoding):
        out = torch.empty(n_head * hd, device=dev)
        fn(None, torch.from_numpy(q).to(dev), torch.from_numpy(pool).to(dev), i32(table, dev),
           out, n_head, n_kv, hd, bt, n, qp, True)
        torch.cuda.synchronize()
        check_close(out.cpu().numpy(), ref, KvDataType.F32)


@pytest.mark.parametrize("sweep", [(512, 8, 4, 16, 0x5EED), (256, 4, 2, 32, 0xAAA5)])
def test_scattered_parity_sweep(dev, sweep):
    # paged_attention_parity.rs:19-148: contexts 1..2048 over scattered pages
    bt, n_head, n_kv, hd, seed = sweep
    pa = PagedAttention(0)
    nb = 2048 // bt
    table = np.random.default_rng(seed).permutation(nb).astype(np.uint32)
    pool = np.zeros(nb * bt * 2 * n_kv * hd, np.float32)
    orc.fill_pool_paged(pool, table, bt, n_kv, hd, seed, nb * bt)
    q = orc.xorshift_a(seed ^ 0xC0FFEE, n_head * hd)
    dq, dp, dt = torch.from_numpy(q).to(dev), torch.from_numpy(pool).to(dev), i32(table, dev)
    out = torch.empty(n_head * hd, device=dev)
    for seq in [1, 2, 3, 15, 16, 17, 255, 256, 257, 511, 512, 513, 1000, 1024, 2047, 2048]:
        ref = orc.sdpa_decode(pool, table, bt, seq, q, n_head, n_kv, hd, True, seq - 1)
        for fn in (pa.launch, pa.launch_flash_decoding):
            fn(None, dq, dp, dt, out, n_head, n_kv, hd, bt, seq, seq - 1, True)
            torch.cuda.synchronize()
            g = out.cpu().numpy()
            assert cosine(g, ref) >= 0.9999
            check_close(g, ref, KvDataType.F32)


@pytest.mark.parametrize("dtype", [KvDataType.F16, KvDataType.BF16, KvDataType.F32])
def test_batched_decode_ragged(dev, dtype):
    rng = np.random.default_rng(21)
    n_head, n_kv, hd, bt = 12, 2, 128, 16
    lens = np.array([1, 17, 300, 0, 64, 1031, 16, 5], np.int64)
    stride = int(max((l + bt - 1) // bt for l in lens))
    nb = int(sum((l + bt - 1) // bt for l in lens)) + 7
    perm = rng.permutation(nb).astype(np.uint32)
    tab = np.full((len(lens), stride), 0xFFFFFFFF, np.uint32)
    pos = 0
    for b, l in enumerate(lens):
        c = (int(l) + bt - 1) // bt
        tab[b, :c] = perm[pos:pos + c]
        pos += c
    pool, pool_f32 = make_pool(rng, nb, bt, n_kv, hd, dtype, dev)
    q = rng.standard_normal((len(lens), n_head, hd)).astype(np.float32)
    ref = orc.sdpa_decode_batched(pool_f32, tab, lens.astype(np.uint32), bt, q, n_head, n_kv, hd)
    pa = PagedAttention(0)
    for tps in (0, 16, 64, 100, 1024):
        plan = PagedAttention.plan(len(lens), n_head, n_kv, hd, bt, int(lens.max()), tps, dtype)
        ws = PagedAttention.workspace(plan)
        out = torch.full((len(lens), n_head, hd), float("nan"), device=dev)
        pa.decode_batched(None, torch.from_numpy(q).to(dev), pool, i32(tab, dev),
                          i32(lens, dev), out, n_head, n_kv, hd, bt, dtype, plan, ws)
        torch.cuda.synchronize()
        check_close(out.cpu().numpy(), ref, dtype)


SHAPES = [  # (n_head, n_kv, head_dim, block_tokens): every slot-major head grouping,
    (8, 8, 128, 16), (16, 8, 64, 16), (6, 2, 64, 16), (4, 1, 128, 32), (8, 1, 128, 16),
    (14, 2, 128, 16), (24, 2, 128, 8), (32, 1, 64, 16), (64, 2, 128, 16), (10, 2, 64, 16),
    (12, 4, 128, 1), (12, 3, 128, 16), (12, 4, 128, 6), (8, 2, 32, 16)]  # ... and fallbacks


@pytest.mark.parametrize("dtype", [KvDataType.F16, KvDataType.BF16])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_batched_decode_head_groupings(dev, dtype, shape):
    n_head, n_kv, hd, bt = shape
    rng = np.random.default_rng(sum(shape))
    lens = np.array([0, 1, 33, 250, 700], np.int64)
    stride = int(max((l + bt - 1) // bt for l in lens))
    nb = int(sum((l + bt - 1) // bt for l in lens)) + 3
    perm = rng.permutation(nb).astype(np.uint32)
    tab = np.full((len(lens), stride), 0xFFFFFFFF, np.uint32)
    pos = 0
    for b, l in enumerate(lens):
        c = (int(l) + bt - 1) // bt
        tab[b, :c] = perm[pos:pos + c]
        pos += c
    pool, pool_f32 = make_pool(rng, nb, bt, n_kv, hd, dtype, dev)
    q = rng.standard_normal((len(lens), n_head, hd)).astype(np.float32)
    ref = orc.sdpa_decode_batched(pool_f32, tab, lens.astype(np.uint32), bt, q, n_head, n_kv, hd)
    pa = PagedAttention(0)
    for tps in (0, 128):
        plan = PagedAttention.plan(len(lens), n_head, n_kv, hd, bt, int(lens.max()), tps, dtype)
        ws = PagedAttention.workspace(plan)
        out = torch.full((len(lens), n_head, hd), float("nan"), device=dev)
        pa.decode_batched(None, torch.from_numpy(q).to(dev), pool, i32(tab, dev),
                          i32(lens, dev), out, n_head, n_kv, hd, bt, dtype, plan, ws)
        torch.cuda.synchronize()
        check_close(out.cpu().numpy(), ref, dtype)


@pytest.mark.parametrize("dtype", [KvDataType.F16, KvDataType.BF16])
def test_batched_decode_workspace_reuse(dev, dtype):
    """One workspace serves repeated calls, a smaller plan after a larger
    one, and a larger one again: nothing a call leaves in it changes the next
    call's result."""
    rng = np.random.default_rng(5)
    n_head, n_kv, hd, bt = 12, 2, 128, 16
    pa = PagedAttention(0)
    big = PagedAttention.plan(8, n_head, n_kv, hd, bt, 3000, 64, dtype)
    ws = PagedAttention.workspace(big)
    for batch, max_ctx, tps in ((8, 3000, 64), (8, 3000, 64), (3, 900, 32), (8, 3000, 128)):
        lens = rng.integers(0, max_ctx + 1, size=batch).astype(np.int64)
        lens[0] = max_ctx
        stride = (max_ctx + bt - 1) // bt
        nb = batch * stride
        tab = rng.permutation(nb).astype(np.uint32).reshape(batch, stride)
        pool, pool_f32 = make_pool(rng, nb, bt, n_kv, hd, dtype, dev)
        q = rng.standard_normal((batch, n_head, hd)).astype(np.float32)
        ref = orc.sdpa_decode_batched(pool_f32, tab, lens.astype(np.uint32), bt, q, n_head,
                                      n_kv, hd)
        plan = PagedAttention.plan(batch, n_head, n_kv, hd, bt, max_ctx, tps, dtype)
        assert plan[1] > 1 and plan[2] <= big[2]
        out = torch.full((batch, n_head, hd), float("nan"), device=dev)
        pa.decode_batched(None, torch.from_numpy(q).to(dev), pool, i32(tab, dev),
                          i32(lens, dev), out, n_head, n_kv, hd, bt, dtype, plan, ws)
        torch.cuda.synchronize()
        check_close(out.cpu().numpy(), ref, dtype)


def test_config1_append_then_decode(dev):
    """Benchmark config 1: f32, B=1, 14/2 heads, hd 64, page 16; 511 cached
    tokens + 1 appended token (512 attended) on the first 32 pages of a seeded
    permutation of a 64-page pool, N(0,1) data from seed 0."""
    s = synth.config1(0)
    rng = np.random.default_rng(0)
    rl = s.row_len
    table = s.free_order[:32].copy()
    layout = PagedKvLayout(64, 16, rl, KvDataType.F32)
    c = orc.Cache(64, 16, s.n_head_kv, s.head_dim)
    c.seed_free_list(s.free_order)
    seq = c.new_sequence()
    rows = rng.standard_normal((512, 2, rl)).astype(np.float32)
    for t in range(511):
        c.append(seq, rows[t, 0], rows[t, 1])
    pool = torch.from_numpy(c.buffer()).to(dev)
    c.append(seq, rows[511, 0], rows[511, 1])
    assert np.array_equal(c.seq_block_table(seq), table)
    q = rng.standard_normal(s.n_head * s.head_dim).astype(np.float32)
    kv, pa = PagedKvGpu(0), PagedAttention(0)
    dt = i32(table, dev)
    kv.append_kv(None, layout, pool, torch.from_numpy(rows[511, 0]).to(dev),
                 torch.from_numpy(rows[511, 1]).to(dev), dt, 511, 1)
    out = torch.empty(s.n_head * s.head_dim, device=dev)
    pa.launch_flash_decoding(None, torch.from_numpy(q).to(dev), pool, dt, out, s.n_head,
                             s.n_head_kv, s.head_dim, 16, 512, 511, True)
    torch.cuda.synchronize()
    assert np.array_equal(pool.cpu().numpy(), c.buffer())
    ref = orc.sdpa_decode(c.buffer(), table, 16, 512, q, s.n_head, s.n_head_kv, s.head_dim,
                          True, 511)
    check_close(out.cpu().numpy(), ref, KvDataType.F32)


def test_config2_one_layer_full_size(dev):
    """Benchmark config 2 at full size for one layer: 32 sequences, ctx
    U[128,4096], 12/2 heads, hd 128, f16 pool of 1.2x tokens on a shuffled
    free list; append one token per sequence, then batched decode."""
    s = synth.config2(0, extra_tokens=1)
    rng = np.random.default_rng(1)
    tab = synth.block_tables(s, extra_tokens=1)
    pool_dev, pool_f32 = make_pool(rng, s.n_blocks, 16, 2, 128, KvDataType.F16, dev)
    newk = torch.from_numpy(rng.standard_normal((32, s.row_len)).astype(np.float32)).half()
    newv = torch.from_numpy(rng.standard_normal((32, s.row_len)).astype(np.float32)).half()
    layout = PagedKvLayout(s.n_blocks, 16, s.row_len, KvDataType.F16)
    kv, pa = PagedKvGpu(0), PagedAttention(0)
    dt = i32(tab, dev)
    cu = i32(np.arange(33), dev)
    kv.append_kv_batched(None, layout, pool_dev, newk.to(dev), newv.to(dev), dt, cu,
                         i32(s.ctx_lens, dev), 32)
    lens = s.ctx_lens + 1
    q = rng.standard_normal((32, 12, 128)).astype(np.float32)
    plan = PagedAttention.plan(32, 12, 2, 128, 16, int(lens.max()))
    ws = PagedAttention.workspace(plan)
    out = torch.empty((32, 12, 128), device=dev)
    pa.decode_batched(None, torch.from_numpy(q).to(dev), pool_dev, dt, i32(lens, dev), out, 12, 2,
                      128, 16, KvDataType.F16, plan, ws)
    torch.cuda.synchronize()
    # oracle: same append on the host copy, then sdpa on the widened pool
    page = 16 * 2 * s.row_len
    p = pool_f32.reshape(-1, 16, 2, s.row_len)
    for b in range(32):
        L = int(s.ctx_lens[b])
        p[tab[b, L // 16], L % 16, 0] = newk[b].float().numpy()
        p[tab[b, L // 16], L % 16, 1] = newv[b].float().numpy()
    got_pool = pool_dev.float().cpu().numpy()
    assert np.array_equal(got_pool, pool_f32.reshape(-1))
    ref = orc.sdpa_decode_batched(pool_f32.reshape(-1), tab, lens.astype(np.uint32), 16, q, 12, 2,
                                  128)
    check_close(out.cpu().numpy(), ref, KvDataType.F16)
    del page


def test_long_context_split_covers_all_tokens(dev):
    """Config 5 shape at reduced batch: 32768 tokens, 32/8 heads, f16, 1% of
    K rows scaled x8.  The reference drops tokens >= 8192; every one counts here."""
    rng = np.random.default_rng(5)
    n_head, n_kv, hd, bt, ctx = 32, 8, 128, 16, 32768
    nb = ctx // bt + 5
    table = rng.permutation(nb)[: ctx // bt].astype(np.uint32)
    host = rng.standard_normal((nb, bt, 2, n_kv * hd)).astype(np.float32)
    hot = rng.random((nb, bt)) < 0.01
    host[:, :, 0][hot] *= 8.0
    pool16 = torch.from_numpy(host.reshape(-1)).half()
    pool_f32 = pool16.float().numpy()
    q = rng.standard_normal((1, n_head, hd)).astype(np.float32)
    ref = orc.sdpa_decode_batched(pool_f32, table[None], np.array([ctx], np.uint32), bt, q,
                                  n_head, n_kv, hd)
    pa = PagedAttention(0)
    plan = PagedAttention.plan(1, n_head, n_kv, hd, bt, ctx)
    ws = PagedAttention.workspace(plan)
    out = torch.empty((1, n_head, hd), device=dev)
    pa.decode_batched(None, torch.from_numpy(q).to(dev), pool16.to(dev), i32(table[None], dev),
                      i32(np.array([ctx]), dev), out, n_head, n_kv, hd, bt, KvDataType.F16, plan,
                      ws)
    torch.cuda.synchronize()
    check_close(out.cpu().numpy(), ref, KvDataType.F16)
    # the single-sequence split-K entry point on the same data
    out2 = torch.empty(n_head * hd, device=dev)
    pa.launch_flash_decoding(None, torch.from_numpy(q.ravel()).to(dev), pool16.to(dev),
                             i32(table, dev), out2, n_head, n_kv, hd, bt, ctx, ctx - 1, True,
                             kv_dtype=KvDataType.F16)
    torch.cuda.synchronize()
    check_close(out2.cpu().numpy(), ref.ravel(), KvDataType.F16)


def test_graph_replay_with_device_position(dev):
    """graph_dynamic_params_test.rs:19-226: append + attention captured once
    with pos_ptr, replayed for positions 0..7 against eager launches."""
    n_head, n_kv, hd, bt, nb = 4, 2, 64, 16, 4
    rl = n_kv * hd
    layout = PagedKvLayout(nb, bt, rl)
    kv, pa = PagedKvGpu(0), PagedAttention(0)
    rng = np.random.default_rng(9)
    table = i32(np.arange(nb), dev)
    pool_g = torch.zeros(layout.floats_total(), device=dev)
    pool_e = torch.zeros(layout.floats_total(), device=dev)
    k = torch.empty(rl, device=dev)
    v = torch.empty(rl, device=dev)
    q = torch.empty(n_head * hd, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    out_g = torch.empty(n_head * hd, device=dev)
    out_e = torch.empty(n_head * hd, device=dev)
    # eager warm-up resolves every kernel handle before capture
    kv.append_kv_with_pos_ptr(None, layout, pool_g, k, v, table, 0, 1, pos)
    pa.launch_flash_decoding(None, q, pool_g, table, out_g, n_head, n_kv, hd, bt, 1, 0, True, pos)
    torch.cuda.synchronize()
    pool_g.zero_()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            kv.append_kv_with_pos_ptr(s, layout, pool_g, k, v, table, 0, 1, pos)
            pa.launch_flash_decoding(s, q, pool_g, table, out_g, n_head, n_kv, hd, bt, 1, 0, True,
                                     pos)
    torch.cuda.synchronize()
    for step in range(8):
        k.copy_(torch.from_numpy(rng.standard_normal(rl).astype(np.float32)))
        v.copy_(torch.from_numpy(rng.standard_normal(rl).astype(np.float32)))
        q.copy_(torch.from_numpy(rng.standard_normal(n_head * hd).astype(np.float32)))
        pos.fill_(step)
        torch.cuda.synchronize()
        kv.append_kv(None, layout, pool_e, k, v, table, step, 1)
        pa.launch(None, q, pool_e, table, out_e, n_head, n_kv, hd, bt, step + 1, step, True)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(pool_g, pool_e)
        assert torch.max(torch.abs(out_g - out_e)).item() < 1e-5


def test_attention_validation_errors(dev):
    pa = PagedAttention(0)
    q = torch.zeros(64, device=dev)
    pool = torch.zeros(1024, device=dev)
    bt = i32(np.array([0, 1]), dev)
    out = torch.zeros(64, device=dev)
    with pytest.raises(HipError) as e:
        pa.launch(None, q, pool, bt, out, 3, 2, 16, 4, 4, 3, True)
    assert (e.value.expected, e.value.actual) == (2, 1)        # n_head % n_head_kv
    with pytest.raises(HipError) as e:
        pa.launch(None, q, pool, bt, out, 4, 2, 16, 4, 0, 0, True)
    assert (e.value.expected, e.value.actual) == (1, 0)        # seq_tokens < 1
    with pytest.raises(HipError) as e:
        pa.launch(None, q, pool, bt, out, 4, 2, 16, 4, 12, 11, True)
    assert (e.value.expected, e.value.actual) == (12, 8)       # block table too short
    with pytest.raises(HipError) as e:
        pa.launch(None, q, pool, bt, out, 4, 2, 24, 4, 4, 3, True)
    assert e.value.kind in ("InvalidSize", "Unsupported")


def test_config1_fused_step(dev):
    """Benchmark config 1 as one launch (eh_append_flash_decoding): the pool
    equals the oracle cache after the append, the output is within the f32
    bar of sdpa_decode."""
    s = synth.config1(0)
    rng = np.random.default_rng(0)
    rl = s.row_len
    table = s.free_order[:32].copy()
    c = orc.Cache(64, 16, s.n_head_kv, s.head_dim)
    c.seed_free_list(s.free_order)
    seq = c.new_sequence()
    rows = rng.standard_normal((512, 2, rl)).astype(np.float32)
    for t in range(511):
        c.append(seq, rows[t, 0], rows[t, 1])
    pool = torch.from_numpy(c.buffer()).to(dev)
    c.append(seq, rows[511, 0], rows[511, 1])
    q = rng.standard_normal(s.n_head * s.head_dim).astype(np.float32)
    out = torch.full((s.n_head * s.head_dim,), float("nan"), device=dev)
    PagedAttention(0).append_flash_decoding(None, torch.from_numpy(rows[511, 0]).to(dev),
                                            torch.from_numpy(rows[511, 1]).to(dev),
                                            torch.from_numpy(q).to(dev), pool, i32(table, dev), out,
                                            s.n_head, s.n_head_kv, s.head_dim, 16, 511)
    torch.cuda.synchronize()
    assert np.array_equal(pool.cpu().numpy(), c.buffer())
    ref = orc.sdpa_decode(c.buffer(), table, 16, 512, q, s.n_head, s.n_head_kv, s.head_dim,
                          True, 511)
    check_close(out.cpu().numpy(), ref, KvDataType.F32)


@pytest.mark.parametrize("dtype,cfg", [(KvDataType.F32, (14, 2, 64, 16)),
                                       (KvDataType.F16, (12, 2, 128, 16)),
                                       (KvDataType.BF16, (8, 8, 128, 8)),
                                       (KvDataType.F16, (4, 1, 32, 4))])
def test_fused_step_matches_append_then_decode(dev, dtype, cfg):
    """eh_append_flash_decoding equals append_kv + launch_flash_decoding:
    pool bit for bit, output within the dtype's bar of sdpa_decode, at
    positions on every slot of a page and past a page boundary, host and
    device positions."""
    n_head, n_kv, hd, bt = cfg
    rl = n_kv * hd
    rng = np.random.default_rng(hd + n_kv)
    nb = 40
    table = rng.permutation(nb).astype(np.uint32)
    td = {KvDataType.F32: torch.float32, KvDataType.F16: torch.float16,
          KvDataType.BF16: torch.bfloat16}[dtype]
    base = torch.from_numpy(rng.standard_normal(nb * bt * 2 * rl).astype(np.float32)).to(td)
    layout = PagedKvLayout(nb, bt, rl, dtype)
    kv, pa = PagedKvGpu(0), PagedAttention(0)
    dt = i32(table, dev)
    for p in (0, bt - 1, bt, 3 * bt + 2, nb * bt - 1):
        for dev_pos in (False, True):
            k = torch.from_numpy(rng.standard_normal(rl).astype(np.float32)).to(td).to(dev)
            v = torch.from_numpy(rng.standard_normal(rl).astype(np.float32)).to(td).to(dev)
            q = torch.from_numpy(rng.standard_normal(n_head * hd).astype(np.float32)).to(dev)
            pos = i32([p], dev) if dev_pos else None
            pool_a, pool_b = base.to(dev), base.to(dev)
            kv.append_kv(None, layout, pool_a, k, v, dt, p, 1)
            out_b = torch.full((n_head * hd,), float("nan"), device=dev)
            pa.append_flash_decoding(None, k, v, q, pool_b, dt, out_b, n_head, n_kv, hd, bt,
                                     0 if dev_pos else p, pos, dtype)
            torch.cuda.synchronize()
            assert torch.equal(pool_a.view(torch.uint8), pool_b.view(torch.uint8)), (p, dev_pos)
            pf = pool_a.float().cpu().numpy()
            ref = orc.sdpa_decode(pf, table, bt, p + 1, q.cpu().numpy(), n_head, n_kv, hd, True, p)
            check_close(out_b.cpu().numpy(), ref, dtype)


def test_fused_step_errors(dev):
    """eh_append_flash_decoding rejects FP8 pools, short rows and a host
    position past the block table before any launch."""
    n_head, n_kv, hd, bt, nb = 4, 2, 64, 16, 4
    rl = n_kv * hd
    pool = torch.zeros(nb * bt * 2 * rl, device=dev)
    table = i32(np.arange(nb), dev)
    k = torch.zeros(rl, device=dev)
    q = torch.zeros(n_head * hd, device=dev)
    out = torch.empty_like(q)
    pa = PagedAttention(0)
    with pytest.raises(HipError):       # rows shorter than row_len
        pa.append_flash_decoding(None, k[:rl - 4], k, q, pool, table, out, n_head, n_kv, hd, bt, 3)
    with pytest.raises(HipError):       # position 64 needs a fifth page
        pa.append_flash_decoding(None, k, k, q, pool, table, out, n_head, n_kv, hd, bt, nb * bt)
    with pytest.raises(HipError):       # FP8 pools: the scale-aware entries only
        pa.append_flash_decoding(None, k, k, q, pool, table, out, n_head, n_kv, hd, bt, 3,
                                 kv_dtype=KvDataType.FP8)
    pa.append_flash_decoding(None, k, k, q, pool, table, out, n_head, n_kv, hd, bt, nb * bt - 1)
    torch.cuda.synchronize()
    assert torch.all(torch.isfinite(out))


@pytest.mark.parametrize("case", ["none_entry", "past_pool", "past_table"])
def test_fused_step_masked_page_device_position(dev, case):
    """eh_append_flash_decoding with a device position whose page is masked
    (table entry 0xFFFFFFFF, a page id past the pool, or a position past the
    table): EH_OK, the pool is unchanged, and q attends the tokens 0..pos that
    sit on valid pages."""
    n_head, n_kv, hd, bt = 12, 2, 128, 16
    rl = n_kv * hd
    rng = np.random.default_rng(41)
    nb = 6
    table = rng.permutation(nb)[:4].astype(np.uint32)
    pos = {"none_entry": 40, "past_pool": 20, "past_table": 64}[case]
    if case == "none_entry":
        table[2] = 0xFFFFFFFF
    elif case == "past_pool":
        table[1] = nb + 3
    base = rng.standard_normal(nb * bt * 2 * rl).astype(np.float32)
    pool = torch.from_numpy(base).half().to(dev)
    pool_f32 = torch.from_numpy(base).half().float().numpy()
    before = pool.clone()
    k = torch.from_numpy(rng.standard_normal(rl).astype(np.float32)).half().to(dev)
    v = torch.from_numpy(rng.standard_normal(rl).astype(np.float32)).half().to(dev)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    out = torch.full((n_head * hd,), float("nan"), device=dev)
    PagedAttention(0).append_flash_decoding(None, k, v, torch.from_numpy(q).to(dev), pool,
                                            i32(table, dev), out, n_head, n_kv, hd, bt, 0,
                                            i32([pos], dev), KvDataType.F16)
    torch.cuda.synchronize()
    assert torch.equal(pool.view(torch.int16), before.view(torch.int16)), "row written"
    valid = [j for j in range(pos // bt + 1) if j < len(table) and table[j] < nb]
    assert valid == list(range(len(valid))), "masked pages are the trailing ones"
    n = min(pos + 1, bt * len(valid))
    ref = orc.sdpa_decode(pool_f32, table[:len(valid)], bt, n, q, n_head, n_kv, hd, True, n - 1)
    check_close(out.cpu().numpy(), ref, KvDataType.F16)


def test_single_sequence_calls_with_own_workspace(dev):
    """The _ws forms of eh_paged_attention / eh_flash_decoding /
    eh_append_flash_decoding: with a workspace of the context scratch's size
    they equal the shared-scratch calls bit for bit; with a smaller one the
    split grows and the result stays within the bar of the oracle; a
    workspace too small for the longest split is InvalidSize naming the
    least that fits; calls on two streams with their own workspaces overlap
    and both match the oracle."""
    n_head, n_kv, hd, bt = 12, 2, 128, 16
    rl = n_kv * hd
    rng = np.random.default_rng(57)
    n = 20000
    nb = n // bt + 8
    table = rng.permutation(nb)[:n // bt + 1].astype(np.uint32)
    base = rng.standard_normal(nb * bt * 2 * rl).astype(np.float32)
    pool = torch.from_numpy(base).half().to(dev)
    pf = torch.from_numpy(base).half().float().numpy()
    dt = i32(table, dev)
    pa = PagedAttention(0)
    full = torch.empty(PagedAttention.single_workspace_bytes() // 4, device=dev)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    dq = torch.from_numpy(q).to(dev)
    ref = orc.sdpa_decode(pf, table, bt, n, q, n_head, n_kv, hd, True, n - 1)
    for call in ("launch_flash_decoding", "launch_with_pos_ptr"):
        a = torch.empty(n_head * hd, device=dev)
        b = torch.empty_like(a)
        args = (None, dq, pool, dt)
        tail = (n_head, n_kv, hd, bt, n, n - 1, True)
        if call == "launch_flash_decoding":
            pa.launch_flash_decoding(*args, a, *tail, kv_dtype=KvDataType.F16)
            pa.launch_flash_decoding(*args, b, *tail, kv_dtype=KvDataType.F16, workspace=full)
        else:
            pa.launch_with_pos_ptr(*args, a, *tail, None, KvDataType.F16)
            pa.launch_with_pos_ptr(*args, b, *tail, None, KvDataType.F16, workspace=full)
        torch.cuda.synchronize()
        assert torch.equal(a.view(torch.int32), b.view(torch.int32)), call
        check_close(b.cpu().numpy(), ref, KvDataType.F16, call + " _ws")
    # a small workspace: longer splits, same result within the bar
    small = torch.empty(12 * 1024, device=dev)
    c = torch.empty(n_head * hd, device=dev)
    pa.launch_flash_decoding(None, dq, pool, dt, c, n_head, n_kv, hd, bt, n, n - 1, True,
                             kv_dtype=KvDataType.F16, workspace=small)
    torch.cuda.synchronize()
    check_close(c.cpu().numpy(), ref, KvDataType.F16, "flash_decoding small workspace")
    with pytest.raises(HipError) as e:
        pa.launch_flash_decoding(None, dq, pool, dt, c, n_head, n_kv, hd, bt, n, n - 1, True,
                                 kv_dtype=KvDataType.F16, workspace=torch.empty(16, device=dev))
    assert e.value.kind == "InvalidSize" and e.value.actual == 64 and e.value.expected > 64
    # no workspace at all (null, 0 bytes): a context that one pass covers needs
    # no partials; a longer one is InvalidSize
    short = 300
    a1 = torch.empty(n_head * hd, device=dev)
    pa.launch_with_pos_ptr(None, dq, pool, dt, a1, n_head, n_kv, hd, bt, short, short - 1, True,
                           None, KvDataType.F16, workspace=(0, 0))
    torch.cuda.synchronize()
    ref_s = orc.sdpa_decode(pf, table, bt, short, q, n_head, n_kv, hd, True, short - 1)
    check_close(a1.cpu().numpy(), ref_s, KvDataType.F16, "single pass, no workspace")
    with pytest.raises(HipError) as e:
        pa.launch_flash_decoding(None, dq, pool, dt, c, n_head, n_kv, hd, bt, n, n - 1, True,
                                 kv_dtype=KvDataType.F16, workspace=(0, 0))
    assert e.value.kind == "InvalidSize" and e.value.actual == 0
    # the fused step: same pool bytes and output with and without a workspace
    p0, p1 = pool.clone(), pool.clone()
    k = torch.from_numpy(rng.standard_normal(rl).astype(np.float32)).half().to(dev)
    v = torch.from_numpy(rng.standard_normal(rl).astype(np.float32)).half().to(dev)
    o0, o1 = torch.empty(n_head * hd, device=dev), torch.empty(n_head * hd, device=dev)
    pa.append_flash_decoding(None, k, v, dq, p0, dt, o0, n_head, n_kv, hd, bt, n, None,
                             KvDataType.F16)
    pa.append_flash_decoding(None, k, v, dq, p1, dt, o1, n_head, n_kv, hd, bt, n, None,
                             KvDataType.F16, workspace=full)
    torch.cuda.synchronize()
    assert torch.equal(p0.view(torch.int16), p1.view(torch.int16))
    assert torch.equal(o0.view(torch.int32), o1.view(torch.int32))
    # two streams, one workspace each, no synchronisation between the calls
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    w1, w2 = torch.empty_like(full), torch.empty_like(full)
    q2 = rng.standard_normal(n_head * hd).astype(np.float32)
    dq2 = torch.from_numpy(q2).to(dev)
    r1, r2 = torch.empty(n_head * hd, device=dev), torch.empty(n_head * hd, device=dev)
    torch.cuda.synchronize()
    for _ in range(3):
        pa.launch_flash_decoding(s1, dq, pool, dt, r1, n_head, n_kv, hd, bt, n, n - 1, True,
                                 kv_dtype=KvDataType.F16, workspace=w1)
        pa.launch_flash_decoding(s2, dq2, pool, dt, r2, n_head, n_kv, hd, bt, n - 1000, n - 1001,
                                 True, kv_dtype=KvDataType.F16, workspace=w2)
    torch.cuda.synchronize()
    check_close(r1.cpu().numpy(), ref, KvDataType.F16, "stream 1")
    ref2 = orc.sdpa_decode(pf, table, bt, n - 1000, q2, n_head, n_kv, hd, True, n - 1001)
    check_close(r2.cpu().numpy(), ref2, KvDataType.F16, "stream 2")


def test_graph_replay_split_count_follows_device_position(dev):
    """The reference sizes its split grid on the host from seq_tokens and
    freezes it at capture (forward_driver.rs:2230-2243), and drops tokens
    past 8192 (paged_attention.cu:244-247).  Here append(pos_ptr) +
    flash_decoding(pos_ptr) are captured once over a 12288-token block table
    and replayed at device positions that cross split boundaries and 8192;
    every replay must equal sdpa_decode over tokens 0..pos (f32, 1e-5) and
    write its row (graph_dynamic_params_test.rs:17-229 pattern)."""
    n_head, n_kv, hd, bt, cap = 14, 2, 64, 16, 12288
    rl = n_kv * hd
    n_pages = cap // bt
    nb = n_pages + 5
    rng = np.random.default_rng(8192)
    table_h = rng.permutation(nb)[:n_pages].astype(np.uint32)
    layout = PagedKvLayout(nb, bt, rl)
    host = rng.standard_normal(layout.floats_total()).astype(np.float32)
    pool = torch.from_numpy(host).to(dev)
    table = i32(table_h, dev)
    kv, pa = PagedKvGpu(0), PagedAttention(0)
    k = torch.empty(rl, device=dev)
    v = torch.empty(rl, device=dev)
    q = torch.empty(n_head * hd, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    out = torch.empty(n_head * hd, device=dev)
    kv.append_kv_with_pos_ptr(None, layout, pool, k, v, table, 0, 1, pos)   # warm-up
    pa.launch_flash_decoding(None, q, pool, table, out, n_head, n_kv, hd, bt, 1, 0, True, pos)
    torch.cuda.synchronize()
    pool.copy_(torch.from_numpy(host))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            kv.append_kv_with_pos_ptr(s, layout, pool, k, v, table, 0, 1, pos)
            pa.launch_flash_decoding(s, q, pool, table, out, n_head, n_kv, hd, bt, 1, 0, True,
                                     pos)
    torch.cuda.synchronize()
    page = bt * 2 * rl
    for p in (0, 255, 256, 4095, 8191, 8192, 12287, 100):
        kn = rng.standard_normal(rl).astype(np.float32)
        vn = rng.standard_normal(rl).astype(np.float32)
        qn = rng.standard_normal(n_head * hd).astype(np.float32)
        k.copy_(torch.from_numpy(kn))
        v.copy_(torch.from_numpy(vn))
        q.copy_(torch.from_numpy(qn))
        pos.fill_(p)
        torch.cuda.synchronize()
        print(f"[replay] position {p}", flush=True)
        g.replay()
        torch.cuda.synchronize()
        base = int(table_h[p // bt]) * page + (p % bt) * 2 * rl
        host[base:base + rl] = kn
        host[base + rl:base + 2 * rl] = vn
        assert np.array_equal(pool.cpu().numpy(), host), f"pool after replay at {p}"
        ref = orc.sdpa_decode(host, table_h, bt, p + 1, qn, n_head, n_kv, hd, True, p)
        check_close(out.cpu().numpy(), ref, KvDataType.F32, what=f"replay pos {p}")
