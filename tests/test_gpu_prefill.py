"""GPU parity of the MFMA causal chunked prefill against the oracle.

The oracle's prefill_causal restates the reference's causal window
(flash_attention_2.cu:44-68: query i at p0+i attends keys 0..=p0+i) with the
f64 sdpa of forward_cpu.rs:424-510, on the exactly widened f32 pool.
Tolerances: f32 KV max-abs 1e-5; f16 and bf16 KV max-abs <= 2e-3 and |gpu - ref| <= 2e-3 +
1e-3*|ref|.  Operands: f16 pages run f16 MFMAs with q as hi + lo f16 halves
for the scores and P one f16; bf16 pages are widened to f16 as they are
staged (exact below 2^16) and take the same path, and a tile holding a bf16
value of magnitude 2^16 or more is re-staged raw and run on bf16 MFMAs with q
and P as hi + lo bf16 pairs.  Shapes: the
reference's own FA2 test (flash_attention_parity.rs:45-207), ragged chunks on
scattered pages, GQA groups 1..8, both compiled head sizes, benchmark
config 3 (sampled rows at full size), a whole 8192-token prompt in one chunk,
and one captured graph replayed over successive chunks.
"""
import numpy as np
import pytest
import torch

from oracle import orc
from titan_amd import HipError, KvDataType, PagedKvGpu, PagedKvLayout
from titan_amd.flash_attention import FlashAttention2

import parity
from e4m3_data import all_codes, gauss_codes

pytestmark = pytest.mark.gpu

TD = {KvDataType.F32: torch.float32, KvDataType.F16: torch.float16,
      KvDataType.BF16: torch.bfloat16}


def i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(dev)


def check_close(gpu, ref, dtype, what="", stress=False):
    parity.check_close(gpu, ref, f32=dtype == KvDataType.F32,
                       what=what or KvDataType(dtype).name, stress=stress)


def cosine(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return a @ b / (np.linalg.norm(a) * np.linalg.norm(b))


def make_pool(rng, n_blocks, bt, n_kv, hd, dtype, dev):
    host = rng.standard_normal(n_blocks * bt * 2 * n_kv * hd).astype(np.float32)
    t = torch.from_numpy(host).to(TD[dtype])
    return t.to(dev), t.to(torch.float32).numpy()


@pytest.mark.parametrize("seq_tokens", [1, 4, 16, 64, 128])
def test_fa2_reference_shapes(dev, seq_tokens):
    # flash_attention_parity.rs:45-207: 16/2 heads, hd 128, page 64, pool of 4
    # pages mapped 0..3, K/V appended through PagedKvGpu, pos_offset 0.
    nh, nkv, hd, bt = 16, 2, 128, 64
    layout = PagedKvLayout(4, bt, nkv * hd, KvDataType.F32)
    pool = torch.zeros(layout.floats_total(), device=dev)
    table = np.arange(4, dtype=np.uint32)
    t = np.arange(seq_tokens)[:, None, None]
    kvh = np.arange(nkv)[None, :, None]
    hq = np.arange(nh)[None, :, None]
    d = np.arange(hd)[None, None, :]
    keys = (np.sin(((t * 100 + kvh * 10 + d).astype(np.float32) * np.float32(0.013)))
            * np.float32(0.5)).astype(np.float32)
    vals = (np.cos(((t * 100 + kvh * 10 + d).astype(np.float32) * np.float32(0.017)))
            * np.float32(0.5)).astype(np.float32)
    q = (np.sin(((t * 50 + hq * 5 + d).astype(np.float32) * np.float32(0.019)))
         * np.float32(0.5)).astype(np.float32)
    PagedKvGpu(0).append_kv(None, layout, pool, torch.from_numpy(keys.reshape(seq_tokens, -1)).to(dev),
                            torch.from_numpy(vals.reshape(seq_tokens, -1)).to(dev), i32(table, dev),
                            0, seq_tokens)
    out = torch.empty((seq_tokens, nh, hd), device=dev)
    FlashAttention2(0).launch(None, torch.from_numpy(q).to(dev), pool, i32(table, dev), out, nh,
                              nkv, hd, bt, seq_tokens, 0)
    torch.cuda.synchronize()
    ref = orc.prefill_causal(pool.cpu().numpy(), table, bt, q, seq_tokens, 0, nh, nkv, hd)
    g = out.cpu().numpy()
    for qp in range(seq_tokens):
        for h in range(nh):
            assert cosine(g[qp, h], ref[qp, h]) >= 0.9999
    check_close(g, ref, KvDataType.F32)


CASES = [
    # (dtype, n_head, n_kv, hd, bt, pos_offset, q_tokens)
    (KvDataType.F32, 8, 2, 128, 16, 0, 1),
    (KvDataType.F32, 8, 8, 64, 16, 37, 45),
    (KvDataType.F32, 14, 2, 64, 16, 511, 1),
    (KvDataType.F32, 32, 4, 128, 16, 100, 70),
    (KvDataType.F16, 12, 2, 128, 16, 0, 1),
    (KvDataType.F16, 12, 2, 128, 16, 3, 5),
    (KvDataType.F16, 32, 8, 128, 16, 300, 200),
    (KvDataType.F16, 8, 1, 64, 32, 1000, 33),
    (KvDataType.F16, 7, 7, 128, 8, 65, 130),
    (KvDataType.BF16, 32, 8, 128, 16, 0, 1),
    (KvDataType.BF16, 32, 8, 128, 16, 2, 14),
    (KvDataType.BF16, 32, 8, 128, 16, 500, 300),
    (KvDataType.BF16, 16, 2, 64, 16, 64, 64),
    (KvDataType.BF16, 4, 4, 128, 1, 20, 31),
    (KvDataType.BF16, 12, 4, 128, 6, 90, 77),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0].name}-{c[1]}x{c[2]}-hd{c[3]}"
                         f"-bt{c[4]}-p{c[5]}-q{c[6]}")
def test_chunk_on_scattered_context(dev, case):
    dtype, nh, nkv, hd, bt, p0, nq = case
    rng = np.random.default_rng(1000 + CASES.index(case))
    total = p0 + nq
    n_pages = -(-total // bt)
    pool_pages = n_pages + 5
    table = rng.permutation(pool_pages)[:n_pages].astype(np.uint32)
    dpool, hpool = make_pool(rng, pool_pages, bt, nkv, hd, dtype, dev)
    q = rng.standard_normal((nq, nh, hd)).astype(np.float32)
    out = torch.full((nq, nh, hd), float("nan"), device=dev)
    FlashAttention2(0).launch(None, torch.from_numpy(q).to(dev), dpool, i32(table, dev), out, nh,
                              nkv, hd, bt, nq, p0, kv_dtype=dtype)
    torch.cuda.synchronize()
    ref = orc.prefill_causal(hpool, table, bt, q, nq, p0, nh, nkv, hd)
    check_close(out.cpu().numpy(), ref, dtype, str(case))


@pytest.mark.parametrize("hd,nh,nkv", [(128, 32, 8), (64, 16, 2)])
def test_bf16_values_beyond_f16_range(dev, hd, nh, nkv):
    """bf16 pages are staged as f16 (exact below 2^16); a tile holding a finite
    value of magnitude >= 2^16 takes the exact bf16 path.  Large V values in
    some tiles, a large K value in another (its key then dominates the
    softmax), normal tiles around them: every row against the oracle."""
    bt, p0, nq = 16, 700, 140
    rng = np.random.default_rng(4242 + hd)
    total = p0 + nq
    n_pages = -(-total // bt)
    pool_pages = n_pages + 5
    table = rng.permutation(pool_pages)[:n_pages].astype(np.uint32)
    host = rng.standard_normal((pool_pages, bt, 2, nkv, hd)).astype(np.float32)
    # V values beyond f16's range on the page holding keys 64.. (first tile)
    host[table[4], 3, 1, 0, :8] = [7.0e4, -3.1e5, 1.0e6, 65536.0, -65536.0, 2.5e7, 9.0e4, -7.0e4]
    # a K value beyond f16's range on the page holding keys 512..
    host[table[32], 5, 0, nkv - 1, 3] = 1.2e5
    # near the limit but in range (65280 is the largest bf16 below 2^16): f16 path
    host[table[20], 0, 1, 0, :2] = [65280.0, -65280.0]
    t = torch.from_numpy(host.reshape(-1)).to(torch.bfloat16)
    dpool, hpool = t.to(dev), t.to(torch.float32).numpy()
    q = rng.standard_normal((nq, nh, hd)).astype(np.float32)
    out = torch.full((nq, nh, hd), float("nan"), device=dev)
    FlashAttention2(0).launch(None, torch.from_numpy(q).to(dev), dpool, i32(table, dev), out, nh,
                              nkv, hd, bt, nq, p0, kv_dtype=KvDataType.BF16)
    torch.cuda.synchronize()
    ref = orc.prefill_causal(hpool, table, bt, q, nq, p0, nh, nkv, hd)
    g = out.cpu().numpy()
    assert np.abs(ref).max() > 1e3                       # the large values reach the output
    check_close(g, ref, KvDataType.BF16, "bf16 beyond f16 range", stress=True)


@pytest.mark.parametrize("which", ["k", "v"])
def test_bf16_late_tile_beyond_f16_range(dev, monkeypatch, which):
    """One bf16 value of magnitude >= 2^16 in the K (or V) rows of a late tile
    only: the ping-pong kernel stages K and V on different halves of the
    workgroup, so each half's range flag is met mid-run, after many tiles on
    the f16 path; every workgroup then restarts on the exact path.  Against
    the oracle and bit-identical to the single-phase kernel."""
    nh, nkv, hd, bt, p0, nq = 32, 8, 128, 16, 1500, 200
    rng = np.random.default_rng(515 + (which == "v"))
    total = p0 + nq
    n_pages = -(-total // bt)
    pool_pages = n_pages + 3
    table = rng.permutation(pool_pages)[:n_pages].astype(np.uint32)
    host = rng.standard_normal((pool_pages, bt, 2, nkv, hd)).astype(np.float32)
    page = table[1400 // bt]  # key 1400 + slot: tile 21 of 27
    host[page, 7, 0 if which == "k" else 1, 3, 5] = -2.0e5 if which == "k" else 7.5e4
    t = torch.from_numpy(host.reshape(-1)).to(torch.bfloat16)
    dpool, hpool = t.to(dev), t.to(torch.float32).numpy()
    q = rng.standard_normal((nq, nh, hd)).astype(np.float32)
    outs = {}
    for kern in ("single", "pp"):
        monkeypatch.setenv("EH_PREFILL_KERNEL", kern)
        out = torch.full((nq, nh, hd), float("nan"), device=dev)
        FlashAttention2(0).launch(None, torch.from_numpy(q).to(dev), dpool, i32(table, dev), out,
                                  nh, nkv, hd, bt, nq, p0, kv_dtype=KvDataType.BF16)
        torch.cuda.synchronize()
        outs[kern] = out.cpu().numpy()
    assert np.array_equal(outs["pp"].view(np.uint32), outs["single"].view(np.uint32))
    ref = orc.prefill_causal(hpool, table, bt, q, nq, p0, nh, nkv, hd)
    assert np.abs(ref).max() > (100.0 if which == "v" else 0.0)  # the large V value reaches the output
    check_close(outs["pp"], ref, KvDataType.BF16, f"bf16 late {which}", stress=which == "v")


@pytest.mark.parametrize("kstd", [4.0, 16.0, 64.0])
@pytest.mark.parametrize("dtype", [KvDataType.F16, KvDataType.BF16])
def test_large_keys_within_f16_range(dev, dtype, kstd):
    """K of standard deviation 4-64 (every value inside f16's range, so bf16
    pages take the f16-staged path) with N(0,1) q and V, under the strict
    bar.  The score error of the f16 operands grows with |K|: q rounded once
    to f16 reaches 7e-3 at a K deviation of 16; q as hi + lo halves keeps
    every case near 5e-4."""
    nh, nkv, hd, bt, p0, nq = 32, 8, 128, 16, 900, 160
    rng = np.random.default_rng(77 + int(kstd) + 1000 * int(dtype))
    total = p0 + nq
    n_pages = -(-total // bt)
    pool_pages = n_pages + 3
    table = rng.permutation(pool_pages)[:n_pages].astype(np.uint32)
    host = rng.standard_normal((pool_pages, bt, 2, nkv, hd)).astype(np.float32)
    host[:, :, 0] *= np.float32(kstd)
    t = torch.from_numpy(host.reshape(-1)).to(TD[dtype])
    dpool, hpool = t.to(dev), t.to(torch.float32).numpy()
    assert np.abs(hpool).max() < 65504.0
    q = rng.standard_normal((nq, nh, hd)).astype(np.float32)
    out = torch.full((nq, nh, hd), float("nan"), device=dev)
    FlashAttention2(0).launch(None, torch.from_numpy(q).to(dev), dpool, i32(table, dev), out, nh,
                              nkv, hd, bt, nq, p0, kv_dtype=dtype)
    torch.cuda.synchronize()
    ref = orc.prefill_causal(hpool, table, bt, q, nq, p0, nh, nkv, hd)
    check_close(out.cpu().numpy(), ref, dtype, f"{dtype.name} K std {kstd:g}")


def test_pos_ptr_overrides_offset(dev):
    # flash_attention_2.cu:43: a device position replaces the host pos_offset.
    dtype, nh, nkv, hd, bt = KvDataType.F16, 8, 2, 128, 16
    rng = np.random.default_rng(7)
    table = rng.permutation(40).astype(np.uint32)
    dpool, hpool = make_pool(rng, 40, bt, nkv, hd, dtype, dev)
    nq = 24
    q = rng.standard_normal((nq, nh, hd)).astype(np.float32)
    fa = FlashAttention2(0)
    dq, dt = torch.from_numpy(q).to(dev), i32(table, dev)
    for pos in (0, 17, 200, 40 * bt - nq):
        pos_t = torch.tensor([pos], dtype=torch.int32, device=dev)
        out = torch.empty((nq, nh, hd), device=dev)
        fa.launch_with_pos_ptr(None, dq, dpool, dt, out, nh, nkv, hd, bt, nq, 0, pos_t,
                               kv_dtype=dtype)
        torch.cuda.synchronize()
        ref = orc.prefill_causal(hpool, table, bt, q, nq, pos, nh, nkv, hd)
        check_close(out.cpu().numpy(), ref, dtype, f"pos {pos}")


@pytest.mark.parametrize("dtype", [KvDataType.F16, KvDataType.BF16, KvDataType.F32])
def test_batched_ragged_chunks(dev, dtype):
    nh, nkv, hd, bt = 16, 4, 128, 16
    rng = np.random.default_rng(11 + int(dtype))
    starts = [0, 5, 130, 1000]
    lens = [33, 1, 200, 64]
    stride = max(-(-(s + n) // bt) for s, n in zip(starts, lens)) + 2
    n_pages = sum(-(-(s + n) // bt) for s, n in zip(starts, lens)) + 3
    perm = rng.permutation(n_pages).astype(np.uint32)
    tables = np.full((len(starts), stride), 0xFFFFFFFF, np.uint32)
    o = 0
    for b, (s, n) in enumerate(zip(starts, lens)):
        k = -(-(s + n) // bt)
        tables[b, :k] = perm[o:o + k]
        o += k
    dpool, hpool = make_pool(rng, n_pages, bt, nkv, hd, dtype, dev)
    total = sum(lens)
    q = rng.standard_normal((total, nh, hd)).astype(np.float32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    out = torch.full((total, nh, hd), float("nan"), device=dev)
    FlashAttention2(0).launch_batched(None, torch.from_numpy(q).to(dev), dpool, i32(tables, dev),
                                      i32(cu, dev), i32(np.array(starts, np.uint32), dev), out,
                                      nh, nkv, hd, bt, max(lens), kv_dtype=dtype)
    torch.cuda.synchronize()
    g = out.cpu().numpy()
    for b, (s, n) in enumerate(zip(starts, lens)):
        k = -(-(s + n) // bt)
        ref = orc.prefill_causal(hpool, tables[b, :k], bt, q[cu[b]:cu[b + 1]], n, s, nh, nkv, hd)
        check_close(g[cu[b]:cu[b + 1]], ref, dtype, f"seq {b}")


PP_CASES = [
    # (dtype, n_head, n_kv, hd, bt, starts, lens)
    (KvDataType.BF16, 32, 8, 128, 16, [2048, 0, 700], [512, 300, 129]),
    (KvDataType.F16, 32, 8, 128, 16, [2048, 0, 700], [512, 300, 129]),
    (KvDataType.FP8, 32, 8, 128, 16, [2048, 0, 700], [512, 300, 129]),
    (KvDataType.BF16, 16, 2, 64, 8, [0, 5, 1000], [33, 1, 260]),
    (KvDataType.F16, 12, 4, 128, 4, [90, 3], [77, 140]),
]


@pytest.mark.parametrize("case", PP_CASES, ids=lambda c: f"{c[0].name}-{c[1]}x{c[2]}-hd{c[3]}-bt{c[4]}")
def test_pingpong_matches_single_phase(dev, monkeypatch, case):
    """The two prefill kernels (eh_prefill_pp_*: the workgroup's halves take
    turns at MFMAs and softmax; eh_prefill_*: every wave does both) compute the
    same products in the same order per accumulator: outputs bit-identical on
    ragged chunks over scattered pages, with one table entry pointing outside
    the pool (its keys masked), for every page type the ping-pong kernel
    takes; and the ping-pong output against the oracle."""
    dtype, nh, nkv, hd, bt, starts, lens = case
    rng = np.random.default_rng(77 + PP_CASES.index(case))
    stride = max(-(-(s + n) // bt) for s, n in zip(starts, lens)) + 1
    n_pages = sum(-(-(s + n) // bt) for s, n in zip(starts, lens)) + 3
    perm = rng.permutation(n_pages).astype(np.uint32)
    tables = np.full((len(starts), stride), 0xFFFFFFFF, np.uint32)
    o = 0
    for b, (s0, n) in enumerate(zip(starts, lens)):
        k = -(-(s0 + n) // bt)
        tables[b, :k] = perm[o:o + k]
        o += k
    tables[0, 3] = n_pages + 7  # outside the pool: masked by both kernels
    total = sum(lens)
    q = rng.standard_normal((total, nh, hd)).astype(np.float32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    fa = FlashAttention2(0)
    if dtype == KvDataType.FP8:
        codes, ks, vs = gauss_codes(rng, n_pages, bt, nkv, hd)
        dpool = torch.from_numpy(codes).to(dev)
        f = orc.e4m3_to_f32(codes).reshape(n_pages, bt, 2, nkv, hd)
        f[:, :, 0] *= ks[None, None, :, None]
        f[:, :, 1] *= vs[None, None, :, None]
        hpool = f.reshape(-1)
        dks, dvs = torch.from_numpy(ks).to(dev), torch.from_numpy(vs).to(dev)
    else:
        dpool, hpool = make_pool(rng, n_pages, bt, nkv, hd, dtype, dev)
    outs = {}
    for kern in ("single", "pp"):
        monkeypatch.setenv("EH_PREFILL_KERNEL", kern)
        out = torch.full((total, nh, hd), float("nan"), device=dev)
        args = (None, torch.from_numpy(q).to(dev), dpool, i32(tables, dev), i32(cu, dev),
                i32(np.array(starts, np.uint32), dev), out, nh, nkv, hd, bt, max(lens))
        if dtype == KvDataType.FP8:
            fa.launch_batched_e4m3(*args, dks, dvs)
        else:
            fa.launch_batched(*args, kv_dtype=dtype)
        torch.cuda.synchronize()
        outs[kern] = out.cpu().numpy()
    if hd == 128:  # both kernels walk 64-key tiles: one running-max update per tile each
        assert np.array_equal(outs["pp"].view(np.uint32), outs["single"].view(np.uint32))
    else:  # head_dim 64: the single-phase kernel's tiles hold 128 keys, so the
        # lazy rescale points differ; both within the bar of each other
        check_close(outs["pp"], outs["single"], KvDataType.F16, "pp vs single-phase")
    # the oracle reads every table entry: sequences 1.. (sequence 0 holds the
    # masked entry, pinned above by bit identity and by test_invalid_pages_are_masked)
    for b, (s0, n) in enumerate(zip(starts, lens)):
        if b == 0:
            continue
        k = -(-(s0 + n) // bt)
        ref = orc.prefill_causal(hpool, tables[b, :k], bt, q[cu[b]:cu[b + 1]], n, s0, nh, nkv, hd)
        check_close(outs["pp"][cu[b]:cu[b + 1]], ref,
                    KvDataType.F16 if dtype == KvDataType.FP8 else dtype, f"pp seq {b}")


def test_invalid_pages_are_masked(dev):
    # Entries past the pool mask their keys: the result equals attention over
    # the remaining keys (a sequence whose first page is invalid).
    dtype, nh, nkv, hd, bt = KvDataType.F16, 4, 1, 64, 16
    rng = np.random.default_rng(5)
    dpool, hpool = make_pool(rng, 8, bt, nkv, hd, dtype, dev)
    table = np.array([0xFFFFFF, 3, 5], np.uint32)
    nq, p0 = 8, 40
    q = rng.standard_normal((nq, nh, hd)).astype(np.float32)
    out = torch.empty((nq, nh, hd), device=dev)
    FlashAttention2(0).launch(None, torch.from_numpy(q).to(dev), dpool, i32(table, dev), out, nh,
                              nkv, hd, bt, nq, p0, kv_dtype=dtype)
    torch.cuda.synchronize()
    # Masking page 0's keys equals attention over keys bt..p0+i, i.e. the
    # oracle's prefill over the table without its first entry, bt earlier.
    ref = orc.prefill_causal(hpool, table[1:], bt, q, nq, p0 - bt, nh, nkv, hd)
    check_close(out.cpu().numpy(), ref, dtype, "masked first page")


def test_config3_sampled_rows(dev):
    """Benchmark config 3 at full size: 8 sequences each append a 512-token
    chunk onto 2048 cached tokens (32/8 heads, hd 128, page 16, bf16 KV) and
    run causal prefill over the chunk.  The append is checked bit-exactly by
    gathering the chunk back; attention is checked on 96 sampled query rows
    against the oracle (full-size oracle runs take minutes)."""
    from titan_amd import synth
    dtype, B, nh, nkv, hd, bt = KvDataType.BF16, 8, 32, 8, 128, 16
    shape = synth.config3(0)
    assert (shape.batch, shape.n_head, shape.n_head_kv, shape.head_dim) == (B, nh, nkv, hd)
    rl = nkv * hd
    rng = np.random.default_rng(3)
    tables = synth.block_tables(shape, extra_tokens=512)
    layout = PagedKvLayout(shape.n_blocks, bt, rl, dtype)
    dpool, _ = make_pool(rng, shape.n_blocks, bt, nkv, hd, dtype, dev)
    newk = torch.randn((B * 512, rl), device=dev).to(torch.bfloat16)
    newv = torch.randn((B * 512, rl), device=dev).to(torch.bfloat16)
    cu = np.arange(0, B * 512 + 1, 512, dtype=np.uint32)
    starts = np.full(B, 2048, np.uint32)
    dtab, dcu, dst = i32(tables, dev), i32(cu, dev), i32(starts, dev)
    PagedKvGpu(0).append_kv_batched(None, layout, dpool, newk, newv, dtab, dcu, dst, B * 512)
    q = torch.randn((B * 512, nh, hd), device=dev)
    out = torch.empty_like(q)
    FlashAttention2(0).launch_batched(None, q, dpool, dtab, dcu, dst, out, nh, nkv, hd, bt, 512,
                                      kv_dtype=dtype)
    torch.cuda.synchronize()
    hpool = dpool.to(torch.float32).cpu().numpy()
    # append bit-exactness: the chunk read back through the tables
    kv = PagedKvGpu(0)
    for b in (0, B - 1):
        got = torch.empty((512, rl), device=dev, dtype=torch.bfloat16)
        kv.read_keys(None, layout, dpool, dtab[b], got, 2048, 512)
        torch.cuda.synchronize()
        assert torch.equal(got.cpu(), newk[b * 512:(b + 1) * 512].cpu())
    g = out.cpu().numpy()
    hq = q.cpu().numpy()
    picks = np.random.default_rng(9).integers(0, B * 512, size=96)
    for r in np.concatenate([[0, 511, 512 * 7 + 511], picks]):
        b, i = divmod(int(r), 512)
        ref = orc.prefill_causal(hpool, tables[b], bt, hq[r:r + 1], 1, 2048 + i, nh, nkv, hd)
        check_close(g[r:r + 1], ref, dtype, f"row {r}")


def test_validation_errors(dev):
    fa = FlashAttention2(0)
    q = torch.zeros((4, 8, 128), device=dev)
    out = torch.zeros_like(q)
    pool = torch.zeros(16 * 2 * 2 * 128 * 4, device=dev)
    table = torch.zeros(1, dtype=torch.int32, device=dev)
    with pytest.raises(HipError) as e:
        fa.launch(None, q[:2], pool, table, out, 8, 2, 128, 16, 4, 0)
    assert e.value.kind == "InvalidSize" and e.value.expected == 4 * 8 * 128 * 4
    with pytest.raises(HipError) as e:   # table must cover pos_offset + q_tokens
        fa.launch(None, q, pool, table, out, 8, 2, 128, 16, 4, 13)
    assert e.value.kind == "InvalidSize" and e.value.expected == 8
    with pytest.raises(HipError) as e:
        fa.launch(None, q, pool, table, out, 8, 2, 96, 16, 4, 0)
    assert e.value.kind == "Unsupported"
    # zero tokens is a no-op success
    fa.launch(None, q, pool, table, out, 8, 2, 128, 16, 0, 0)


@pytest.mark.parametrize("data", ["gauss", "codes"])
@pytest.mark.parametrize("hd,nh,nkv", [(128, 16, 4), (64, 8, 8), (128, 32, 8)])
def test_batched_ragged_chunks_e4m3(dev, hd, nh, nkv, data):
    """Chunked prefill over an E4M3 pool (per-kv-head scales) against the
    oracle's causal attention on the dequantised pool, decode(code) * scale.
    "gauss": quantised N(0,1) K/V (scales max|x| / 448), the contract's data,
    strict bar; "codes": every E4M3 code with random scales (|x| up to ~22),
    a stress case under the per-element bound."""
    bt = 16
    rng = np.random.default_rng(23 + hd + nh)
    starts = [0, 5, 130, 1000]
    lens = [33, 1, 200, 64]
    stride = max(-(-(s + n) // bt) for s, n in zip(starts, lens)) + 2
    n_pages = sum(-(-(s + n) // bt) for s, n in zip(starts, lens)) + 3
    perm = rng.permutation(n_pages).astype(np.uint32)
    tables = np.full((len(starts), stride), 0xFFFFFFFF, np.uint32)
    o = 0
    for b, (s, n) in enumerate(zip(starts, lens)):
        k = -(-(s + n) // bt)
        tables[b, :k] = perm[o:o + k]
        o += k
    codes, ks, vs = (gauss_codes if data == "gauss" else all_codes)(rng, n_pages, bt, nkv, hd)
    f = orc.e4m3_to_f32(codes).reshape(n_pages, bt, 2, nkv, hd)
    f[:, :, 0] *= ks[None, None, :, None]
    f[:, :, 1] *= vs[None, None, :, None]
    hpool = f.reshape(-1)
    total = sum(lens)
    q = rng.standard_normal((total, nh, hd)).astype(np.float32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    out = torch.full((total, nh, hd), float("nan"), device=dev)
    FlashAttention2(0).launch_batched_e4m3(None, torch.from_numpy(q).to(dev),
                                           torch.from_numpy(codes).to(dev), i32(tables, dev),
                                           i32(cu, dev), i32(np.array(starts, np.uint32), dev), out,
                                           nh, nkv, hd, bt, max(lens), torch.from_numpy(ks).to(dev),
                                           torch.from_numpy(vs).to(dev))
    torch.cuda.synchronize()
    g = out.cpu().numpy()
    for b, (s, n) in enumerate(zip(starts, lens)):
        k = -(-(s + n) // bt)
        ref = orc.prefill_causal(hpool, tables[b, :k], bt, q[cu[b]:cu[b + 1]], n, s, nh, nkv, hd)
        check_close(g[cu[b]:cu[b + 1]], ref, KvDataType.F16, f"seq {b}", stress=data == "codes")


def test_e4m3_prefill_rejects_other_entries(dev):
    """An E4M3 pool goes through the scale-aware prefill only."""
    pool = torch.zeros(4 * 16 * 2 * 256, dtype=torch.uint8, device=dev)
    q = torch.zeros((4, 8, 128), device=dev)
    out = torch.empty_like(q)
    tab = torch.zeros((1, 4), dtype=torch.int32, device=dev)
    cu = torch.tensor([0, 4], dtype=torch.int32, device=dev)
    st = torch.zeros(1, dtype=torch.int32, device=dev)
    with pytest.raises(HipError):
        FlashAttention2(0).launch_batched(None, q, pool, tab, cu, st, out, 8, 2, 128, 16, 4,
                                          kv_dtype=KvDataType.FP8)


def _random_prefill_case(seed):
    """One seeded random batched prefill: f32/f16/bf16 pages, head_dim 64 or
    128, 1/2/4/8 kv heads with 1-8 q heads each (at most 16 q heads, so the
    oracle stays fast), pages of 16/32/64 tokens, 1-4 sequences with chunks of
    1-200 tokens on contexts of 0-800."""
    rng = np.random.default_rng(30_000 + seed)
    dtype = (KvDataType.F32, KvDataType.F16, KvDataType.BF16)[int(rng.integers(3))]
    hd = int(rng.choice([64, 128]))
    nkv = int(rng.choice([1, 2, 4, 8]))
    g = int(rng.choice([g for g in (1, 2, 3, 4, 7, 8) if g * nkv <= 16]))
    bt = int(rng.choice([16, 32, 64]))
    B = int(rng.integers(1, 5))
    starts = rng.choice([0, 0, bt - 1, bt, int(rng.integers(1, 800))], B).astype(np.int64)
    lens = rng.integers(1, 201, B).astype(np.int64)
    return dtype, (g * nkv, nkv, hd, bt), starts, lens


@pytest.mark.parametrize("seed", range(12))
def test_prefill_random_sweep(dev, seed):
    """The batched prefill on random shapes against the oracle's causal
    prefill, sequence by sequence."""
    dtype, (nh, nkv, hd, bt), starts, lens = _random_prefill_case(seed)
    print(f"[prefill sweep {seed}] {dtype.name} heads {nh}/{nkv} hd {hd} page {bt} "
          f"starts {starts.tolist()} lens {lens.tolist()}", flush=True)
    rng = np.random.default_rng(40_000 + seed)
    pages = [-(-(int(s) + int(n)) // bt) for s, n in zip(starts, lens)]
    stride = max(pages) + 1
    n_pages = sum(pages) + 2
    perm = rng.permutation(n_pages).astype(np.uint32)
    tables = np.full((len(starts), stride), 0xFFFFFFFF, np.uint32)
    o = 0
    for b, k in enumerate(pages):
        tables[b, :k] = perm[o:o + k]
        o += k
    dpool, hpool = make_pool(rng, n_pages, bt, nkv, hd, dtype, dev)
    total = int(lens.sum())
    q = rng.standard_normal((total, nh, hd)).astype(np.float32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    out = torch.full((total, nh, hd), float("nan"), device=dev)
    FlashAttention2(0).launch_batched(None, torch.from_numpy(q).to(dev), dpool, i32(tables, dev),
                                      i32(cu, dev), i32(starts.astype(np.uint32), dev), out,
                                      nh, nkv, hd, bt, int(lens.max()), kv_dtype=dtype)
    torch.cuda.synchronize()
    g = out.cpu().numpy()
    for b, (s, n) in enumerate(zip(starts, lens)):
        ref = orc.prefill_causal(hpool, tables[b, :pages[b]], bt, q[cu[b]:cu[b + 1]], int(n),
                                 int(s), nh, nkv, hd)
        check_close(g[cu[b]:cu[b + 1]], ref, dtype, f"prefill sweep {seed} seq {b}")


@pytest.mark.parametrize("seed", range(16))
def test_pingpong_random_sweep(dev, monkeypatch, seed):
    """The two prefill kernels on seeded random shapes: f16, bf16 and E4M3
    pages; head_dim 64 or 128; 1-8 kv heads with 1-8 q heads each; pages of
    4-64 tokens; 1-5 sequences with chunks of 1-700 tokens on contexts of
    0-3000; up to two table entries pointing outside the pool.  Bit-identical
    at head_dim 128 (both walk 64-key tiles), within the bar of each other at
    64; every fourth shape also against the oracle (sequences without an
    invalid entry)."""
    rng = np.random.default_rng(90_000 + seed)
    dtype = (KvDataType.F16, KvDataType.BF16, KvDataType.FP8)[int(rng.integers(3))]
    hd = int(rng.choice([64, 128, 128]))
    nkv = int(rng.choice([1, 2, 4, 8]))
    g = int(rng.choice([1, 2, 3, 4, 6, 7, 8]))
    bt = int(rng.choice([4, 8, 16, 32, 64]))
    B = int(rng.integers(1, 6))
    starts = rng.choice([0, 0, bt - 1, bt, int(rng.integers(1, 3000))], B).astype(np.int64)
    lens = rng.integers(1, 700, B).astype(np.int64)
    nh = g * nkv
    print(f"[pp sweep {seed}] {dtype.name} heads {nh}/{nkv} hd {hd} page {bt} "
          f"starts {starts.tolist()} lens {lens.tolist()}", flush=True)
    pages = [-(-(int(s0) + int(n)) // bt) for s0, n in zip(starts, lens)]
    stride = max(pages) + int(rng.integers(0, 3))
    n_pages = sum(pages) + 2
    perm = rng.permutation(n_pages).astype(np.uint32)
    tables = np.full((B, stride), 0xFFFFFFFF, np.uint32)
    o = 0
    for b, k in enumerate(pages):
        tables[b, :k] = perm[o:o + k]
        o += k
    bad_seqs = set()
    for _ in range(int(rng.integers(0, 3))):
        b = int(rng.integers(B))
        tables[b, int(rng.integers(pages[b]))] = n_pages + 5 + int(rng.integers(100))
        bad_seqs.add(b)
    total = int(lens.sum())
    q = rng.standard_normal((total, nh, hd)).astype(np.float32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    fa = FlashAttention2(0)
    if dtype == KvDataType.FP8:
        codes, ks, vs = gauss_codes(rng, n_pages, bt, nkv, hd)
        dpool = torch.from_numpy(codes).to(dev)
        f = orc.e4m3_to_f32(codes).reshape(n_pages, bt, 2, nkv, hd)
        f[:, :, 0] *= ks[None, None, :, None]
        f[:, :, 1] *= vs[None, None, :, None]
        hpool = f.reshape(-1)
        dks, dvs = torch.from_numpy(ks).to(dev), torch.from_numpy(vs).to(dev)
    else:
        dpool, hpool = make_pool(rng, n_pages, bt, nkv, hd, dtype, dev)
    outs = {}
    for kern in ("single", "pp"):
        monkeypatch.setenv("EH_PREFILL_KERNEL", kern)
        out = torch.full((total, nh, hd), float("nan"), device=dev)
        args = (None, torch.from_numpy(q).to(dev), dpool, i32(tables, dev), i32(cu, dev),
                i32(np.array(starts, np.uint32), dev), out, nh, nkv, hd, bt, int(lens.max()))
        if dtype == KvDataType.FP8:
            fa.launch_batched_e4m3(*args, dks, dvs)
        else:
            fa.launch_batched(*args, kv_dtype=dtype)
        torch.cuda.synchronize()
        outs[kern] = out.cpu().numpy()
    if hd == 128:
        assert np.array_equal(outs["pp"].view(np.uint32), outs["single"].view(np.uint32))
    else:
        check_close(outs["pp"], outs["single"], KvDataType.F16, "pp vs single-phase")
    if seed % 4 == 0:
        for b in range(B):
            if b in bad_seqs:
                continue
            ref = orc.prefill_causal(hpool, tables[b, :pages[b]], bt, q[cu[b]:cu[b + 1]],
                                     int(lens[b]), int(starts[b]), nh, nkv, hd)
            check_close(outs["pp"][cu[b]:cu[b + 1]], ref,
                        KvDataType.F16 if dtype == KvDataType.FP8 else dtype, f"pp seq {b}")


@pytest.mark.parametrize("dtype", [KvDataType.BF16, KvDataType.F16, KvDataType.FP8],
                         ids=lambda d: d.name)
def test_graph_replay_successive_chunks(dev, dtype):
    """Batched chunked prefill captured once in a HIP graph, then replayed for
    successive chunks. Before each replay the caller writes the chunk's q,
    cu_q and start positions into the captured buffers (eager copies and a
    synchronisation, as a serving loop does). Every replay equals an eager
    call on the same inputs bit for bit, and every chunk matches the oracle
    (f16 bar; E4M3 on decode(code) * scale). Chunks are ragged and one
    sequence has an empty chunk. bf16 pages run the ping-pong kernel, f16 and
    E4M3 pages the single-phase kernel."""
    nh, nkv, hd, bt = 16, 4, 128, 16
    B, C, n_chunks = 3, 96, 4
    rng = np.random.default_rng(4100 + int(dtype))
    ctx0 = np.array([0, 37, 300], np.int64)
    lens = rng.integers(1, C + 1, size=(n_chunks, B))
    lens[2, 1] = 0
    stride = -(-(int(ctx0.max()) + n_chunks * C) // bt) + 1
    n_pages = B * stride + 3
    perm = rng.permutation(n_pages).astype(np.uint32)
    tables = perm[:B * stride].reshape(B, stride).copy()
    if dtype == KvDataType.FP8:
        codes, ks, vs = gauss_codes(rng, n_pages, bt, nkv, hd)
        dpool = torch.from_numpy(codes).to(dev)
        f = orc.e4m3_to_f32(codes).reshape(n_pages, bt, 2, nkv, hd)
        f[:, :, 0] *= ks[None, None, :, None]
        f[:, :, 1] *= vs[None, None, :, None]
        hpool = f.reshape(-1)
        dks, dvs = torch.from_numpy(ks).to(dev), torch.from_numpy(vs).to(dev)
    else:
        dpool, hpool = make_pool(rng, n_pages, bt, nkv, hd, dtype, dev)
    fa = FlashAttention2(0)
    q_s = torch.zeros((B * C, nh, hd), device=dev)
    cu_s = i32(np.zeros(B + 1, np.uint32), dev)
    sp_s = i32(np.zeros(B, np.uint32), dev)
    dtab = i32(tables, dev)
    out_g = torch.empty_like(q_s)
    out_e = torch.empty_like(q_s)

    def call(stream, out):
        if dtype == KvDataType.FP8:
            fa.launch_batched_e4m3(stream, q_s, dpool, dtab, cu_s, sp_s, out, nh, nkv, hd, bt, C,
                                   dks, dvs)
        else:
            fa.launch_batched(stream, q_s, dpool, dtab, cu_s, sp_s, out, nh, nkv, hd, bt, C,
                              kv_dtype=dtype)

    call(None, out_g)                                               # warm-up on empty chunks
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            call(s, out_g)
    torch.cuda.synchronize()
    done = ctx0.copy()
    for k in range(n_chunks):
        cu = np.concatenate([[0], np.cumsum(lens[k])]).astype(np.uint32)
        q = rng.standard_normal((B * C, nh, hd)).astype(np.float32)
        q_s.copy_(torch.from_numpy(q))
        cu_s.copy_(i32(cu, dev))
        sp_s.copy_(i32(done.astype(np.uint32), dev))
        out_g.fill_(float("nan"))
        out_e.fill_(float("nan"))
        torch.cuda.synchronize()
        call(None, out_e)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g.view(torch.int32), out_e.view(torch.int32)), k
        gh = out_g.cpu().numpy()
        for b in range(B):
            n, st = int(lens[k, b]), int(done[b])
            if n == 0:
                continue
            pages = -(-(st + n) // bt)
            ref = orc.prefill_causal(hpool, tables[b, :pages], bt, q[cu[b]:cu[b + 1]], n, st, nh,
                                     nkv, hd)
            check_close(gh[cu[b]:cu[b + 1]], ref,
                        KvDataType.F16 if dtype == KvDataType.FP8 else dtype, f"chunk {k} seq {b}")
        assert np.isnan(gh[cu[B]:]).all()                            # rows past the chunks untouched
        done += lens[k]


@pytest.mark.parametrize("dtype", [KvDataType.BF16, KvDataType.F16, KvDataType.FP8],
                         ids=lambda d: d.name)
def test_long_prompt_in_one_chunk(dev, dtype):
    """A whole 8192-token prompt in one chunk (position 0) beside a
    3000-token chunk continuing at position 5000, 32/8 heads, hd 128, pages
    of 16 on scattered tables: each row block walks up to 128 key tiles
    (the random sweeps stop near 700-token chunks).  40 sampled query rows
    against the oracle (first and last rows, row-block edges, random),
    strict bar; bf16 pages run the ping-pong kernel."""
    nh, nkv, hd, bt = 32, 8, 128, 16
    starts, lens = np.array([0, 5000]), np.array([8192, 3000])
    rng = np.random.default_rng(5100 + int(dtype))
    need = [-(-(s + n) // bt) for s, n in zip(starts, lens)]
    n_pages = sum(need) + 3
    perm = rng.permutation(n_pages).astype(np.uint32)
    tables = np.full((2, max(need)), 0xFFFFFFFF, np.uint32)
    tables[0, :need[0]] = perm[:need[0]]
    tables[1, :need[1]] = perm[need[0]:need[0] + need[1]]
    if dtype == KvDataType.FP8:
        codes, ks, vs = gauss_codes(rng, n_pages, bt, nkv, hd)
        dpool = torch.from_numpy(codes).to(dev)
        f = orc.e4m3_to_f32(codes).reshape(n_pages, bt, 2, nkv, hd)
        f[:, :, 0] *= ks[None, None, :, None]
        f[:, :, 1] *= vs[None, None, :, None]
        hpool = f.reshape(-1)
    else:
        dpool, hpool = make_pool(rng, n_pages, bt, nkv, hd, dtype, dev)
    total = int(lens.sum())
    q = rng.standard_normal((total, nh, hd)).astype(np.float32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    out = torch.full((total, nh, hd), float("nan"), device=dev)
    args = (None, torch.from_numpy(q).to(dev), dpool, i32(tables, dev), i32(cu, dev),
            i32(starts.astype(np.uint32), dev), out, nh, nkv, hd, bt, int(lens.max()))
    if dtype == KvDataType.FP8:
        FlashAttention2(0).launch_batched_e4m3(*args, torch.from_numpy(ks).to(dev),
                                               torch.from_numpy(vs).to(dev))
    else:
        FlashAttention2(0).launch_batched(*args, kv_dtype=dtype)
    torch.cuda.synchronize()
    g = out.cpu().numpy()
    assert not np.isnan(g).any()
    edges = [0, 1, 63, 64, 8191, 8192, 8192 + 2999, 4096 - 1, 4096, 8192 + 1500]
    for r in np.concatenate([edges, rng.integers(0, total, size=30)]):
        b = 0 if r < lens[0] else 1
        i = int(r - cu[b])
        ref = orc.prefill_causal(hpool, tables[b, :need[b]], bt, q[r:r + 1], 1, int(starts[b]) + i,
                                 nh, nkv, hd)
        check_close(g[r:r + 1], ref, KvDataType.F16 if dtype == KvDataType.FP8 else dtype,
                    f"row {r}")
