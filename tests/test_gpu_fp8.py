"""GPU parity of FP8 (E4M3) KV storage: quantising append, dequantising
gather and the token-balanced decode over an E4M3 pool, against the oracle's
E4M3 restatement (tests/test_oracle_fp8.py pins it).

Bars: append and gather bit-exact (codes; dequantised f32 bits, NaN where the
code is NaN); decode over quantised N(0,1) K/V (scale max|x| / 448, as a
quantiser stores the contract's data) max-abs <= 2e-3 and
|gpu - ref| <= 2e-3 + 1e-3*|ref| (tests/parity.py) against sdpa_decode on
the dequantised pool (decode(code) * scale); decode over every code (|x| up
to ~22, a stress case) the per-element bound only; and the acceptance of the
reference's FP8 KV spec (openspec/archive/2026-08-28-fp8-kv-cache-quantization/
specs/kv-compression/spec.md:12-15): cosine similarity >= 0.999 between the
E4M3 attention output and the f16 one on the same K/V.
"""
import numpy as np
import pytest
import torch

from oracle import orc
from titan_amd import HipError, KvDataType, PagedAttention, PagedKvGpu, PagedKvLayout

import parity
from e4m3_data import all_codes, gauss_codes

pytestmark = pytest.mark.gpu

NONE = 0xFFFFFFFF


def i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(dev)


def make_tables(rng, lens, bt, spare=3):
    need = [(int(l) + bt - 1) // bt for l in lens]
    stride = max(max(need), 1)
    nb = sum(need) + spare
    perm = rng.permutation(nb).astype(np.uint32)
    tab = np.full((len(lens), stride), NONE, np.uint32)
    pos = 0
    for b, c in enumerate(need):
        tab[b, :c] = perm[pos:pos + c]
        pos += c
    return tab, nb


def dequant_pool(codes, nb, bt, n_kv, hd, ks, vs):
    """decode(code) * scale of the element's (K or V, kv head)."""
    f = orc.e4m3_to_f32(codes).reshape(nb, bt, 2, n_kv, hd)
    f[:, :, 0] *= np.asarray(ks, np.float32)[None, None, :, None]
    f[:, :, 1] *= np.asarray(vs, np.float32)[None, None, :, None]
    return f.reshape(-1)


def test_e4m3_append_bit_exact(dev):
    """Ragged batch of f32 rows -> codes equal the oracle's quantisation,
    including ties, saturation, subnormals, signed zeros and NaN."""
    rng = np.random.default_rng(21)
    n_kv, hd, bt = 2, 128, 16
    rl = n_kv * hd
    starts = np.array([0, 5, 31, 100], np.int64)
    ns = np.array([17, 1, 40, 3], np.int64)
    tab, nb = make_tables(rng, starts + ns, bt)
    T = int(ns.sum())
    ks = np.array([0.05, 1.7], np.float32)
    vs = np.array([3.0, 0.011], np.float32)
    keys = (rng.standard_normal((T, rl)) * 10.0 ** rng.uniform(-3, 2.5, (T, rl))).astype(np.float32)
    vals = (rng.standard_normal((T, rl)) * 10.0 ** rng.uniform(-3, 2.5, (T, rl))).astype(np.float32)
    tbl = orc.e4m3_to_f32(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    mids = ((tbl[1:] + tbl[:-1]) / 2).astype(np.float32)
    keys[0, :126] = mids * ks[0]                     # exact ties of head 0 (scaled back)
    keys[1, :8] = [np.nan, np.inf, -np.inf, 1e9, -0.0, 2.0 ** -12, -500 * ks[0], 447.9 * ks[0]]
    pool = torch.zeros(nb * bt * 2 * rl, dtype=torch.uint8, device=dev)
    lay = PagedKvLayout(nb, bt, rl, KvDataType.FP8)
    cu = np.concatenate([[0], np.cumsum(ns)]).astype(np.uint32)
    PagedKvGpu(0).append_kv_e4m3_batched(None, lay, pool, torch.from_numpy(keys).to(dev),
                                         torch.from_numpy(vals).to(dev), i32(tab, dev), i32(cu, dev),
                                         i32(starts, dev), T, hd, torch.from_numpy(ks).to(dev),
                                         torch.from_numpy(vs).to(dev))
    torch.cuda.synchronize()
    want = np.zeros((nb, bt, 2, n_kv, hd), np.uint8)
    t = 0
    for b in range(len(starts)):
        for i in range(int(ns[b])):
            p = int(starts[b]) + i
            page, slot = tab[b, p // bt], p % bt
            for h in range(n_kv):
                want[page, slot, 0, h] = orc.f32_to_e4m3(keys[t, h * hd:(h + 1) * hd], ks[h])
                want[page, slot, 1, h] = orc.f32_to_e4m3(vals[t, h * hd:(h + 1) * hd], vs[h])
            t += 1
    got = pool.cpu().numpy().reshape(want.shape)
    bad = np.argwhere(got != want)
    assert bad.size == 0, (bad[:4], got[tuple(bad[0])], want[tuple(bad[0])])


def test_e4m3_gather_all_codes(dev):
    """Every code through the dequantising read: decode(code) * scale, bit-exact."""
    n_kv, hd, bt = 2, 128, 16
    rl = n_kv * hd
    nb = 4
    codes = np.tile(np.arange(256, dtype=np.uint8), nb * bt * 2 * rl // 256)
    np.random.default_rng(2).shuffle(codes)
    pool = torch.from_numpy(codes).to(dev)
    lay = PagedKvLayout(nb, bt, rl, KvDataType.FP8)
    tab = np.array([2, 0, 3, 1], np.uint32)
    ks = np.array([0.25, 3.3], np.float32)
    vs = np.array([1.0, 0.07], np.float32)
    pk = PagedKvGpu(0)
    for is_value, sc in ((0, ks), (1, vs)):
        out = torch.zeros((nb * bt, rl), device=dev)
        pk.read_e4m3(None, lay, pool, i32(tab, dev), out, 0, nb * bt, is_value, hd,
                     torch.from_numpy(sc).to(dev))
        torch.cuda.synchronize()
        rows = codes.reshape(nb, bt, 2, n_kv, hd)[tab, :, is_value].reshape(nb * bt, n_kv, hd)
        want = (orc.e4m3_to_f32(rows) * sc[None, :, None]).astype(np.float32).reshape(nb * bt, rl)
        got = out.cpu().numpy()
        assert np.array_equal(np.isnan(got), np.isnan(want))
        ok = ~np.isnan(want)
        assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))


def run_decode_e4m3(dev, lens, shape, seed, grid=None, data="gauss"):
    n_head, n_kv, hd, bt = shape
    rng = np.random.default_rng(seed)
    tab, nb = make_tables(rng, lens, bt)
    codes, ks, vs = (gauss_codes if data == "gauss" else all_codes)(rng, nb, bt, n_kv, hd)
    B = len(lens)
    q = rng.standard_normal((B, n_head, hd)).astype(np.float32)
    plan = PagedAttention.plan(B, n_head, n_kv, hd, bt, int(max(lens)), 0, KvDataType.FP8)
    assert plan[0] == 0
    if grid is not None:
        plan = PagedAttention.with_grid(plan, grid, B, n_head)
    ws = PagedAttention.workspace(plan)
    out = torch.full((B, n_head, hd), float("nan"), device=dev)
    PagedAttention(0).decode_batched_e4m3(None, torch.from_numpy(q).to(dev),
                                          torch.from_numpy(codes).to(dev), i32(tab, dev),
                                          i32(lens, dev), out, n_head, n_kv, hd, bt,
                                          torch.from_numpy(ks).to(dev), torch.from_numpy(vs).to(dev),
                                          plan, ws)
    torch.cuda.synchronize()
    pool_f32 = dequant_pool(codes, nb, bt, n_kv, hd, ks, vs)
    ref = orc.sdpa_decode_batched(pool_f32, tab, np.asarray(lens, np.uint32), bt, q, n_head, n_kv, hd)
    return out.cpu().numpy(), ref


def check_close(gpu, ref, what="e4m3", stress=False):
    parity.check_close(gpu, ref, what=what, stress=stress)


@pytest.mark.parametrize("shape", [(12, 2, 128, 16), (32, 8, 128, 16), (8, 1, 128, 32),
                                   (16, 4, 128, 16), (14, 2, 128, 16)],
                         ids=lambda s: "x".join(map(str, s)))
def test_e4m3_decode_matches_sdpa(dev, shape):
    lens = np.array([0, 1, 15, 16, 17, 300, 2049, 0, 33, 1000, 7], np.int64)
    out, ref = run_decode_e4m3(dev, lens, shape, 40 + sum(shape))
    check_close(out, ref)


@pytest.mark.parametrize("shape", [(12, 2, 128, 16), (32, 8, 128, 16)],
                         ids=lambda s: "x".join(map(str, s)))
def test_e4m3_decode_all_codes_stress(dev, shape):
    """Every E4M3 code (random scales, |K|, |V| up to ~22): outputs of
    magnitude up to ~20, checked with the per-element bound."""
    lens = np.array([0, 1, 15, 16, 17, 300, 2049, 0, 33, 1000, 7], np.int64)
    out, ref = run_decode_e4m3(dev, lens, shape, 40 + sum(shape), data="codes")
    check_close(out, ref, stress=True)


@pytest.mark.parametrize("grid", [1, 3, 64])
def test_e4m3_decode_small_grids(dev, grid):
    lens = np.array([3000, 1, 2000, 0, 5, 1500, 16, 31, 777], np.int64)
    out, ref = run_decode_e4m3(dev, lens, (12, 2, 128, 16), 90 + grid, grid)
    check_close(out, ref)


def test_e4m3_cosine_vs_f16(dev):
    """The same K/V stored as f16 and as E4M3 (per-head scale max|x| / 448).

    The spec's acceptance (cosine >= 0.999 against f16) is stated for a real
    model's KV (Llama 3.2 3B); no weights exist here, so that figure is not
    reproduced.  On i.i.d. Gaussian K/V, E4M3's 3-bit mantissa (~3.6 % RMS
    relative rounding) bounds the cosine near 0.998 on average (V noise
    ~0.9993, K noise perturbing random scores of spread ~2 by ~7 %): the test
    asserts mean >= 0.998 and min >= 0.99 over 96 output rows."""
    rng = np.random.default_rng(33)
    n_head, n_kv, hd, bt = 12, 2, 128, 16
    rl = n_kv * hd
    lens = rng.integers(128, 4097, 8).astype(np.int64)
    tab, nb = make_tables(rng, lens, bt)
    kvf = rng.standard_normal((nb * bt, 2, n_kv, hd)).astype(np.float32)
    kvf[:, 0] *= 2.0                                   # K spread wider than V
    ks = (np.abs(kvf[:, 0]).max(axis=(0, 2)) / 448.0).astype(np.float32)
    vs = (np.abs(kvf[:, 1]).max(axis=(0, 2)) / 448.0).astype(np.float32)
    codes = np.empty(kvf.shape, np.uint8)
    for h in range(n_kv):
        codes[:, 0, h] = orc.f32_to_e4m3(kvf[:, 0, h], ks[h])
        codes[:, 1, h] = orc.f32_to_e4m3(kvf[:, 1, h], vs[h])
    q = rng.standard_normal((len(lens), n_head, hd)).astype(np.float32)
    pa = PagedAttention(0)
    dq, dl, dt = torch.from_numpy(q).to(dev), i32(lens, dev), i32(tab, dev)
    p8 = PagedAttention.plan(len(lens), n_head, n_kv, hd, bt, 4096, 0, KvDataType.FP8)
    o8 = torch.empty((len(lens), n_head, hd), device=dev)
    pa.decode_batched_e4m3(None, dq, torch.from_numpy(codes.reshape(-1)).to(dev), dt, dl, o8,
                           n_head, n_kv, hd, bt, torch.from_numpy(ks).to(dev),
                           torch.from_numpy(vs).to(dev), p8, PagedAttention.workspace(p8))
    p16 = PagedAttention.plan(len(lens), n_head, n_kv, hd, bt, 4096, 0, KvDataType.F16)
    o16 = torch.empty_like(o8)
    pa.decode_batched(None, dq, torch.from_numpy(kvf.reshape(-1)).half().to(dev), dt, dl, o16,
                      n_head, n_kv, hd, bt, KvDataType.F16, p16, PagedAttention.workspace(p16))
    torch.cuda.synchronize()
    a, b = o8.cpu().double().reshape(-1, hd), o16.cpu().double().reshape(-1, hd)
    cos = (a * b).sum(1) / (a.norm(dim=1) * b.norm(dim=1))
    assert cos.mean().item() >= 0.998 and cos.min().item() >= 0.99, (cos.mean().item(),
                                                                      cos.min().item())


def e4m3_scales_np(rows, n_kv, hd):
    """The dynamic per-head scale rule: max(amax / 448, FLT_MIN) over the
    finite elements of each head, 1 when none is nonzero (all in f32)."""
    out = np.empty(n_kv, np.float32)
    for h in range(n_kv):
        a = np.abs(rows[:, h * hd:(h + 1) * hd].astype(np.float32))
        a = a[np.isfinite(a)]
        m = np.float32(a.max()) if a.size else np.float32(0)
        out[h] = max(m / np.float32(448), np.float32(np.finfo(np.float32).tiny)) if m > 0 else 1.0
    return out


def test_e4m3_dynamic_scales_exact(dev):
    """eh_kv_e4m3_scales: per kv head, max(amax / 448, FLT_MIN) over the finite
    elements, bit for bit; NaN and infinities ignored, an all-zero head gets 1,
    a head of tiny values gets the FLT_MIN floor."""
    rng = np.random.default_rng(71)
    n_kv, hd, n = 5, 128, 777
    rl = n_kv * hd
    k = (rng.standard_normal((n, rl)) * 3).astype(np.float32)
    v = rng.standard_normal((n, rl)).astype(np.float32)
    k[123, 0 * hd + 7] = 913.25          # head 0's amax
    k[5, 1 * hd + 3] = np.nan            # ignored
    k[6, 1 * hd + 4] = -np.inf           # ignored
    k[:, 2 * hd:3 * hd] = 0.0            # all zero: scale 1
    v[:, 3 * hd:4 * hd] *= 1e-38         # amax / 448 below FLT_MIN: the floor
    v[400, 4 * hd + 127] = -1.5e7        # the sign does not matter
    layout = PagedKvLayout(4, 16, rl, KvDataType.FP8)
    ks, vs = torch.full((n_kv,), -1.0, device=dev), torch.full((n_kv,), -1.0, device=dev)
    PagedKvGpu(0).e4m3_scales(None, layout, torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev),
                              hd, ks, vs)
    torch.cuda.synchronize()
    assert np.array_equal(ks.cpu().numpy().view(np.uint32), e4m3_scales_np(k, n_kv, hd).view(np.uint32))
    assert np.array_equal(vs.cpu().numpy().view(np.uint32), e4m3_scales_np(v, n_kv, hd).view(np.uint32))
    assert ks[2].item() == 1.0 and vs[3].item() == np.finfo(np.float32).tiny


def test_e4m3_dynamic_scales_end_to_end(dev):
    """The FP8 spec's flow (specs/kv-compression/spec.md:8-14): scales from the
    prompt's own K/V on the device, the quantising append with them, E4M3
    decode against the same K/V in f16.  Pool bytes equal the oracle's
    quantisation with those scales; output cosine as test_e4m3_cosine_vs_f16
    (i.i.d. data, no model weights here); and the spec's memory bound for its
    scenario -- Llama 3.2 3B (28 layers, 8 kv heads, head_dim 128), 4096
    tokens -- holds for the E4M3 layout (<= 300 MB)."""
    n_layers, kv3b, hd3b, ctx = 28, 8, 128, 4096
    per_layer = PagedKvLayout(ctx // 16, 16, kv3b * hd3b, KvDataType.FP8).bytes_total()
    assert n_layers * per_layer <= 300 * 10**6

    rng = np.random.default_rng(72)
    n_head, n_kv, hd, bt = 12, 2, 128, 16
    rl = n_kv * hd
    lens = rng.integers(200, 2049, 6).astype(np.int64)
    B, T = len(lens), int(lens.sum())
    tab, nb = make_tables(rng, lens, bt)
    k = (rng.standard_normal((T, rl)) * 2).astype(np.float32)
    v = rng.standard_normal((T, rl)).astype(np.float32)
    layout = PagedKvLayout(nb, bt, rl, KvDataType.FP8)
    dk, dv = torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev)
    ks, vs = torch.empty(n_kv, device=dev), torch.empty(n_kv, device=dev)
    kvg = PagedKvGpu(0)
    kvg.e4m3_scales(None, layout, dk, dv, hd, ks, vs)
    pool = torch.zeros(layout.bytes_total(), dtype=torch.uint8, device=dev)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    kvg.append_kv_e4m3_batched(None, layout, pool, dk, dv, i32(tab, dev), i32(cu, dev),
                               i32(np.zeros(B), dev), T, hd, ks, vs)
    torch.cuda.synchronize()
    ksn, vsn = ks.cpu().numpy(), vs.cpu().numpy()
    assert np.array_equal(ksn.view(np.uint32), e4m3_scales_np(k, n_kv, hd).view(np.uint32))
    # oracle pool: each token's row quantised with the device scales at its page slot
    want = np.zeros((nb, bt, 2, n_kv, hd), np.uint8)
    for b in range(B):
        for t in range(int(lens[b])):
            r = cu[b] + t
            for h in range(n_kv):
                want[tab[b, t // bt], t % bt, 0, h] = orc.f32_to_e4m3(k[r, h * hd:(h + 1) * hd], ksn[h])
                want[tab[b, t // bt], t % bt, 1, h] = orc.f32_to_e4m3(v[r, h * hd:(h + 1) * hd], vsn[h])
    assert np.array_equal(pool.cpu().numpy(), want.reshape(-1)), "pool bytes"
    q = rng.standard_normal((B, n_head, hd)).astype(np.float32)
    pa = PagedAttention(0)
    dq, dl, dt = torch.from_numpy(q).to(dev), i32(lens, dev), i32(tab, dev)
    p8 = PagedAttention.plan(B, n_head, n_kv, hd, bt, 2048, 0, KvDataType.FP8)
    o8 = torch.empty((B, n_head, hd), device=dev)
    pa.decode_batched_e4m3(None, dq, pool, dt, dl, o8, n_head, n_kv, hd, bt, ks, vs, p8,
                           PagedAttention.workspace(p8))
    # the same rows as f16 pages
    f16 = np.zeros((nb, bt, 2, rl), np.float16)
    for b in range(B):
        for t in range(int(lens[b])):
            f16[tab[b, t // bt], t % bt, 0] = k[cu[b] + t]
            f16[tab[b, t // bt], t % bt, 1] = v[cu[b] + t]
    p16 = PagedAttention.plan(B, n_head, n_kv, hd, bt, 2048, 0, KvDataType.F16)
    o16 = torch.empty_like(o8)
    pa.decode_batched(None, dq, torch.from_numpy(f16.reshape(-1)).to(dev), dt, dl, o16, n_head,
                      n_kv, hd, bt, KvDataType.F16, p16, PagedAttention.workspace(p16))
    torch.cuda.synchronize()
    a, c = o8.cpu().double().reshape(-1, hd), o16.cpu().double().reshape(-1, hd)
    cos = (a * c).sum(1) / (a.norm(dim=1) * c.norm(dim=1))
    assert cos.mean().item() >= 0.998 and cos.min().item() >= 0.99, (cos.mean().item(),
                                                                      cos.min().item())


def test_e4m3_dynamic_scales_errors(dev):
    rl, hd = 256, 128
    layout = PagedKvLayout(4, 16, rl, KvDataType.FP8)
    rows = torch.zeros((8, rl), device=dev)
    sc = torch.empty(2, device=dev)
    kvg = PagedKvGpu(0)
    with pytest.raises(HipError):                         # scale arrays shorter than n_kv
        kvg.e4m3_scales(None, layout, rows, rows, hd, sc[:1], sc)
    with pytest.raises(HipError):                         # not an FP8 layout
        kvg.e4m3_scales(None, PagedKvLayout(4, 16, rl, KvDataType.F16), rows, rows, hd, sc, sc)
    with pytest.raises(HipError):                         # head_dim must divide row_len
        kvg.e4m3_scales(None, layout, rows, rows, 96, sc, sc)


def test_e4m3_entry_rejects_other_paths(dev):
    """An E4M3 pool goes through the scale-aware entry points only."""
    from titan_amd import HipError
    with pytest.raises(HipError):
        PagedAttention.plan(4, 12, 2, 128, 16, 100, 64, KvDataType.FP8)   # fixed splits
    with pytest.raises(HipError):
        PagedAttention.plan(4, 12, 2, 64, 16, 100, 0, KvDataType.FP8)     # head_dim 64


def test_e4m3_entry_errors(dev):
    """Null scales, short buffers and non-FP8 layouts are rejected before any launch."""
    from titan_amd import HipError, KvCacheError
    n_kv, hd, bt, nb = 2, 128, 16, 4
    rl = n_kv * hd
    pool = torch.zeros(nb * bt * 2 * rl, dtype=torch.uint8, device=dev)
    lay = PagedKvLayout(nb, bt, rl, KvDataType.FP8)
    keys = torch.zeros((3, rl), device=dev)
    tab = torch.zeros((1, nb), dtype=torch.int32, device=dev)
    cu = torch.tensor([0, 3], dtype=torch.int32, device=dev)
    st = torch.zeros(1, dtype=torch.int32, device=dev)
    sc = torch.ones(n_kv, device=dev)
    pk = PagedKvGpu(0)
    with pytest.raises(HipError):       # keys shorter than total_tokens rows
        pk.append_kv_e4m3_batched(None, lay, pool, keys, keys, tab, cu, st, 4, hd, sc, sc)
    with pytest.raises(HipError):       # a 16-bit layout
        pk.append_kv_e4m3_batched(None, PagedKvLayout(nb, bt, rl, KvDataType.F16), pool, keys,
                                  keys, tab, cu, st, 3, hd, sc, sc)
    with pytest.raises((HipError, KvCacheError)):   # null scale arrays
        pk.append_kv_e4m3_batched(None, lay, pool, keys, keys, tab, cu, st, 3, hd, None, None)
    plan = PagedAttention.plan(1, 12, n_kv, hd, bt, 64, 0, KvDataType.FP8)
    q = torch.zeros((1, 12, hd), device=dev)
    out = torch.empty_like(q)
    lens = torch.tensor([20], dtype=torch.int32, device=dev)
    ws = PagedAttention.workspace(plan)
    with pytest.raises((HipError, KvCacheError)):
        PagedAttention(0).decode_batched_e4m3(None, q, pool, tab, lens, out, 12, n_kv, hd, bt,
                                              None, None, plan, ws)
    with pytest.raises(HipError):       # E4M3 pools only through the scale-aware entries
        PagedAttention(0).decode_batched(None, q, pool, tab, lens, out, 12, n_kv, hd, bt,
                                         KvDataType.FP8, plan, ws)


@pytest.mark.parametrize("shape,grid", [((12, 2, 128, 16), None), ((32, 8, 128, 16), None),
                                        ((12, 2, 128, 16), 5)])
def test_e4m3_fused_step_matches_separate(dev, shape, grid):
    """eh_append_decode_batched_e4m3 (quantising append + decode in one launch)
    leaves the pool bit-identical to eh_append_kv_e4m3_batched and its output
    bit-identical to eh_paged_decode_batched_e4m3 after that append (lens =
    start_pos + 1), and within tolerance of sdpa_decode on the dequantised
    pool.  The appended rows include values that saturate (|x/scale| >= 448),
    and contexts that end on every slot of a page.  Pool: quantised N(0,1)
    K/V (scales max|x| / 448)."""
    n_head, n_kv, hd, bt = shape
    rng = np.random.default_rng(77 + n_kv)
    pos = np.concatenate([[0, 1, 15, 16, 17, 31, 32, 255], rng.integers(1, 700, 8)]).astype(np.uint32)
    B, rl = len(pos), n_kv * hd
    tab, nb = make_tables(rng, pos + 1, bt)
    codes, ks, vs = gauss_codes(rng, nb, bt, n_kv, hd)
    newk = rng.standard_normal((B, rl)).astype(np.float32)
    newv = rng.standard_normal((B, rl)).astype(np.float32)
    newk[0, :4] = [30.0, -30.0, 1e-7, 0.0]               # saturating, subnormal, zero
    q = rng.standard_normal((B, n_head, hd)).astype(np.float32)
    plan = PagedAttention.plan(B, n_head, n_kv, hd, bt, int(pos.max()) + 1, 0, KvDataType.FP8)
    assert plan[0] == 0
    if grid is not None:
        plan = PagedAttention.with_grid(plan, grid, B, n_head)
    lay = PagedKvLayout(nb, bt, rl, KvDataType.FP8)
    t = lambda a: torch.from_numpy(a).to(dev)
    dks, dvs, dq, dtab = t(ks), t(vs), t(q), i32(tab, dev)
    pa = PagedAttention(0)
    # separate: quantising append, then decode over lens = pos + 1
    pool_a = t(codes.copy())
    PagedKvGpu(0).append_kv_e4m3_batched(None, lay, pool_a, t(newk), t(newv), dtab,
                                         i32(np.arange(B + 1), dev), i32(pos, dev), B, hd, dks, dvs)
    out_a = torch.full((B, n_head, hd), float("nan"), device=dev)
    pa.decode_batched_e4m3(None, dq, pool_a, dtab, i32(pos + 1, dev), out_a, n_head, n_kv, hd, bt,
                           dks, dvs, plan, PagedAttention.workspace(plan))
    # fused
    pool_b = t(codes.copy())
    out_b = torch.full((B, n_head, hd), float("nan"), device=dev)
    pa.append_decode_batched_e4m3(None, lay, pool_b, t(newk), t(newv), dtab, i32(pos, dev), dq,
                                  out_b, n_head, hd, plan, PagedAttention.workspace(plan), dks, dvs)
    torch.cuda.synchronize()
    pa_np, pb_np = pool_a.cpu().numpy(), pool_b.cpu().numpy()
    bad = np.argwhere(pa_np != pb_np)
    assert bad.size == 0, (bad[:4], pa_np[bad[0]], pb_np[bad[0]])
    oa, ob = out_a.cpu().numpy(), out_b.cpu().numpy()
    assert np.array_equal(oa.view(np.uint32), ob.view(np.uint32)), np.max(np.abs(oa - ob))
    ref = orc.sdpa_decode_batched(dequant_pool(pb_np, nb, bt, n_kv, hd, ks, vs), tab, pos + 1, bt,
                                  q, n_head, n_kv, hd)
    check_close(ob, ref)


def test_e4m3_fused_step_graph_replay(dev):
    """The fused E4M3 step captured once and replayed as positions grow (the
    work split follows the device lengths): every replay equals eager
    quantising append + E4M3 decode, pool and output bit for bit."""
    n_head, n_kv, hd, bt = 12, 2, 128, 16
    rl, B, steps = n_kv * hd, 6, 5
    rng = np.random.default_rng(13)
    start0 = np.array([0, 14, 31, 500, 1023, 77], np.int64)
    tab, nb = make_tables(rng, start0 + steps + 1, bt)
    codes = rng.integers(0, 256, nb * bt * 2 * rl).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x3C
    host = torch.from_numpy(codes)
    pool_g, pool_e = host.to(dev), host.to(dev)
    lay = PagedKvLayout(nb, bt, rl, KvDataType.FP8)
    dtab, pos, cu = i32(tab, dev), i32(start0, dev), i32(np.arange(B + 1), dev)
    ks = torch.from_numpy(rng.uniform(0.002, 0.05, n_kv).astype(np.float32)).to(dev)
    vs = torch.from_numpy(rng.uniform(0.002, 0.05, n_kv).astype(np.float32)).to(dev)
    k = torch.empty((B, rl), device=dev)
    v = torch.empty_like(k)
    q = torch.empty((B, n_head, hd), device=dev)
    out_g, out_e = torch.empty_like(q), torch.empty_like(q)
    plan = PagedAttention.plan(B, n_head, n_kv, hd, bt, int(start0.max()) + steps + 1, 0,
                               KvDataType.FP8)
    ws_g, ws_e = PagedAttention.workspace(plan), PagedAttention.workspace(plan)
    pa, kv = PagedAttention(0), PagedKvGpu(0)
    k.zero_(); v.zero_(); q.zero_()
    pa.append_decode_batched_e4m3(None, lay, pool_g, k, v, dtab, pos, q, out_g, n_head, hd, plan,
                                  ws_g, ks, vs)
    torch.cuda.synchronize()
    pool_g.copy_(host.to(dev))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            pa.append_decode_batched_e4m3(s, lay, pool_g, k, v, dtab, pos, q, out_g, n_head, hd,
                                          plan, ws_g, ks, vs)
    torch.cuda.synchronize()
    for step in range(steps):
        k.copy_(torch.from_numpy(rng.standard_normal((B, rl)).astype(np.float32)))
        v.copy_(torch.from_numpy(rng.standard_normal((B, rl)).astype(np.float32)))
        q.copy_(torch.from_numpy(rng.standard_normal((B, n_head, hd)).astype(np.float32)))
        pos.copy_(i32(start0 + step, dev))
        torch.cuda.synchronize()
        kv.append_kv_e4m3_batched(None, lay, pool_e, k, v, dtab, cu, pos, B, hd, ks, vs)
        pa.decode_batched_e4m3(None, q, pool_e, dtab, pos + 1, out_e, n_head, n_kv, hd, bt, ks, vs,
                               plan, ws_e)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(pool_g, pool_e), step
        assert torch.equal(out_g.view(torch.int32), out_e.view(torch.int32)), step


def test_e4m3_fused_step_errors(dev):
    """The fused E4M3 step needs an FP8 layout, both scales and f32 rows; the
    16-bit fused step refuses FP8 pools.  All before any launch."""
    from titan_amd import HipError, KvCacheError
    n_kv, hd, bt, nb, B = 2, 128, 16, 8, 2
    rl = n_kv * hd
    pool = torch.zeros(nb * bt * 2 * rl, dtype=torch.uint8, device=dev)
    lay = PagedKvLayout(nb, bt, rl, KvDataType.FP8)
    keys = torch.zeros((B, rl), device=dev)
    tab = torch.zeros((B, 4), dtype=torch.int32, device=dev)
    pos = torch.zeros(B, dtype=torch.int32, device=dev)
    q = torch.zeros((B, 12, hd), device=dev)
    out = torch.empty_like(q)
    sc = torch.ones(n_kv, device=dev)
    plan = PagedAttention.plan(B, 12, n_kv, hd, bt, 64, 0, KvDataType.FP8)
    ws = PagedAttention.workspace(plan)
    pa = PagedAttention(0)
    with pytest.raises(HipError):       # f32 rows shorter than B x row_len
        pa.append_decode_batched_e4m3(None, lay, pool, keys[:1], keys, tab, pos, q, out, 12, hd,
                                      plan, ws, sc, sc)
    with pytest.raises((HipError, KvCacheError)):   # a 16-bit layout
        pa.append_decode_batched_e4m3(None, PagedKvLayout(nb, bt, rl, KvDataType.F16), pool, keys,
                                      keys, tab, pos, q, out, 12, hd, plan, ws, sc, sc)
    with pytest.raises((HipError, KvCacheError)):   # null scale arrays
        pa.append_decode_batched_e4m3(None, lay, pool, keys, keys, tab, pos, q, out, 12, hd, plan,
                                      ws, None, None)
    with pytest.raises(HipError):       # FP8 pools only through the scale-aware fused step
        pa.append_decode_batched(None, lay, pool, keys, keys, tab, pos, q, out, 12, hd, plan, ws)


@pytest.mark.parametrize("seed", range(12))
def test_e4m3_scheduled_step_random_sweep(dev, seed):
    """The scheduled E4M3 step (quantising append + decode in one launch, the
    split read from a step schedule) on random shapes: 1/2/4/8 kv heads with
    1-8 q heads each, pages of 16/32/64 tokens, 1-24 sequences mixing zeros,
    page boundaries and long contexts.  The pool equals the quantising
    append's bit for bit; outputs match sdpa_decode on the dequantised pool."""
    rng = np.random.default_rng(50_000 + seed)
    n_kv = int(rng.choice([1, 2, 4, 8]))
    n_head = n_kv * int(rng.choice([1, 2, 3, 4, 6, 7, 8]))
    hd, bt = 128, int(rng.choice([16, 32, 64]))
    B = int(rng.integers(1, 25))
    kind = rng.integers(0, 3, B)
    pos = np.where(kind == 0, rng.integers(0, 40, B),
                   np.where(kind == 1, rng.integers(40, 1500, B),
                            rng.choice([0, bt - 1, bt, 2 * bt - 1], B))).astype(np.uint32)
    print(f"[e4m3 sweep {seed}] heads {n_head}/{n_kv} page {bt} B {B} max pos {int(pos.max())}",
          flush=True)
    rl = n_kv * hd
    tab, nb = make_tables(rng, pos + 1, bt)
    codes, ks, vs = gauss_codes(rng, nb, bt, n_kv, hd)
    newk = rng.standard_normal((B, rl)).astype(np.float32)
    newv = rng.standard_normal((B, rl)).astype(np.float32)
    q = rng.standard_normal((B, n_head, hd)).astype(np.float32)
    plan = PagedAttention.plan(B, n_head, n_kv, hd, bt, int(pos.max()) + 1, 0, KvDataType.FP8)
    assert plan[0] == 0
    lay = PagedKvLayout(nb, bt, rl, KvDataType.FP8)
    t = lambda a: torch.from_numpy(a).to(dev)
    dks, dvs, dtab, dpos = t(ks), t(vs), i32(tab, dev), i32(pos, dev)
    pool_a = t(codes.copy())
    PagedKvGpu(0).append_kv_e4m3_batched(None, lay, pool_a, t(newk), t(newv), dtab,
                                         i32(np.arange(B + 1), dev), dpos, B, hd, dks, dvs)
    pa = PagedAttention(0)
    sched = PagedAttention.schedule_buffer(B, tab.shape[1], bt, plan)
    pa.build_schedule(None, lay, dtab, dpos, 1, plan, sched)
    pool_b = t(codes.copy())
    out = torch.full((B, n_head, hd), float("nan"), device=dev)
    pa.append_decode_scheduled(None, lay, pool_b, t(newk), t(newv), sched, tab.shape[1], t(q), out,
                               n_head, hd, plan, PagedAttention.workspace(plan), dks, dvs)
    torch.cuda.synchronize()
    pa_np, pb_np = pool_a.cpu().numpy(), pool_b.cpu().numpy()
    assert np.array_equal(pa_np, pb_np), np.argwhere(pa_np != pb_np)[:4]
    ref = orc.sdpa_decode_batched(dequant_pool(pb_np, nb, bt, n_kv, hd, ks, vs), tab, pos + 1, bt,
                                  q, n_head, n_kv, hd)
    check_close(out.cpu().numpy(), ref)
