"""Bytes outside the attended tokens never reach an output.

A page handed out by the allocator holds whatever its last owner (or the
allocator) left.  Here every slot past a sequence's length, every
unreferenced page and the tail of each sequence's last page hold NaN (the
pages of an E4M3 pool the NaN code).  A kernel that let a zero weight meet
such a V row (0 * NaN = NaN) would fail.  The paths covered:
  * the token-balanced decode, self-scheduled and from a step schedule, with
    the fused append, including appends that open a new tile (old length 0,
    16, 32, ...), whose tile's other rows are not written;
  * the same over E4M3 pages;
  * the fixed-split and slot-major kernels of one sequence, with host and
    device positions, the fused append onto a new page, and invalid table
    entries inside the attended range (their stand-in, page 0, is NaN);
  * the single-pass decode of one sequence and the batched fixed-split
    decode;
  * decode over the protected-sinks range, with every unattended row NaN,
    on fixed and seeded random shapes;
  * chunked prefill, both kernels, over f32, f16, bf16 and E4M3 pages, also
    with invalid table entries inside a chunk's causal window (page 0 NaN).
Outputs are compared with the oracle, which reads only the attended tokens,
or, where the table has invalid entries, with a float64 numpy attention over
the tokens on valid pages; the bar is the usual one (tests/parity.py), and
every output must be finite.
"""
import numpy as np
import pytest
import torch

from oracle import orc
from titan_amd import KvDataType, PagedAttention, PagedKvLayout
from titan_amd.flash_attention import FlashAttention2

import parity

pytestmark = pytest.mark.gpu

NONE = 0xFFFFFFFF
TDT = {KvDataType.F32: torch.float32, KvDataType.F16: torch.float16,
       KvDataType.BF16: torch.bfloat16}


def i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(dev)


def tables(rng, n_tok, bt, spare=4):
    need = [(int(n) + bt - 1) // bt for n in n_tok]
    nb = sum(need) + spare
    perm = rng.permutation(nb).astype(np.uint32)
    tab = np.full((len(n_tok), max(max(need), 1)), NONE, np.uint32)
    o = 0
    for b, c in enumerate(need):
        tab[b, :c] = perm[o:o + c]
        o += c
    return tab, nb


def nan_pool(rng, nb, bt, rl, tab, n_tok, dtype):
    """Host pool [nb, bt, 2, rl] of NaN with N(0,1) K/V rows at tokens
    0..n_tok[b]-1 of every sequence (rounded to `dtype`, as f32), and the
    device pool holding exactly those values."""
    host = np.full((nb, bt, 2, rl), np.nan, np.float32)
    for b, n in enumerate(n_tok):
        for t in range(int(n)):
            host[tab[b, t // bt], t % bt] = rng.standard_normal((2, rl)).astype(np.float32)
    t = torch.from_numpy(host.reshape(-1)).to(TDT[dtype])
    return t, t.to(torch.float32).numpy()


def check(gpu, ref, f32, what):
    assert np.isfinite(gpu).all(), what
    parity.check_close(gpu, ref, f32=f32, what=what)


def np_attend(host, table, toks, q, n_head, n_kv, hd):
    """float64 softmax attention of q [n_head, hd] over tokens `toks` of one
    sequence (host pool [nb, bt, 2, rl], GQA: q head h reads kv head
    h // (n_head / n_kv)), scale 1/sqrt(hd)."""
    bt = host.shape[1]
    rows = np.stack([host[table[t // bt], t % bt] for t in toks]).astype(np.float64)
    k = rows[:, 0].reshape(len(toks), n_kv, hd)
    v = rows[:, 1].reshape(len(toks), n_kv, hd)
    out = np.zeros((n_head, hd))
    for h in range(n_head):
        kv = h // (n_head // n_kv)
        s = k[:, kv] @ q[h].astype(np.float64) / np.sqrt(hd)
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ v[:, kv]
    return out


@pytest.mark.parametrize("dtype", [KvDataType.F16, KvDataType.BF16], ids=lambda d: d.name)
def test_balanced_decode_and_steps(dev, dtype):
    """Token-balanced decode (self-scheduled), then the fused step both
    self-scheduled and from a step schedule (append at position len, attend
    len + 1 tokens), on a NaN-tailed pool: 12/2 heads, hd 128, pages of 16,
    lengths on and off the tile and page edges (the appends at 0, 16, 32 and
    1024 open a new tile), one empty sequence."""
    n_head, n_kv, hd, bt = 12, 2, 128, 16
    rl = n_kv * hd
    rng = np.random.default_rng(61 + int(dtype))
    lens = np.array([1, 15, 16, 17, 32, 250, 0, 1024, 47], np.int64)
    B = len(lens)
    tab, nb = tables(rng, lens + 1, bt)
    pool0, host = nan_pool(rng, nb, bt, rl, tab, lens, dtype)
    q = rng.standard_normal((B, n_head, hd)).astype(np.float32)
    dq = torch.from_numpy(q).to(dev)
    pa = PagedAttention(0)
    plan = PagedAttention.plan(B, n_head, n_kv, hd, bt, int(lens.max()) + 1, 0, dtype)
    assert plan[0] == 0
    ws = PagedAttention.workspace(plan)
    dtab = i32(tab, dev)
    out = torch.full((B, n_head, hd), float("nan"), device=dev)
    pool = pool0.to(dev)
    pa.decode_batched(None, dq, pool, dtab, i32(lens, dev), out, n_head, n_kv, hd, bt, dtype,
                      plan, ws)
    torch.cuda.synchronize()
    ref = orc.sdpa_decode_batched(host.reshape(-1), tab, lens.astype(np.uint32), bt, q, n_head,
                                  n_kv, hd)
    check(out.cpu().numpy(), ref, False, f"{dtype.name} decode")
    layout = PagedKvLayout(nb, bt, rl, dtype)
    nk = torch.from_numpy(rng.standard_normal((B, rl)).astype(np.float32)).to(TDT[dtype]).to(dev)
    nv = torch.from_numpy(rng.standard_normal((B, rl)).astype(np.float32)).to(TDT[dtype]).to(dev)
    h = host.reshape(nb, bt, 2, rl).copy()
    for b in range(B):
        L = int(lens[b])
        h[tab[b, L // bt], L % bt, 0] = nk[b].float().cpu().numpy()
        h[tab[b, L // bt], L % bt, 1] = nv[b].float().cpu().numpy()
    ref = orc.sdpa_decode_batched(h.reshape(-1), tab, (lens + 1).astype(np.uint32), bt, q,
                                  n_head, n_kv, hd)
    pos = i32(lens, dev)
    for form in ("self-scheduled", "scheduled"):
        pool = pool0.to(dev)
        out.fill_(float("nan"))
        if form == "scheduled":
            sched = PagedAttention.schedule_buffer(B, tab.shape[1], bt, plan)
            pa.build_schedule(None, layout, dtab, pos, 1, plan, sched)
            pa.append_decode_scheduled(None, layout, pool, nk, nv, sched, tab.shape[1], dq, out,
                                       n_head, hd, plan, ws)
        else:
            pa.append_decode_batched(None, layout, pool, nk, nv, dtab, pos, dq, out, n_head, hd,
                                     plan, ws)
        torch.cuda.synchronize()
        check(out.cpu().numpy(), ref, False, f"{dtype.name} fused step, {form}")


def test_e4m3_decode_and_step(dev):
    """Token-balanced decode over E4M3 pages whose unused slots hold the NaN
    code (0x7F), then the fused E4M3 step (the f32 rows quantised in the
    launch) with appends that open a new tile."""
    n_head, n_kv, hd, bt = 12, 2, 128, 16
    rl = n_kv * hd
    rng = np.random.default_rng(67)
    lens = np.array([3, 16, 31, 300, 0, 77, 32], np.int64)
    B = len(lens)
    tab, nb = tables(rng, lens + 1, bt)
    ks = np.full(n_kv, 4.0 / 448, np.float32)
    vs = np.full(n_kv, 4.0 / 448, np.float32)
    codes = np.full((nb, bt, 2, n_kv, hd), 0x7F, np.uint8)
    for b, n in enumerate(lens):
        for t in range(int(n)):
            x = rng.standard_normal((2, n_kv, hd)).astype(np.float32)
            for hh in range(n_kv):
                codes[tab[b, t // bt], t % bt, 0, hh] = orc.f32_to_e4m3(x[0, hh], ks[hh])
                codes[tab[b, t // bt], t % bt, 1, hh] = orc.f32_to_e4m3(x[1, hh], vs[hh])

    def dequant(c):
        f = orc.e4m3_to_f32(c.reshape(-1)).reshape(nb, bt, 2, n_kv, hd)
        f[:, :, 0] *= ks[None, None, :, None]
        f[:, :, 1] *= vs[None, None, :, None]
        return f.reshape(-1)

    q = rng.standard_normal((B, n_head, hd)).astype(np.float32)
    dq = torch.from_numpy(q).to(dev)
    dks, dvs = torch.from_numpy(ks).to(dev), torch.from_numpy(vs).to(dev)
    plan = PagedAttention.plan(B, n_head, n_kv, hd, bt, int(lens.max()) + 1, 0, KvDataType.FP8)
    ws = PagedAttention.workspace(plan)
    pa = PagedAttention(0)
    dtab = i32(tab, dev)
    out = torch.full((B, n_head, hd), float("nan"), device=dev)
    pool = torch.from_numpy(codes.reshape(-1)).to(dev)
    pa.decode_batched_e4m3(None, dq, pool, dtab, i32(lens, dev), out, n_head, n_kv, hd, bt, dks,
                           dvs, plan, ws)
    torch.cuda.synchronize()
    ref = orc.sdpa_decode_batched(dequant(codes), tab, lens.astype(np.uint32), bt, q, n_head,
                                  n_kv, hd)
    check(out.cpu().numpy(), ref, False, "E4M3 decode")
    nk = rng.standard_normal((B, rl)).astype(np.float32)
    nv = rng.standard_normal((B, rl)).astype(np.float32)
    layout = PagedKvLayout(nb, bt, rl, KvDataType.FP8)
    out.fill_(float("nan"))
    pa.append_decode_batched_e4m3(None, layout, pool, torch.from_numpy(nk).to(dev),
                                  torch.from_numpy(nv).to(dev), dtab, i32(lens, dev), dq, out,
                                  n_head, hd, plan, ws, dks, dvs)
    torch.cuda.synchronize()
    c2 = pool.cpu().numpy().reshape(nb, bt, 2, n_kv, hd)
    for b in range(B):  # the appended codes landed where the oracle's quantiser puts them
        L = int(lens[b])
        for hh in range(n_kv):
            assert np.array_equal(c2[tab[b, L // bt], L % bt, 0, hh],
                                  orc.f32_to_e4m3(nk[b, hh * hd:(hh + 1) * hd], ks[hh]))
            assert np.array_equal(c2[tab[b, L // bt], L % bt, 1, hh],
                                  orc.f32_to_e4m3(nv[b, hh * hd:(hh + 1) * hd], vs[hh]))
    ref = orc.sdpa_decode_batched(dequant(c2), tab, (lens + 1).astype(np.uint32), bt, q, n_head,
                                  n_kv, hd)
    check(out.cpu().numpy(), ref, False, "E4M3 fused step")


@pytest.mark.parametrize("dtype,hd", [(KvDataType.F32, 64), (KvDataType.F16, 64),
                                      (KvDataType.F16, 128)], ids=["f32-64", "f16-64", "f16-128"])
def test_single_sequence_decode(dev, dtype, hd):
    """Split-K decode of one sequence (f32: the fixed-split kernel, config
    1's; f16: the slot-major kernel), 14/2 heads, pages of 16, NaN-tailed:
    host position, device position under a larger grid bound, and (f32,
    which has it) the fused append onto a new page (position 512, the first
    row of its page, not written before the launch)."""
    n_head, n_kv, bt = 14, 2, 16
    rl = n_kv * hd
    rng = np.random.default_rng(71 + hd + int(dtype))
    n = 512
    tab, nb = tables(rng, [n + 200], bt)
    pool0, host = nan_pool(rng, nb, bt, rl, tab, [n], dtype)
    pool = pool0.to(dev)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    dq = torch.from_numpy(q).to(dev)
    f32 = dtype == KvDataType.F32
    ref = orc.sdpa_decode(host.reshape(-1), tab[0], bt, n, q, n_head, n_kv, hd, True, n - 1)
    pa = PagedAttention(0)
    dtab = i32(tab[0], dev)
    out = torch.full((n_head * hd,), float("nan"), device=dev)
    pa.launch_flash_decoding(None, dq, pool, dtab, out, n_head, n_kv, hd, bt, n, n - 1, True,
                             kv_dtype=dtype)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), ref, f32, f"{dtype.name} hd{hd} host position")
    pos = torch.tensor([n - 1], dtype=torch.int32, device=dev)
    out.fill_(float("nan"))
    pa.launch_flash_decoding(None, dq, pool, dtab, out, n_head, n_kv, hd, bt, n + 199, n + 198,
                             True, pos, kv_dtype=dtype)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), ref, f32, f"{dtype.name} hd{hd} device position")
    if f32:
        nk = rng.standard_normal(rl).astype(np.float32)
        nv = rng.standard_normal(rl).astype(np.float32)
        out.fill_(float("nan"))
        pa.append_flash_decoding(None, torch.from_numpy(nk).to(dev), torch.from_numpy(nv).to(dev),
                                 dq, pool, dtab, out, n_head, n_kv, hd, bt, n)
        torch.cuda.synchronize()
        h = host.reshape(nb, bt, 2, rl).copy()
        h[tab[0, n // bt], n % bt, 0] = nk
        h[tab[0, n // bt], n % bt, 1] = nv
        ref = orc.sdpa_decode(h.reshape(-1), tab[0], bt, n + 1, q, n_head, n_kv, hd, True, n)
        check(out.cpu().numpy(), ref, True, "f32 fused append onto a new page")


@pytest.mark.parametrize("dtype,hd", [(KvDataType.F32, 64), (KvDataType.F16, 64),
                                      (KvDataType.F16, 128)], ids=["f32-64", "f16-64", "f16-128"])
def test_single_sequence_invalid_pages(dev, dtype, hd):
    """Invalid table entries inside the attended range mask their tokens;
    the kernels read page 0 in their place, and page 0 here is all NaN.
    Compared with a float64 attention over the tokens on valid pages."""
    n_head, n_kv, bt = 14, 2, 16
    rl = n_kv * hd
    rng = np.random.default_rng(79 + hd + int(dtype))
    n = 300
    n_pg = -(-n // bt)
    nb = n_pg + 3
    table = (1 + rng.permutation(nb - 1)[:n_pg]).astype(np.uint32)   # page 0 is never used
    bad = [2, 7, n_pg - 1]
    table[bad] = [NONE, nb + 40, NONE]
    host = np.full((nb, bt, 2, rl), np.nan, np.float32)
    live = [t for t in range(n) if t // bt not in bad]
    for t in live:
        host[table[t // bt], t % bt] = rng.standard_normal((2, rl)).astype(np.float32)
    pool_t = torch.from_numpy(host.reshape(-1)).to(TDT[dtype])
    host = pool_t.to(torch.float32).numpy().reshape(nb, bt, 2, rl)
    q = rng.standard_normal((n_head, hd)).astype(np.float32)
    ref = np_attend(host, table, live, q, n_head, n_kv, hd).reshape(-1)
    out = torch.full((n_head * hd,), float("nan"), device=dev)
    PagedAttention(0).launch_flash_decoding(None, torch.from_numpy(q.reshape(-1)).to(dev),
                                            pool_t.to(dev), i32(table, dev), out, n_head, n_kv,
                                            hd, bt, n, n - 1, True, kv_dtype=dtype)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), ref, dtype == KvDataType.F32, f"{dtype.name} hd{hd}")


@pytest.mark.parametrize("dtype,kern,hd", [
    (KvDataType.F16, "single", 128), (KvDataType.F16, "pp", 128),
    (KvDataType.BF16, "single", 128), (KvDataType.BF16, "pp", 128),
    (KvDataType.F16, "single", 64), (KvDataType.BF16, "pp", 64),
    (KvDataType.F32, "single", 128), (KvDataType.F32, "single", 64)],
    ids=lambda v: getattr(v, "name", str(v)))
def test_prefill(dev, monkeypatch, dtype, kern, hd):
    """Causal chunked prefill over NaN-tailed pages, both kernels (f32 pages
    have one): keys past each chunk's last position (the rest of its last
    page) and unreferenced pages hold NaN."""
    monkeypatch.setenv("EH_PREFILL_KERNEL", kern)
    nh, nkv, bt = 16, 4, 16
    rl = nkv * hd
    rng = np.random.default_rng(73 + int(dtype))
    starts, lens = np.array([0, 37, 200]), np.array([45, 100, 9])
    n_tok = starts + lens
    tab, nb = tables(rng, n_tok, bt)
    pool, host = nan_pool(rng, nb, bt, rl, tab, n_tok, dtype)
    total = int(lens.sum())
    q = rng.standard_normal((total, nh, hd)).astype(np.float32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    out = torch.full((total, nh, hd), float("nan"), device=dev)
    FlashAttention2(0).launch_batched(None, torch.from_numpy(q).to(dev), pool.to(dev),
                                      i32(tab, dev), i32(cu, dev), i32(starts, dev), out, nh, nkv,
                                      hd, bt, int(lens.max()), kv_dtype=dtype)
    torch.cuda.synchronize()
    g = out.cpu().numpy()
    for b in range(len(lens)):
        k = (int(n_tok[b]) + bt - 1) // bt
        ref = orc.prefill_causal(host.reshape(-1), tab[b, :k], bt, q[cu[b]:cu[b + 1]],
                                 int(lens[b]), int(starts[b]), nh, nkv, hd)
        check(g[cu[b]:cu[b + 1]], ref, dtype == KvDataType.F32, f"{dtype.name} {kern} seq {b}")


@pytest.mark.parametrize("dtype,kern", [
    (KvDataType.F16, "single"), (KvDataType.F16, "pp"), (KvDataType.BF16, "single"),
    (KvDataType.BF16, "pp"), (KvDataType.F32, "single")],
    ids=lambda v: getattr(v, "name", str(v)))
def test_prefill_invalid_pages(dev, monkeypatch, dtype, kern):
    """Invalid table entries inside a prefill chunk's causal window mask
    their keys; both kernels read page 0 in their place, and page 0 here is
    all NaN.  Every query row against a float64 attention over its causal
    keys on valid pages."""
    monkeypatch.setenv("EH_PREFILL_KERNEL", kern)
    nh, nkv, hd, bt = 8, 2, 128, 16
    rl = nkv * hd
    rng = np.random.default_rng(83 + int(dtype))
    p0, nq = 40, 90
    n = p0 + nq
    n_pg = -(-n // bt)
    nb = n_pg + 3
    table = (1 + rng.permutation(nb - 1)[:n_pg]).astype(np.uint32)   # page 0 is never used
    bad = [1, 5]
    table[bad] = [NONE, nb + 9]
    host = np.full((nb, bt, 2, rl), np.nan, np.float32)
    for t in range(n):
        if t // bt not in bad:
            host[table[t // bt], t % bt] = rng.standard_normal((2, rl)).astype(np.float32)
    pool_t = torch.from_numpy(host.reshape(-1)).to(TDT[dtype])
    host = pool_t.to(torch.float32).numpy().reshape(nb, bt, 2, rl)
    q = rng.standard_normal((nq, nh, hd)).astype(np.float32)
    out = torch.full((nq, nh, hd), float("nan"), device=dev)
    FlashAttention2(0).launch_batched(None, torch.from_numpy(q).to(dev), pool_t.to(dev),
                                      i32(table[None, :], dev), i32(np.array([0, nq]), dev),
                                      i32(np.array([p0]), dev), out, nh, nkv, hd, bt, nq,
                                      kv_dtype=dtype)
    torch.cuda.synchronize()
    g = out.cpu().numpy()
    assert np.isfinite(g).all()
    ref = np.stack([np_attend(host, table, [t for t in range(p0 + i + 1) if t // bt not in bad],
                              q[i], nh, nkv, hd) for i in range(nq)])
    check(g, ref, dtype == KvDataType.F32, f"{dtype.name} {kern}")


def e4m3_pool(rng, nb, bt, n_kv, hd, rows):
    """E4M3 pool [nb, bt, 2, n_kv, hd] of the NaN code (0x7F) with quantised
    N(0,1) K/V at the (page, slot) pairs in `rows`, scales 4 / 448; returns
    the codes, the dequantised f32 pool and the scales."""
    ks = np.full(n_kv, 4.0 / 448, np.float32)
    vs = np.full(n_kv, 4.0 / 448, np.float32)
    codes = np.full((nb, bt, 2, n_kv, hd), 0x7F, np.uint8)
    for pg, sl in rows:
        x = rng.standard_normal((2, n_kv, hd)).astype(np.float32)
        for hh in range(n_kv):
            codes[pg, sl, 0, hh] = orc.f32_to_e4m3(x[0, hh], ks[hh])
            codes[pg, sl, 1, hh] = orc.f32_to_e4m3(x[1, hh], vs[hh])
    f = orc.e4m3_to_f32(codes.reshape(-1)).reshape(nb, bt, 2, n_kv, hd)
    f[:, :, 0] *= ks[None, None, :, None]
    f[:, :, 1] *= vs[None, None, :, None]
    return codes, f.reshape(nb, bt, 2, n_kv * hd), ks, vs


@pytest.mark.parametrize("kern", ["single", "pp"])
def test_e4m3_prefill(dev, monkeypatch, kern):
    """Causal chunked prefill over E4M3 pages, both kernels: NaN codes past
    each chunk's last position and on unreferenced pages, then a chunk whose
    table has invalid entries inside its causal window (page 0, their
    stand-in, all NaN codes)."""
    monkeypatch.setenv("EH_PREFILL_KERNEL", kern)
    nh, nkv, hd, bt = 16, 4, 128, 16
    rng = np.random.default_rng(89)
    starts, lens = np.array([0, 37, 200]), np.array([45, 100, 9])
    n_tok = starts + lens
    tab, nb = tables(rng, n_tok, bt)
    rows = [(int(tab[b, t // bt]), t % bt) for b, n in enumerate(n_tok) for t in range(int(n))]
    codes, host, ks, vs = e4m3_pool(rng, nb, bt, nkv, hd, rows)
    dks, dvs = torch.from_numpy(ks).to(dev), torch.from_numpy(vs).to(dev)
    total = int(lens.sum())
    q = rng.standard_normal((total, nh, hd)).astype(np.float32)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    out = torch.full((total, nh, hd), float("nan"), device=dev)
    fa = FlashAttention2(0)
    fa.launch_batched_e4m3(None, torch.from_numpy(q).to(dev),
                           torch.from_numpy(codes.reshape(-1)).to(dev), i32(tab, dev),
                           i32(cu, dev), i32(starts, dev), out, nh, nkv, hd, bt,
                           int(lens.max()), dks, dvs)
    torch.cuda.synchronize()
    g = out.cpu().numpy()
    for b in range(len(lens)):
        k = (int(n_tok[b]) + bt - 1) // bt
        ref = orc.prefill_causal(host.reshape(-1), tab[b, :k], bt, q[cu[b]:cu[b + 1]],
                                 int(lens[b]), int(starts[b]), nh, nkv, hd)
        check(g[cu[b]:cu[b + 1]], ref, False, f"E4M3 {kern} seq {b}")

    p0, nq = 40, 90
    n = p0 + nq
    n_pg = -(-n // bt)
    nb = n_pg + 3
    table = (1 + rng.permutation(nb - 1)[:n_pg]).astype(np.uint32)   # page 0 is never used
    bad = [1, 5]
    table[bad] = [NONE, nb + 9]
    rows = [(int(table[t // bt]), t % bt) for t in range(n) if t // bt not in bad]
    codes, host, ks, vs = e4m3_pool(rng, nb, bt, nkv, hd, rows)
    q = rng.standard_normal((nq, nh, hd)).astype(np.float32)
    out = torch.full((nq, nh, hd), float("nan"), device=dev)
    fa.launch_batched_e4m3(None, torch.from_numpy(q).to(dev),
                           torch.from_numpy(codes.reshape(-1)).to(dev), i32(table[None, :], dev),
                           i32(np.array([0, nq]), dev), i32(np.array([p0]), dev), out, nh, nkv,
                           hd, bt, nq, dks, dvs)
    torch.cuda.synchronize()
    ref = np.stack([np_attend(host, table, [t for t in range(p0 + i + 1) if t // bt not in bad],
                              q[i], nh, nkv, hd) for i in range(nq)])
    check(out.cpu().numpy(), ref, False, f"E4M3 {kern} invalid pages")


@pytest.mark.parametrize("dtype", [KvDataType.F16, KvDataType.BF16, KvDataType.FP8],
                         ids=lambda d: d.name)
@pytest.mark.parametrize("sink,window", [(4, 15), (0, 40), (5, 3), (20, 100), (17, 1)])
def test_window_decode_unattended_rows(dev, dtype, sink, window):
    """Decode over the protected-sinks range where every token outside the
    sinks and the window holds NaN on its valid page (and the page tails and
    unreferenced pages too): tiles that the range cuts (the sink edge, the
    window's first tile, the last tile) mix attended and NaN rows.  Output and
    per-page H2O mass against the oracle, which reads only attended tokens."""
    n_head, n_kv, hd, bt = 12, 2, 128, 16
    rl = n_kv * hd
    rng = np.random.default_rng(71 + 3 * sink + window + int(dtype))
    lens = np.array([0, 1, 5, 17, 33, 300, 2049, 100, 7, 64], np.int64)
    B = len(lens)
    tab, nb = tables(rng, lens, bt)

    def attended(n):
        if n == 0:
            return []
        lo = max(sink, n - 1 - window)
        return [t for t in range(n) if t < sink or t >= lo]

    ks = vs = None
    if dtype == KvDataType.FP8:
        ksn = np.full(n_kv, 4.0 / 448, np.float32)
        vsn = np.full(n_kv, 4.0 / 448, np.float32)
        codes = np.full((nb, bt, 2, n_kv, hd), 0x7F, np.uint8)
        for b, n in enumerate(lens):
            for t in attended(int(n)):
                x = rng.standard_normal((2, n_kv, hd)).astype(np.float32)
                for hh in range(n_kv):
                    codes[tab[b, t // bt], t % bt, 0, hh] = orc.f32_to_e4m3(x[0, hh], ksn[hh])
                    codes[tab[b, t // bt], t % bt, 1, hh] = orc.f32_to_e4m3(x[1, hh], vsn[hh])
        f = orc.e4m3_to_f32(codes.reshape(-1)).reshape(nb, bt, 2, n_kv, hd)
        f[:, :, 0] *= ksn[None, None, :, None]
        f[:, :, 1] *= vsn[None, None, :, None]
        host = f.reshape(-1)
        pool = torch.from_numpy(codes.reshape(-1)).to(dev)
        ks, vs = torch.from_numpy(ksn).to(dev), torch.from_numpy(vsn).to(dev)
    else:
        h = np.full((nb, bt, 2, rl), np.nan, np.float32)
        for b, n in enumerate(lens):
            for t in attended(int(n)):
                h[tab[b, t // bt], t % bt] = rng.standard_normal((2, rl)).astype(np.float32)
        t16 = torch.from_numpy(h.reshape(-1)).to(TDT[dtype])
        host, pool = t16.to(torch.float32).numpy(), t16.to(dev)
    q = rng.standard_normal((B, n_head, hd)).astype(np.float32)
    plan = PagedAttention.plan(B, n_head, n_kv, hd, bt, int(lens.max()), 0, dtype)
    extra = PagedAttention.mass_workspace_bytes(B, tab.shape[1], bt, n_head)
    ws = torch.zeros((plan[2] + extra + 3) // 4, device=dev)
    mass = torch.zeros((nb,), device=dev)
    out = torch.full((B, n_head, hd), float("nan"), device=dev)
    PagedAttention(0).decode_batched_window(None, torch.from_numpy(q).to(dev), pool, i32(tab, dev),
                                            i32(lens, dev), out, n_head, n_kv, hd, bt, dtype, sink,
                                            window, plan, ws, ks, vs, block_mass=mass)
    torch.cuda.synchronize()
    ref, ref_mass = orc.sdpa_decode_window_batched(host, tab, lens.astype(np.uint32), bt, q, n_head,
                                                   n_kv, hd, sink, window, n_blocks=nb)
    check(out.cpu().numpy(), ref, False, f"{dtype.name} window {sink}/{window}")
    got = mass.cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all()
    bad = np.abs(got - ref_mass) > 2e-4 * n_head + 1e-3 * ref_mass
    assert not bad.any(), (np.argwhere(bad)[:4], got[bad][:4], ref_mass[bad][:4])


@pytest.mark.parametrize("seed", range(12))
def test_window_random_sweep(dev, seed):
    """Decode over the protected-sinks range on seeded random shapes: f16,
    bf16 or E4M3 pages; 1/2/4/8 kv heads with 1-8 q heads each; pages of 16,
    32 or 64 tokens; 1-16 sequences of 0-2500 tokens; sinks and windows on and
    off tile edges; a planner or forced grid.  Every unattended row holds NaN.
    Output and per-page H2O mass against the oracle."""
    rng = np.random.default_rng(500_000 + seed)
    dtype = (KvDataType.F16, KvDataType.BF16, KvDataType.FP8)[int(rng.integers(3))]
    n_kv = int(rng.choice([1, 2, 4, 8]))
    g = int(rng.choice([1, 2, 3, 4, 6, 8]))
    n_head, hd, bt = g * n_kv, 128, int(rng.choice([16, 32, 64]))
    rl = n_kv * hd
    B = int(rng.integers(1, 17))
    lens = np.where(rng.integers(0, 2, B) == 0, rng.integers(0, 70, B),
                    rng.integers(70, 2500, B)).astype(np.int64)
    sink = int(rng.choice([0, 1, 4, 15, 16, 17, 40]))
    window = int(rng.choice([1, 3, 15, 16, 31, 64, 100, 700]))
    tab, nb = tables(rng, lens, bt)

    def attended(n):
        if n == 0:
            return []
        lo = max(sink, n - 1 - window)
        return [t for t in range(n) if t < sink or t >= lo]

    ks = vs = None
    if dtype == KvDataType.FP8:
        rows = [(int(tab[b, t // bt]), t % bt) for b, n in enumerate(lens) for t in attended(int(n))]
        codes, host, ksn, vsn = e4m3_pool(rng, nb, bt, n_kv, hd, rows)
        host = host.reshape(-1)
        pool = torch.from_numpy(codes.reshape(-1)).to(dev)
        ks, vs = torch.from_numpy(ksn).to(dev), torch.from_numpy(vsn).to(dev)
    else:
        h = np.full((nb, bt, 2, rl), np.nan, np.float32)
        for b, n in enumerate(lens):
            for t in attended(int(n)):
                h[tab[b, t // bt], t % bt] = rng.standard_normal((2, rl)).astype(np.float32)
        t16 = torch.from_numpy(h.reshape(-1)).to(TDT[dtype])
        host, pool = t16.to(torch.float32).numpy(), t16.to(dev)
    q = rng.standard_normal((B, n_head, hd)).astype(np.float32)
    plan = PagedAttention.plan(B, n_head, n_kv, hd, bt, max(int(lens.max()), 1), 0, dtype)
    assert plan[0] == 0
    if rng.integers(2):
        plan = PagedAttention.with_grid(plan, int(rng.choice([1, 2, 7, 64, 333])), B, n_head)
    extra = PagedAttention.mass_workspace_bytes(B, tab.shape[1], bt, n_head)
    ws = torch.zeros((plan[2] + extra + 3) // 4, device=dev)
    mass = torch.zeros((nb,), device=dev)
    out = torch.full((B, n_head, hd), float("nan"), device=dev)
    print(f"[window sweep {seed}] {dtype.name} heads {n_head}/{n_kv} page {bt} B {B} sink {sink} "
          f"window {window} max len {int(lens.max())}", flush=True)
    PagedAttention(0).decode_batched_window(None, torch.from_numpy(q).to(dev), pool, i32(tab, dev),
                                            i32(lens, dev), out, n_head, n_kv, hd, bt, dtype, sink,
                                            window, plan, ws, ks, vs, block_mass=mass)
    torch.cuda.synchronize()
    ref, ref_mass = orc.sdpa_decode_window_batched(host, tab, lens.astype(np.uint32), bt, q, n_head,
                                                   n_kv, hd, sink, window, n_blocks=nb)
    check(out.cpu().numpy(), ref, False, f"window sweep {seed}")
    got = mass.cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all()
    bad = np.abs(got - ref_mass) > 2e-4 * n_head + 1e-3 * ref_mass
    assert not bad.any(), (np.argwhere(bad)[:4], got[bad][:4], ref_mass[bad][:4])


@pytest.mark.parametrize("dtype,hd", [(KvDataType.F32, 64), (KvDataType.F16, 64),
                                      (KvDataType.BF16, 32), (KvDataType.F16, 128)],
                         ids=lambda v: getattr(v, "name", str(v)))
def test_single_pass_and_fixed_split_batched(dev, dtype, hd):
    """The single-pass decode of one sequence (`eh_paged_attention`, host and
    device positions) and the batched fixed-split decode (head sizes outside
    the balanced kernel, or a caller's tokens_per_split) over NaN-tailed
    pages, against the oracle."""
    n_head, n_kv, bt = 8, 2, 16
    rl = n_kv * hd
    rng = np.random.default_rng(97 + hd + int(dtype))
    f32 = dtype == KvDataType.F32
    pa = PagedAttention(0)
    n = 300
    tab, nb = tables(rng, [n + 40], bt)
    pool0, host = nan_pool(rng, nb, bt, rl, tab, [n], dtype)
    pool = pool0.to(dev)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    ref = orc.sdpa_decode(host.reshape(-1), tab[0], bt, n, q, n_head, n_kv, hd, True, n - 1)
    out = torch.full((n_head * hd,), float("nan"), device=dev)
    pa.launch(None, torch.from_numpy(q).to(dev), pool, i32(tab[0], dev), out, n_head, n_kv, hd, bt,
              n, n - 1, True, kv_dtype=dtype)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), ref, f32, f"{dtype.name} hd{hd} single pass")
    out.fill_(float("nan"))
    pa.launch_with_pos_ptr(None, torch.from_numpy(q).to(dev), pool, i32(tab[0], dev), out, n_head,
                           n_kv, hd, bt, n + 39, n + 38, True,
                           torch.tensor([n - 1], dtype=torch.int32, device=dev), kv_dtype=dtype)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), ref, f32, f"{dtype.name} hd{hd} single pass, device position")

    lens = np.array([1, 15, 16, 17, 250, 0, 600, 47], np.int64)
    B = len(lens)
    tab, nb = tables(rng, lens, bt)
    pool0, host = nan_pool(rng, nb, bt, rl, tab, lens, dtype)
    qb = rng.standard_normal((B, n_head, hd)).astype(np.float32)
    plan = PagedAttention.plan(B, n_head, n_kv, hd, bt, int(lens.max()), 64, dtype)
    assert plan[0] != 0  # fixed splits (16-bit pages round the hint up to 256 tokens)
    out = torch.full((B, n_head, hd), float("nan"), device=dev)
    pa.decode_batched(None, torch.from_numpy(qb).to(dev), pool0.to(dev), i32(tab, dev),
                      i32(lens, dev), out, n_head, n_kv, hd, bt, dtype, plan,
                      PagedAttention.workspace(plan))
    torch.cuda.synchronize()
    ref = orc.sdpa_decode_batched(host.reshape(-1), tab, lens.astype(np.uint32), bt, qb, n_head,
                                  n_kv, hd)
    check(out.cpu().numpy(), ref, f32, f"{dtype.name} hd{hd} fixed-split batched")
