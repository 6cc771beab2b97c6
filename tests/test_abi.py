"""CPU checks of the C-ABI library: it loads, exports every declared symbol,
the code objects hold every kernel the launcher names, host-only entry points
behave, and the host bookkeeping equals the oracle's PagedKvCache bit for bit.
No GPU compute is called."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from oracle import orc
from titan_amd import _lib
from titan_amd.errors import KvCacheError, check

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in sorted(os.listdir(os.path.join(ROOT, "include"))):
        text = open(os.path.join(ROOT, "include", h)).read()
        names |= set(re.findall(r"\b(eh_\w+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol():
    L = _lib.load()
    missing = [n for n in sorted(declared_symbols()) if not hasattr(L, n)]
    assert not missing, missing
    assert declared_symbols() == set(_lib.EXPORTED)


def test_rust_binding_declares_every_entry_point():
    """The integration guide's complete extern block names exactly the
    functions the headers declare (the Rust side a maintainer would add)."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = text[text.index("## Appendix: the complete `extern \"C\"` block"):]
    declared_in_rust = set(re.findall(r"pub fn (eh_\w+)\(", block))
    assert declared_in_rust == declared_symbols()


def test_code_objects_contain_launched_kernels():
    kv = open(os.path.join(_lib.LIB_DIR, "paged_kv.hsaco"), "rb").read()
    for ch in (16, 8, 4, 2):
        for k in ("eh_append_kv_c", "eh_gather_kv_c", "eh_copy_pages_c"):
            assert f"{k}{ch}".encode() in kv
    for k in ("eh_remap_block_tables", "eh_page_refcounts", "eh_fill_u32", "eh_append_kv_e4m3",
              "eh_gather_kv_e4m3", "eh_kv_e4m3_scales", "eh_stream_pages_d1",
              "eh_stream_pages_d2", "eh_stream_pages_heads"):
        assert k.encode() in kv
    for dt in ("f32", "f16", "bf16"):
        dec = open(os.path.join(_lib.LIB_DIR, f"paged_decode_{dt}.hsaco"), "rb").read()
        for hd in (4, 8, 16, 32, 64, 128, 256):
            for g in (1, 2, 4, 6, 7, 8):
                assert f"eh_decode_split_{dt}_hd{hd}_g{g}".encode() in dec
        assert b"eh_decode_merge" in dec
    for dt in ("f16", "bf16", "fp8"):
        tl = open(os.path.join(_lib.LIB_DIR, f"paged_decode_tiles_{dt}.hsaco"), "rb").read()
        for g in (1, 2, 4, 6, 8):
            assert f"eh_decode_tiles_{dt}_hd128_g{g}".encode() in tl
            assert f"eh_decode_tiles_{dt}_hd128_g{g}_ext".encode() in tl
            assert f"eh_decode_tiles_{dt}_hd128_g{g}_sched".encode() in tl
        assert b"eh_decode_tiles_merge" in tl and b"eh_decode_tiles_mass" in tl
        assert b"eh_decode_tiles_merge_sched" in tl and b"eh_decode_tiles_schedule" in tl
    pf = open(os.path.join(_lib.LIB_DIR, "paged_prefill.hsaco"), "rb").read()
    for dt in ("f32", "f16", "bf16"):
        for hd in (64, 128):
            assert f"eh_prefill_{dt}_hd{hd}".encode() in pf


def test_status_names_and_layout_bytes():
    L = _lib.load()
    assert L.eh_status_name(1) == b"InvalidSize" and L.eh_status_name(20) == b"PoolExhausted"
    lay = _lib.eh_kv_layout(10, 16, 256, 1, 0)
    assert L.eh_kv_layout_bytes_total(C.byref(lay)) == 10 * 16 * 2 * 256 * 2
    assert [L.eh_kv_element_bytes(d) for d in range(4)] == [4, 2, 1, 2]


def test_null_context_is_rejected_before_any_hip_call():
    L = _lib.load()
    lay = _lib.eh_kv_layout(1, 1, 1, 0, 0)
    st = L.eh_append_kv(None, None, C.byref(lay), None, 0, None, 0, None, 0, None, 0, 0, 0, None)
    assert st == 21


def test_decode_plan():
    L = _lib.load()
    tps, ms, ws = C.c_uint32(), C.c_uint32(), C.c_uint64()
    assert L.eh_decode_plan(1, 32, 12, 2, 128, 16, 4096, 256, C.byref(tps), C.byref(ms),
                            C.byref(ws)) == 0
    assert (tps.value, ms.value) == (256, 16)
    assert ws.value == 32 * 12 * 16 * (128 + 2) * 4
    # the split bound is capped at 256 by growing the split size
    assert L.eh_decode_plan(1, 1, 32, 8, 128, 16, 1 << 20, 64, C.byref(tps), C.byref(ms),
                            C.byref(ws)) == 0
    assert ms.value <= 256 and tps.value * ms.value >= 1 << 20
    assert L.eh_decode_plan(1, 1, 12, 2, 128, 16, 100, 256, C.byref(tps), C.byref(ms),
                            C.byref(ws)) == 0
    assert ms.value == 1 and ws.value == 0
    assert L.eh_decode_plan(1, 1, 12, 5, 128, 16, 100, 0, C.byref(tps), C.byref(ms),
                            C.byref(ws)) == 21
    # a split's block-table slice must fit the 1024-entry LDS stage
    assert L.eh_decode_plan(1, 1, 12, 2, 128, 1, 100000, 2048, C.byref(tps), C.byref(ms),
                            C.byref(ws)) == 1
    # fixed-split kernel (f32): the split granularity is one round of its four
    # waves (4 tokens each at head_dim 64), so a hint of 20 rounds up to 32
    assert L.eh_decode_plan(0, 1, 14, 2, 64, 16, 512, 20, C.byref(tps), C.byref(ms),
                            C.byref(ws)) == 0
    assert (tps.value, ms.value) == (32, 16)
    assert ws.value == 14 * 16 * (64 + 2) * 4


_SIZE_CHECKS = r"""
import ctypes as C, json, sys
sys.path.insert(0, sys.argv[1])
from titan_amd import _lib
L = _lib.load()
ctx = C.c_void_p(64)   # never dereferenced: every case is rejected before the context is used
U64 = 2**64 - 1

def err():
    e, a = C.c_uint64(), C.c_uint64()
    L.eh_last_error(C.byref(e), C.byref(a), None, None)
    return e.value, a.value

def lay(nb, bt, rl, dt=1):
    return _lib.eh_kv_layout(nb, bt, rl, dt, 0)

out = {}
def run(name, st):
    out[name] = (st, *err())

buf = C.c_void_p(4096)
for name, l in (("bt0", lay(4, 0, 256)), ("bt_big", lay(4, 2**31, 256)), ("rl0", lay(4, 16, 0)),
                ("row_big", lay(4, 16, 2**30, 0)), ("pool_wrap", lay(2**62, 16, 256))):
    run("append_" + name, L.eh_append_kv(ctx, None, C.byref(l), buf, 1 << 20, buf, 1 << 20, buf,
                                         1 << 20, buf, 64, 0, 1, None))
run("gather_bt0", L.eh_gather_kv(ctx, None, C.byref(lay(4, 0, 256)), buf, 1 << 20, buf, 64, buf,
                                 1 << 20, 0, 1, 0))
run("copy_bt0", L.eh_copy_pages(ctx, None, C.byref(lay(4, 0, 256)), buf, 1 << 20, buf, buf, 1))
run("sched_rl0", L.eh_decode_schedule(ctx, None, C.byref(lay(4, 16, 0)), buf, 64, 1, buf, 1, 1, 1,
                                      buf, 1 << 20))
# a page of 2^30 tokens x 2 x 2^30 kv heads x 128 x 4 B is 2^70 bytes: it wrapped to 0 before
run("prefill_page_wrap", L.eh_flash_attention_prefill(ctx, None, 0, buf, 2**40, buf, 1 << 20, buf,
                                                      4, buf, 2**40, 2**30, 2**30, 128, 2**30, 1,
                                                      0, None))
# measurement aids: layout, page size, depth, grid and buffer checks
f16 = lay(4, 16, 256)  # 16 KiB pages, pool 64 KiB
run("stream_bt0", L.eh_stream_pages(ctx, None, C.byref(lay(4, 0, 256)), buf, 1 << 20, buf, 64, 1,
                                    1, 1, buf, 64))
run("stream_page", L.eh_stream_pages(ctx, None, C.byref(lay(4, 8, 256)), buf, 1 << 20, buf, 64, 1,
                                     1, 1, buf, 64))
run("stream_pool", L.eh_stream_pages(ctx, None, C.byref(f16), buf, 1000, buf, 64, 1, 1, 1, buf, 64))
run("stream_depth", L.eh_stream_pages(ctx, None, C.byref(f16), buf, 1 << 16, buf, 64, 1, 3, 1, buf,
                                      64))
run("stream_grid0", L.eh_stream_pages(ctx, None, C.byref(f16), buf, 1 << 16, buf, 64, 1, 1, 0, buf,
                                      64))
run("stream_ids", L.eh_stream_pages(ctx, None, C.byref(f16), buf, 1 << 16, buf, 8, 10, 1, 1, buf,
                                    64))
run("stream_out", L.eh_stream_pages(ctx, None, C.byref(f16), buf, 1 << 16, buf, 64, 1, 1, 4, buf,
                                    64))
run("heads_bt32", L.eh_stream_pages_heads(ctx, None, C.byref(lay(4, 32, 256)), buf, 1 << 20, buf,
                                          64, 1, 128, 1, buf, 64))
run("heads_hd96", L.eh_stream_pages_heads(ctx, None, C.byref(f16), buf, 1 << 16, buf, 64, 1, 96, 1,
                                          buf, 64))
run("heads_hd64", L.eh_stream_pages_heads(ctx, None, C.byref(f16), buf, 1 << 16, buf, 64, 1, 64, 1,
                                          buf, 64))
run("heads_nkv3", L.eh_stream_pages_heads(ctx, None, C.byref(lay(4, 16, 384)), buf, 1 << 20, buf,
                                          64, 1, 128, 1, buf, 64))
run("heads_grid0", L.eh_stream_pages_heads(ctx, None, C.byref(f16), buf, 1 << 16, buf, 64, 1, 128,
                                           0, buf, 64))
run("heads_out", L.eh_stream_pages_heads(ctx, None, C.byref(f16), buf, 1 << 16, buf, 64, 1, 128, 4,
                                         buf, 64))
print(json.dumps(out))
"""


def test_layout_and_size_checks_before_any_hip_call():
    """Pool layouts that would divide by zero or pass a wrapped size, and a
    prefill whose page size passes 64 bits, are rejected with InvalidSize
    before the context is used: block_tokens 0 or above 2^31 - 1, row_len 0,
    rows of 2^31 bytes or more, and a pool or page size beyond 64 bits (the
    expected size saturates at UINT64_MAX). The read-ceiling measurement aids
    reject page sizes, depths, head shapes, grids and short buffers outside
    their contract with the status and (expected, actual) pair of each rule.
    The calls run in a child process, so a regression shows as a failed test,
    not a crashed run."""
    import json
    import subprocess
    import sys
    r = subprocess.run([sys.executable, "-c", _SIZE_CHECKS, ROOT], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    got = json.loads(r.stdout.strip().splitlines()[-1])
    bad, uns = 1, 30  # EH_INVALID_SIZE, EH_UNSUPPORTED
    imax, u64 = 2**31 - 1, 2**64 - 1
    want = {
        "append_bt0": (bad, 1, 0), "append_bt_big": (bad, imax, 2**31), "append_rl0": (bad, 1, 0),
        "append_row_big": (bad, imax, 2**32), "append_pool_wrap": (bad, u64, 1 << 20),
        "gather_bt0": (bad, 1, 0), "copy_bt0": (bad, 1, 0), "sched_rl0": (bad, 1, 0),
        "prefill_page_wrap": (bad, u64, 1 << 20),
        "stream_bt0": (bad, 1, 0), "stream_page": (uns, 16384, 8192),
        "stream_pool": (bad, 1 << 16, 1000), "stream_depth": (uns, 2, 3),
        "stream_grid0": (bad, 1, 0), "stream_ids": (bad, 40, 8), "stream_out": (bad, 128, 64),
        "heads_bt32": (uns, 16, 32), "heads_hd96": (bad, 96, 256), "heads_hd64": (uns, 256, 128),
        "heads_nkv3": (uns, 8, 3), "heads_grid0": (bad, 1, 0), "heads_out": (bad, 128, 64),
    }
    assert {k: tuple(v) for k, v in got.items()} == want


def test_grid_workspace_bytes():
    """Workspace of a token-balanced decode at a caller-chosen grid: one
    (acc, m, l) partial per run and per sequence, 4 * (grid + batch) * n_head
    * 130 bytes, saturating at UINT64_MAX where that leaves 64 bits."""
    L = _lib.load()
    assert L.eh_decode_grid_workspace_bytes(1024, 32, 12) == 4 * (1024 + 32) * 12 * 130
    assert L.eh_decode_grid_workspace_bytes(1, 0, 1) == 520
    assert L.eh_decode_grid_workspace_bytes(0, 0, 7) == 0
    big = 4 * (2**32 - 1 + 2**32 - 1) * (2**32 - 1) * 130
    assert big >= 2**64
    assert L.eh_decode_grid_workspace_bytes(2**32 - 1, 2**32 - 1, 2**32 - 1) == 2**64 - 1
    # either side of the 64-bit limit at n_head = 2^32 - 1
    h = 2**32 - 1
    assert 520 * 8_000_000 * h < 2**64 <= 520 * 9_000_000 * h
    assert L.eh_decode_grid_workspace_bytes(8_000_000, 0, h) == 520 * 8_000_000 * h
    assert L.eh_decode_grid_workspace_bytes(8_999_000, 1_000, h) == 2**64 - 1


class HostCache:
    """Thin driver of the product's host bookkeeping through the C-ABI."""

    def __init__(self, *cfg):
        self.L = _lib.load()
        h = C.c_void_p()
        check(self.L.eh_kvcache_new(*cfg, 0, C.byref(h)), host=True)
        self.h = h

    def __del__(self):
        if getattr(self, "h", None):
            self.L.eh_kvcache_destroy(self.h)

    def table(self, s):
        n = self.L.eh_kvcache_block_table(self.h, s, None, 0)
        out = np.zeros(max(n, 1), np.uint32)
        self.L.eh_kvcache_block_table(self.h, s, out.ctypes.data, n)
        return out[:n].tolist()

    def reserve(self, s, n):
        st = C.c_uint64()
        check(self.L.eh_kvcache_reserve(self.h, s, n, C.byref(st)), host=True)
        return st.value


@pytest.mark.parametrize("args,msg", [
    ((0, 16, 1, 1), "n_blocks must be non-zero"),
    ((1, 0, 1, 1), "block_tokens must be non-zero"),
    ((1, 1, 0, 1), "heads and head_dim must be non-zero"),
])
def test_host_cache_invalid_config(args, msg):
    with pytest.raises(KvCacheError) as e:
        HostCache(*args)
    assert e.value.kind == "InvalidArgs" and e.value.msg == msg


def test_host_bookkeeping_matches_oracle_random_schedule():
    """Random interleaving of new/append/free on both implementations: block
    tables, counts, usage and exhaustion points agree exactly."""
    rng = np.random.default_rng(1234)
    nb, bt = 37, 5
    o = orc.Cache(nb, bt, 1, 2)
    order = rng.permutation(nb)
    o.seed_free_list(order)
    p = HostCache(nb, bt, 1, 2)
    check(p.L.eh_kvcache_seed_free_list(p.h, order.astype(np.uint32).ctypes.data, nb), host=True)
    seqs = []
    row = np.zeros(2, np.float32)
    for it in range(3000):
        r = rng.random()
        if r < 0.05 or not seqs:
            seqs.append(o.new_sequence())
            assert p.L.eh_kvcache_new_sequence(p.h) == seqs[-1]
        elif r < 0.1:
            s = int(rng.choice(seqs))
            o.free_sequence(s)
            p.L.eh_kvcache_free_sequence(p.h, s)
        else:
            s = int(rng.choice(seqs))
            err_o = err_p = None
            try:
                o.append(s, row, row)
            except orc.KvCacheError as e:
                err_o = (e.kind, e.blocks_used, e.blocks_total)
            try:
                p.reserve(s, 1)
            except KvCacheError as e:
                err_p = (e.kind, e.blocks_used, e.blocks_total)
            assert err_o == err_p
        assert o.blocks_used() == p.L.eh_kvcache_blocks_used(p.h)
    for s in seqs:
        assert o.seq_block_table(s).tolist() == p.table(s)
        assert o.token_count(s) == p.L.eh_kvcache_token_count(p.h, s)


def test_host_reserve_many_equals_repeated_single():
    o = orc.Cache(50, 4, 1, 2)
    p = HostCache(50, 4, 1, 2)
    s = o.new_sequence()
    p.L.eh_kvcache_new_sequence(p.h)
    row = np.zeros(2, np.float32)
    for n in (3, 1, 9, 4, 0, 17):
        for _ in range(n):
            o.append(s, row, row)
        p.reserve(s, n)
        assert o.seq_block_table(s).tolist() == p.table(s)
    # all-or-nothing exhaustion
    with pytest.raises(KvCacheError) as e:
        p.reserve(s, 1000)
    assert e.value.kind == "PoolExhausted"
    assert p.table(s) == o.seq_block_table(s).tolist()


def _seed(p, order):
    o = np.ascontiguousarray(order, dtype=np.uint32)
    check(p.L.eh_kvcache_seed_free_list(p.h, o.ctypes.data, o.size), host=True)


def test_host_seed_free_list_rejects_unsafe_orders():
    p = HostCache(8, 4, 1, 2)
    for bad, msg in (([0, 1, 2, 3, 4, 5, 6, 6], "duplicate page id"),
                     ([0, 1, 2, 3, 4, 5, 6], "order must list every free page exactly once"),
                     ([0, 1, 2, 3, 4, 5, 6, 9], "page id out of range")):
        with pytest.raises(KvCacheError) as e:
            _seed(p, bad)
        assert e.value.kind == "InvalidArgs" and e.value.msg == msg
    assert p.L.eh_kvcache_blocks_used(p.h) == 0
    _seed(p, [5, 3, 0, 1, 2, 4, 6, 7])
    s = p.L.eh_kvcache_new_sequence(p.h)
    p.reserve(s, 5)                              # pops pages 5 and 3
    assert p.table(s) == [5, 3]
    # a page a sequence holds cannot be seeded again (it would get two owners)
    with pytest.raises(KvCacheError) as e:
        _seed(p, [5, 0, 1, 2, 4, 6])
    assert e.value.msg == "page is in use"
    # a permutation of the pages that are still free is accepted
    _seed(p, [7, 6, 4, 2, 1, 0])
    t = p.L.eh_kvcache_new_sequence(p.h)
    p.reserve(t, 9)
    assert p.table(t) == [7, 6, 4]
    assert p.L.eh_kvcache_blocks_used(p.h) == 5


def test_host_reserve_batch_all_or_nothing():
    nb, bt = 10, 4
    p, q = HostCache(nb, bt, 1, 2), HostCache(nb, bt, 1, 2)
    for c in (p, q):
        for _ in range(4):
            c.L.eh_kvcache_new_sequence(c.h)
    lens = [3, 4, 0, 7]
    for s, n in enumerate(lens):
        p.reserve(s, n)
        q.reserve(s, n)
    seqs = np.array([0, 1, 2, 3], np.uint64)
    starts = np.zeros(4, np.uint64)
    ones = np.ones(4, np.uint64)
    check(p.L.eh_kvcache_reserve_batch(p.h, seqs.ctypes.data, 4, ones.ctypes.data,
                                       starts.ctypes.data), host=True)
    assert starts.tolist() == lens
    for s in range(4):                            # equals the single reserves in list order
        q.reserve(s, 1)
        assert p.table(s) == q.table(s)
    # exhaustion mid-batch: pages left = 10 - 7 = 3; the batch of 5 tokens each needs more
    used = p.L.eh_kvcache_blocks_used(p.h)
    before = [(p.table(s), p.L.eh_kvcache_token_count(p.h, s)) for s in range(4)]
    with pytest.raises(KvCacheError) as e:
        fives = np.full(4, 5, np.uint64)
        check(p.L.eh_kvcache_reserve_batch(p.h, seqs.ctypes.data, 4, fives.ctypes.data,
                                           starts.ctypes.data), host=True)
    assert e.value.kind == "PoolExhausted"
    assert (e.value.blocks_used, e.value.blocks_total) == (used, nb)
    assert [(p.table(s), p.L.eh_kvcache_token_count(p.h, s)) for s in range(4)] == before
    assert p.L.eh_kvcache_blocks_used(p.h) == used
    # an unknown or repeated sequence changes nothing either
    for bad in ([0, 9], [1, 1]):
        b = np.array(bad, np.uint64)
        with pytest.raises(KvCacheError):
            check(p.L.eh_kvcache_reserve_batch(p.h, b.ctypes.data, 2, ones.ctypes.data,
                                               starts.ctypes.data), host=True)
        assert [(p.table(s), p.L.eh_kvcache_token_count(p.h, s)) for s in range(4)] == before


def test_host_reserve_of_a_huge_count_is_exhaustion():
    """A token count near 2^64 must not wrap the page arithmetic into a small
    request: it cannot fit the pool, so PoolExhausted, with nothing changed."""
    nb, bt = 6, 4
    p = HostCache(nb, bt, 1, 2)
    for _ in range(2):
        p.L.eh_kvcache_new_sequence(p.h)
    p.reserve(0, 5)
    before = [(p.table(s), p.L.eh_kvcache_token_count(p.h, s)) for s in range(2)]
    huge = (1 << 64) - 3                           # 5 + huge + 3 wraps to 5 in 64 bits
    start = C.c_uint64(0)
    with pytest.raises(KvCacheError) as e:
        check(p.L.eh_kvcache_reserve(p.h, 0, huge, C.byref(start)), host=True)
    assert e.value.kind == "PoolExhausted"
    seqs = np.array([1, 0], np.uint64)
    counts = np.array([1, huge], np.uint64)
    starts = np.zeros(2, np.uint64)
    with pytest.raises(KvCacheError) as e:
        check(p.L.eh_kvcache_reserve_batch(p.h, seqs.ctypes.data, 2, counts.ctypes.data,
                                           starts.ctypes.data), host=True)
    assert e.value.kind == "PoolExhausted"
    assert [(p.table(s), p.L.eh_kvcache_token_count(p.h, s)) for s in range(2)] == before
    assert p.L.eh_kvcache_blocks_used(p.h) == 2


def test_host_truncate_restores_free_list_order():
    p, q = HostCache(12, 4, 1, 2), HostCache(12, 4, 1, 2)
    for c in (p, q):
        _seed(c, [3, 9, 1, 0, 11, 2, 5, 4, 6, 7, 8, 10])
        for _ in range(2):
            c.L.eh_kvcache_new_sequence(c.h)
        c.reserve(0, 6)
    p.reserve(1, 9)                               # pops 1, 0, 11
    assert p.table(1) == [1, 0, 11]
    check(p.L.eh_kvcache_truncate(p.h, 1, 0), host=True)
    p.reserve(0, 3)                               # 6 -> 9 tokens: pops 1 again
    q.reserve(0, 3)
    assert p.table(0) == q.table(0) == [3, 9, 1]
    p.reserve(1, 5)
    q.reserve(1, 5)
    assert p.table(1) == q.table(1) == [0, 11]
    assert p.L.eh_kvcache_truncate(p.h, 0, 10) == 21    # past the count
    check(p.L.eh_kvcache_truncate(p.h, 0, 5), host=True)
    assert p.table(0) == [3, 9] and p.L.eh_kvcache_token_count(p.h, 0) == 5
