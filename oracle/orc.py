"""ctypes view of the CPU oracle (liborc_kv.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product package
(titan_amd) never imports this module.
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# TITAN_ORACLE_LIB selects another build (the sanitized one).
_LIB_PATH = os.environ.get("TITAN_ORACLE_LIB") or os.path.join(_HERE, "liborc_kv.so")

OK, POOL_EXHAUSTED, INVALID_ARGS = 0, 20, 21

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle not built: {_LIB_PATH} (run make -C oracle)")
        L = C.CDLL(_LIB_PATH)
        vp, sz, u32, i32, f32 = C.c_void_p, C.c_size_t, C.c_uint32, C.c_int, C.c_float
        P = C.POINTER
        sigs = {
            "orc_cache_new": (i32, [sz, sz, sz, sz, sz, P(vp), P(C.c_char_p)]),
            "orc_cache_destroy": (None, [vp]),
            "orc_cache_seed_free_list": (None, [vp, vp, sz]),
            "orc_cache_new_sequence": (sz, [vp]),
            "orc_cache_free_sequence": (None, [vp, sz]),
            "orc_cache_token_count": (sz, [vp, sz]),
            "orc_cache_blocks_total": (sz, [vp]),
            "orc_cache_blocks_used": (sz, [vp]),
            "orc_cache_sequences": (sz, [vp]),
            "orc_cache_block_table": (C.c_long, [vp, sz, vp, sz]),
            "orc_cache_append": (i32, [vp, sz, vp, sz, vp, sz, P(sz), P(sz), P(C.c_char_p)]),
            "orc_cache_read_row": (i32, [vp, sz, sz, i32, vp, P(C.c_char_p)]),
            "orc_cache_read_all": (i32, [vp, sz, i32, vp, P(C.c_char_p)]),
            "orc_cache_buffer": (vp, [vp, P(sz)]),
            "orc_sdpa_decode": (None, [vp, vp, sz, sz, vp, sz, sz, sz, i32, sz, vp]),
            "orc_sdpa_decode_batched": (None, [vp, vp, sz, vp, sz, sz, vp, sz, sz, sz, vp]),
            "orc_sdpa_decode_window_batched": (None, [vp, vp, sz, vp, sz, sz, vp, sz, sz, sz, sz, sz,
                                                      vp, vp]),
            "orc_prefill_causal": (None, [vp, vp, sz, vp, sz, sz, sz, sz, sz, vp]),
            "orc_f16_to_f32": (f32, [C.c_uint16]),
            "orc_f16_to_f32_array": (None, [vp, vp, sz]),
            "orc_f32_to_f16_rne": (C.c_uint16, [f32]),
            "orc_f32_to_bf16_rne": (C.c_uint16, [f32]),
            "orc_bf16_to_f32_array": (None, [vp, vp, sz]),
            "orc_e4m3_to_f32": (f32, [C.c_uint8]),
            "orc_f32_to_e4m3": (C.c_uint8, [f32, f32]),
            "orc_e4m3_to_f32_array": (None, [vp, vp, sz, f32]),
            "orc_f32_to_e4m3_array": (None, [vp, vp, sz, f32]),
            "orc_xorshift_a_f32": (None, [u32, vp, sz]),
            "orc_generate_rows_b": (None, [u32, sz, sz, vp, vp]),
            "orc_fill_pool_paged": (None, [vp, vp, sz, sz, sz, u32, sz]),
            "orc_cow_new": (vp, []),
            "orc_cow_fork": (vp, [vp]),
            "orc_cow_destroy": (None, [vp]),
            "orc_cow_append_block": (None, [vp, u32]),
            "orc_cow_is_shared": (i32, [vp, sz]),
            "orc_cow_tail_needs_cow": (i32, [vp]),
            "orc_cow_perform_tail_cow": (None, [vp, u32]),
            "orc_cow_ids": (sz, [vp, vp, sz]),
            "orc_cow_len": (sz, [vp]),
            "orc_cow_is_dirty": (i32, [vp, sz]),
            "orc_cow_refcount": (sz, [vp, sz]),
            "orc_radix_new": (vp, [sz]),
            "orc_radix_destroy": (None, [vp]),
            "orc_radix_match_prefix": (sz, [vp, vp, sz, vp, sz, P(sz)]),
            "orc_radix_insert": (None, [vp, vp, sz, vp, sz, i32]),
            "orc_radix_evict_lru": (sz, [vp, sz, vp, sz]),
            "orc_radix_total_cached_blocks": (sz, [vp]),
            "orc_radix_invalidate_physical_blocks": (None, [vp, vp, sz]),
            "orc_radix_set_ref_count": (i32, [vp, vp, sz, sz]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return C.c_void_p(a.ctypes.data) if a is not None and a.size else None


class KvCacheError(Exception):
    def __init__(self, kind, msg=None, blocks_used=None, blocks_total=None):
        super().__init__(kind, msg, blocks_used, blocks_total)
        self.kind, self.msg = kind, msg
        self.blocks_used, self.blocks_total = blocks_used, blocks_total


class Cache:
    """PagedKvCache restatement (engine-kvcache/src/cache.rs)."""

    def __init__(self, n_blocks, block_tokens, heads, head_dim, dtype=np.float32):
        self.dtype = np.dtype(dtype)
        self.row_len = heads * head_dim
        self.n_blocks, self.block_tokens = n_blocks, block_tokens
        h = C.c_void_p()
        msg = C.c_char_p()
        rc = lib().orc_cache_new(n_blocks, block_tokens, heads, head_dim, self.dtype.itemsize,
                                 C.byref(h), C.byref(msg))
        if rc != OK:
            self._h = None
            raise KvCacheError("InvalidArgs", msg.value.decode())
        self._h = h

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_cache_destroy(self._h)
            self._h = None

    def seed_free_list(self, order):
        o = np.ascontiguousarray(order, dtype=np.uint32)
        lib().orc_cache_seed_free_list(self._h, _p(o), o.size)

    def new_sequence(self):
        return lib().orc_cache_new_sequence(self._h)

    def free_sequence(self, seq):
        lib().orc_cache_free_sequence(self._h, seq)

    def token_count(self, seq):
        return lib().orc_cache_token_count(self._h, seq)

    def blocks_total(self):
        return lib().orc_cache_blocks_total(self._h)

    def blocks_used(self):
        return lib().orc_cache_blocks_used(self._h)

    def sequences(self):
        return lib().orc_cache_sequences(self._h)

    def seq_block_table(self, seq):
        n = lib().orc_cache_block_table(self._h, seq, None, 0)
        if n < 0:
            return None
        out = np.zeros(max(n, 1), dtype=np.uint32)
        lib().orc_cache_block_table(self._h, seq, _p(out), n)
        return out[:n]

    def append(self, seq, key, value):
        k = np.ascontiguousarray(key, dtype=self.dtype)
        v = np.ascontiguousarray(value, dtype=self.dtype)
        used, total, msg = C.c_size_t(), C.c_size_t(), C.c_char_p()
        rc = lib().orc_cache_append(self._h, seq, _p(k), k.size, _p(v), v.size,
                                    C.byref(used), C.byref(total), C.byref(msg))
        if rc == POOL_EXHAUSTED:
            raise KvCacheError("PoolExhausted", None, used.value, total.value)
        if rc != OK:
            raise KvCacheError("InvalidArgs", msg.value.decode())

    def _row(self, seq, token, is_value):
        out = np.zeros(self.row_len, dtype=self.dtype)
        msg = C.c_char_p()
        rc = lib().orc_cache_read_row(self._h, seq, token, int(is_value), _p(out), C.byref(msg))
        if rc != OK:
            raise KvCacheError("InvalidArgs", msg.value.decode())
        return out

    def read_key(self, seq, token):
        return self._row(seq, token, False)

    def read_value(self, seq, token):
        return self._row(seq, token, True)

    def _all(self, seq, is_value):
        n = self.token_count(seq)
        out = np.zeros(max(n * self.row_len, 1), dtype=self.dtype)
        msg = C.c_char_p()
        rc = lib().orc_cache_read_all(self._h, seq, int(is_value), _p(out), C.byref(msg))
        if rc != OK:
            raise KvCacheError("InvalidArgs", msg.value.decode())
        return out[: n * self.row_len]

    def read_keys(self, seq):
        return self._all(seq, False)

    def read_values(self, seq):
        return self._all(seq, True)

    def buffer(self):
        nbytes = C.c_size_t()
        ptr = lib().orc_cache_buffer(self._h, C.byref(nbytes))
        raw = (C.c_ubyte * nbytes.value).from_address(ptr)
        return np.frombuffer(bytes(raw), dtype=self.dtype).copy()


def sdpa_decode(pool, block_table, block_tokens, seq_tokens, query, n_head, n_head_kv,
                head_dim, causal, query_pos):
    """forward_cpu.rs:424-510 over an f32 pool (elements)."""
    pool = np.ascontiguousarray(pool, dtype=np.float32)
    bt = np.ascontiguousarray(block_table, dtype=np.uint32)
    q = np.ascontiguousarray(query, dtype=np.float32)
    out = np.zeros(n_head * head_dim, dtype=np.float32)
    if n_head * head_dim == 0:
        return out
    lib().orc_sdpa_decode(_p(pool), _p(bt), block_tokens, seq_tokens, _p(q), n_head,
                          n_head_kv, head_dim, int(causal), query_pos, _p(out))
    return out


def sdpa_decode_batched(pool, bt, lens, block_tokens, q, n_head, n_head_kv, head_dim):
    pool = np.ascontiguousarray(pool, dtype=np.float32)
    bt = np.ascontiguousarray(bt, dtype=np.uint32)
    lens = np.ascontiguousarray(lens, dtype=np.uint32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    B = lens.size
    out = np.zeros((B, n_head, head_dim), dtype=np.float32)
    lib().orc_sdpa_decode_batched(_p(pool), _p(bt), bt.shape[1], _p(lens), B, block_tokens,
                                  _p(q), n_head, n_head_kv, head_dim, _p(out))
    return out


def sdpa_decode_window_batched(pool, bt, lens, block_tokens, q, n_head, n_head_kv, head_dim,
                               sink, window, n_blocks=None):
    """sdpa_decode over [0, sink) U [max(sink, n-1-window), n-1]; window 0 = all.
    With n_blocks, also returns the per-page attention mass (f64 [n_blocks])."""
    pool = np.ascontiguousarray(pool, dtype=np.float32)
    bt = np.ascontiguousarray(bt, dtype=np.uint32)
    lens = np.ascontiguousarray(lens, dtype=np.uint32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    B = len(lens)
    out = np.zeros((B, n_head, head_dim), dtype=np.float32)
    mass = None if n_blocks is None else np.zeros(n_blocks, dtype=np.float64)
    lib().orc_sdpa_decode_window_batched(_p(pool), _p(bt), bt.shape[1], _p(lens), B, block_tokens,
                                         _p(q), n_head, n_head_kv, head_dim, int(sink), int(window),
                                         _p(out), None if mass is None else _p(mass))
    return out if mass is None else (out, mass)


def prefill_causal(pool, block_table, block_tokens, q, q_tokens, pos_offset, n_head,
                   n_head_kv, head_dim):
    pool = np.ascontiguousarray(pool, dtype=np.float32)
    bt = np.ascontiguousarray(block_table, dtype=np.uint32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.zeros((q_tokens, n_head, head_dim), dtype=np.float32)
    lib().orc_prefill_causal(_p(pool), _p(bt), block_tokens, _p(q), q_tokens, pos_offset,
                             n_head, n_head_kv, head_dim, _p(out))
    return out


def f16_bits_to_f32(bits):
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.zeros(b.shape, dtype=np.float32)
    lib().orc_f16_to_f32_array(_p(b), _p(out), b.size)
    return out


def bf16_bits_to_f32(bits):
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.zeros(b.shape, dtype=np.float32)
    lib().orc_bf16_to_f32_array(_p(b), _p(out), b.size)
    return out


def f32_to_f16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    return np.array([lib().orc_f32_to_f16_rne(float(v)) for v in x], dtype=np.uint16)


def f32_to_bf16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    return np.array([lib().orc_f32_to_bf16_rne(float(v)) for v in x], dtype=np.uint16)


def e4m3_to_f32(codes, scale=1.0):
    """decode(code) * scale (f32) for FP8 E4M3 codes."""
    c = np.ascontiguousarray(codes, dtype=np.uint8)
    out = np.zeros(c.shape, dtype=np.float32)
    lib().orc_e4m3_to_f32_array(_p(c), _p(out), c.size, float(scale))
    return out


def f32_to_e4m3(x, scale=1.0):
    """E4M3 codes of x / scale (RNE, saturating at 448)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.shape, dtype=np.uint8)
    lib().orc_f32_to_e4m3_array(_p(x), _p(out), x.size, float(scale))
    return out


def xorshift_a(seed, n):
    out = np.zeros(n, dtype=np.float32)
    lib().orc_xorshift_a_f32(seed, _p(out), n)
    return out


def generate_rows_b(seed, n_tokens, row_len):
    k = np.zeros(n_tokens * row_len, dtype=np.float32)
    v = np.zeros(n_tokens * row_len, dtype=np.float32)
    lib().orc_generate_rows_b(seed, n_tokens, row_len, _p(k), _p(v))
    return k, v


def fill_pool_paged(pool, block_table, block_tokens, n_head_kv, head_dim, seed, n_tokens):
    assert pool.dtype == np.float32 and pool.flags.c_contiguous
    bt = np.ascontiguousarray(block_table, dtype=np.uint32)
    lib().orc_fill_pool_paged(_p(pool), _p(bt), block_tokens, n_head_kv, head_dim, seed,
                              n_tokens)


class Cow:
    """CowBlockTable restatement (engine-kvcache/src/cow.rs)."""

    def __init__(self, handle=None):
        self._h = handle if handle is not None else lib().orc_cow_new()

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_cow_destroy(self._h)
            self._h = None

    def fork(self):
        return Cow(lib().orc_cow_fork(self._h))

    def append_block(self, bid):
        lib().orc_cow_append_block(self._h, bid)

    def is_shared(self, idx):
        return bool(lib().orc_cow_is_shared(self._h, idx))

    def tail_needs_cow(self):
        return bool(lib().orc_cow_tail_needs_cow(self._h))

    def perform_tail_cow(self, new_id):
        lib().orc_cow_perform_tail_cow(self._h, new_id)

    def physical_block_ids(self):
        n = lib().orc_cow_len(self._h)
        out = np.zeros(max(n, 1), dtype=np.uint32)
        lib().orc_cow_ids(self._h, _p(out), n)
        return [int(x) for x in out[:n]]

    def __len__(self):
        return lib().orc_cow_len(self._h)

    def is_dirty(self, idx):
        return bool(lib().orc_cow_is_dirty(self._h, idx))

    def refcount(self, idx):
        return lib().orc_cow_refcount(self._h, idx)


class Radix:
    """RadixTree restatement (engine-kvcache/src/radix.rs), logical clock."""

    def __init__(self, block_tokens):
        self._h = lib().orc_radix_new(block_tokens)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_radix_destroy(self._h)
            self._h = None

    def match_prefix(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        cap = 1 << 16
        out = np.zeros(cap, dtype=np.uint32)
        nb = C.c_size_t()
        m = lib().orc_radix_match_prefix(self._h, _p(t), t.size, _p(out), cap, C.byref(nb))
        return m, [int(x) for x in out[: nb.value]]

    def insert(self, tokens, blocks, is_pinned):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        b = np.ascontiguousarray(blocks, dtype=np.uint32)
        lib().orc_radix_insert(self._h, _p(t), t.size, _p(b), b.size, int(is_pinned))

    def evict_lru(self, target):
        cap = 1 << 20
        out = np.zeros(cap, dtype=np.uint32)
        n = lib().orc_radix_evict_lru(self._h, target, _p(out), cap)
        return [int(x) for x in out[:n]]

    def total_cached_blocks(self):
        return lib().orc_radix_total_cached_blocks(self._h)

    def invalidate_physical_blocks(self, blocks):
        b = np.ascontiguousarray(blocks, dtype=np.uint32)
        lib().orc_radix_invalidate_physical_blocks(self._h, _p(b), b.size)

    def set_ref_count(self, tokens, ref):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        return lib().orc_radix_set_ref_count(self._h, _p(t), t.size, ref)


class Streaming:
    """StreamingKvConfig / StreamingKvManager restatement (engine-kvcache/src/streaming.rs)."""

    class Cfg(C.Structure):
        _fields_ = [("sink_tokens", C.c_size_t), ("recent_window_tokens", C.c_size_t),
                    ("max_budget_tokens", C.c_size_t), ("block_tokens", C.c_size_t)]

    def __init__(self, sink=None, recent=None, budget=None, bt=None):
        L = lib()
        L.orc_stream_cfg_new.restype = Streaming.Cfg
        L.orc_stream_cfg_new.argtypes = [C.c_size_t] * 4
        L.orc_stream_cfg_default.restype = Streaming.Cfg
        L.orc_stream_cfg_default.argtypes = []
        for f in ("orc_stream_sink_blocks", "orc_stream_recent_blocks",
                  "orc_stream_max_active_blocks"):
            getattr(L, f).restype = C.c_size_t
            getattr(L, f).argtypes = [Streaming.Cfg]
        L.orc_stream_new.restype = C.c_void_p
        L.orc_stream_new.argtypes = [Streaming.Cfg]
        L.orc_stream_destroy.restype = None
        L.orc_stream_destroy.argtypes = [C.c_void_p]
        L.orc_stream_record_attention_mass.restype = None
        L.orc_stream_record_attention_mass.argtypes = [C.c_void_p, C.c_uint32, C.c_float]
        L.orc_stream_scores_len.restype = C.c_size_t
        L.orc_stream_scores_len.argtypes = [C.c_void_p]
        L.orc_stream_prune_blocks.restype = None
        L.orc_stream_prune_blocks.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p,
                                              C.POINTER(C.c_size_t), C.c_void_p,
                                              C.POINTER(C.c_size_t)]
        self.cfg = L.orc_stream_cfg_default() if sink is None else L.orc_stream_cfg_new(
            sink, recent, budget, bt)
        self._h = L.orc_stream_new(self.cfg)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_stream_destroy(self._h)
            self._h = None

    def sink_blocks(self):
        return lib().orc_stream_sink_blocks(self.cfg)

    def recent_blocks(self):
        return lib().orc_stream_recent_blocks(self.cfg)

    def max_active_blocks(self):
        return lib().orc_stream_max_active_blocks(self.cfg)

    def record_attention_mass(self, block, mass):
        lib().orc_stream_record_attention_mass(self._h, block, mass)

    def scores_len(self):
        return lib().orc_stream_scores_len(self._h)

    def prune_blocks(self, table):
        t = np.ascontiguousarray(table, dtype=np.uint32)
        r = np.zeros(max(t.size, 1), np.uint32)
        e = np.zeros(max(t.size, 1), np.uint32)
        nr, ne = C.c_size_t(), C.c_size_t()
        lib().orc_stream_prune_blocks(self._h, _p(t), t.size, _p(r), C.byref(nr), _p(e),
                                      C.byref(ne))
        return [int(x) for x in r[:nr.value]], [int(x) for x in e[:ne.value]]


def compaction_plan(block_tables, n_used, n_blocks):
    """Gather-compaction plan, restated with sets (the product policy has no
    reference counterpart: the copy step of a compaction is only sketched in
    openspec/changes/archive/2026-08-28-agent-runtime-optimizations/
    design.md:134-148).  Rule: with k live pages, every live page at or
    above id k moves to a free id below k, the i-th smallest such page to
    the i-th smallest hole.  Returns (src, dst, remap) like
    titan_amd.share.compaction_plan."""
    bt = np.asarray(block_tables, dtype=np.uint32)
    live = set()
    for b in range(bt.shape[0]):
        live.update(int(p) for p in bt[b, :int(n_used[b])])
    if any(p >= n_blocks for p in live):
        raise ValueError("a live block-table entry is outside the pool")
    k = len(live)
    movers = sorted(p for p in live if p >= k)
    holes = sorted(set(range(k)) - live)
    assert len(movers) == len(holes)
    remap = np.arange(n_blocks, dtype=np.uint32)
    for p, h in zip(movers, holes):
        remap[p] = h
    return (np.array(movers, dtype=np.uint32), np.array(holes, dtype=np.uint32), remap)
