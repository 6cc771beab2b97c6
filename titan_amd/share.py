"""Prefix-sharing bookkeeping -- the engine-kvcache `CowBlockTable`,
`RadixTree` and `StreamingKvManager` surfaces over libengine_hip.so
(include/kv_share.h).

Names and argument meaning follow engine-kvcache/src/{cow,radix,streaming}.rs.
The objects hold integers only; the pages they name live in an HBM pool and
are moved with PagedKvGpu.copy_pages / remap_block_tables.
"""
import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib


def _u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


class CowBlockTable:
    """cow.rs:17-97: reference-counted shared blocks, O(1)-per-entry fork."""

    def __init__(self, _handle=None):
        self._L = _lib.load()
        self._h = _handle if _handle is not None else self._L.eh_cow_new()

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._L.eh_cow_destroy(h)
            self._h = None

    def fork(self):
        return CowBlockTable(self._L.eh_cow_fork(self._h))

    def append_block(self, block_id):
        self._L.eh_cow_append_block(self._h, int(block_id))

    def is_shared(self, block_index):
        return bool(self._L.eh_cow_is_shared(self._h, int(block_index)))

    def tail_needs_cow(self):
        return bool(self._L.eh_cow_tail_needs_cow(self._h))

    def perform_tail_cow(self, new_block_id):
        self._L.eh_cow_perform_tail_cow(self._h, int(new_block_id))

    def physical_block_ids(self):
        n = self._L.eh_cow_len(self._h)
        out = np.zeros(max(n, 1), dtype=np.uint32)
        self._L.eh_cow_block_ids(self._h, _p(out), n)
        return [int(x) for x in out[:n]]

    def __len__(self):
        return self._L.eh_cow_len(self._h)

    def is_empty(self):
        return len(self) == 0

    def is_dirty(self, block_index):
        return bool(self._L.eh_cow_is_dirty(self._h, int(block_index)))

    def ref_count(self, block_index):
        """Arc::strong_count of the entry (0 past the end)."""
        return self._L.eh_cow_ref_count(self._h, int(block_index))

    @property
    def seq_len(self):
        return self._L.eh_cow_seq_len(self._h)

    @seq_len.setter
    def seq_len(self, v):
        self._L.eh_cow_set_seq_len(self._h, int(v))


@dataclass
class RadixMatchResult:
    """radix.rs:45-51"""
    matched_tokens: int
    matched_blocks: list


class RadixTree:
    """radix.rs:57-290 with a logical access clock (reproducible LRU)."""

    def __init__(self, block_tokens):
        self._L = _lib.load()
        self.block_tokens = int(block_tokens)
        self._h = self._L.eh_radix_new(self.block_tokens)
        if not self._h:
            raise ValueError("block_tokens must be non-zero")

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._L.eh_radix_destroy(h)
            self._h = None

    def match_prefix(self, tokens):
        t = _u32(tokens)
        cap = max(t.size // max(self.block_tokens, 1) + 1, 1) + self.total_cached_blocks()
        out = np.zeros(cap, dtype=np.uint32)
        nb = C.c_uint64()
        m = self._L.eh_radix_match_prefix(self._h, _p(t), t.size, _p(out), cap, C.byref(nb))
        return RadixMatchResult(int(m), [int(x) for x in out[:min(nb.value, cap)]])

    def insert(self, tokens, blocks, is_pinned):
        t, b = _u32(tokens), _u32(blocks)
        self._L.eh_radix_insert(self._h, _p(t), t.size, _p(b), b.size, 1 if is_pinned else 0)

    def evict_lru(self, target_blocks_to_free):
        cap = max(self.total_cached_blocks(), 1)
        out = np.zeros(cap, dtype=np.uint32)
        n = self._L.eh_radix_evict_lru(self._h, int(target_blocks_to_free), _p(out), cap)
        return [int(x) for x in out[:min(n, cap)]]

    def total_cached_blocks(self):
        return self._L.eh_radix_total_cached_blocks(self._h)

    def invalidate_physical_blocks(self, freed_blocks):
        b = _u32(freed_blocks)
        self._L.eh_radix_invalidate_physical_blocks(self._h, _p(b), b.size)

    def set_ref_count(self, tokens, ref_count):
        """ref_count of the node ending exactly at `tokens` (False if none)."""
        t = _u32(tokens)
        return self._L.eh_radix_set_ref_count(self._h, _p(t), t.size, int(ref_count)) == 0


class StreamingKvConfig:
    """streaming.rs:9-65"""

    def __init__(self, sink_tokens=None, recent_window_tokens=None, max_budget_tokens=None,
                 block_tokens=None, _raw=None):
        L = _lib.load()
        if _raw is not None:
            self._c = _raw
        elif sink_tokens is None:
            self._c = L.eh_stream_cfg_default()
        else:
            self._c = L.eh_stream_cfg_new(int(sink_tokens), int(recent_window_tokens),
                                          int(max_budget_tokens), int(block_tokens))

    @classmethod
    def default(cls):
        return cls()

    sink_tokens = property(lambda s: s._c.sink_tokens)
    recent_window_tokens = property(lambda s: s._c.recent_window_tokens)
    max_budget_tokens = property(lambda s: s._c.max_budget_tokens)
    block_tokens = property(lambda s: s._c.block_tokens)

    def sink_blocks(self):
        return _lib.load().eh_stream_sink_blocks(self._c)

    def recent_blocks(self):
        return _lib.load().eh_stream_recent_blocks(self._c)

    def max_active_blocks(self):
        return _lib.load().eh_stream_max_active_blocks(self._c)


class StreamingKvManager:
    """streaming.rs:68-142"""

    def __init__(self, cfg):
        self._L = _lib.load()
        self.cfg = cfg
        self._h = self._L.eh_stream_new(cfg._c)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._L.eh_stream_destroy(h)
            self._h = None

    def record_attention_mass(self, block_id, mass):
        self._L.eh_stream_record_attention_mass(self._h, int(block_id), float(mass))

    def record_attention_masses(self, masses):
        """record_attention_mass(i, masses[i]) for every non-zero entry: the
        per-page masses a decode launch accumulated (block_mass), on the host."""
        m = np.ascontiguousarray(masses, dtype=np.float32)
        self._L.eh_stream_record_attention_masses(self._h, _p(m), m.size)

    @property
    def block_scores(self):
        n = self._L.eh_stream_scores_len(self._h)
        return [self._L.eh_stream_score(self._h, i) for i in range(n)]

    def prune_blocks(self, block_table):
        """-> (retained, evicted)"""
        t = _u32(block_table)
        n = t.size
        r = np.zeros(max(n, 1), dtype=np.uint32)
        e = np.zeros(max(n, 1), dtype=np.uint32)
        nr, ne = C.c_uint64(), C.c_uint64()
        self._L.eh_stream_prune_blocks(self._h, _p(t), n, _p(r), C.byref(nr), _p(e), C.byref(ne))
        return [int(x) for x in r[:nr.value]], [int(x) for x in e[:ne.value]]


def compaction_plan(block_tables, n_used, n_blocks):
    """Gather-compaction of live pages to the lowest ids.

    block_tables [B, stride] u32 and n_used [B] (host arrays).  Returns
    (src, dst, remap) uint32 arrays: copy src[k] -> dst[k] with
    PagedKvGpu.copy_pages, then rewrite tables through remap."""
    bt = _u32(block_tables)
    if bt.ndim != 2:
        raise ValueError("block_tables must be [B, stride]")
    nu = _u32(n_used)
    B, stride = bt.shape
    src = np.zeros(max(int(n_blocks), 1), dtype=np.uint32)
    dst = np.zeros_like(src)
    remap = np.zeros(max(int(n_blocks), 1), dtype=np.uint32)
    n = _lib.load().eh_compaction_plan(_p(bt), stride, _p(nu), B, int(n_blocks), _p(src), _p(dst),
                                       _p(remap))
    if n < 0:
        raise ValueError("a live block-table entry is outside the pool")
    return src[:n].copy(), dst[:n].copy(), remap[:int(n_blocks)].copy()
