"""PagedKvCache with its pool in HBM -- the engine-kvcache `PagedKvCache` surface.

Same API and error behaviour as engine-kvcache/src/cache.rs (`new`,
`new_sequence`, `append`, `free_sequence`, `read_key`/`read_value`,
`read_keys`/`read_values`, `seq_block_table`, `token_count`, `blocks_used`,
`blocks_total`, `sequences`, `config`).  Page bookkeeping runs in the native
host library (kv_host.cpp); page bytes are written and read by the gfx950
kernels.  Rows are tensors in the pool's element type.
"""
import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .errors import KvCacheError, check
from .paged_kv import KvDataType, PagedKvGpu, PagedKvLayout

TORCH_DTYPE = {
    KvDataType.F32: torch.float32,
    KvDataType.F16: torch.float16,
    KvDataType.BF16: torch.bfloat16,
    KvDataType.FP8: torch.uint8,
}


@dataclass(frozen=True)
class PagedKvCacheConfig:
    """engine-kvcache/src/cache.rs:8-40"""
    n_blocks: int
    block_tokens: int
    heads: int
    head_dim: int

    def row_len(self):
        return self.heads * self.head_dim

    def floats_per_token(self):
        return 2 * self.row_len()

    def floats_per_block(self):
        return self.block_tokens * self.floats_per_token()

    def floats_total(self):
        return self.n_blocks * self.floats_per_block()


class PagedKvCache:
    """engine-kvcache/src/cache.rs:49-256 with the pool on `device`."""

    def __init__(self, cfg, dtype=KvDataType.F32, device=0):
        self._L = _lib.load()
        self._cfg = cfg
        self.dtype = KvDataType(dtype)
        h = C.c_void_p()
        check(self._L.eh_kvcache_new(cfg.n_blocks, cfg.block_tokens, cfg.heads, cfg.head_dim,
                                     int(self.dtype), C.byref(h)), host=True)
        self._h = h
        self.device = torch.device("cuda", device if isinstance(device, int) else device.index or 0)
        self.layout = PagedKvLayout(cfg.n_blocks, cfg.block_tokens, cfg.row_len(), self.dtype)
        # cache.rs:78-79: the pool starts zero-filled.
        self.pool = torch.zeros(cfg.floats_total(), dtype=TORCH_DTYPE[self.dtype], device=self.device)
        self._kv = PagedKvGpu(self.device.index)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._L.eh_kvcache_destroy(h)
            self._h = None

    # ---- bookkeeping (cache.rs:98-149) ----------------------------------------
    def config(self):
        return self._cfg

    def blocks_total(self):
        return self._L.eh_kvcache_blocks_total(self._h)

    def blocks_used(self):
        return self._L.eh_kvcache_blocks_used(self._h)

    def sequences(self):
        return self._L.eh_kvcache_sequences(self._h)

    def seq_block_table(self, seq):
        n = self._L.eh_kvcache_block_table(self._h, seq, None, 0)
        if n < 0:
            return None
        out = np.zeros(max(n, 1), dtype=np.uint32)
        self._L.eh_kvcache_block_table(self._h, seq, out.ctypes.data, n)
        return out[:n].tolist()

    def free_sequence(self, seq):
        self._L.eh_kvcache_free_sequence(self._h, seq)

    def new_sequence(self):
        return self._L.eh_kvcache_new_sequence(self._h)

    def token_count(self, seq):
        return self._L.eh_kvcache_token_count(self._h, seq)

    def seed_free_list(self, order):
        """Extension: successive page pops return order[0], order[1], ..."""
        o = np.ascontiguousarray(order, dtype=np.uint32)
        check(self._L.eh_kvcache_seed_free_list(self._h, o.ctypes.data, o.size), host=True)

    def reserve(self, seq, n_tokens):
        """Allocate pages for n more tokens of `seq`; returns the first position."""
        start = C.c_uint64()
        check(self._L.eh_kvcache_reserve(self._h, seq, n_tokens, C.byref(start)), host=True)
        return start.value

    # ---- data path -------------------------------------------------------------
    def _row_tensor(self, x):
        t = torch.as_tensor(x)
        if t.dtype != TORCH_DTYPE[self.dtype]:
            t = t.to(TORCH_DTYPE[self.dtype])
        return t.reshape(-1).to(self.device).contiguous()

    def _table_dev(self, seq):
        bt = self.seq_block_table(seq)
        return torch.tensor(bt if bt else [0], dtype=torch.int32, device=self.device)

    def truncate(self, seq, n_tokens):
        """Extension: roll a reservation back to n_tokens; the released pages
        return to the free list in the order they were popped from."""
        check(self._L.eh_kvcache_truncate(self._h, int(seq), int(n_tokens)), host=True)

    def append(self, seq, key, value, stream=None):
        """cache.rs:153-192: one token's K and V rows.  All or nothing, as the
        reference: the row lengths and the sequence are checked first
        (same order, same messages); if the launch fails after the page
        was reserved, the reservation is rolled back before the error
        propagates."""
        k, v = self._row_tensor(key), self._row_tensor(value)
        m = self._cfg.row_len()
        if k.numel() != m or v.numel() != m:
            raise KvCacheError("InvalidArgs", "key/value length must equal heads * head_dim")
        if seq >= self.sequences():
            raise KvCacheError("InvalidArgs", "unknown sequence id")
        before = self.token_count(seq)
        pos = self.reserve(seq, 1)
        try:
            self._kv.append_kv(stream, self.layout, self.pool, k, v, self._table_dev(seq), pos, 1)
        except BaseException:
            self.truncate(seq, before)
            raise

    def _read(self, seq, start, n, is_value, stream=None):
        out = torch.empty(max(n, 1) * self._cfg.row_len(), dtype=TORCH_DTYPE[self.dtype],
                          device=self.device)
        if n:
            fn = self._kv.read_values if is_value else self._kv.read_keys
            fn(stream, self.layout, self.pool, self._table_dev(seq), out, start, n)
        return out[: n * self._cfg.row_len()]

    def _check_row(self, seq, token):
        if seq >= self.sequences():
            raise KvCacheError("InvalidArgs", "unknown sequence id")
        if token >= self.token_count(seq):
            raise KvCacheError("InvalidArgs", "token out of range")

    def read_key(self, seq, token):
        """cache.rs:195-197"""
        self._check_row(seq, token)
        return self._read(seq, token, 1, False)

    def read_value(self, seq, token):
        """cache.rs:200-202"""
        self._check_row(seq, token)
        return self._read(seq, token, 1, True)

    def read_keys(self, seq):
        """cache.rs:230-232"""
        if seq >= self.sequences():
            raise KvCacheError("InvalidArgs", "unknown sequence id")
        return self._read(seq, 0, self.token_count(seq), False)

    def read_values(self, seq):
        """cache.rs:235-237"""
        if seq >= self.sequences():
            raise KvCacheError("InvalidArgs", "unknown sequence id")
        return self._read(seq, 0, self.token_count(seq), True)

    # ---- batched extensions -------------------------------------------------
    def block_tables(self, seqs, stride=None):
        """Dense device [len(seqs), stride] u32 tables (pad 0xFFFFFFFF) and token counts."""
        seqs_a = np.ascontiguousarray(seqs, dtype=np.uint64)
        if stride is None:
            stride = max(1, max(len(self.seq_block_table(int(s)) or []) for s in seqs))
        tab = np.zeros((len(seqs), stride), dtype=np.uint32)
        lens = np.zeros(len(seqs), dtype=np.uint32)
        check(self._L.eh_kvcache_export_tables(self._h, seqs_a.ctypes.data, seqs_a.size,
                                               tab.ctypes.data, stride, lens.ctypes.data),
              host=True)
        return (torch.from_numpy(tab.view(np.int32)).to(self.device),
                torch.from_numpy(lens.view(np.int32)).to(self.device))

    def reserve_batch(self, seqs, counts):
        """Extension: reserve counts[i] tokens for seqs[i], all or nothing
        (PoolExhausted leaves every sequence unchanged); returns the first
        new position of each sequence."""
        seqs_a = np.ascontiguousarray([int(s) for s in seqs], dtype=np.uint64)
        cnt = np.ascontiguousarray([int(n) for n in counts], dtype=np.uint64)
        if cnt.size != seqs_a.size:
            raise KvCacheError("InvalidArgs", "one count per sequence")
        starts = np.zeros(max(seqs_a.size, 1), dtype=np.uint64)
        check(self._L.eh_kvcache_reserve_batch(self._h, seqs_a.ctypes.data, seqs_a.size,
                                               cnt.ctypes.data, starts.ctypes.data), host=True)
        return starts[:seqs_a.size].astype(np.int64)

    def extend_batch(self, seqs, counts, keys, values, stream=None, stride=None):
        """Append counts[i] tokens to seqs[i] for every listed sequence with one
        kernel launch (a ragged batch: prompt prefill, or one token each at
        decode).  keys/values: [sum(counts), row_len] device tensors in the
        pool dtype, sequence by sequence.  Returns (device block tables
        [B, stride], device start positions [B] int32, host token counts
        after the append).

        All or nothing: shapes, dtype, device and the table stride are checked
        before any page is reserved; the batch's pages are reserved in one
        step (PoolExhausted leaves every sequence unchanged); a failed launch
        rolls every reservation back."""
        B = len(seqs)
        counts = [int(n) for n in counts]
        if len(counts) != B:
            raise KvCacheError("InvalidArgs", "one count per sequence")
        if any(n < 0 for n in counts):
            raise KvCacheError("InvalidArgs", "token counts must not be negative")
        m = self._cfg.row_len()
        total = sum(counts)
        if total >= 1 << 31:
            raise KvCacheError("InvalidArgs", "at most 2^31 - 1 rows per launch")
        want = TORCH_DTYPE[self.dtype]
        for t in (keys, values):
            if tuple(t.shape) != (total, m):
                raise KvCacheError("InvalidArgs", "key/value length must equal heads * head_dim")
            if t.dtype != want or t.device != self.device:
                raise KvCacheError("InvalidArgs", "keys/values must be pool-dtype tensors on the "
                                                  "pool's device")
        for s in seqs:
            if int(s) >= self.sequences():
                raise KvCacheError("InvalidArgs", "unknown sequence id")
        before = [self.token_count(int(s)) for s in seqs]
        bt = self._cfg.block_tokens
        need = max([(n + c + bt - 1) // bt for n, c in zip(before, counts)] or [1])
        if stride is None:
            stride = max(1, need)
        elif stride < need:
            raise KvCacheError("InvalidArgs", "stride shorter than a block table")
        starts = self.reserve_batch(seqs, counts)
        try:
            tables, _ = self.block_tables(seqs, stride)
            cu = torch.from_numpy(np.concatenate([[0], np.cumsum(counts)]).astype(np.int32))
            sp = torch.from_numpy(starts.astype(np.int32)).to(self.device)
            if total:
                self._kv.append_kv_batched(stream, self.layout, self.pool, keys.contiguous(),
                                           values.contiguous(), tables, cu.to(self.device), sp,
                                           total)
        except BaseException:
            for s, n in reversed(list(zip(seqs, before))):
                self.truncate(int(s), n)
            raise
        return tables, sp, [n + c for n, c in zip(before, counts)]

    def append_batch(self, seqs, keys, values, stream=None, stride=None):
        """Append one token to every sequence in `seqs` with one kernel launch
        (extend_batch with a count of 1 each; same all-or-nothing rule).
        keys/values: [len(seqs), row_len] device tensors in the pool dtype."""
        return self.extend_batch(seqs, [1] * len(seqs), keys, values, stream, stride)
