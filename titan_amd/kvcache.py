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

    def append(self, seq, key, value, stream=None):
        """cache.rs:153-192: one token's K and V rows."""
        k, v = self._row_tensor(key), self._row_tensor(value)
        m = self._cfg.row_len()
        if k.numel() != m or v.numel() != m:
            raise KvCacheError("InvalidArgs", "key/value length must equal heads * head_dim")
        pos = self.reserve(seq, 1)
        self._kv.append_kv(stream, self.layout, self.pool, k, v, self._table_dev(seq), pos, 1)

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

    def append_batch(self, seqs, keys, values, stream=None, stride=None):
        """Append one token to every sequence in `seqs` with one kernel launch.
        keys/values: [len(seqs), row_len] device tensors in the pool dtype."""
        starts = [self.reserve(int(s), 1) for s in seqs]
        tables, _ = self.block_tables(seqs, stride)
        B = len(seqs)
        cu = torch.arange(B + 1, dtype=torch.int32, device=self.device)
        sp = torch.tensor(starts, dtype=torch.int32, device=self.device)
        self._kv.append_kv_batched(stream, self.layout, self.pool, keys.contiguous(),
                                   values.contiguous(), tables, cu, sp, B)
        return tables
