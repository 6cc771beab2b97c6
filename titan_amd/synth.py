"""Seeded synthetic workloads for the paged KV path (the five benchmark shapes).

Inputs are drawn with numpy's PCG64 (`np.random.default_rng(seed)`), N(0,1)
in f64, then rounded to the storage type (f32, or f16/bf16 with
round-to-nearest-even).  Queries stay f32 (the reference API is f32).
Block tables come from a seeded shuffled free list: sequence b pops its
pages in order, so logically adjacent pages sit at scattered physical ids.
"""
from dataclasses import dataclass, field

import numpy as np
import torch

from .paged_kv import KvDataType

NP_STORAGE = {KvDataType.F32: np.float32, KvDataType.F16: np.float16}


def round_to(x, dtype):
    """f32/f64 array -> torch tensor in the storage dtype (RNE), on the CPU."""
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    return t.to({KvDataType.F32: torch.float32, KvDataType.F16: torch.float16,
                 KvDataType.BF16: torch.bfloat16}[KvDataType(dtype)])


def widen(t):
    """Storage tensor -> exact f32 numpy array."""
    return t.detach().to("cpu").to(torch.float32).numpy()


@dataclass
class DecodeShape:
    batch: int
    n_head: int
    n_head_kv: int
    head_dim: int
    block_tokens: int
    dtype: KvDataType
    ctx_lens: np.ndarray          # tokens already cached per sequence
    n_blocks: int                 # pool pages
    free_order: np.ndarray        # page pop order (seeded shuffle)
    meta: dict = field(default_factory=dict)

    @property
    def row_len(self):
        return self.n_head_kv * self.head_dim


def config1(seed=0):
    """B=1, 14/2 heads, hd 64, page 16, f32: 511 cached tokens + 1 appended = 512
    attended, on the first 32 pages of a seeded permutation of a 64-page pool."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(64).astype(np.uint32)
    return DecodeShape(1, 14, 2, 64, 16, KvDataType.F32, np.array([511], dtype=np.int64), 64,
                       perm, {"seed": seed})


def config2(seed=0, extra_tokens=64):
    """B=32, 12/2 heads, hd 128, page 16, f16.  ctx ~ U[128, 4096]; pool =
    ceil(1.2 * sum(ctx) / 16) pages (at least what ctx + extra_tokens needs)."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(128, 4096, size=32, endpoint=True).astype(np.int64)
    need = int(sum((int(l) + extra_tokens + 15) // 16 for l in lens))
    n_blocks = max(int(np.ceil(1.2 * lens.sum() / 16)), need)
    perm = rng.permutation(n_blocks).astype(np.uint32)
    return DecodeShape(32, 12, 2, 128, 16, KvDataType.F16, lens, n_blocks, perm, {"seed": seed})


def config3(seed=0, chunk=512, cached=2048):
    """B=8, 32/8 heads, hd 128, page 16, bf16: each sequence holds `cached`
    tokens and appends a `chunk`-token prefill chunk.  Pool = ceil(1.2 x the
    pages the chunks end on), seeded shuffled free list."""
    rng = np.random.default_rng(seed)
    need = 8 * ((cached + chunk + 15) // 16)
    n_blocks = int(np.ceil(1.2 * need))
    perm = rng.permutation(n_blocks).astype(np.uint32)
    return DecodeShape(8, 32, 8, 128, 16, KvDataType.BF16, np.full(8, cached, dtype=np.int64),
                       n_blocks, perm, {"seed": seed, "chunk": chunk})


def config5(seed=0, n_blocks=None, batch=4, ctx=32768):
    """B=4 at 32768 tokens, 32/8 heads, hd 128, page 16, f16.  Pages scattered
    by a seeded permutation over `n_blocks` pages."""
    rng = np.random.default_rng(seed)
    need = batch * ((ctx + 1 + 15) // 16)
    n_blocks = max(n_blocks or need, need)
    perm = rng.permutation(n_blocks).astype(np.uint32)
    return DecodeShape(batch, 32, 8, 128, 16, KvDataType.F16,
                       np.full(batch, ctx, dtype=np.int64), n_blocks, perm, {"seed": seed})


def block_tables(shape, extra_tokens=0):
    """Pop pages for ctx_lens[b] + extra_tokens tokens per sequence in order
    b = 0..B-1.  Returns [B, stride] uint32 (pad 0xFFFFFFFF)."""
    bt = shape.block_tokens
    counts = [(int(l) + extra_tokens + bt - 1) // bt for l in shape.ctx_lens]
    stride = max(counts)
    tab = np.full((shape.batch, stride), 0xFFFFFFFF, dtype=np.uint32)
    pos = 0
    for b, c in enumerate(counts):
        if pos + c > shape.n_blocks:
            raise ValueError("pool too small for the requested contexts")
        tab[b, :c] = shape.free_order[pos:pos + c]
        pos += c
    return tab


def normal(rng, shape):
    return rng.standard_normal(shape)
