"""Two reference call sites driven through this library exactly as a
maintainer would rebind them (the walkthroughs in the integration notes).

1. The streaming forward driver's per-layer KV step
   (engine/engine-core/src/streaming_forward_driver.rs:514-540): each layer
   owns an f32 pool of ONE page of `capacity` tokens (layout n_blocks 1,
   block_tokens capacity, :178-183; block table [0], :273); per token p it
   calls PagedKvGpu::append_kv(p, 1) and then PagedAttention::launch with
   seq_tokens p + 1, query_pos p, causal.  Every layer's output against
   orc.sdpa_decode on the oracle cache built by the same appends, the pools
   byte for byte; the one-launch form (eh_append_flash_decoding) gives the
   same pool bytes and the same output to the f32 bar; a position past the
   page is the reference's InvalidSize.
2. The server's continuous-batching scheduler over the CPU cache
   (engine/engine-server/src/scheduler.rs:20-99, session.rs:40-83): sessions
   are added (new_sequence + one appended row), advanced one token per round
   (append, read the key row back, digest, next token), retired or cancelled
   (free_sequence).  Here the same loop runs over PagedKvCache (pool in HBM)
   and over orc.Cache side by side: produced tokens, blocks in use, block
   tables and pool bytes agree every round; the reference's own scheduler
   tests (scheduler.rs:235-271) hold; a session that does not fit is
   PoolExhausted with nothing changed (cache.rs:164-177, no partial state).
"""
import numpy as np
import pytest
import torch

from oracle import orc
from titan_amd import HipError, KvDataType, PagedAttention, PagedKvGpu, PagedKvLayout
from titan_amd.errors import KvCacheError
from titan_amd.kvcache import PagedKvCache, PagedKvCacheConfig

import parity

pytestmark = pytest.mark.gpu


def test_streaming_driver_layer_loop(dev):
    nh, nkv, hd, capacity, layers = 14, 2, 64, 256, 3
    row = nkv * hd
    rng = np.random.default_rng(514)
    layout = PagedKvLayout(1, capacity, row, KvDataType.F32)
    pkv, pa = PagedKvGpu(0), PagedAttention(0)
    bt = torch.zeros(1, dtype=torch.int32, device=dev)       # the driver's [0] table
    pools = [torch.zeros(capacity * 2 * row, dtype=torch.float32, device=dev)
             for _ in range(layers)]
    fused = [torch.zeros_like(p) for p in pools]            # the one-launch form's pools
    oracle = [orc.Cache(1, capacity, nkv, hd) for _ in range(layers)]
    seqs = [o.new_sequence() for o in oracle]
    out = torch.empty(nh * hd, dtype=torch.float32, device=dev)
    out1 = torch.empty_like(out)
    # tokens 0..23, then the last positions of the page after a bulk prefix
    steps = list(range(24)) + [capacity - 2, capacity - 1]
    for p in steps:
        if p == capacity - 2:   # fill 24 .. capacity-3 as a prompt would
            n = capacity - 2 - 24
            for l in range(layers):
                k = rng.standard_normal((n, row)).astype(np.float32)
                v = rng.standard_normal((n, row)).astype(np.float32)
                kd, vd = torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev)
                pkv.append_kv(None, layout, pools[l], kd, vd, bt, 24, n)
                pkv.append_kv(None, layout, fused[l], kd, vd, bt, 24, n)
                for t in range(n):
                    oracle[l].append(seqs[l], k[t], v[t])
        for l in range(layers):
            k = rng.standard_normal(row).astype(np.float32)
            v = rng.standard_normal(row).astype(np.float32)
            q = rng.standard_normal(nh * hd).astype(np.float32)
            kd, vd, qd = (torch.from_numpy(x).to(dev) for x in (k, v, q))
            # d. append K, V to the resident layer pool; e. paged attention
            pkv.append_kv(None, layout, pools[l], kd, vd, bt, p, 1)
            pa.launch(None, qd, pools[l], bt, out, nh, nkv, hd, capacity, p + 1, p, True)
            pa.append_flash_decoding(None, kd, vd, qd, fused[l], bt, out1, nh, nkv, hd,
                                     capacity, p)
            oracle[l].append(seqs[l], k, v)
            ref = orc.sdpa_decode(oracle[l].buffer(), np.zeros(1, np.uint32), capacity, p + 1,
                                  q, nh, nkv, hd, True, p)
            torch.cuda.synchronize()
            parity.check_close(out.cpu().numpy(), ref, f32=True, what=f"driver p={p} l={l}")
            parity.check_close(out1.cpu().numpy(), ref, f32=True, what=f"one-launch p={p} l={l}")
    torch.cuda.synchronize()
    for l in range(layers):
        want = oracle[l].buffer().view(np.uint8)
        assert np.array_equal(pools[l].cpu().numpy().view(np.uint8), want)
        assert np.array_equal(fused[l].cpu().numpy().view(np.uint8), want)
    # the driver refuses p >= block_tokens itself (:383-388); the append's own
    # validation is the same InvalidSize
    kd = torch.zeros(row, dtype=torch.float32, device=dev)
    with pytest.raises(HipError) as e:
        pkv.append_kv(None, layout, pools[0], kd, kd, bt, capacity, 1)
    assert e.value.kind == "InvalidSize"


# ---- the server's placeholder session (session.rs:85-128), restated ----------

def kv_row(token, row_len):
    """session.rs:113-128: deterministic rows from the token id (u32 wrap)."""
    i = np.arange(row_len, dtype=np.uint64)
    ki = ((token * 7) % 2**32 + i) % 2**32 % 97
    vi = ((token * 13) % 2**32 + i) % 2**32 % 89
    return ki.astype(np.float32) * np.float32(0.25), vi.astype(np.float32) * np.float32(0.5)


def digest_layer(row):
    """session.rs:104-111: FNV-1a over trunc(|v| * 1000) computed in f32."""
    h = 1469598103934665603
    for v in np.abs(np.asarray(row, np.float32)) * np.float32(1000.0):
        h = ((h ^ int(v)) * 1099511628211) % 2**64
    return h


def stub_next_token(token, digest, vocab):
    """session.rs:90-96"""
    a = (token * 2654435761) % 2**32
    return ((a ^ (digest & 0xFFFF)) % vocab) + 1


class Session:
    """session.rs:40-83 over either cache (the product's PagedKvCache or
    orc.Cache): the cache is the scheduler's, the session holds its ids."""

    def __init__(self, cache, seq, vocab, prompt_token, max_tokens):
        k, v = kv_row(prompt_token, cache_row_len(cache))
        cache.append(seq, k, v)
        self.seq, self.current, self.steps = seq, prompt_token, 0
        self.vocab, self.max_tokens = vocab, max_tokens

    def finished(self):
        return self.max_tokens == 0 or self.steps >= self.max_tokens

    def step(self, cache):
        if self.finished():
            return None
        index = cache.token_count(self.seq)
        k, v = kv_row(self.current, cache_row_len(cache))
        cache.append(self.seq, k, v)
        back = cache.read_key(self.seq, index)
        back = back.cpu().numpy() if torch.is_tensor(back) else np.asarray(back)
        d = (digest_layer(back) * 31 + self.current) % 2**64
        self.current = stub_next_token(self.current, d, self.vocab)
        self.steps += 1
        return self.current


def cache_row_len(cache):
    cfg = cache.config()
    return cfg.row_len() if callable(getattr(cfg, "row_len", None)) else cfg


class Scheduler:
    """scheduler.rs:12-99: one cache, sessions advanced one token per round,
    retired or cancelled sessions free their pages."""

    def __init__(self, cache):
        self.cache, self.active = cache, []

    def add(self, vocab, prompt_token, max_tokens):
        seq = self.cache.new_sequence()
        self.active.append(Session(self.cache, seq, vocab, prompt_token, max_tokens))
        return len(self.active) - 1

    def advance(self):
        produced, nxt = [], []
        for s in self.active:
            if s.finished():
                self.cache.free_sequence(s.seq)
                continue
            t = s.step(self.cache)
            if t is not None:
                produced.append(t)
            if s.finished():
                self.cache.free_sequence(s.seq)
            else:
                nxt.append(s)
        self.active = nxt
        return produced

    def cancel(self, index):
        if index < len(self.active):
            self.cache.free_sequence(self.active.pop(index).seq)


class _OrcCfg:
    def __init__(self, row):
        self._row = row

    def row_len(self):
        return self._row


def pair(n_blocks, block_tokens, heads, head_dim):
    c = PagedKvCache(PagedKvCacheConfig(n_blocks, block_tokens, heads, head_dim), KvDataType.F32)
    o = orc.Cache(n_blocks, block_tokens, heads, head_dim)
    o.config = lambda: _OrcCfg(heads * head_dim)
    return Scheduler(c), Scheduler(o)


def same_state(a, b):
    torch.cuda.synchronize()
    assert a.cache.blocks_used() == b.cache.blocks_used()
    assert [s.seq for s in a.active] == [s.seq for s in b.active]
    for s in a.active:
        assert list(a.cache.seq_block_table(s.seq)) == list(b.cache.seq_block_table(s.seq))
    got = a.cache.pool.cpu().numpy().view(np.uint8)
    assert np.array_equal(got, b.cache.buffer().view(np.uint8))


def test_scheduler_reference_scenarios(dev):
    # scheduler.rs:225-233 config; :235-255 and :257-271
    a, b = pair(16, 128, 1, 1)
    for s in (a, b):
        s.add(1000, 3, 2)
        s.add(1000, 7, 5)
    rounds = []
    while a.active:
        pa_, pb_ = a.advance(), b.advance()
        assert pa_ == pb_
        rounds.append(len(pa_))
        same_state(a, b)
    assert rounds == [2, 2, 1, 1, 1] and not b.active
    assert a.cache.blocks_used() == 0
    a, b = pair(16, 128, 1, 1)
    for s in (a, b):
        s.add(1000, 11, 64)
    assert a.cache.blocks_used() > 0
    same_state(a, b)
    a.cancel(0)
    b.cancel(0)
    assert a.cache.blocks_used() == 0 and not a.active
    same_state(a, b)


def test_scheduler_page_reuse_and_exhaustion(dev):
    """Sessions of ragged budgets on 16-token pages: retired pages are reused
    by later admissions in the reference's order, a cancel mid-run, and an
    admission that does not fit raises PoolExhausted with nothing changed."""
    a, b = pair(24, 16, 2, 64)
    budgets = [5, 40, 17, 0, 33, 12]
    for i, m in enumerate(budgets):
        for s in (a, b):
            s.add(50000, 100 + i, m)
    same_state(a, b)
    for r in range(60):   # the last admission (round 20, budget 30) retires at 51
        pa_, pb_ = a.advance(), b.advance()
        assert pa_ == pb_, f"round {r}"
        same_state(a, b)
        if r == 8:
            for s in (a, b):
                s.cancel(1)
            same_state(a, b)
        if r in (10, 20):
            for s in (a, b):
                s.add(50000, 900 + r, 30)
            same_state(a, b)
    assert not a.active and a.cache.blocks_used() == 0
    # fill the pool, then one more admission must fail with no partial state
    for s in (a, b):
        for i in range(24):
            s.add(50000, 7 + i, 100)
    same_state(a, b)
    used = a.cache.blocks_used()
    with pytest.raises(KvCacheError) as e:
        a.add(50000, 1, 5)
    assert e.value.kind == "PoolExhausted"
    with pytest.raises(orc.KvCacheError):
        b.add(50000, 1, 5)
    assert a.cache.blocks_used() == used == a.cache.blocks_total()
    assert a.cache.token_count(a.cache.sequences() - 1) == 0
    same_state(a, b)
