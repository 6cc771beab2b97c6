"""Prefix-shared KV with copy-on-write, LRU eviction and gather-compaction
(benchmark config 4), driven through the engine-kvcache surfaces.

Flow (each step uses the reference's bookkeeping semantics; page bytes move
on the GPU):
  1. a 1024-token prefix fills 64 pages of a pinned prefix table;
  2. each of the 64 sequences forks the prefix table
     (CowBlockTable::fork, cow.rs:40-45) and appends a private suffix of
     U[64, 512] tokens;
  3. each sequence forks a child branch; the child appends 16 tokens.  When
     the child's tail page is shared AND partially filled, it is copied to a
     fresh page first (eh_copy_pages) and swapped in with perform_tail_cow
     (cow.rs:73-81).  tail_needs_cow (cow.rs:64-70) looks only at the
     reference count, so a full shared tail is left alone: the append opens a
     new page and never writes into the shared one;
  4. the parents retire; pages no table references any more return to the
     free list;
  5. the children are indexed in a RadixTree under the pinned prefix node
     (radix.rs:120-204), touched in a seeded order (match_prefix), and
     evict_lru (radix.rs:208-222) frees at least 25 % of the live pages; the
     evicted children are dropped;
  6. survivors are gather-compacted to the lowest page ids
     (eh_compaction_plan -> eh_copy_pages -> eh_remap_block_tables), and
     page reference counts are recounted on the device (eh_page_refcounts).

The bookkeeping classes are parameters so the same flow can be run on the
product objects (titan_amd.share) or on any object with the reference's
method names.
"""
from dataclasses import dataclass, field

import numpy as np


def _match(radix, tokens):
    r = radix.match_prefix(tokens)
    if isinstance(r, tuple):
        return r[0], list(r[1])
    return r.matched_tokens, list(r.matched_blocks)


@dataclass
class AppendOp:
    tables: np.ndarray      # [B, stride] u32 (pad 0xFFFFFFFF)
    cu: np.ndarray          # [B+1] u32
    start: np.ndarray       # [B] u32
    keys: np.ndarray        # [T, row_len] f16
    values: np.ndarray      # [T, row_len] f16


@dataclass
class CopyOp:
    src: np.ndarray
    dst: np.ndarray


@dataclass
class Plan:
    ops: list = field(default_factory=list)
    tables: dict = field(default_factory=dict)          # seq -> final page ids (pre-compaction)
    compacted: dict = field(default_factory=dict)       # seq -> page ids after compaction
    tokens: dict = field(default_factory=dict)          # seq -> token count
    rows: dict = field(default_factory=dict)            # seq -> (keys, values) f16 [n, row_len]
    victims: list = field(default_factory=list)         # pages freed by evict_lru, in order
    evicted_seqs: list = field(default_factory=list)
    cow_pairs: int = 0
    strong_counts: dict = field(default_factory=dict)   # page -> CoW strong count (survivors)
    remap: np.ndarray = None
    compaction: CopyOp = None
    n_blocks: int = 0
    live_before_evict: int = 0


class PrefixShareScenario:
    def __init__(self, seed=0, n_seqs=64, prefix_tokens=1024, suffix=(64, 512), append=16,
                 n_kv=8, head_dim=128, block_tokens=16, evict_frac=0.25, cow_cls=None,
                 radix_cls=None, compaction_plan=None):
        if cow_cls is None or radix_cls is None or compaction_plan is None:
            from .share import CowBlockTable, RadixTree, compaction_plan as cp
            cow_cls = cow_cls or CowBlockTable
            radix_cls = radix_cls or RadixTree
            compaction_plan = compaction_plan or cp
        self.cow_cls, self.radix_cls, self.compaction_plan = cow_cls, radix_cls, compaction_plan
        self.rng = np.random.default_rng(seed)
        # The touch order that drives LRU eviction has a generator of its own,
        # created before any row is drawn: the plan (victims, tables, remap)
        # then depends on the seed and the page counts only, not on how many
        # random values the rows consumed (row_len).
        self.touch_rng = np.random.default_rng([seed, 0x70C4])
        self.n_seqs, self.prefix_tokens, self.append = n_seqs, prefix_tokens, append
        self.n_kv, self.head_dim, self.bt = n_kv, head_dim, block_tokens
        self.row_len = n_kv * head_dim
        self.evict_frac = evict_frac
        self.suffix = self.rng.integers(suffix[0], suffix[1], size=n_seqs, endpoint=True)
        bt = block_tokens
        need = -(-prefix_tokens // bt) + sum(-(-(int(l) + append) // bt) + 2 for l in self.suffix)
        self.n_blocks = int(need * 1.25) + 8
        self.free = [int(x) for x in self.rng.permutation(self.n_blocks)[::-1]]  # pop() from end

    # ------------------------------------------------------------------ helpers
    def _rows(self, n):
        k = self.rng.standard_normal((n, self.row_len)).astype(np.float16)
        v = self.rng.standard_normal((n, self.row_len)).astype(np.float16)
        return k, v

    def _append_op(self, seqs, tables, starts, rows):
        stride = max(len(tables[s]) for s in seqs)
        tab = np.full((len(seqs), stride), 0xFFFFFFFF, np.uint32)
        for i, s in enumerate(seqs):
            tab[i, :len(tables[s])] = tables[s]
        lens = [rows[s][0].shape[0] for s in seqs]
        cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
        return AppendOp(tab, cu, np.array([starts[s] for s in seqs], np.uint32),
                        np.concatenate([rows[s][0] for s in seqs]),
                        np.concatenate([rows[s][1] for s in seqs]))

    # ------------------------------------------------------------------ plan
    def plan(self):
        bt, P = self.bt, Plan()
        P.n_blocks = self.n_blocks
        n_pre_pages = -(-self.prefix_tokens // bt)
        # 1. prefix
        prefix = self.cow_cls()
        for _ in range(n_pre_pages):
            prefix.append_block(self.free.pop())
        pk, pv = self._rows(self.prefix_tokens)
        pre_ids = prefix.physical_block_ids()
        P.ops.append(self._append_op(["p"], {"p": pre_ids}, {"p": 0}, {"p": (pk, pv)}))
        # 2. parents fork the prefix and append their suffix
        parents, ids, rows, starts = [], {}, {}, {}
        for s in range(self.n_seqs):
            parents.append(prefix.fork())
            L = int(self.suffix[s])
            for _ in range(-(-(self.prefix_tokens + L) // bt) - n_pre_pages):
                parents[s].append_block(self.free.pop())
            ids[s] = parents[s].physical_block_ids()
            rows[s] = self._rows(L)
            starts[s] = self.prefix_tokens
        P.ops.append(self._append_op(list(range(self.n_seqs)), ids, starts, rows))
        seq_rows = {s: (np.concatenate([pk, rows[s][0]]), np.concatenate([pv, rows[s][1]]))
                    for s in range(self.n_seqs)}
        # 3. children fork and append, copy-on-write of shared partial tails
        children, cow_src, cow_dst = [], [], []
        crow, cids, cstart = {}, {}, {}
        for s in range(self.n_seqs):
            children.append(parents[s].fork())
            c = children[s]
            pos = self.prefix_tokens + int(self.suffix[s])
            if pos % bt != 0 and c.tail_needs_cow():
                new = self.free.pop()
                cow_src.append(c.physical_block_ids()[-1])
                cow_dst.append(new)
                c.perform_tail_cow(new)
            end = pos + self.append
            while len(c) * bt < end:
                c.append_block(self.free.pop())
            cids[s] = c.physical_block_ids()
            crow[s] = self._rows(self.append)
            cstart[s] = pos
        P.cow_pairs = len(cow_src)
        if cow_src:
            P.ops.append(CopyOp(np.array(cow_src, np.uint32), np.array(cow_dst, np.uint32)))
        P.ops.append(self._append_op(list(range(self.n_seqs)), cids, cstart, crow))
        for s in range(self.n_seqs):
            seq_rows[s] = (np.concatenate([seq_rows[s][0], crow[s][0]]),
                           np.concatenate([seq_rows[s][1], crow[s][1]]))
        # 4. parents and the prefix table retire; unreferenced pages are freed
        del c
        parents.clear()
        del prefix
        live = set()
        for c in children:
            live.update(c.physical_block_ids())
        allocated = set(range(self.n_blocks)) - set(self.free)
        for p in sorted(allocated - live):
            self.free.append(p)
        P.live_before_evict = len(live)
        # 5. radix index, seeded touches, LRU eviction of >= evict_frac of pages
        radix = self.radix_cls(bt)
        pre_tokens = list(range(self.prefix_tokens))
        radix.insert(pre_tokens, pre_ids, True)
        tok = {}
        for s in range(self.n_seqs):
            n_tok = self.prefix_tokens + int(self.suffix[s]) + self.append
            tok[s] = pre_tokens + [1_000_000 + s * 10_000 + i for i in range(n_tok - self.prefix_tokens)]
            radix.insert(tok[s], cids[s], False)
        for s in self.touch_rng.permutation(self.n_seqs):
            m, blk = _match(radix, tok[int(s)])
            assert m == len(tok[int(s)]) and blk == cids[int(s)]
        target = int(np.ceil(self.evict_frac * len(live)))
        P.victims = list(radix.evict_lru(target))
        gone = set(P.victims)
        survivors = []
        for s in range(self.n_seqs):
            if gone.intersection(cids[s][n_pre_pages:]):
                P.evicted_seqs.append(s)
            else:
                survivors.append(s)
        for s in P.evicted_seqs:
            children[s] = None
        self.free.extend(P.victims)
        # 6. compaction over the survivors
        stride = max(len(cids[s]) for s in survivors)
        tab = np.full((len(survivors), stride), 0xFFFFFFFF, np.uint32)
        n_used = np.array([len(cids[s]) for s in survivors], np.uint32)
        for i, s in enumerate(survivors):
            tab[i, :len(cids[s])] = cids[s]
        src, dst, remap = self.compaction_plan(tab, n_used, self.n_blocks)
        P.compaction = CopyOp(src, dst)
        P.remap = remap
        for i, s in enumerate(survivors):
            P.tables[s] = cids[s]
            P.compacted[s] = [int(remap[p]) for p in cids[s]]
            P.tokens[s] = self.prefix_tokens + int(self.suffix[s]) + self.append
            P.rows[s] = seq_rows[s]
            c = children[s]
            for j, p in enumerate(cids[s]):
                P.strong_counts[int(remap[p])] = int(c.ref_count(j)) if hasattr(c, "ref_count") \
                    else int(c.refcount(j))
        self.survivors = survivors
        self.survivor_table = tab
        self.survivor_used = n_used
        return P


def model_pool(scn, plan):
    """Host model of the pool bytes after every op of `plan` (copies are
    exact, so the model is the expected device state bit for bit)."""
    bt, rl = scn.bt, scn.row_len
    pool = np.zeros((plan.n_blocks, bt, 2, rl), dtype=np.float16)
    for op in plan.ops:
        if isinstance(op, CopyOp):
            pool[op.dst] = pool[op.src]
            continue
        for b in range(op.tables.shape[0]):
            for i in range(int(op.cu[b]), int(op.cu[b + 1])):
                pos = int(op.start[b]) + i - int(op.cu[b])
                page = int(op.tables[b, pos // bt])
                pool[page, pos % bt, 0] = op.keys[i]
                pool[page, pos % bt, 1] = op.values[i]
    if plan.compaction is not None and len(plan.compaction.src):
        pool[plan.compaction.dst] = pool[plan.compaction.src]
    return pool


def run_on_gpu(scn, plan, device=0, stream=None):
    """Executes the plan's page moves on the GPU; returns the device pool, the
    remapped device tables and the device reference counts."""
    import torch

    from .paged_kv import KvDataType, PagedKvGpu, PagedKvLayout

    dev = torch.device("cuda", device)
    kv = PagedKvGpu(device)
    layout = PagedKvLayout(plan.n_blocks, scn.bt, scn.row_len, KvDataType.F16)
    pool = torch.zeros(layout.floats_total(), dtype=torch.float16, device=dev)

    def i32(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).to(dev)

    for op in plan.ops:
        if isinstance(op, CopyOp):
            kv.copy_pages(stream, layout, pool, i32(op.src), i32(op.dst))
        else:
            kv.append_kv_batched(stream, layout, pool, torch.from_numpy(op.keys).to(dev),
                                 torch.from_numpy(op.values).to(dev), i32(op.tables),
                                 i32(op.cu), i32(op.start), int(op.cu[-1]))
    tables = i32(scn.survivor_table)
    if len(plan.compaction.src):
        kv.copy_pages(stream, layout, pool, i32(plan.compaction.src), i32(plan.compaction.dst))
    kv.remap_block_tables(stream, tables, i32(plan.remap))
    counts = torch.zeros(plan.n_blocks, dtype=torch.int32, device=dev)
    kv.page_refcounts(stream, tables, i32(scn.survivor_used), counts)
    torch.cuda.synchronize()
    return pool, tables, counts, layout
