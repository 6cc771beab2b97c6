"""eh_append_decode_batched_noalloc: the fused decode step with the library's
per-GPU static scratch in place of a caller workspace (for callers that
cannot allocate device memory).  It has no counterpart in the reference.

Checked through the C-ABI against eh_append_decode_batched (the same kernels
with a torch workspace) on the same inputs: pool bytes and outputs bit for
bit, on two calls in a row -- the second with a smaller batch and shorter
contexts, so stale partials of the first call sit in the shared scratch --
and against the oracle within the parity bar.  Also: no device allocation
across repeated calls, and a shape whose partials exceed the 32 MiB scratch
is rejected before any launch.
"""
import numpy as np
import pytest
import torch

from oracle import orc
from titan_amd import HipError, KvDataType, PagedAttention, PagedKvLayout

import parity

pytestmark = pytest.mark.gpu

NONE = 0xFFFFFFFF


def i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(dev)


def case(dev, rng, pos, n_head=12, n_kv=2, hd=128, bt=16):
    rl = n_kv * hd
    B = len(pos)
    need = [(int(p) + 1 + bt - 1) // bt for p in pos]
    nb = sum(need) + 3
    perm = rng.permutation(nb).astype(np.uint32)
    tab = np.full((B, max(need)), NONE, np.uint32)
    o = 0
    for b, c in enumerate(need):
        tab[b, :c] = perm[o:o + c]
        o += c
    host = rng.standard_normal(nb * bt * 2 * rl).astype(np.float16)
    k = rng.standard_normal((B, rl)).astype(np.float16)
    v = rng.standard_normal((B, rl)).astype(np.float16)
    q = rng.standard_normal((B, n_head, hd)).astype(np.float32)
    return dict(tab=tab, nb=nb, host=host, k=k, v=v, q=q, pos=np.asarray(pos, np.uint32),
                shape=(n_head, n_kv, hd, bt))


def run_pair(dev, c):
    n_head, n_kv, hd, bt = c["shape"]
    B = len(c["pos"])
    layout = PagedKvLayout(c["nb"], bt, n_kv * hd, KvDataType.F16)
    plan = PagedAttention.plan(B, n_head, n_kv, hd, bt, int(c["pos"].max()) + 1)
    assert plan[0] == 0
    t = lambda a: torch.from_numpy(a).to(dev)
    dtab, dpos, dk, dv, dq = i32(c["tab"], dev), i32(c["pos"], dev), t(c["k"]), t(c["v"]), t(c["q"])
    pa = PagedAttention(0)
    pool_a, pool_b = t(c["host"].copy()), t(c["host"].copy())
    out_a = torch.full((B, n_head, hd), float("nan"), device=dev)
    out_b = torch.full((B, n_head, hd), float("nan"), device=dev)
    pa.append_decode_batched(None, layout, pool_a, dk, dv, dtab, dpos, dq, out_a, n_head, hd, plan,
                             PagedAttention.workspace(plan))
    pa.append_decode_batched_noalloc(None, layout, pool_b, dk, dv, dtab, dpos, dq, out_b, n_head,
                                     hd, plan[1])
    torch.cuda.synchronize()
    assert torch.equal(pool_a.view(torch.int16), pool_b.view(torch.int16))
    oa, ob = out_a.cpu().numpy(), out_b.cpu().numpy()
    assert np.array_equal(oa.view(np.uint32), ob.view(np.uint32))
    want = c["host"].reshape(c["nb"], bt, 2, n_kv * hd).copy()
    for b, p in enumerate(c["pos"]):
        want[c["tab"][b, p // bt], p % bt, 0] = c["k"][b]
        want[c["tab"][b, p // bt], p % bt, 1] = c["v"][b]
    ref = orc.sdpa_decode_batched(want.reshape(-1).astype(np.float32), c["tab"], c["pos"] + 1, bt,
                                  c["q"], n_head, n_kv, hd)
    parity.check_close(ob, ref, what="noalloc")
    return layout, pool_b, dk, dv, dtab, dpos, dq, out_b, plan


def test_noalloc_equals_workspace_entry_two_calls(dev):
    rng = np.random.default_rng(2718)
    # first call: config 2's shape (batch 32, contexts U[128, 4096])
    first = case(dev, rng, rng.integers(127, 4096, size=32))
    run_pair(dev, first)
    # second call, smaller: 5 sequences, short contexts, page-boundary positions
    second = case(dev, rng, [0, 15, 16, 300, 33])
    layout, pool, dk, dv, dtab, dpos, dq, out, plan = run_pair(dev, second)
    # repeated calls allocate nothing
    pa = PagedAttention(0)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    n_alloc = torch.cuda.memory_stats()["allocation.all.allocated"]
    for _ in range(50):
        pa.append_decode_batched_noalloc(None, layout, pool, dk, dv, dtab, dpos, dq, out, 12, 128,
                                         plan[1])
    torch.cuda.synchronize()
    assert torch.cuda.memory_stats()["allocation.all.allocated"] == n_alloc
    assert torch.cuda.mem_get_info()[0] >= free0


def test_noalloc_rejects_shapes_beyond_the_scratch(dev):
    # (grid + batch) * n_head * 130 * 4 bytes > 32 MiB: 2048 sequences x 64 heads
    n_head, n_kv, hd, bt, B = 64, 8, 128, 16, 2048
    layout = PagedKvLayout(4, bt, n_kv * hd, KvDataType.F16)
    plan = PagedAttention.plan(B, n_head, n_kv, hd, bt, 64)
    need = 4 * (plan[1] + B) * n_head * 130
    assert need > 32 << 20
    tiny = torch.zeros(16, device=dev)
    tab = torch.zeros((B, 1), dtype=torch.int32, device=dev)
    with pytest.raises(HipError) as e:
        PagedAttention(0).append_decode_batched_noalloc(None, layout, tiny, tiny, tiny, tab, tiny,
                                                        tiny, tiny, n_head, hd, plan[1])
    assert e.value.kind == "InvalidSize"
    assert (e.value.expected, e.value.actual) == (32 << 20, need)
