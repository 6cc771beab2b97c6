"""Launches allocate no device memory.

The reference asserts that its live-allocation counter is unchanged across
paged-attention launches (engine-cuda/tests/paged_attention_parity.rs:
196-216, counter at engine-cuda/src/device_buffer.rs:160-163).  Here the
device's free memory (hipMemGetInfo, through torch.cuda.mem_get_info) is
read before and after 100 launches of every entry point, after one warm-up
launch each (which may load a code object); every buffer is created before
the first reading and torch's own allocation counter confirms that the loop
itself allocated nothing.
"""
import numpy as np
import pytest
import torch

from titan_amd import FlashAttention2, KvDataType, PagedAttention, PagedKvGpu, PagedKvLayout

pytestmark = pytest.mark.gpu


def i32(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(dev)


def test_launches_do_not_allocate(dev):
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    kv, pa, fa = PagedKvGpu(0), PagedAttention(0), FlashAttention2(0)
    B, nh, nkv, hd, bt = 8, 12, 2, 128, 16
    rl = nkv * hd
    nb = 8 * 40 + 4
    tab = np.arange(nb - 4, dtype=np.uint32).reshape(8, 40)
    d_tab = i32(tab, dev)
    lay16 = PagedKvLayout(nb, bt, rl, KvDataType.F16)
    pool16 = torch.randn(lay16.floats_total(), generator=g, device=dev).half()
    lay32 = PagedKvLayout(nb, bt, rl, KvDataType.F32)
    pool32 = torch.randn(lay32.floats_total(), generator=g, device=dev)
    lay8 = PagedKvLayout(nb, bt, rl, KvDataType.FP8)
    pool8 = torch.randint(0, 0x7E, (lay8.floats_total(),), generator=g, device=dev,
                          dtype=torch.uint8)
    scales = torch.full((nkv,), 0.02, device=dev)
    lens = torch.full((B,), 500, dtype=torch.int32, device=dev)
    pos = lens - 1
    cu = torch.arange(B + 1, dtype=torch.int32, device=dev)
    q = torch.randn((B, nh, hd), generator=g, device=dev)
    out = torch.empty_like(q)
    k16 = torch.randn((B, rl), generator=g, device=dev).half()
    v16 = torch.randn((B, rl), generator=g, device=dev).half()
    k32 = torch.randn((B, rl), generator=g, device=dev)
    v32 = torch.randn((B, rl), generator=g, device=dev)
    gout = torch.empty((300, rl), device=dev, dtype=torch.float16)
    gout32 = torch.empty((300, rl), device=dev)
    row_tab = d_tab[0].contiguous()
    plan = PagedAttention.plan(B, nh, nkv, hd, bt, 640)
    ws = PagedAttention.workspace(plan)
    plan_fx = PagedAttention.plan(B, nh, nkv, hd, bt, 640, 64)
    ws_fx = PagedAttention.workspace(plan_fx)
    plan8 = PagedAttention.plan(B, nh, nkv, hd, bt, 640, 0, KvDataType.FP8)
    ws8 = PagedAttention.workspace(plan8)
    mass = torch.zeros(nb, device=dev)
    mws = torch.empty(int(PagedAttention.mass_workspace_bytes(B, 40, bt, nh)) // 4 + plan[2] // 4 + 1,
                      device=dev)
    pq = torch.randn((B * 64, nh, hd), generator=g, device=dev)
    pout = torch.empty_like(pq)
    cu_q = torch.arange(0, B * 64 + 1, 64, dtype=torch.int32, device=dev)
    sp_q = torch.full((B,), 400, dtype=torch.int32, device=dev)
    src = i32(np.arange(0, 8), dev)
    dst = i32(np.arange(nb - 4, nb - 4 + 8) % nb, dev)[:4].contiguous()
    src4 = src[:4].contiguous()
    remap = i32(np.arange(nb), dev)
    counts = torch.zeros(nb, dtype=torch.int32, device=dev)
    used = torch.full((B,), 32, dtype=torch.int32, device=dev)
    q1 = q[0].contiguous()
    o1 = out[0].contiguous()
    pos1 = pos[:1].contiguous()
    sws = torch.empty(1 << 16, device=dev)   # caller-owned single-sequence workspace

    calls = {
        "eh_append_kv": lambda: kv.append_kv(None, lay16, pool16, k16[:1], v16[:1], row_tab, 499, 1),
        "eh_append_kv(pos_ptr)": lambda: kv.append_kv_with_pos_ptr(None, lay16, pool16, k16[:1],
                                                                   v16[:1], row_tab, 0, 1, pos1),
        "eh_gather_kv": lambda: kv.read_keys(None, lay16, pool16, row_tab, gout, 0, 300),
        "eh_append_kv_batched": lambda: kv.append_kv_batched(None, lay16, pool16, k16, v16, d_tab,
                                                             cu, pos, B),
        "eh_append_kv_e4m3_batched": lambda: kv.append_kv_e4m3_batched(
            None, lay8, pool8, k32, v32, d_tab, cu, pos, B, hd, scales, scales),
        "eh_gather_kv_e4m3": lambda: kv.read_e4m3(None, lay8, pool8, row_tab, gout32, 0, 300, 0,
                                                  hd, scales),
        "eh_copy_pages": lambda: kv.copy_pages(None, lay16, pool16, src4, dst),
        "eh_remap_block_tables": lambda: kv.remap_block_tables(None, d_tab, remap),
        "eh_page_refcounts": lambda: kv.page_refcounts(None, d_tab, used, counts),
        "eh_paged_attention": lambda: pa.launch(None, q1, pool32, row_tab, o1, nh, nkv, hd, bt,
                                                500, 499, True),
        "eh_flash_decoding": lambda: pa.launch_flash_decoding(None, q1, pool32, row_tab, o1, nh,
                                                              nkv, hd, bt, 500, 499, True),
        "eh_flash_decoding(pos_ptr)": lambda: pa.launch_flash_decoding(
            None, q1, pool16, row_tab, o1, nh, nkv, hd, bt, 500, 499, True, pos1,
            kv_dtype=KvDataType.F16),
        "eh_append_flash_decoding": lambda: pa.append_flash_decoding(
            None, k16[0].contiguous(), v16[0].contiguous(), q1, pool16, row_tab, o1, nh, nkv, hd,
            bt, 499, kv_dtype=KvDataType.F16),
        "eh_paged_attention_ws": lambda: pa.launch_with_pos_ptr(
            None, q1, pool32, row_tab, o1, nh, nkv, hd, bt, 500, 499, True, None, workspace=sws),
        "eh_flash_decoding_ws": lambda: pa.launch_flash_decoding(
            None, q1, pool16, row_tab, o1, nh, nkv, hd, bt, 500, 499, True, pos1,
            kv_dtype=KvDataType.F16, workspace=sws),
        "eh_append_flash_decoding_ws": lambda: pa.append_flash_decoding(
            None, k16[0].contiguous(), v16[0].contiguous(), q1, pool16, row_tab, o1, nh, nkv, hd,
            bt, 499, kv_dtype=KvDataType.F16, workspace=sws),
        "eh_paged_decode_batched (balanced)": lambda: pa.decode_batched(
            None, q, pool16, d_tab, lens, out, nh, nkv, hd, bt, KvDataType.F16, plan, ws),
        "eh_paged_decode_batched (fixed splits)": lambda: pa.decode_batched(
            None, q, pool16, d_tab, lens, out, nh, nkv, hd, bt, KvDataType.F16, plan_fx, ws_fx),
        "eh_paged_decode_batched_e4m3": lambda: pa.decode_batched_e4m3(
            None, q, pool8, d_tab, lens, out, nh, nkv, hd, bt, scales, scales, plan8, ws8),
        "eh_paged_decode_batched_window (+mass)": lambda: pa.decode_batched_window(
            None, q, pool16, d_tab, lens, out, nh, nkv, hd, bt, KvDataType.F16, 4, 64, plan, mws,
            block_mass=mass),
        "eh_append_decode_batched": lambda: pa.append_decode_batched(
            None, lay16, pool16, k16, v16, d_tab, pos, q, out, nh, hd, plan, ws),
        "eh_append_decode_batched_e4m3": lambda: pa.append_decode_batched_e4m3(
            None, lay8, pool8, k32, v32, d_tab, pos, q, out, nh, hd, plan8, ws8, scales, scales),
        "eh_flash_attention_prefill": lambda: fa.launch(None, pq[:64].contiguous(), pool16,
                                                        row_tab, pout[:64].contiguous(), nh, nkv,
                                                        hd, bt, 64, 400, kv_dtype=KvDataType.F16),
        "eh_prefill_batched": lambda: fa.launch_batched(None, pq, pool16, d_tab, cu_q, sp_q, pout,
                                                        nh, nkv, hd, bt, 64,
                                                        kv_dtype=KvDataType.F16),
        "eh_prefill_batched_e4m3": lambda: fa.launch_batched_e4m3(None, pq, pool8, d_tab, cu_q,
                                                                  sp_q, pout, nh, nkv, hd, bt, 64,
                                                                  scales, scales),
    }
    for name, fn in calls.items():
        fn()                                   # warm-up: resolves the kernel handles
    torch.cuda.synchronize()
    for name, fn in calls.items():
        print(f"[alloc] {name}", flush=True)
        torch.cuda.synchronize()
        n_alloc = torch.cuda.memory_stats()["allocation.all.allocated"]
        free0, _ = torch.cuda.mem_get_info()
        for _ in range(100):
            fn()
        torch.cuda.synchronize()
        free1, _ = torch.cuda.mem_get_info()
        assert torch.cuda.memory_stats()["allocation.all.allocated"] == n_alloc, name
        assert free1 >= free0, f"{name}: free device memory dropped by {free0 - free1} bytes"
