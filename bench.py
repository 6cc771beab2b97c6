"""Benchmark of the paged KV-cache hot path on one MI355X.

Workload (benchmark config 2): batch 32 GQA decode step, 12 query / 2 KV
heads, head_dim 128, page 16 tokens, f16 KV with f32 accumulation, context
lengths U[128, 4096] from the seed, pool of 1.2x the cached tokens per layer
on a shuffled free list, 28 layers with 28 distinct pools (2.3 GB, far above
the 256 MB Infinity Cache).  One step = for each layer: append one token per
sequence (batched append kernel), then batched paged decode over every
cached token.  Inputs are resident in HBM before timing; contexts grow by one
token per step on the device.

Prints ONE JSON line: value = KV bytes read by decode per second over the
whole step (GB/s); tok/s = 32 tokens per step.  `roofline` times the decode
kernel alone with HIP events (per launch, on the launch stream);
`cpu_baseline` times the oracle (C restatement of the reference's
single-threaded PagedKvCache::append + sdpa_decode) on a bounded sample.
"""
import argparse
import json
import os
import platform
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "paged-decode KV read GB/s (% HBM peak) + decode tok/s, B=32 ctx 4k, 1 GPU"
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, AMD published


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--layers", type=int, default=28)
    p.add_argument("--tps", type=int, default=0, help="tokens per split (0 = planner)")
    p.add_argument("--graph", type=int, default=1, help="replay the step as a HIP graph")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline budget")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--roofline-iters", type=int, default=10)
    p.add_argument("--fuse", type=int, default=1,
                   help="one fused append+decode launch per layer when the balanced kernel applies")
    return p.parse_args()


def cpu_model():
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        for ln in out.splitlines():
            if ln.startswith("Model name"):
                return ln.split(":", 1)[1].strip()
    except Exception:
        pass
    return platform.processor() or "unknown"


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus above 1 is not supported "
                          "(see DESIGN.md for how the path shards)", "n_gpus": args.gpus}))
        sys.exit(2)

    import numpy as np
    import torch

    from titan_amd import KvDataType, PagedAttention, PagedKvGpu, PagedKvLayout, synth

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    L = args.layers
    extra = args.warmup + args.steps + 2 + args.roofline_iters
    shape = synth.config2(0, extra_tokens=extra)
    B, NQ, NKV, HD, BT = shape.batch, shape.n_head, shape.n_head_kv, shape.head_dim, shape.block_tokens
    rl = shape.row_len
    tab = synth.block_tables(shape, extra_tokens=extra)
    layout = PagedKvLayout(shape.n_blocks, BT, rl, KvDataType.F16)
    print(f"[bench] config2: B={B} heads {NQ}/{NKV} hd {HD} page {BT} f16, ctx sum "
          f"{int(shape.ctx_lens.sum())}, pool {shape.n_blocks} pages x {L} layers "
          f"({layout.bytes_total() * L / 1e9:.2f} GB)", file=sys.stderr, flush=True)

    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    pools = [torch.randn(layout.floats_total(), generator=gen, device=dev, dtype=torch.float16)
             for _ in range(L)]
    qs = [torch.randn((B, NQ, HD), generator=gen, device=dev) for _ in range(L)]
    newk = [torch.randn((B, rl), generator=gen, device=dev, dtype=torch.float16) for _ in range(L)]
    newv = [torch.randn((B, rl), generator=gen, device=dev, dtype=torch.float16) for _ in range(L)]
    outs = [torch.empty((B, NQ, HD), device=dev) for _ in range(L)]
    d_tab = torch.from_numpy(tab.view(np.int32)).to(dev)
    cu = torch.arange(B + 1, dtype=torch.int32, device=dev)
    start = torch.from_numpy(shape.ctx_lens.astype(np.int32)).to(dev)   # next write position
    lens = start + 1                                                     # tokens attended
    max_ctx = int(shape.ctx_lens.max()) + extra
    plan = PagedAttention.plan(B, NQ, NKV, HD, BT, max_ctx, args.tps)
    ws = PagedAttention.workspace(plan)
    kname = PagedAttention.kernel_name(NQ, NKV, HD, BT, KvDataType.F16)
    balanced = plan[0] == 0
    fused = balanced and bool(args.fuse)
    kv, pa = PagedKvGpu(0), PagedAttention(0)

    def layer(i, s=None):
        if fused:  # append + decode in one launch of the balanced kernel
            pa.append_decode_batched(s, layout, pools[i], newk[i], newv[i], d_tab, start, qs[i],
                                     outs[i], NQ, HD, plan, ws)
        else:
            kv.append_kv_batched(s, layout, pools[i], newk[i], newv[i], d_tab, cu, start, B)
            pa.decode_batched(s, qs[i], pools[i], d_tab, lens, outs[i], NQ, NKV, HD, BT,
                              KvDataType.F16, plan, ws)

    def step(s=None):
        for i in range(L):
            layer(i, s)
        start.add_(1)
        lens.add_(1)

    # warm-up (eager) resolves every kernel handle
    for _ in range(max(args.warmup, 1)):
        step()
    torch.cuda.synchronize()

    runner = step
    if args.graph:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                step(s)
        torch.cuda.synchronize()
        # capture does not execute: contexts are unchanged here
        runner = g.replay

    ctx_before = int(start.sum().item())
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        runner()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = e0.elapsed_time(e1)
    elapsed = max(gpu_ms / 1e3, 1e-9)
    # KV bytes the decode reads: every attended row once per kv head (K and V).
    kv_bytes = 0
    for k in range(args.steps):
        attended = ctx_before + B * (k + 1)
        kv_bytes += L * attended * NKV * HD * 2 * 2
    value = kv_bytes / elapsed / 1e9
    ms_step = gpu_ms / args.steps
    tok_s = B * args.steps / elapsed
    print(f"[bench] {args.steps} steps: {ms_step:.3f} ms/step (wall {wall * 1e3 / args.steps:.3f}),"
          f" {value:.1f} GB/s, {tok_s:.0f} tok/s", file=sys.stderr, flush=True)

    # Roofline of the decode launch (split kernel + merge; with --fuse the
    # same launch also appends the step's rows): the 28 layers' calls are
    # captured in a graph on their own stream and replayed between two events
    # on that stream, so host enqueue time never enters the measured interval.
    # Replays rewrite the same rows at the same positions.
    dstream = torch.cuda.Stream()
    dstream.wait_stream(torch.cuda.current_stream())
    dgraph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(dstream):
        with torch.cuda.graph(dgraph, stream=dstream):
            for i in range(L):
                if fused:
                    pa.append_decode_batched(dstream, layout, pools[i], newk[i], newv[i], d_tab,
                                             start, qs[i], outs[i], NQ, HD, plan, ws)
                else:
                    pa.decode_batched(dstream, qs[i], pools[i], d_tab, lens, outs[i], NQ, NKV, HD,
                                      BT, KvDataType.F16, plan, ws)
    torch.cuda.synchronize()
    ra, rb = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(dstream):  # replay() launches on the current stream
        dgraph.replay()  # warm
        ra.record(dstream)
        for _ in range(args.roofline_iters):
            dgraph.replay()
        rb.record(dstream)
    torch.cuda.synchronize()
    avg_ms = ra.elapsed_time(rb) / (args.roofline_iters * L)
    attended = int(lens.sum().item())
    # KV rows read once per kv head; a fused launch also reads and writes the
    # appended rows (B x 2 rows)
    per_launch_bytes = attended * NKV * HD * 2 * 2 + (2 * B * 2 * rl * 2 if fused else 0)
    achieved = per_launch_bytes / (avg_ms / 1e3) / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "decode_config2_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tr = json.load(f)
        if tr.get("kernel") == kname:
            traffic = tr.get("hbm_bytes_per_launch")
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": kname + (" + eh_decode_tiles_merge" if balanced else " + eh_decode_merge")
                + (" (fused append)" if fused else ""),
                "avg_launch_us": round(avg_ms * 1e3, 2),
                "algorithmic_bytes_per_launch": per_launch_bytes}

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args, shape, tab, pools[0], qs[0], newk[0], newv[0])

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic (seeded N(0,1) K/V/Q, seeded U[128,4096] contexts, shuffled free list)",
        "config": {"workload": "config2: batch-32 GQA paged decode step, 12/2 heads, hd 128, "
                               "page 16, f16 KV, ctx U[128,4096], 28 layers (append + decode)",
                   "batch": B, "layers": L, "n_head": NQ, "n_head_kv": NKV, "head_dim": HD,
                   "block_tokens": BT, "ctx_sum": ctx_before, "tokens_per_split": plan[0],
                   "grid": plan[1], "fused_append": fused, "graph": bool(args.graph)},
        "tok_s": round(tok_s, 1), "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": roofline, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def cpu_baseline(args, shape, tab, pool0, q0, k0, v0):
    """Oracle append + sdpa_decode (single thread) on whole layer-steps of the
    same workload, repeated until the time budget is spent."""
    import numpy as np

    from oracle import orc

    B, NQ, NKV, HD, BT = shape.batch, shape.n_head, shape.n_head_kv, shape.head_dim, shape.block_tokens
    rl = shape.row_len
    pool = pool0.float().cpu().numpy().copy()           # exact widening, untimed
    q = q0.cpu().numpy()
    kn, vn = k0.float().cpu().numpy(), v0.float().cpu().numpy()
    lens = shape.ctx_lens.astype(np.int64)
    page = BT * 2 * rl
    n_layers, secs, kv_bytes = 0, 0.0, 0
    while secs < args.cpu_seconds and n_layers < 64:
        t0 = time.perf_counter()
        for b in range(B):                               # PagedKvCache::append row copies
            L_b = int(lens[b])
            base = int(tab[b, L_b // BT]) * page + (L_b % BT) * 2 * rl
            pool[base:base + rl] = kn[b]
            pool[base + rl:base + 2 * rl] = vn[b]
        orc.sdpa_decode_batched(pool, tab, (lens + 1).astype(np.uint32), BT, q, NQ, NKV, HD)
        secs += time.perf_counter() - t0
        kv_bytes += int((lens + 1).sum()) * NKV * HD * 2 * 2
        n_layers += 1
    return {"value": round(kv_bytes / secs / 1e9, 4), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": f"{n_layers} layer-steps of config 2 (32 sequences, append + decode over "
                      f"the f32-widened pool), {secs:.1f} s on 1 thread of {cpu_model()} "
                      f"({os.cpu_count()} logical CPUs visible)",
            "tok_s": round(B * n_layers / 28 / secs, 3)}


if __name__ == "__main__":
    main()
