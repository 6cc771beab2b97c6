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
import shutil
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
    p.add_argument("--cpu-child", action="store_true", help=argparse.SUPPRESS)
    p.add_argument("--roofline-iters", type=int, default=20)
    p.add_argument("--fuse", type=int, default=1,
                   help="one fused append+decode launch per layer when the balanced kernel applies")
    p.add_argument("--sched", type=int, default=1,
                   help="build the step's work split once per step (eh_decode_schedule) and run "
                        "every layer from it")
    p.add_argument("--suite", action="store_true",
                   help="instead of the headline line, time the other benchmark configurations "
                        "(1, 3, 4, 5) and append/gather, one JSON line each")
    p.add_argument("--append-tokens", type=int, default=1,
                   help="suite append part: tokens appended per sequence per call (config 2: 1)")
    p.add_argument("--c5-pool-frac", type=float, default=0.9,
                   help="config 5 pool size as a fraction of free HBM")
    p.add_argument("--parts", default="c1,append,e4m3,bf16,ceiling,c2u,c3,c4,c5",
                   help="suite parts to run (comma list of c1, append, e4m3, bf16, ceiling, "
                        "c2u, c3, c4, c5)")
    return p.parse_args()


def cpu_model():
    """lscpu's model name with its family/model/stepping numbers (a VM may
    report a generic name), and /proc/cpuinfo's when lscpu is absent."""
    fields = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        for ln in out.splitlines():
            k, _, v = ln.partition(":")
            fields[k.strip()] = v.strip()
    except Exception:
        pass
    name = fields.get("Model name")
    if not name:
        try:
            with open("/proc/cpuinfo") as f:
                for ln in f:
                    if ln.startswith("model name"):
                        name = ln.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
    name = name or platform.processor() or "unknown"
    ids = [f"{k.lower()} {fields[k]}" for k in ("CPU family", "Model", "Stepping") if fields.get(k)]
    return name + (f" ({', '.join(ids)})" if ids else "")


def start_cpu_baseline(args):
    """Starts the CPU baseline in a child process pinned to one core
    (`taskset -c <cpu>`, the first core this process may use) BEFORE anything
    touches the GPU; the child sees no GPU at all.  Returns the Popen."""
    cpu = min(os.sched_getaffinity(0))
    cmd = [sys.executable, os.path.abspath(__file__), "--cpu-child",
           "--cpu-seconds", str(args.cpu_seconds)]
    taskset = shutil.which("taskset")
    cmd = ([taskset, "-c", str(cpu)] + cmd) if taskset else cmd
    env = dict(os.environ, HIP_VISIBLE_DEVICES="", CUDA_VISIBLE_DEVICES="",
               ROCR_VISIBLE_DEVICES="", TITAN_CPU_PIN=str(cpu),
               TITAN_CPU_AVAIL=str(len(os.sched_getaffinity(0))),
               TITAN_CPU_PINNER="taskset" if taskset else "sched_setaffinity")
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                            env=env)


def finish_cpu_baseline(proc):
    try:
        out, err = proc.communicate(timeout=600)
    except subprocess.TimeoutExpired:
        proc.kill()
        return {"error": "cpu baseline timed out"}
    lines = [ln for ln in out.splitlines() if ln.startswith("{")]
    if proc.returncode != 0 or not lines:
        return {"error": f"cpu baseline exited {proc.returncode}: {err[-400:]}"}
    return json.loads(lines[-1])


def main():
    args = parse()
    if args.cpu_child:
        cpu_child(args)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU; --gpus above 1 is not supported "
                          "(the path shards by sequence or by kv head with no exchange inside it; one "
                          "GPU's share is what is measured)", "n_gpus": args.gpus}))
        sys.exit(2)

    # the CPU baseline's child starts before this process touches the GPU
    cpu_proc = None if (args.no_cpu or args.suite) else start_cpu_baseline(args)

    import numpy as np
    import torch

    from titan_amd import KvDataType, PagedAttention, PagedKvGpu, PagedKvLayout, synth

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.suite:
        suite(args, dev)
        return
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
    scheduled = fused and bool(args.sched)
    stride = int(tab.shape[1])
    sched = PagedAttention.schedule_buffer(B, stride, BT, plan) if scheduled else None
    kv, pa = PagedKvGpu(0), PagedAttention(0)

    def layer(i, s=None):
        if scheduled:  # append + decode in one launch, split read from the step schedule
            pa.append_decode_scheduled(s, layout, pools[i], newk[i], newv[i], sched, stride, qs[i],
                                       outs[i], NQ, HD, plan, ws)
        elif fused:  # append + decode in one launch of the balanced kernel
            pa.append_decode_batched(s, layout, pools[i], newk[i], newv[i], d_tab, start, qs[i],
                                     outs[i], NQ, HD, plan, ws)
        else:
            kv.append_kv_batched(s, layout, pools[i], newk[i], newv[i], d_tab, cu, start, B)
            pa.decode_batched(s, qs[i], pools[i], d_tab, lens, outs[i], NQ, NKV, HD, BT,
                              KvDataType.F16, plan, ws)

    def step(s=None):
        if scheduled:  # the step's work split, shared by its 28 layers
            pa.build_schedule(s, layout, d_tab, start, 1, plan, sched)
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
    # one event between consecutive steps: the first-to-last interval is the
    # timed region, the consecutive pairs give per-step times for the median
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    t0 = time.perf_counter()
    ev[0].record()
    for k in range(args.steps):
        runner()
        ev[k + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev[0].elapsed_time(ev[-1])
    step_ms = [ev[k].elapsed_time(ev[k + 1]) for k in range(args.steps)]
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
            if scheduled:
                pa.build_schedule(dstream, layout, d_tab, start, 1, plan, sched)
            for i in range(L):
                if scheduled:
                    pa.append_decode_scheduled(dstream, layout, pools[i], newk[i], newv[i], sched,
                                               stride, qs[i], outs[i], NQ, HD, plan, ws)
                elif fused:
                    pa.append_decode_batched(dstream, layout, pools[i], newk[i], newv[i], d_tab,
                                             start, qs[i], outs[i], NQ, HD, plan, ws)
                else:
                    pa.decode_batched(dstream, qs[i], pools[i], d_tab, lens, outs[i], NQ, NKV, HD,
                                      BT, KvDataType.F16, plan, ws)
    torch.cuda.synchronize()
    rev = [torch.cuda.Event(enable_timing=True) for _ in range(args.roofline_iters + 1)]
    with torch.cuda.stream(dstream):  # replay() launches on the current stream
        dgraph.replay()  # warm
        rev[0].record(dstream)
        for k in range(args.roofline_iters):
            dgraph.replay()
            rev[k + 1].record(dstream)
    torch.cuda.synchronize()
    avg_ms = rev[0].elapsed_time(rev[-1]) / (args.roofline_iters * L)
    med_ms = float(np.median([rev[k].elapsed_time(rev[k + 1])
                              for k in range(args.roofline_iters)])) / L
    attended = int(lens.sum().item())
    # KV rows read once per kv head; a fused launch also reads and writes the
    # appended rows (B x 2 rows)
    per_launch_bytes = attended * NKV * HD * 2 * 2 + (2 * B * 2 * rl * 2 if fused else 0)
    achieved = per_launch_bytes / (avg_ms / 1e3) / 1e9
    # HBM traffic per call from the committed counter profile, used only when
    # it was captured from these exact kernel and launcher sources
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "decode_config2_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tr = json.load(f)
        if tr.get("kernel") == kname and tr.get("source_sha256") == decode_source_digest():
            traffic = tr.get("hbm_bytes_per_launch")
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": (kname + "_sched + eh_decode_tiles_merge_sched (fused append; "
                           "+ 1/28 of eh_decode_tiles_schedule per step)") if scheduled else
                (kname + (" + eh_decode_tiles_merge" if balanced else " + eh_decode_merge")
                 + (" (fused append)" if fused else "")),
                "avg_launch_us": round(avg_ms * 1e3, 2),
                "median_launch_us": round(med_ms * 1e3, 2),
                "timing": f"HIP events on the graph's stream around each of {args.roofline_iters} "
                          f"replays of {L} calls (+ one schedule build); avg = total / calls, "
                          "median over the replays",
                "algorithmic_bytes_per_launch": per_launch_bytes}

    cpu = finish_cpu_baseline(cpu_proc) if cpu_proc is not None else None

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "ms_per_step_median": round(float(np.median(step_ms)), 4),
        "ms_per_step_min_max": [round(min(step_ms), 4), round(max(step_ms), 4)],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic (seeded N(0,1) K/V/Q, seeded U[128,4096] contexts, shuffled free list)",
        "config": {"workload": "config2: batch-32 GQA paged decode step, 12/2 heads, hd 128, "
                               "page 16, f16 KV, ctx U[128,4096], 28 layers (append + decode)",
                   "batch": B, "layers": L, "n_head": NQ, "n_head_kv": NKV, "head_dim": HD,
                   "block_tokens": BT, "ctx_sum": ctx_before, "tokens_per_split": plan[0],
                   "grid": plan[1], "fused_append": fused, "step_schedule": scheduled,
                   "graph": bool(args.graph)},
        "tok_s": round(tok_s, 1), "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": roofline, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)



def graph_time_us(fn, iters=20, per_graph=20, stream=None, warm_s=0.05):
    """Capture per_graph back-to-back calls fn(stream) in one graph, replay it
    for warm_s seconds (the compute clock settles under sustained load: short
    runs of the MFMA-bound prefill measured up to 18 % slower), then iters
    times between two events on the capture stream; mean microseconds per
    call (graph launch cost amortised over per_graph calls)."""
    import torch
    s = stream or torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    fn(None)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for _ in range(per_graph):
                fn(s)
    torch.cuda.synchronize()
    t_end = time.perf_counter() + warm_s
    while True:
        with torch.cuda.stream(s):
            g.replay()
        torch.cuda.synchronize()
        if time.perf_counter() >= t_end:
            break
    with torch.cuda.stream(s):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(s)
        for _ in range(iters):
            g.replay()
        b.record(s)
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / (iters * per_graph)


DECODE_SOURCES = ("titan_amd/csrc/kernels/paged_decode_tiles.hip", "titan_amd/csrc/engine_hip.cpp")


def decode_source_digest():
    """sha256 over the decode kernel and launcher sources (the GPU box has no
    .git, so a content hash ties a counter profile to the code it measured)."""
    import hashlib
    h = hashlib.sha256()
    for rel in DECODE_SOURCES:
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def emit(d):
    print(json.dumps(d), flush=True)


def suite(args, dev):
    """The benchmark configurations other than the headline (config 2), each
    on synthetic seeded inputs resident in HBM; timings are HIP events around
    graph replays (launch cost inside the graph, host enqueue outside).
    --parts selects: c1 (config 1), append (config 2 append / gather), e4m3
    (config 2 decode over E4M3 pages), bf16 (config 2 decode over bf16 pages
    beside f16), ceiling (config 2's read ceilings), c2u (config 2's shape at a
    uniform 4 k context), c3 (config 3 prefill), c4 (config 4 compaction), c5 (config 5
    long-context decode on a ~90 % HBM pool)."""
    import numpy as np
    import torch

    from titan_amd import (FlashAttention2, KvDataType, PagedAttention, PagedKvGpu,
                           PagedKvLayout, synth)

    kv, pa, fa = PagedKvGpu(0), PagedAttention(0), FlashAttention2(0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    parts = set(args.parts.split(","))

    def pools_graph_us(call, pools, reps=20):
        """µs per call: one call per pool (the headline step's rotation) in one
        graph, median of `reps` replays after 50 ms of warm replays."""
        st = torch.cuda.Stream()
        st.wait_stream(torch.cuda.current_stream())
        call(None, pools[0])
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(st):
            with torch.cuda.graph(g, stream=st):
                for p in pools:
                    call(st, p)
        torch.cuda.synchronize()
        t_end = time.perf_counter() + 0.05
        while time.perf_counter() < t_end:
            with torch.cuda.stream(st):
                g.replay()
            torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        with torch.cuda.stream(st):
            ev[0].record(st)
            for k in range(reps):
                g.replay()
                ev[k + 1].record(st)
        torch.cuda.synchronize()
        return (float(np.median([ev[k].elapsed_time(ev[k + 1]) for k in range(reps)])) * 1e3 /
                len(pools))

    if "c1" in parts:  # f32, B=1, 14/2 heads, hd 64, page 16, 511 cached + 1 appended
        s1 = synth.config1(0)
        rl = s1.row_len
        lay1 = PagedKvLayout(64, 16, rl, KvDataType.F32)
        pool1 = torch.randn(lay1.floats_total(), generator=gen, device=dev)
        tab1 = torch.from_numpy(s1.free_order[:32].astype(np.uint32).view(np.int32)).to(dev)
        k1 = torch.randn(rl, generator=gen, device=dev)
        v1 = torch.randn(rl, generator=gen, device=dev)
        q1 = torch.randn(s1.n_head * s1.head_dim, generator=gen, device=dev)
        o1 = torch.empty_like(q1)

        def step1(st):
            kv.append_kv(st, lay1, pool1, k1, v1, tab1, 511, 1)
            pa.launch_flash_decoding(st, q1, pool1, tab1, o1, s1.n_head, s1.n_head_kv,
                                     s1.head_dim, 16, 512, 511, True)
        us1 = graph_time_us(step1, 20)
        emit({"config": 1, "what": "append 1 token + flash-decoding attention, f32, B=1, 14/2 "
              "heads, hd 64, ctx 512", "latency_us": round(us1, 2),
              "kv_bytes": 512 * rl * 2 * 4, "GB/s": round(512 * rl * 2 * 4 / us1 / 1e3, 1)})

        def step1f(st):
            pa.append_flash_decoding(st, k1, v1, q1, pool1, tab1, o1, s1.n_head, s1.n_head_kv,
                                     s1.head_dim, 16, 511)
        us1f = graph_time_us(step1f, 20)
        emit({"config": 1, "what": "the same step in one launch (eh_append_flash_decoding)",
              "latency_us": round(us1f, 2), "kv_bytes": 512 * rl * 2 * 4,
              "GB/s": round(512 * rl * 2 * 4 / us1f / 1e3, 1)})

    s2 = synth.config2(0, extra_tokens=1)
    tab2 = synth.block_tables(s2, extra_tokens=1)
    dtab2 = torch.from_numpy(tab2.view(np.int32)).to(dev)
    if "append" in parts:  # append / gather at config 2's shape (one layer)
        A = max(args.append_tokens, 1)
        sa = synth.config2(0, extra_tokens=A) if A > 1 else s2
        taba = synth.block_tables(sa, extra_tokens=A) if A > 1 else tab2
        dtaba = torch.from_numpy(taba.view(np.int32)).to(dev)
        lay2 = PagedKvLayout(sa.n_blocks, 16, sa.row_len, KvDataType.F16)
        pool2 = torch.randn(lay2.floats_total(), generator=gen, device=dev, dtype=torch.float16)
        nk2 = torch.randn((32 * A, sa.row_len), generator=gen, device=dev, dtype=torch.float16)
        nv2 = torch.randn((32 * A, sa.row_len), generator=gen, device=dev, dtype=torch.float16)
        cu2 = torch.arange(0, 32 * A + 1, A, dtype=torch.int32, device=dev)
        st2 = torch.from_numpy(sa.ctx_lens.astype(np.int32)).to(dev)
        us_app = graph_time_us(lambda st: kv.append_kv_batched(st, lay2, pool2, nk2, nv2, dtaba,
                                                               cu2, st2, 32 * A), 20)
        app_bytes = 32 * A * 2 * sa.row_len * 2 * 2
        emit({"config": 2, "what": f"batched append of {A} token(s) per sequence "
              f"({32 * A} x 1 KiB rows), f16", "latency_us": round(us_app, 2),
              "GB/s": round(app_bytes / us_app / 1e3, 2)})
        del pool2
        lay2 = PagedKvLayout(s2.n_blocks, 16, s2.row_len, KvDataType.F16)
        pool2 = torch.randn(lay2.floats_total(), generator=gen, device=dev, dtype=torch.float16)
        L0 = int(s2.ctx_lens[0])
        gout = torch.empty((L0, s2.row_len), dtype=torch.float16, device=dev)
        tab_row = dtab2[0].contiguous()
        us_g = graph_time_us(lambda st: kv.read_keys(st, lay2, pool2, tab_row, gout, 0, L0), 20)
        g_bytes = L0 * s2.row_len * 2 * 2
        emit({"config": 2, "what": f"gather of one sequence's K rows ({L0} tokens x 512 B), f16",
              "latency_us": round(us_g, 2), "GB/s": round(g_bytes / us_g / 1e3, 1)})
        del pool2

    if "e4m3" in parts:  # config 2's decode over E4M3 pages, 16 rotated pools (> the 256 MB MALL)
        lay8 = PagedKvLayout(s2.n_blocks, 16, s2.row_len, KvDataType.FP8)
        pools8 = [torch.randint(0, 0x7E, (lay8.floats_total(),), generator=gen, device=dev,
                                dtype=torch.uint8) for _ in range(16)]
        q8 = torch.randn((32, 12, 128), generator=gen, device=dev)
        o8 = torch.empty_like(q8)
        ks8 = torch.full((2,), 0.01, device=dev)
        vs8 = torch.full((2,), 0.02, device=dev)
        lens8 = torch.from_numpy((s2.ctx_lens + 1).astype(np.int32)).to(dev)
        plan8 = PagedAttention.plan(32, 12, 2, 128, 16, int(s2.ctx_lens.max()) + 1, 0,
                                    KvDataType.FP8)
        ws8 = PagedAttention.workspace(plan8)
        stride2 = int(tab2.shape[1])
        sched8 = PagedAttention.schedule_buffer(32, stride2, 16, plan8)
        pa.build_schedule(None, lay8, dtab2, lens8, 0, plan8, sched8)
        turn = [0]
        b8 = int((s2.ctx_lens + 1).sum()) * 2 * 128 * 2 * 1

        def dec8(st):
            p = pools8[turn[0] % len(pools8)]
            turn[0] += 1
            pa.decode_batched_e4m3(st, q8, p, dtab2, lens8, o8, 12, 2, 128, 16, ks8, vs8, plan8,
                                   ws8)
        us8 = graph_time_us(dec8, 20, 32)
        emit({"config": 2, "what": "decode over E4M3 pages (fp8 KV, per-kv-head scales), B=32, "
              "12/2 heads, hd 128, one layer (self-scheduled)", "latency_us": round(us8, 2),
              "kv_bytes": b8, "GB/s": round(b8 / us8 / 1e3, 1),
              "hbm_frac_of_8TB/s": round(b8 / us8 / 1e3 / 8000.0, 4)})

        def dec8s(st):
            p = pools8[turn[0] % len(pools8)]
            turn[0] += 1
            pa.append_decode_scheduled(st, lay8, p, None, None, sched8, stride2, q8, o8, 12, 128,
                                       plan8, ws8, ks8, vs8)
        us8s = graph_time_us(dec8s, 20, 32)
        emit({"config": 2, "what": "the same E4M3 decode from a step schedule (built once)",
              "latency_us": round(us8s, 2), "kv_bytes": b8, "GB/s": round(b8 / us8s / 1e3, 1),
              "hbm_frac_of_8TB/s": round(b8 / us8s / 1e3 / 8000.0, 4),
              "kernel": PagedAttention.kernel_name(12, 2, 128, 16, KvDataType.FP8) +
              "_sched + eh_decode_tiles_merge_sched"})
        # the fused step: the appended f32 rows quantised inside the decode launch
        pos8 = torch.from_numpy(s2.ctx_lens.astype(np.int32)).to(dev)
        nk8 = torch.randn((32, s2.row_len), generator=gen, device=dev)
        nv8 = torch.randn((32, s2.row_len), generator=gen, device=dev)
        sched8f = PagedAttention.schedule_buffer(32, stride2, 16, plan8)
        pa.build_schedule(None, lay8, dtab2, pos8, 1, plan8, sched8f)

        def step8(st):
            p = pools8[turn[0] % len(pools8)]
            turn[0] += 1
            pa.append_decode_scheduled(st, lay8, p, nk8, nv8, sched8f, stride2, q8, o8, 12, 128,
                                       plan8, ws8, ks8, vs8)
        us8f = graph_time_us(step8, 20, 32)
        emit({"config": 2, "what": "fused E4M3 decode step from a step schedule (quantising "
              "append of the 32 new f32 rows + decode in one launch), B=32, 12/2 heads, hd 128, "
              "one layer", "latency_us": round(us8f, 2), "kv_bytes": b8,
              "GB/s": round(b8 / us8f / 1e3, 1)})
        del pools8

    if "ceiling" in parts:
        # The read floor of the headline call: config 2's decode (schedule +
        # fused append + decode, 28 rotated pools as the headline step) and a
        # pure read of the same pages through the same tables (whole 16 KiB
        # pages, sequence-major as the decode walks them) over the same 28
        # pools, each as a graph of 28 calls replayed between events.
        L = 28
        lay2 = PagedKvLayout(s2.n_blocks, 16, s2.row_len, KvDataType.F16)
        pools = [torch.randn(lay2.floats_total(), generator=gen, device=dev, dtype=torch.float16)
                 for _ in range(L)]
        pos2 = torch.from_numpy(s2.ctx_lens.astype(np.int32)).to(dev)
        n_tok = s2.ctx_lens.astype(np.int64) + 1
        ids = np.concatenate([tab2[b, :(int(n_tok[b]) + 15) // 16] for b in range(32)])
        dids = torch.from_numpy(ids.astype(np.uint32).view(np.int32)).to(dev)
        page_b = lay2.page_bytes()
        plan2 = PagedAttention.plan(32, 12, 2, 128, 16, int(n_tok.max()))
        ws2 = PagedAttention.workspace(plan2)
        stride2 = int(tab2.shape[1])
        sched2 = PagedAttention.schedule_buffer(32, stride2, 16, plan2)
        q2 = torch.randn((32, 12, 128), generator=gen, device=dev)
        o2 = torch.empty_like(q2)
        nk2 = torch.randn((32, s2.row_len), generator=gen, device=dev, dtype=torch.float16)
        nv2 = torch.randn((32, s2.row_len), generator=gen, device=dev, dtype=torch.float16)
        xo = torch.empty(1024 * 8, dtype=torch.int32, device=dev)
        dec_bytes = int(n_tok.sum()) * 2 * 128 * 2 * 2 + 2 * 32 * 2 * s2.row_len * 2

        def graph_us(call):
            return pools_graph_us(call, pools)

        pa.build_schedule(None, lay2, dtab2, pos2, 1, plan2, sched2)
        us_dec = graph_us(lambda st, p: pa.append_decode_scheduled(
            st, lay2, p, nk2, nv2, sched2, stride2, q2, o2, 12, 128, plan2, ws2))
        best = None
        sweep = {}
        for depth in (1, 2):
            for grid in (256, 512, 1024):
                us = graph_us(lambda st, p: kv.stream_pages(st, lay2, p, dids, xo, depth, grid))
                sweep[f"d{depth}_g{grid}"] = round(us, 2)
                if best is None or us < best[0]:
                    best = (us, depth, grid)
        # the same pages in the decode's own pattern: one wave per kv head, the two waves
        # of a group reading only their head's K and V rows of the same pages
        heads = {}
        for grid in (256, 512, 1024):
            heads[f"g{grid}"] = round(graph_us(
                lambda st, p: kv.stream_pages_heads(st, lay2, p, dids, xo, 128, grid)), 2)
        hk = min(heads, key=heads.get)
        st_bytes = len(ids) * page_b
        emit({"config": 2, "what": "read ceiling: the decode's pages (whole 16 KiB pages through "
              "the same tables, sequence-major) streamed once per call by eh_stream_pages, 28 "
              "rotated pools as the headline step, and in the decode's per-kv-head pattern by "
              "eh_stream_pages_heads; the decode call (schedule + fused append + decode) timed "
              "the same way in the same process",
              "pages": int(len(ids)), "stream_bytes": st_bytes, "decode_bytes": dec_bytes,
              "ceiling_us": round(best[0], 2), "ceiling_depth": best[1], "ceiling_grid": best[2],
              "ceiling_GB/s": round(st_bytes / best[0] / 1e3, 1),
              "ceiling_frac_of_8TB/s": round(st_bytes / best[0] / 1e3 / 8000.0, 4),
              "sweep_us": sweep, "decode_us": round(us_dec, 2),
              "decode_GB/s": round(dec_bytes / us_dec / 1e3, 1),
              "decode_frac_of_8TB/s": round(dec_bytes / us_dec / 1e3 / 8000.0, 4),
              "decode_frac_of_ceiling": round((dec_bytes / us_dec) / (st_bytes / best[0]), 4),
              "heads_ceiling_us": heads[hk], "heads_ceiling_grid": int(hk[1:]),
              "heads_sweep_us": heads,
              "decode_frac_of_heads_ceiling": round((dec_bytes / us_dec) /
                                                    (st_bytes / heads[hk]), 4)})
        del pools

    if "c2u" in parts:
        # Config 2's shape with every sequence at a full 4 k context (the
        # north star's "batch-32 ... at 4k context"): 4095 cached tokens + the
        # appended one, 256 pages each drawn in shuffled order from a pool of
        # 1.2x the pages, 28 rotated pools as the headline step.  The fused
        # step from a step schedule, then the read ceilings of the same pages
        # timed the same way, then a check of the last call against a float64
        # numpy attention over a host copy of its pages.
        L = 28
        n_pg = 32 * 256
        nbu = n_pg * 6 // 5
        tabu = np.random.default_rng(4096).permutation(nbu)[:n_pg].astype(np.uint32)
        tabu = tabu.reshape(32, 256)
        layu = PagedKvLayout(nbu, 16, 256, KvDataType.F16)
        poolsu = [torch.randn(layu.floats_total(), generator=gen, device=dev, dtype=torch.float16)
                  for _ in range(L)]
        dtabu = torch.from_numpy(tabu.view(np.int32)).to(dev)
        posu = torch.full((32,), 4095, dtype=torch.int32, device=dev)
        planu = PagedAttention.plan(32, 12, 2, 128, 16, 4096)
        wsu = PagedAttention.workspace(planu)
        schedu = PagedAttention.schedule_buffer(32, 256, 16, planu)
        qu = torch.randn((32, 12, 128), generator=gen, device=dev)
        ou = torch.full((32, 12, 128), float("nan"), device=dev)
        nku = torch.randn((32, 256), generator=gen, device=dev, dtype=torch.float16)
        nvu = torch.randn((32, 256), generator=gen, device=dev, dtype=torch.float16)
        pa.build_schedule(None, layu, dtabu, posu, 1, planu, schedu)
        us_u = pools_graph_us(lambda st, p: pa.append_decode_scheduled(
            st, layu, p, nku, nvu, schedu, 256, qu, ou, 12, 128, planu, wsu), poolsu)
        torch.cuda.synchronize()
        host = poolsu[-1].view(nbu, 16, 2, 2, 128)[dtabu.long()].cpu().numpy()
        host = host.reshape(32, 4096, 2, 2, 128)
        app_ok = bool(np.array_equal(host[:, 4095, 0].reshape(32, 256).view(np.uint16),
                                     nku.cpu().numpy().view(np.uint16)) and
                      np.array_equal(host[:, 4095, 1].reshape(32, 256).view(np.uint16),
                                     nvu.cpu().numpy().view(np.uint16)))
        ref = np_decode_f64(host, qu.cpu().numpy())
        del host
        d = np.abs(ou.cpu().numpy().astype(np.float64) - ref)
        ok = bool(np.isfinite(d).all() and d.max() <= 2e-3 and
                  (d <= 2e-3 + 1e-3 * np.abs(ref)).all())
        ids = torch.from_numpy(tabu.reshape(-1).view(np.int32)).to(dev)
        xo = torch.empty(1024 * 8, dtype=torch.int32, device=dev)
        whole = {f"d{dp}_g{g}": round(pools_graph_us(
            lambda st, p: kv.stream_pages(st, layu, p, ids, xo, dp, g), poolsu), 2)
            for dp in (1, 2) for g in (256, 512, 1024)}
        heads = {g: round(pools_graph_us(
            lambda st, p: kv.stream_pages_heads(st, layu, p, ids, xo, 128, g), poolsu), 2)
            for g in (256, 512, 1024)}
        c_us, h_us = min(whole.values()), min(heads.values())
        st_b = n_pg * layu.page_bytes()
        dec_b = 32 * 4096 * 2 * 128 * 2 * 2 + 2 * 32 * 2 * 256 * 2
        emit({"config": "2u", "what": "config 2's shape at a uniform 4 k context: B=32, 12/2 "
              "heads, hd 128, page 16, f16, 4095 cached + 1 appended per sequence, fused append "
              "+ decode from a step schedule, 28 rotated pools; read ceilings of the same 8192 "
              "pages (whole pages, eh_stream_pages, 1 or 2 pages in flight; per-kv-head pattern, "
              "eh_stream_pages_heads) timed the same way",
              "latency_us": round(us_u, 2), "kv_bytes": dec_b,
              "GB/s": round(dec_b / us_u / 1e3, 1),
              "frac_of_8TB/s": round(dec_b / us_u / 1e3 / 8000.0, 4),
              "step_ms_28_layers": round(28 * us_u / 1e3, 4),
              "ceiling_us": whole, "heads_ceiling_us": heads,
              "frac_of_ceiling": round((dec_b / us_u) / (st_b / c_us), 4),
              "frac_of_heads_ceiling": round((dec_b / us_u) / (st_b / h_us), 4),
              "check_vs_numpy_f64": {"max_abs": float(d.max()), "within_bar": ok,
                                     "appended_rows_bit_exact": app_ok},
              "kernel": PagedAttention.kernel_name(12, 2, 128, 16, KvDataType.F16) +
              "_sched + eh_decode_tiles_merge_sched"})
        del poolsu
        torch.cuda.empty_cache()

    if "bf16" in parts:  # config 2's decode over bf16 pages beside f16, 16 rotated pools each
        lens16 = torch.from_numpy((s2.ctx_lens + 1).astype(np.int32)).to(dev)
        q16 = torch.randn((32, 12, 128), generator=gen, device=dev)
        b16 = int((s2.ctx_lens + 1).sum()) * 2 * 128 * 2 * 2
        st16 = int(tab2.shape[1])
        for dt, tdt in ((KvDataType.F16, torch.float16), (KvDataType.BF16, torch.bfloat16)):
            lay16 = PagedKvLayout(s2.n_blocks, 16, s2.row_len, dt)
            pools16 = [torch.randn(lay16.floats_total(), generator=gen, device=dev, dtype=tdt)
                       for _ in range(16)]
            plan16 = PagedAttention.plan(32, 12, 2, 128, 16, int(s2.ctx_lens.max()) + 1, 0, dt)
            ws16 = PagedAttention.workspace(plan16)
            sched16 = PagedAttention.schedule_buffer(32, st16, 16, plan16)
            pa.build_schedule(None, lay16, dtab2, lens16, 0, plan16, sched16)
            o16 = torch.empty_like(q16)
            turn = [0]

            def dec16(st):
                p = pools16[turn[0] % len(pools16)]
                turn[0] += 1
                pa.append_decode_scheduled(st, lay16, p, None, None, sched16, st16, q16, o16, 12,
                                           128, plan16, ws16)
            us16 = graph_time_us(dec16, 20, 32)
            emit({"config": 2, "what": f"decode from a step schedule over {dt.name.lower()} pages, "
                  "B=32, 12/2 heads, hd 128, one layer, 16 rotated pools",
                  "latency_us": round(us16, 2), "kv_bytes": b16,
                  "GB/s": round(b16 / us16 / 1e3, 1),
                  "hbm_frac_of_8TB/s": round(b16 / us16 / 1e3 / 8000.0, 4),
                  "kernel": PagedAttention.kernel_name(12, 2, 128, 16, dt) +
                  "_sched + eh_decode_tiles_merge_sched"})
            del pools16
            torch.cuda.empty_cache()

    if "c3" in parts:  # bf16 chunked prefill, B=8, 512 new tokens on 2048 cached, 32/8 heads
        s3 = synth.config3(0)
        tab3 = synth.block_tables(s3, extra_tokens=512)
        lay3 = PagedKvLayout(s3.n_blocks, 16, s3.row_len, KvDataType.BF16)
        pool3 = torch.randn(lay3.floats_total(), generator=gen, device=dev, dtype=torch.bfloat16)
        dtab3 = torch.from_numpy(tab3.view(np.int32)).to(dev)
        T3 = 8 * 512
        k3 = torch.randn((T3, s3.row_len), generator=gen, device=dev, dtype=torch.bfloat16)
        v3 = torch.randn((T3, s3.row_len), generator=gen, device=dev, dtype=torch.bfloat16)
        q3 = torch.randn((T3, 32, 128), generator=gen, device=dev)
        o3 = torch.empty_like(q3)
        cu3 = torch.arange(0, T3 + 1, 512, dtype=torch.int32, device=dev)
        sp3 = torch.full((8,), 2048, dtype=torch.int32, device=dev)
        us_a3 = graph_time_us(lambda st: kv.append_kv_batched(st, lay3, pool3, k3, v3, dtab3, cu3,
                                                              sp3, T3), 10)
        us_p3 = graph_time_us(lambda st: fa.launch_batched(st, q3, pool3, dtab3, cu3, sp3, o3, 32,
                                                           8, 128, 16, 512,
                                                           kv_dtype=KvDataType.BF16), 5, 4)
        flops = 8 * 32 * 4 * 128 * sum(2048 + i + 1 for i in range(512))
        emit({"config": 3, "what": "chunked prefill (causal, MFMA), bf16 KV staged as f16, B=8, "
              "512 on 2048, 32/8 heads, hd 128", "prefill_us": round(us_p3, 2), "flop": flops,
              "TFLOP/s": round(flops / us_p3 / 1e6, 1),
              "mfma_frac_of_2.5PF": round(flops / us_p3 / 1e6 / 2500.0, 4),
              "append_us": round(us_a3, 2),
              "append_GB/s": round(T3 * 2 * s3.row_len * 2 * 2 / us_a3 / 1e3, 1)})
        pool3h = pool3.to(torch.float16)
        us_p3h = graph_time_us(lambda st: fa.launch_batched(st, q3, pool3h, dtab3, cu3, sp3, o3,
                                                            32, 8, 128, 16, 512,
                                                            kv_dtype=KvDataType.F16), 5, 4)
        emit({"config": 3, "what": "the same prefill over f16 pages", "prefill_us": round(us_p3h, 2),
              "TFLOP/s": round(flops / us_p3h / 1e6, 1),
              "mfma_frac_of_2.5PF": round(flops / us_p3h / 1e6 / 2500.0, 4)})
        del pool3h
        lay3e = PagedKvLayout(s3.n_blocks, 16, s3.row_len, KvDataType.FP8)
        pool3e = torch.randint(0, 0x7E, (lay3e.floats_total(),), generator=gen, device=dev,
                               dtype=torch.uint8)
        sc3 = torch.full((8,), 0.01, device=dev)
        us_p3e = graph_time_us(lambda st: fa.launch_batched_e4m3(st, q3, pool3e, dtab3, cu3, sp3,
                                                                 o3, 32, 8, 128, 16, 512, sc3,
                                                                 sc3), 5, 4)
        emit({"config": 3, "what": "chunked prefill (causal, MFMA) over E4M3 pages (fp8 KV, "
              "per-kv-head scales), B=8, 512 on 2048, 32/8 heads, hd 128",
              "prefill_us": round(us_p3e, 2), "flop": flops,
              "TFLOP/s": round(flops / us_p3e / 1e6, 1),
              "mfma_frac_of_2.5PF": round(flops / us_p3e / 1e6 / 2500.0, 4)})
        del pool3, pool3e, k3, v3, q3, o3

    if "c4" in parts:  # prefix-shared CoW + eviction + compaction (page moves on the GPU)
        from titan_amd.prefix_share import PrefixShareScenario, run_on_gpu
        scn = PrefixShareScenario(seed=0)
        plan4 = scn.plan()
        pool4, _, _, lay4 = run_on_gpu(scn, plan4)
        src = torch.from_numpy(np.asarray(plan4.compaction.src, np.uint32).view(np.int32)).to(dev)
        dst = torch.from_numpy(np.asarray(plan4.compaction.dst, np.uint32).view(np.int32)).to(dev)
        npairs = int(src.numel())
        # compaction moves each survivor once; replays re-copy the same bytes
        us4 = graph_time_us(lambda st: kv.copy_pages(st, lay4, pool4, src, dst), 10) if npairs \
            else 0.0
        page = lay4.page_bytes()
        emit({"config": 4, "what": "gather-compaction of surviving pages after prefix-shared "
              "CoW + 25% LRU eviction (64 seqs, 8 kv heads, hd 128, f16)",
              "pages_moved": npairs, "cow_copies": plan4.cow_pairs, "compaction_us": round(us4, 2),
              "GB/s": round(2 * npairs * page / us4 / 1e3, 1) if us4 else None})
        del pool4

    if "c5" in parts:  # B=4 at 32768 tokens, 32/8 heads, f16, pool ~90% of free HBM
        torch.cuda.empty_cache()
        free, _ = torch.cuda.mem_get_info()
        s5 = synth.config5(0, n_blocks=int(args.c5_pool_frac * free) // (16 * 2 * 1024 * 2))
        tab5 = synth.block_tables(s5, extra_tokens=1)
        lay5 = PagedKvLayout(s5.n_blocks, 16, s5.row_len, KvDataType.F16)
        pool5 = torch.empty(lay5.floats_total(), device=dev, dtype=torch.float16)
        # only the pages the tables use are filled (values do not change the
        # timing): N(0,1), with 1 % of the K rows scaled by 8 (the
        # configuration's softmax-range stress)
        ids5 = tab5.reshape(-1)                    # every entry is used: 2049 pages a sequence
        assert (ids5 != 0xFFFFFFFF).all()
        used = torch.from_numpy(ids5.astype(np.int64)).to(dev)
        pg = pool5.view(s5.n_blocks, 16, 2, s5.row_len)
        vals = torch.randn((used.numel(), 16, 2, s5.row_len), generator=gen, device=dev,
                           dtype=torch.float16)
        hot = torch.rand((used.numel(), 16), generator=gen, device=dev) < 0.01
        vals[:, :, 0][hot] *= 8
        pg[used] = vals
        del vals
        dtab5 = torch.from_numpy(tab5.view(np.int32)).to(dev)
        dids5 = torch.from_numpy(ids5.view(np.int32)).to(dev)
        q5 = torch.randn((4, 32, 128), generator=gen, device=dev)
        o5 = torch.empty_like(q5)
        nk5 = torch.randn((4, s5.row_len), generator=gen, device=dev, dtype=torch.float16)
        nv5 = torch.randn((4, s5.row_len), generator=gen, device=dev, dtype=torch.float16)
        st5 = torch.from_numpy(s5.ctx_lens.astype(np.int32)).to(dev)
        plan5 = PagedAttention.plan(4, 32, 8, 128, 16, 32769)
        ws5 = PagedAttention.workspace(plan5)
        stride5 = int(tab5.shape[1])
        sched5 = PagedAttention.schedule_buffer(4, stride5, 16, plan5)
        pa.build_schedule(None, lay5, dtab5, st5, 1, plan5, sched5)
        # evicts the 256 MB MALL by reading 1 GiB of other data: a write-based flush
        # (memset) would leave dirty lines whose write-back competes with the timed reads
        flush = torch.ones(1024 * 1024 * 1024 // 4, device=dev)
        stream = torch.cuda.Stream()
        xo5 = torch.empty(1024 * 8, dtype=torch.int32, device=dev)
        b5 = 4 * 32769 * 8 * 128 * 2 * 2

        def cold_us(call):
            times = []
            with torch.cuda.stream(stream):
                for it in range(12):
                    flush.sum()
                    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    a.record(stream)
                    call()
                    b.record(stream)
                    torch.cuda.synchronize()
                    if it >= 2:
                        times.append(a.elapsed_time(b) * 1e3)
            return float(np.median(times))

        sweep = {}
        for depth in (1, 2):
            for grid in (256, 512, 1024):
                sweep[f"d{depth}_g{grid}"] = round(cold_us(
                    lambda: kv.stream_pages(stream, lay5, pool5, dids5, xo5, depth, grid)), 2)
        c_key = min(sweep, key=sweep.get)
        c_us = sweep[c_key]
        c_bytes = int(ids5.size) * lay5.page_bytes()
        heads5 = {}
        for grid in (256, 512, 1024):
            heads5[f"g{grid}"] = round(cold_us(
                lambda: kv.stream_pages_heads(stream, lay5, pool5, dids5, xo5, 128, grid)), 2)
        h_key = min(heads5, key=heads5.get)
        h_us = heads5[h_key]
        emit({"config": 5, "what": "read ceiling: the 8196 used 64 KiB pages streamed once by "
              "eh_stream_pages through the same tables, and in the decode's per-kv-head pattern "
              "by eh_stream_pages_heads, MALL evicted (1 GiB read) before each timed call",
              "stream_bytes": c_bytes, "ceiling_us": c_us, "best": c_key,
              "sweep_us": sweep, "ceiling_GB/s": round(c_bytes / c_us / 1e3, 1),
              "ceiling_frac_of_8TB/s": round(c_bytes / c_us / 1e3 / 8000.0, 4),
              "heads_ceiling_us": h_us, "heads_best": h_key, "heads_sweep_us": heads5})
        k5 = PagedAttention.kernel_name(32, 8, 128, 16, KvDataType.F16)
        for label, kern, call in (
                ("fused append + decode (self-scheduled)", k5 + " + eh_decode_tiles_merge",
                 lambda: pa.append_decode_batched(stream, lay5, pool5, nk5, nv5, dtab5, st5, q5,
                                                  o5, 32, 128, plan5, ws5)),
                ("fused append + decode from a step schedule",
                 k5 + "_sched + eh_decode_tiles_merge_sched",
                 lambda: pa.append_decode_scheduled(stream, lay5, pool5, nk5, nv5, sched5,
                                                    stride5, q5, o5, 32, 128, plan5, ws5))):
            o5.fill_(float("nan"))
            us5 = cold_us(call)
            # every timed call rewrote the same rows at position 32768 and
            # attended the same 32769 tokens: the appended rows bit for bit and
            # the last call's output against a float64 numpy attention over a
            # compacted host copy of the used pages (the oracle itself stays
            # in tests/, where the same check runs at this pool size)
            host = pg[used].cpu().numpy().reshape(4, 2049 * 16, 2, 8, 128)
            app_ok = all(np.array_equal(host[b, 32768, 0].reshape(-1).view(np.uint16),
                                        nk5[b].cpu().numpy().view(np.uint16)) and
                         np.array_equal(host[b, 32768, 1].reshape(-1).view(np.uint16),
                                        nv5[b].cpu().numpy().view(np.uint16)) for b in range(4))
            ref = np_decode_f64(host[:, :32769], q5.cpu().numpy())
            del host
            d = np.abs(o5.cpu().numpy().astype(np.float64) - ref)
            ok = bool(np.isfinite(d).all() and d.max() <= 2e-3 and
                      (d <= 2e-3 + 1e-3 * np.abs(ref)).all())
            emit({"config": 5, "what": f"{label}, B=4 x 32768 ctx, 32/8 heads, hd 128, f16, 1 % "
                  f"of K rows x 8, pool {lay5.bytes_total() / 1e9:.0f} GB ({s5.n_blocks} pages, "
                  "scattered), MALL evicted (1 GiB read) before each timed call",
                  "latency_us": round(us5, 2), "kv_bytes": b5, "GB/s": round(b5 / us5 / 1e3, 1),
                  "frac_of_8TB/s": round(b5 / us5 / 1e3 / 8000.0, 4),
                  "frac_of_ceiling": round((b5 / us5) / (c_bytes / c_us), 4),
                  "frac_of_heads_ceiling": round((b5 / us5) / (c_bytes / h_us), 4),
                  "check_vs_numpy_f64": {"max_abs": float(d.max()), "within_bar": ok,
                                         "appended_rows_bit_exact": bool(app_ok)},
                  "kernel": kern})
        del pool5, flush


def np_decode_f64(kv, q):
    """Float64 decode attention by numpy: kv [B, T, 2, n_kv, hd] (K then V of
    every attended token), q [B, n_head, hd]; q head h reads kv head
    h // (n_head / n_kv); scale 1 / sqrt(hd)."""
    import numpy as np
    B, T, _, n_kv, hd = kv.shape
    n_head = q.shape[1]
    grp = n_head // n_kv
    out = np.empty(q.shape, np.float64)
    for b in range(B):
        for h in range(n_kv):
            k = kv[b, :, 0, h].astype(np.float64)
            v = kv[b, :, 1, h].astype(np.float64)
            s = k @ q[b, h * grp:(h + 1) * grp].astype(np.float64).T / np.sqrt(hd)
            w = np.exp(s - s.max(axis=0))
            out[b, h * grp:(h + 1) * grp] = (w.T @ v) / w.sum(axis=0)[:, None]
    return out


def cpu_child(args):
    """The CPU baseline itself (runs in the pinned child, never touches a GPU):
    the oracle's restatement of the reference's single-threaded
    PagedKvCache::append row copies + sdpa_decode (cache.rs:153-192,
    forward_cpu.rs:424-510) on whole layer-steps of config 2 -- the same
    contexts, tables and shapes as the GPU run, seeded N(0,1) values widened
    exactly from f16 (untimed).  Each layer-step is timed on its own; at
    least 5 are run (more while the time budget lasts, at most 64) and the
    median is reported."""
    import numpy as np

    from oracle import orc
    from titan_amd import synth

    if os.environ.get("TITAN_CPU_PINNER") == "sched_setaffinity":
        os.sched_setaffinity(0, {int(os.environ["TITAN_CPU_PIN"])})
    shape = synth.config2(0, extra_tokens=1)
    tab = synth.block_tables(shape, extra_tokens=1)
    B, NQ, NKV, HD, BT = shape.batch, shape.n_head, shape.n_head_kv, shape.head_dim, shape.block_tokens
    rl = shape.row_len
    rng = np.random.default_rng(1)
    page = BT * 2 * rl
    pool = rng.standard_normal(shape.n_blocks * page, dtype=np.float32).astype(np.float16)
    pool = pool.astype(np.float32)                       # exact widening, untimed
    q = rng.standard_normal((B, NQ, HD), dtype=np.float32)
    kn = rng.standard_normal((B, rl), dtype=np.float32).astype(np.float16).astype(np.float32)
    vn = rng.standard_normal((B, rl), dtype=np.float32).astype(np.float16).astype(np.float32)
    lens = shape.ctx_lens.astype(np.int64)
    times = []
    total = 0.0
    while len(times) < 64 and (len(times) < 5 or total < args.cpu_seconds):
        t0 = time.perf_counter()
        for b in range(B):                               # PagedKvCache::append row copies
            L_b = int(lens[b])
            base = int(tab[b, L_b // BT]) * page + (L_b % BT) * 2 * rl
            pool[base:base + rl] = kn[b]
            pool[base + rl:base + 2 * rl] = vn[b]
        orc.sdpa_decode_batched(pool, tab, (lens + 1).astype(np.uint32), BT, q, NQ, NKV, HD)
        dt = time.perf_counter() - t0
        times.append(dt)
        total += dt
    med = float(np.median(times))
    kv_bytes = int((lens + 1).sum()) * NKV * HD * 2 * 2
    pin = os.environ.get("TITAN_CPU_PIN", "?")
    print(json.dumps({
        "value": round(kv_bytes / med / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
        "host_logical_cpus": os.cpu_count(),
        "sample": f"config 2 layer-steps (32 sequences, {int((lens + 1).sum())} attended tokens: "
                  f"append + sdpa_decode over the f32-widened pool), median of {len(times)} "
                  f"({total:.1f} s), 1 thread pinned to CPU {pin} "
                  f"({os.environ.get('TITAN_CPU_PINNER', '?')}) of {cpu_model()}: 1 of "
                  f"{os.cpu_count()} logical CPUs on the host ({os.environ.get('TITAN_CPU_AVAIL', '?')} "
                  f"in the benchmark's affinity mask); the reference path is single-threaded",
        "median_layer_step_ms": round(med * 1e3, 2),
        "median_step_ms_28_layers": round(med * 28e3, 1),
        "tok_s": round(B / (28 * med), 3)}), flush=True)


if __name__ == "__main__":
    main()
