"""Benchmark of the MI355X full-attention hot path.

Headline (``value``): paged GQA decode step at B=32, per-sequence contexts
uniform in [128, 2048] (seeded), 8 q / 2 kv heads, d=256, randperm page table.
One step is the decode attention of the model's 6 full-attention layers, each
with its own K/V page pools (~480 MB in all, twice the 256 MB MALL, so K/V
come from HBM), sharing the block table and positions; per layer one launch
does K/V append + split-K partial + merge + sigmoid gate.  The step is one HIP
graph replay; ``--steps`` replays are timed per window with HIP events on the
replay stream, windows repeat until >= 50 ms were timed, and the median window
is reported.  ``value`` is algorithmic HBM GB/s of the step (KV bytes read +
q/gate/out/append/page-table bytes, split scratch excluded).

Also reported: ``roofline`` (the step kernel: average launch = step time / 6),
``roofline_prefill`` (the varlen causal prefill kernel at configs 4 and 3),
``cpu_baseline`` / ``cpu_baseline_prefill`` (the CPU oracle on all host cores,
median of repetitions), and ``extra``: config 1 latency, configs 3/4 prefill,
config 5 long-context decode, the attention block / layer, the config-3
HBM-bound companions, ``gemm_2d`` next to hipBLASLt, the Gated DeltaNet
kernels (``gdn``) and the whole 24-layer model (``model``); ``--only a,b``
selects extras by name.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick] [--only ...]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HQ, HKV, D, PAGE = 8, 2, 256, 16
HBM_PEAK_GBS = 8000.0
ATTN_LAYERS = 6   # full-attention layers of Qwen3.5-0.8B (every 4th of 24)
MFMA_BF16_PEAK_TFLOPS = 2500.0


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ workloads

def decode_workload(lens, dev, seed, kv_scale=1.0, contiguous=False, tight=False):
    """Synthetic decode inputs.  The pool holds B * max_pages pages (every
    table row full width), or with ``tight`` only the pages the sequences use
    plus one each for the append, dealt from one random permutation (an
    engine's shared pool), so a batch with one long sequence does not get a
    pool B times the long sequence."""
    B = len(lens)
    gen = torch.Generator(device=dev).manual_seed(seed)
    max_pages = -(-max(lens) // PAGE) + 1
    if tight:
        need = [-(-n // PAGE) + 1 for n in lens]
        num_pages = sum(need)
        perm = torch.randperm(num_pages, device=dev, generator=gen).to(torch.int32)
        bt = torch.zeros(B, max_pages, dtype=torch.int32, device=dev)
        o = 0
        for b, k in enumerate(need):
            bt[b, :k] = perm[o:o + k]
            o += k
    else:
        num_pages = B * max_pages
    if contiguous:
        bt = torch.arange(num_pages, device=dev, dtype=torch.int32).view(B, max_pages)
    elif not tight:
        bt = torch.randperm(num_pages, device=dev, generator=gen).view(B, max_pages)
        bt = bt.to(torch.int32).contiguous()

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, device=dev, generator=gen) * scale).to(torch.bfloat16)

    kc = rnd(num_pages, HKV, PAGE, D, scale=kv_scale)
    vc = rnd(num_pages, HKV, PAGE, D, scale=kv_scale)
    return dict(
        lens=lens, bt=bt, kc=kc, vc=vc, q=rnd(B, HQ, D), kn=rnd(B, HKV, D), vn=rnd(B, HKV, D),
        gate=rnd(1, HQ, B, D),
        pos=torch.tensor([n - 1 for n in lens], dtype=torch.int64, device=dev),
    )


def decode_bytes(lens):
    """Algorithmic HBM bytes of one decode step (split scratch excluded):
    KV of every attended token, q + gate + gated output, the K/V append
    (read + write), page-table entries and pos."""
    B = len(lens)
    kv = sum(lens) * HKV * D * 2 * 2
    qgo = B * 3 * HQ * D * 2
    append = B * 2 * HKV * D * 2 * 2
    bt = 4 * sum(-(-n // PAGE) for n in lens)
    return kv + qgo + append + bt + 8 * B


def split_kernel_bytes(lens):
    """Algorithmic bytes the split kernel itself must read: KV + q + table."""
    B = len(lens)
    return sum(lens) * HKV * D * 2 * 2 + B * HQ * D * 2 + 4 * sum(-(-n // PAGE) for n in lens) \
        + 8 * B


def config4_lengths():
    """24 lengths log-uniform in [16, 4096], seed 4 (~18.6k tokens)."""
    g4 = torch.Generator().manual_seed(4)
    lens4 = torch.exp(torch.empty(24).uniform_(math.log(16), math.log(4096), generator=g4))
    return [int(x) for x in lens4.round().tolist()]


def prefill_flops(lengths):
    return sum(n * (n + 1) // 2 for n in lengths) * 4 * D * HQ


def profile_traffic(name):
    """HBM bytes per launch measured by rocprofv3 counters, if committed."""
    f = ROOT / "profiles" / f"{name}_traffic.json"
    return json.loads(f.read_text()).get("hbm_bytes_per_launch") if f.exists() else None


# ------------------------------------------------------------------ timing

STEPS_PER_GRAPH = 8


def time_graph(fn, steps, warmup, per_graph=STEPS_PER_GRAPH):
    """`per_graph` back-to-back calls of fn in one graph (as a decode step graph
    holds every attention layer), replayed in windows of ceil(steps/per_graph)
    replays after ceil(warmup/per_graph) untimed ones; median window, ms per
    call (HIP events on the replay stream)."""
    stream = torch.cuda.Stream()
    g = capture(lambda: [fn() for _ in range(per_graph)], stream)
    with torch.cuda.stream(stream):
        ev, _ = time_steps(g, max(1, -(-steps // per_graph)), -(-warmup // per_graph))
    return median(ev) / per_graph


def capture(fn, stream):
    """Warm fn up once on `stream`, then capture one call of it into a graph on
    that same stream (so per-stream workspaces exist before the capture)."""
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fn()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    torch.cuda.synchronize()
    return g


def time_steps(graph, steps, warmup, min_total_s=0.05, min_windows=5):
    """`warmup` untimed replays of `graph` (one step each), then windows of
    exactly `steps` replays, each bracketed by device synchronisation and
    timed with HIP events recorded on the stream the replays run on (plus the
    host clock).  Windows repeat until at least `min_windows` ran and
    `min_total_s` of replays was timed.  Returns per-window ms per step
    (events) and per-window wall ms per step."""
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    ev, wall, total = [], [], 0.0
    while len(ev) < min_windows or total < min_total_s:
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        st.record()
        for _ in range(steps):
            graph.replay()
        en.record()
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        total += dt
        ev.append(st.elapsed_time(en) / steps)
        wall.append(dt * 1e3 / steps)
    return ev, wall


def rnd(x, scale, digits):
    """round(x * scale, digits), None stays None."""
    return None if x is None else round(x * scale, digits)


def median(xs):
    ys = sorted(xs)
    n = len(ys)
    return ys[n // 2] if n % 2 else 0.5 * (ys[n // 2 - 1] + ys[n // 2])


def time_events(fn, iters, warmup=3):
    """Average ms of fn's launches measured with HIP events on the current
    stream (the stream the kernels are launched on)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    for _ in range(iters):
        fn()
    en.record()
    en.synchronize()
    return st.elapsed_time(en) / iters


def time_graph_events(fn, iters):
    """fn captured in a graph of `iters` back-to-back calls, timed with events:
    removes host launch overhead from a per-kernel figure."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(iters):
            fn()
    # bring the clocks to their loaded steady state first (~0.3 s of replays)
    t_end = time.perf_counter() + 0.3
    while True:
        g.replay()
        torch.cuda.synchronize()
        if time.perf_counter() > t_end:
            break
    st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    st.record()
    for _ in range(3):
        g.replay()
    en.record()
    en.synchronize()
    return st.elapsed_time(en) / (3 * iters)


# ------------------------------------------------------------------ main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=2000,
                    help="untimed steps first")
    ap.add_argument("--quick", action="store_true", help="headline only, no extras/CPU")
    ap.add_argument("--only", default="", help="comma list of extras to run")
    ap.add_argument("--mode", default="bench", choices=["bench", "pmc-step", "pmc-copy", "pmc-prefill", "pmc-prefill3", "pmc-gemm",
                             "pmc-gdn", "floor", "trace-c5"],
                    help="pmc-*: eager launches only, for rocprofv3 counter runs; floor: "
                         "vendor kernels over the headline's bytes, for a rocprofv3 trace")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}): the attention path "
              "shards by sequence with no cross-GPU exchange, so the per-GPU figure is the "
              "one-GPU figure.", file=sys.stderr)
        sys.exit(2)

    import __graft_entry__

    pkg = __graft_entry__.load_package()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    pkg._lib.load()

    # ---- headline: config 2 decode step ----------------------------------------
    # One step = the decode attention of every full-attention layer of the
    # model (ATTN_LAYERS): each layer has its own page pools (80 MB of K/V at
    # config 2) and its own q / new K,V / gate, while the sequences (block
    # table, pos) are shared, as in the engine.  The 6 pools (~480 MB) exceed
    # the 256 MB MALL, so replays read K/V from HBM, not from the cache.
    gen = torch.Generator().manual_seed(2)
    lens = torch.randint(128, 2049, (32,), generator=gen).tolist()
    layers = [decode_workload(lens, dev, seed=2 if i == 0 else 200 + i)
              for i in range(ATTN_LAYERS)]
    for lw in layers[1:]:
        lw["bt"], lw["pos"] = layers[0]["bt"], layers[0]["pos"]
    w = layers[0]
    scratch = pkg.allocate_split_scratch(HQ, D, batch=32, device=dev)

    m_p, l_p, acc_p = scratch

    def layer_step(lw):
        return torch.ops.wy_lib.paged_gqa_attention_decode_fused(
            lw["q"], lw["kn"], lw["vn"], lw["kc"], lw["vc"], lw["bt"], lw["pos"], m_p, l_p,
            acc_p, scratch.counters, lw["gate"][0].permute(1, 0, 2))

    def step():
        for lw in layers:
            layer_step(lw)

    def step_one_pool():
        for _ in layers:
            layer_step(w)

    def step_three_ops(lw):
        ctx = pkg.call_paged_gqa_attention_decode_triton(
            lw["q"], lw["kn"], lw["vn"], lw["kc"], lw["vc"], lw["bt"], lw["pos"], tuple(scratch))
        return pkg.attention_gate_pack(ctx.permute(1, 0, 2).unsqueeze(0), lw["gate"])

    if args.mode == "pmc-step":
        for _ in range(10):
            step()
        torch.cuda.synchronize()
        print(json.dumps({"mode": "pmc-step", "launches": 10 * ATTN_LAYERS,
                          "algorithmic_bytes_per_launch": decode_bytes(lens)}))
        return
    if args.mode in ("pmc-prefill", "pmc-prefill3"):
        # config 4 (pmc-prefill) or config 3 (pmc-prefill3): 0.3 s of eager
        # launches first (steady clocks), then 20 more; counters per dispatch
        if args.mode == "pmc-prefill3":
            lens_p, seed_p = [128] * 32, 3
        else:
            lens_p, seed_p = config4_lengths(), 4
        qp, kp, vp, cup = prefill_inputs(dev, lens_p, seed_p)
        run_p = lambda: pkg.gqa_attention_varlen_causal(qp, kp, vp, cup, max(lens_p))
        t_end = time.perf_counter() + 0.3
        n_calls = 0
        while time.perf_counter() < t_end:
            run_p()
            torch.cuda.synchronize()
            n_calls += 1
        for _ in range(20):
            run_p()
        torch.cuda.synchronize()
        print(json.dumps({"mode": args.mode, "flops": prefill_flops(lens_p),
                          "calls": n_calls + 20,
                          "min_hbm_bytes": sum(lens_p) * (HQ * D * 4 + HKV * D * 4)}))
        return
    if args.mode == "pmc-gemm":
        # gemm_2d on the decode (B=32) and prefill (T=4096) projection shapes,
        # 5 eager calls each, for a per-kernel trace
        gg = torch.Generator(device=dev).manual_seed(7)
        for M, N, K in ((32, 5120, 1024), (32, 1024, 2048), (4096, 2048, 1024),
                        (4096, 1024, 2048)):
            x = torch.randn(M, K, device=dev, generator=gg).to(torch.bfloat16)
            wt = torch.randn(N, K, device=dev, generator=gg).to(torch.bfloat16)
            for _ in range(5):
                pkg.gemm_2d(x, wt)
        torch.cuda.synchronize()
        print(json.dumps({"mode": "pmc-gemm"}))
        return
    if args.mode == "pmc-gdn":
        # GDN recurrence decode and the GDN decode block at B=32, 10 eager calls each
        gg = torch.Generator(device=dev).manual_seed(9)
        Bg, Hg, Dg = 32, 16, 128
        q = (torch.randn(Bg, Hg, Dg, device=dev, generator=gg) * 0.08).to(torch.bfloat16)
        k = (torch.randn(Bg, Hg, Dg, device=dev, generator=gg) * 0.08).to(torch.bfloat16)
        v = torch.randn(Bg, Hg, Dg, device=dev, generator=gg).to(torch.bfloat16)
        beta = torch.rand(Bg, Hg, device=dev, generator=gg)
        g = -torch.rand(Bg, Hg, device=dev, generator=gg)
        st = torch.randn(Bg, Hg, Dg, Dg, device=dev, generator=gg) * 0.1
        fused = torch.randn(Bg, 4 * Hg * Dg + 2 * Hg, device=dev, generator=gg).to(torch.bfloat16)
        cs = torch.randn(Bg, 4, 3 * Hg * Dg, device=dev, generator=gg).to(torch.bfloat16)
        cw = (torch.randn(4, 3 * Hg * Dg, device=dev, generator=gg) * 0.5).to(torch.bfloat16)
        a_log = torch.zeros(Hg, device=dev)
        dt = torch.zeros(Hg, device=dev, dtype=torch.bfloat16)
        nw = torch.ones(Dg, device=dev)
        for _ in range(10):
            pkg.gdn_recurrent_decode(q, k, v, beta, g, st)
        for _ in range(10):
            pkg.gdn_decode_block(fused, cs, cw, a_log, dt, nw, st)
        torch.cuda.synchronize()
        print(json.dumps({"mode": "pmc-gdn",
                          "decode_algorithmic_bytes": Bg * Hg * (2 * Dg * Dg * 4 + 4 * Dg * 2 + 8)}))
        return
    if args.mode == "floor":
        # Vendor kernels moving the headline step's bytes, each layer on its
        # own buffers (6 x, > MALL), 40 eager rounds each: a device copy of
        # 40 MB into 40 MB (80 MB of traffic), torch.index_select of the step's
        # K and of its V page rows (each 40 MB read + 40 MB written), a bf16
        # sum of 80 MB, next to wy_page_stream_read and the step itself.
        kvb = sum(lens) * HKV * D * 2 * 2
        src = [torch.ones(kvb // 4, dtype=torch.bfloat16, device=dev) for _ in layers]
        dst = [torch.empty_like(x) for x in src]
        flat = [torch.ones(kvb // 2, dtype=torch.bfloat16, device=dev) for _ in layers]
        btc = layers[0]["bt"].cpu()
        rows = torch.tensor([int(btc[b, p]) * HKV + h for b, n in enumerate(lens)
                             for h in range(HKV) for p in range(-(-n // PAGE))],
                            device=dev, dtype=torch.int64)
        gath = torch.empty(rows.numel(), PAGE * D, dtype=torch.bfloat16, device=dev)
        cases = {
            "copy": lambda i: dst[i].copy_(src[i]),
            "index_select": lambda i: (
                torch.index_select(layers[i]["kc"].view(-1, PAGE * D), 0, rows, out=gath),
                torch.index_select(layers[i]["vc"].view(-1, PAGE * D), 0, rows, out=gath)),
            "sum": lambda i: flat[i].sum(dtype=torch.float32),
            "page_stream_read": lambda i: pkg.page_stream_read(layers[i]["kc"], layers[i]["vc"],
                                                               layers[i]["bt"], layers[i]["pos"]),
            "decode_step": lambda i: layer_step(layers[i]),
        }
        for fn in cases.values():
            for _ in range(40):
                for i in range(ATTN_LAYERS):
                    fn(i)
            torch.cuda.synchronize()
        print(json.dumps({"mode": "floor", "kv_bytes": kvb, "rounds": 40}))
        return
    if args.mode == "trace-c5":
        # config 5 alone (B=64 x 32768, one 4 GiB pool): 5 warm-up steps, then 20,
        # eager, for a kernel trace of the one-launch step at that size
        w5 = decode_workload([32768] * 64, dev, seed=5, kv_scale=0.5)
        sc5 = pkg.allocate_split_scratch(HQ, D, batch=64, device=dev)
        g5 = w5["gate"][0].permute(1, 0, 2)
        for _ in range(25):
            torch.ops.wy_lib.paged_gqa_attention_decode_fused(
                w5["q"], w5["kn"], w5["vn"], w5["kc"], w5["vc"], w5["bt"], w5["pos"], *sc5,
                sc5.counters, g5)
        torch.cuda.synchronize()
        print(json.dumps({"mode": "trace-c5", "launches": 25,
                          "algorithmic_bytes_per_launch": decode_bytes(w5["lens"])}))
        return
    if args.mode == "pmc-copy":
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"mode": "pmc-copy", "bytes_read": 256 << 20,
                          "bytes_written": 256 << 20}))
        return

    log(f"decode config2: sum(L)={sum(lens)} B=32, {ATTN_LAYERS} layers per step")
    stream = torch.cuda.Stream()
    g_step = capture(step, stream)
    with torch.cuda.stream(stream):
        ev, wall = time_steps(g_step, args.steps, args.warmup)
    ms = median(ev)
    layer_bytes = decode_bytes(lens)
    step_bytes = ATTN_LAYERS * layer_bytes
    gbs = step_bytes / (ms * 1e-3) / 1e9
    # the step is ATTN_LAYERS launches of one kernel, back to back in the graph
    kern_ms = ms / ATTN_LAYERS
    kern_gbs = layer_bytes / (kern_ms * 1e-3) / 1e9
    kv_bytes = sum(lens) * HKV * D * 2 * 2
    ms_one = ms_floor = ms3 = ms_copy = None
    if not args.quick:  # companions of the headline (a --quick run times the headline only)
        # the same graph with all 6 launches on one pool (80 MB, stays in the MALL)
        g_one = capture(step_one_pool, stream)
        with torch.cuda.stream(stream):
            ev1, _ = time_steps(g_one, 100, 200)
        ms_one = median(ev1) / ATTN_LAYERS
        # the streaming floor: the same 6 x 80 MB of pages read once, no math,
        # perfectly balanced over 2048 wavefronts (wy_page_stream_read)
        g_fl = capture(lambda: [pkg.page_stream_read(lw["kc"], lw["vc"], lw["bt"], lw["pos"])
                                for lw in layers], stream)
        with torch.cuda.stream(stream):
            evf, _ = time_steps(g_fl, max(args.steps, 20), max(args.warmup, 20))
        ms_floor = median(evf) / ATTN_LAYERS
        # the reference's three-op path, same rotated pools
        g3 = capture(lambda: [step_three_ops(lw) for lw in layers], stream)
        with torch.cuda.stream(stream):
            ev3, _ = time_steps(g3, max(args.steps, 20), max(args.warmup, 20))
        ms3 = median(ev3) / ATTN_LAYERS
        # a vendor floor for the same bytes: torch's device copy (hipMemcpy's
        # blit kernel) of 40 MB into 40 MB, i.e. the step's 80 MB of HBM
        # traffic, one distinct buffer pair per layer, 6 copies in one graph
        half = kv_bytes // 4
        cp_src = [torch.ones(half, dtype=torch.bfloat16, device=dev) for _ in layers]
        cp_dst = [torch.empty_like(x) for x in cp_src]
        g_cp = capture(lambda: [d.copy_(x) for d, x in zip(cp_dst, cp_src)], stream)
        with torch.cuda.stream(stream):
            evc, _ = time_steps(g_cp, max(args.steps, 20), max(args.warmup, 20))
        ms_copy = median(evc) / ATTN_LAYERS
        del g_one, g3, g_fl, g_cp, cp_src, cp_dst
    traffic = profile_traffic("decode_step_config2")

    result = {
        "metric": "decode-attn HBM GB/s (B=32 paged GQA decode step, contexts U[128,2048])",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_layer": round(kern_ms * 1e3, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 q/k/v/gate, randperm page table)",
        "config": {"workload": f"config2: paged GQA decode step B=32, L~U[128,2048], "
                               f"8q/2kv heads, d=256, 16-token pages; one step = the "
                               f"{ATTN_LAYERS} full-attention layers of the model, each "
                               f"with its own K/V page pools",
                   "global_batch": 32, "sum_context_tokens": sum(lens),
                   "layers_per_step": ATTN_LAYERS,
                   "working_set_MB": round(ATTN_LAYERS * 2 * w["kc"].numel() * 2 / 1e6, 1),
                   "step": "per layer one launch: append + split-K + merge + sigmoid gate; "
                           "the step is one HIP graph replay",
                   "timing": f"{len(ev)} windows of exactly {args.steps} steps after "
                             f"{args.warmup} untimed steps; HIP events on the replay stream; "
                             f"median window (wall-clock median "
                             f"{median(wall) * 1e3:.2f} us/step)",
                   "parallelism": "single GPU"},
        "roofline": {"kernel": "paged_decode_split_kernel<true, 4> (one-launch step)",
                     "bound": "hbm",
                     "achieved": round(kern_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(kern_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes_per_launch": layer_bytes,
                     "avg_launch_us": round(kern_ms * 1e3, 3),
                     "stream_floor_us": rnd(ms_floor, 1e3, 3),
                     "stream_floor_GB/s": rnd(ms_floor and kv_bytes / ms_floor, 1e-6, 1),
                     "frac_of_stream_floor": rnd(ms_floor and ms_floor / kern_ms, 1, 4),
                     "vendor_copy_floor_us": rnd(ms_copy, 1e3, 3),
                     "vendor_copy_floor_GB/s": rnd(ms_copy and kv_bytes / ms_copy, 1e-6, 1),
                     "frac_of_vendor_copy_floor": rnd(ms_copy and ms_copy / kern_ms, 1, 4),
                     "single_pool_mall_warm_us": rnd(ms_one, 1e3, 3),
                     "single_pool_mall_warm_frac": rnd(
                         ms_one and layer_bytes / (ms_one * 1e-3) / 1e9 / HBM_PEAK_GBS, 1, 4)},
        "three_op_path_us_per_layer": rnd(ms3, 1e3, 2),
    }
    log(f"  step {ms*1e3:.2f} us ({kern_ms*1e3:.2f} per layer) {gbs:.0f} GB/s; "
        f"one pool {ms_one} ms; stream floor {ms_floor} ms; 3-op {ms3} ms/layer")

    extra = {}
    only = set(filter(None, args.only.split(",")))

    def want(name):
        return not args.quick and (not only or name in only)

    # ---- config 2 as the whole attention block: from the fused projection
    # output (q/k RMSNorm + partial RoPE in the same launch) ----------------------
    if want("block"):
        gen_b = torch.Generator(device=dev).manual_seed(7)
        fused = torch.randn(32, 5120, device=dev, generator=gen_b).to(torch.bfloat16)
        qw = (torch.randn(D, device=dev, generator=gen_b) * 0.3).to(torch.bfloat16)
        kw = (torch.randn(D, device=dev, generator=gen_b) * 0.3).to(torch.bfloat16)
        inv = pkg.rope_inv_freq(64, 1e7, device=dev)

        def block():
            return pkg.decode_attention_block(fused, qw, kw, 1e-6, inv, 64, w["pos"], w["kc"],
                                              w["vc"], w["bt"], scratch)

        msb = time_graph(block, args.steps, args.warmup)
        extra["config2_attention_block"] = {
            "us_per_step": round(msb * 1e3, 2),
            "what": "fused q/gate/k/v projection output -> o_proj input in one launch "
                    "(q/k RMSNorm, partial RoPE, append, split-K, merge, gate)"}

        # the whole attention layer of a decode step (engine/runner.py:444-518):
        # h [32, 1024] -> fused projection GEMM -> block -> o_proj GEMM
        h = torch.randn(32, 1024, device=dev, generator=gen_b).to(torch.bfloat16)
        w_qkvg = (torch.randn(5120, 1024, device=dev, generator=gen_b) * 0.03).to(torch.bfloat16)
        w_o = (torch.randn(1024, 2048, device=dev, generator=gen_b) * 0.03).to(torch.bfloat16)

        def layer(gemm):
            f = gemm(h, w_qkvg)
            packed = pkg.decode_attention_block(f, qw, kw, 1e-6, inv, 64, w["pos"], w["kc"],
                                                w["vc"], w["bt"], scratch)
            return gemm(packed, w_o)

        msl = time_graph(lambda: layer(pkg.gemm_2d), args.steps, args.warmup)
        msl_ref = time_graph(lambda: layer(torch.nn.functional.linear), args.steps, args.warmup)
        extra["config2_attention_layer"] = {
            "us_per_step": round(msl * 1e3, 2),
            "us_per_step_with_hipblaslt_gemms": round(msl_ref * 1e3, 2),
            "what": "h [32,1024] -> gemm_2d [5120,1024] -> attention block -> gemm_2d o_proj "
                    "[1024,2048], one graph (3 launches)"}

    # ---- config 1: B=1, 256 tokens, contiguous table --------------------------
    if want("c1"):
        w1 = decode_workload([256], dev, seed=1, contiguous=True)
        sc1 = pkg.allocate_split_scratch(HQ, D, batch=1, device=dev)

        g1 = w1["gate"][0].permute(1, 0, 2)

        def step1():
            return torch.ops.wy_lib.paged_gqa_attention_decode_fused(
                w1["q"], w1["kn"], w1["vn"], w1["kc"], w1["vc"], w1["bt"], w1["pos"], *sc1,
                sc1.counters, g1)

        ms1 = time_graph(step1, 500, 50)
        extra["config1_decode_B1_L256"] = {"us_per_step": round(ms1 * 1e3, 2),
                                           "GB/s": round(decode_bytes([256]) / ms1 / 1e6, 1)}
        log(f"config1: {ms1*1e3:.2f} us")
        del w1

    # ---- B=1 decode over context length, beside the reference's figures --------
    if want("b1curve"):
        extra["decode_B1_curve"] = b1_curve_bench(pkg, dev)
    # ---- length skew at config 2's total tokens --------------------------------
    if want("skew"):
        extra["decode_length_skew"] = skew_bench(pkg, dev, sum(lens), args.steps, args.warmup)

    # ---- config 3: varlen prefill 32 x 128 -------------------------------------
    if want("c3"):
        extra["config3_prefill_32x128"] = prefill_bench(pkg, dev, [128] * 32, seed=3)
    # ---- config 4: mixed lengths log-uniform [16, 4096] ------------------------
    if want("c4"):
        extra["config4_prefill_mixed"] = prefill_bench(pkg, dev, config4_lengths(), seed=4)
    # ---- the prefill attention path after q/k norm: op sequence vs block ---------
    if want("pblock"):
        extra["config3_prefill_attention_path"] = prefill_path_bench(pkg, dev, [128] * 32, 3)
        extra["config4_prefill_attention_path"] = prefill_path_bench(
            pkg, dev, config4_lengths(), 4)
    # ---- config 5: B=64 x 32768 ------------------------------------------------
    if want("c5"):
        w5 = decode_workload([32768] * 64, dev, seed=5, kv_scale=0.5)
        sc5 = pkg.allocate_split_scratch(HQ, D, batch=64, device=dev)
        m5, l5, a5 = sc5

        def split5():
            torch.ops.wy_lib.paged_gqa_attention_decode_split(
                w5["q"], w5["kc"], w5["vc"], w5["bt"], m5, l5, a5, w5["pos"], 0)

        g5 = w5["gate"][0].permute(1, 0, 2)

        def step5():
            return torch.ops.wy_lib.paged_gqa_attention_decode_fused(
                w5["q"], w5["kn"], w5["vn"], w5["kc"], w5["vc"], w5["bt"], w5["pos"], *sc5,
                sc5.counters, g5)

        ms5 = time_graph(step5, 20, 3)
        sp5 = time_events(split5, 20)
        b5 = decode_bytes(w5["lens"])
        extra["config5_decode_B64_L32768"] = {
            "us_per_step": round(ms5 * 1e3, 1), "GB/s": round(b5 / ms5 / 1e6, 1),
            "split_us": round(sp5 * 1e3, 1),
            "split_GB/s": round(split_kernel_bytes(w5["lens"]) / sp5 / 1e6, 1),
            "frac_of_hbm_peak": round(b5 / ms5 / 1e6 / HBM_PEAK_GBS, 4)}
        log(f"config5: {ms5*1e3:.1f} us")
        del w5, sc5
        torch.cuda.empty_cache()

    # ---- config 3's HBM-bound companions: RoPE, page scatter, gate pack --------
    if want("c3ew"):
        extra["config3_elementwise"] = elementwise_bench(pkg, dev)

    # ---- projection GEMMs around the attention path (wy_lib::gemm_2d) -----------
    if want("gemm"):
        extra["gemm_2d"] = gemm_bench(pkg, dev)

    # ---- the whole model's decode step as one graph ----------------------------
    if want("model"):
        extra["decode_step_full_model"] = decoder_bench(pkg, dev)

    # ---- Gated DeltaNet recurrence (the other mixer of the model) -------------
    if want("gdn"):
        extra["gdn"] = gdn_bench(pkg, dev)

    # ---- prefill roofline: the varlen causal kernel at configs 4 and 3 ----------
    rp = {}
    c4 = extra.get("config4_prefill_mixed")
    if c4:
        rp["config4"] = {
            "kernel": "varlen_causal_prefill_kernel (queue launch)", "bound": "mfma",
            "achieved": c4["TFLOP/s"], "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": c4["frac_of_mfma_peak"], "traffic": profile_traffic("prefill_config4"),
            "algorithmic_flops_per_launch": int(c4["GFLOP"] * 1e9),
            "avg_launch_us": c4["us"]}
    c3 = extra.get("config3_prefill_32x128")
    if c3:
        rp["config3"] = {
            "kernel": "short_prefill_kernel (eight waves per block, one-round grid of sequences <= 128 tokens)",
            "bound": "hbm (arithmetic intensity 51.6 flop/B < ridge 312)",
            "achieved": c3["TFLOP/s"], "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": c3["frac_of_mfma_peak"],
            "attainable": c3["attainable_TFLOP/s"], "frac_of_attainable": c3["frac_of_attainable"],
            "traffic": profile_traffic("prefill_config3"),
            "algorithmic_flops_per_launch": int(c3["GFLOP"] * 1e9),
            "min_hbm_bytes_per_launch": c3["min_hbm_bytes"],
            "avg_launch_us": c3["us"]}
    if rp:
        result["roofline_prefill"] = rp
    if extra:
        result["extra"] = extra

    # ---- CPU baseline: oracle on a bounded sample of config 2 -------------------
    if not args.quick and (not only or "cpu" in only):
        result["cpu_baseline"] = cpu_baseline(w, lens)
        result["cpu_baseline_prefill"] = cpu_baseline_prefill(dev)

    print(json.dumps(result), flush=True)


def decode_layers_us(pkg, dev, lens, steps, warmup, seed=11):
    """One-launch decode step over `lens`, the headline's regime: 6 layers with
    their own tight pools (shared table and pos) in one graph; us per layer."""
    ls = [decode_workload(lens, dev, seed=seed + i, tight=True) for i in range(ATTN_LAYERS)]
    for lw in ls[1:]:
        lw["bt"], lw["pos"] = ls[0]["bt"], ls[0]["pos"]
    sc = pkg.allocate_split_scratch(HQ, D, batch=len(lens), device=dev)

    def step():
        for lw in ls:
            torch.ops.wy_lib.paged_gqa_attention_decode_fused(
                lw["q"], lw["kn"], lw["vn"], lw["kc"], lw["vc"], lw["bt"], lw["pos"], *sc,
                sc.counters, lw["gate"][0].permute(1, 0, 2))

    stream = torch.cuda.Stream()
    g = capture(step, stream)
    with torch.cuda.stream(stream):
        ev, _ = time_steps(g, steps, warmup)
    del g, ls, sc
    torch.cuda.empty_cache()
    return median(ev) / ATTN_LAYERS * 1e3


def skew_bench(pkg, dev, total, steps, warmup):
    """Same total context as config 2 over B=32: uniform lengths vs one long
    sequence and 31 of 128 tokens (the reference measures +20% from uniform to
    extreme skew at equal total, gqa_attention_decode_paged.py:669-673)."""
    B = 32
    uniform = [total // B + (1 if i < total % B else 0) for i in range(B)]
    skew = [total - (B - 1) * 128] + [128] * (B - 1)
    us_u = decode_layers_us(pkg, dev, uniform, steps, warmup)
    us_s = decode_layers_us(pkg, dev, skew, steps, warmup)
    return {"total_tokens": total, "uniform_lengths": f"{B} x ~{total // B}",
            "skew_lengths": f"1 x {skew[0]} + {B - 1} x 128",
            "uniform_us": round(us_u, 2), "skew_us": round(us_s, 2),
            "uniform_GB/s": round(decode_bytes(uniform) / us_u / 1e3, 1),
            "skew_GB/s": round(decode_bytes(skew) / us_s / 1e3, 1),
            "skew_penalty": round(us_s / us_u - 1, 4),
            "reference_skew_penalty_A100": 0.20}


# reference per-call figures on A100 (gqa_attention_decode.py:389-392: the
# three-op split/combine path per call; :604-608: the split-K decode kernel
# with unconditional partial stores)
REF_B1_THREE_OP_US = {64: 12.53, 256: 13.37, 1024: 13.43, 4095: 14.51}
REF_B1_SPLIT_US = {7: 4.74, 128: 7.22, 1024: 9.24, 8192: 14.14}


def b1_curve_bench(pkg, dev):
    """B=1 decode (one layer, one pool, graph of 8 back-to-back calls) at the
    context lengths the reference publishes: the one-launch step and the
    reference's three-op sequence (split + combine + gate pack)."""
    out = {}
    for L in sorted(set(REF_B1_THREE_OP_US) | set(REF_B1_SPLIT_US)):
        w1 = decode_workload([L], dev, seed=100 + L, contiguous=True)
        sc1 = pkg.allocate_split_scratch(HQ, D, batch=1, device=dev)
        g1 = w1["gate"][0].permute(1, 0, 2)

        def step1():
            return torch.ops.wy_lib.paged_gqa_attention_decode_fused(
                w1["q"], w1["kn"], w1["vn"], w1["kc"], w1["vc"], w1["bt"], w1["pos"], *sc1,
                sc1.counters, g1)

        def three1():
            ctx = pkg.call_paged_gqa_attention_decode_triton(
                w1["q"], w1["kn"], w1["vn"], w1["kc"], w1["vc"], w1["bt"], w1["pos"], tuple(sc1))
            return pkg.attention_gate_pack(ctx.permute(1, 0, 2).unsqueeze(0), w1["gate"])

        ms = time_graph(step1, 400, 40)
        ms3 = time_graph(three1, 400, 40)
        out[f"L{L}"] = {"us_one_launch": round(ms * 1e3, 2), "us_three_op": round(ms3 * 1e3, 2),
                        "ref_A100_three_op_us": REF_B1_THREE_OP_US.get(L),
                        "ref_A100_split_kernel_us": REF_B1_SPLIT_US.get(L)}
        del w1, sc1
    return out


def prefill_inputs(dev, lengths, seed):
    gen = torch.Generator(device=dev).manual_seed(seed)
    total = sum(lengths)

    def rnd(*shape):
        return torch.randn(*shape, device=dev, generator=gen).to(torch.bfloat16)

    q, k, v = rnd(total, HQ, D), rnd(total, HKV, D), rnd(total, HKV, D)
    cu_list = [0]
    for n in lengths:
        cu_list.append(cu_list[-1] + n)
    return q, k, v, torch.tensor(cu_list, dtype=torch.int32, device=dev)


def prefill_bench(pkg, dev, lengths, seed):
    """Varlen causal prefill kernel alone, graph-timed with steady clocks."""
    q, k, v, cu = prefill_inputs(dev, lengths, seed)
    total = sum(lengths)
    mx = max(lengths)

    def run():
        return pkg.gqa_attention_varlen_causal(q, k, v, cu, mx)

    ms = time_graph_events(run, 20)
    fl = prefill_flops(lengths)
    tf = fl / (ms * 1e-3) / 1e12
    min_bytes = total * (HQ * D * 2 * 2 + HKV * D * 2 * 2)
    attain = min(MFMA_BF16_PEAK_TFLOPS, fl / (min_bytes / (HBM_PEAK_GBS * 1e9)) / 1e12)
    log(f"prefill {len(lengths)} seqs total {total}: {ms*1e3:.1f} us {tf:.1f} TFLOP/s")
    return {"us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 2), "GFLOP": round(fl / 1e9, 3),
            "min_hbm_bytes": min_bytes,
            "frac_of_mfma_peak": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
            "attainable_TFLOP/s": round(attain, 1), "frac_of_attainable": round(tf / attain, 4),
            "total_tokens": total, "lengths": lengths if len(lengths) <= 32 else None}


def prefill_path_bench(pkg, dev, lengths, seed):
    """The prefill attention path of one layer after the q/k norm (engine/
    runner.py:336-384): RoPE q/k, varlen attention, gate pack, K/V page scatter.
    Timed as the reference's op sequence (6 launches incl. the .contiguous()
    copies) and as the two-launch attention block; both graph-timed."""
    gen = torch.Generator(device=dev).manual_seed(seed)
    T = sum(lengths)

    def rnd(*shape):
        return torch.randn(*shape, device=dev, generator=gen).to(torch.bfloat16)

    q, k, v, gate = rnd(T, HQ, D), rnd(T, HKV, D), rnd(T, HKV * D), rnd(T, HQ * D)
    packed = pkg.build_packed_batch(lengths, device=dev)
    max_pages = -(-max(lengths) // 16)
    num_pages = len(lengths) * max_pages
    bt = torch.randperm(num_pages, device=dev, generator=gen).view(
        len(lengths), max_pages).to(torch.int32)
    kc = torch.zeros(num_pages, HKV, 16, D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    inv = pkg.rope_inv_freq(64, 1e7, device=dev)
    ms_seq = time_graph_events(
        lambda: pkg.prefill_attention_packed(q, k, v, gate, inv, 64, packed, kc, vc, bt), 10)
    ms_blk = time_graph_events(
        lambda: pkg.prefill_attention_block(q, k, v, gate, inv, 64, packed, kc, vc, bt), 10)
    log(f"prefill path {len(lengths)} seqs total {T}: op sequence {ms_seq*1e3:.1f} us, "
        f"block {ms_blk*1e3:.1f} us")
    return {"op_sequence_us": round(ms_seq * 1e3, 2), "block_us": round(ms_blk * 1e3, 2),
            "total_tokens": T,
            "what": "after q/k norm: RoPE q/k + varlen attention + gate pack + K/V page "
                    "scatter; op sequence (reference order, 6 launches) vs the two-launch "
                    "prefill attention block (bit-identical)"}


def decoder_bench(pkg, dev):
    """The whole Qwen3.5 decode step (24 layers: 18 GDN + 6 attention, tied
    248320-word LM head with argmax) as one HIP graph replay, random weights
    of the checkpoint's shapes; attention contexts U[128, 2048] (config 2's
    distribution).  Reported next to the reference's own published decode
    step times (A100, README-EN.md:69-76)."""
    from qwen35_amd.decoder import DecodeModel, DecoderConfig, GraphedDecoder, random_weights
    cfg = DecoderConfig()
    weights = random_weights(cfg, seed=11, device=dev)
    ref_ms = {1: 2.010, 32: 4.662}
    out = {}
    for B in (1, 32):
        hid = torch.randn(B, cfg.hidden, device=dev).to(torch.bfloat16)
        ms = time_graph_events(lambda: pkg.lm_head_argmax(hid, weights[1], False), 10)
        nbytes = weights[1].numel() * 2
        out[f"lm_head_argmax B={B}"] = {
            "us": round(ms * 1e3, 2), "GB/s": round(nbytes / ms / 1e6, 1),
            "frac_of_hbm_peak": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4)}
        log(f"lm_head_argmax B={B}: {out[f'lm_head_argmax B={B}']}")
    for B in (1, 32):
        model = DecodeModel(cfg, weights, batch=B, max_len=2064, device=dev)
        gen = torch.Generator().manual_seed(2)
        lens = torch.randint(128, 2049, (B,), generator=gen)
        model.pos.copy_((lens - 1).to(dev))
        tok = torch.randint(0, cfg.vocab, (B,), generator=gen).to(dev)
        g = GraphedDecoder(model, tok)
        for _ in range(10):
            g.step()
        torch.cuda.synchronize()
        iters = 50
        st, en = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        st.record()
        for _ in range(iters):
            g.step()
        en.record()
        en.synchronize()
        ms = st.elapsed_time(en) / iters
        wbytes = sum(t.numel() * t.element_size() for w in model.layers
                     for t in (w.gate_up, w.down_proj, w.in_proj, w.out_proj))
        wbytes += weights[1].numel() * 2
        sbytes = sum(2 * t.numel() * t.element_size() for t in model.rec_states if t is not None)
        kvbytes = 6 * int((lens + 10).sum()) * 2048
        out[f"B={B}"] = {
            "ms_per_step": round(ms, 4), "tokens_per_s": round(B / ms * 1e3, 1),
            "reference_a100_ms_per_step": ref_ms[B],
            "speedup_vs_reference_a100": round(ref_ms[B] / ms, 2),
            "hbm_bytes_per_step": wbytes + sbytes + kvbytes,
            "GB/s": round((wbytes + sbytes + kvbytes) / ms / 1e6, 1)}
        log(f"decoder B={B}: {out[f'B={B}']}")
        if B == 32:
            # packed prefill of 32 x 128-token prompts into the same caches
            # (eager: the ops read cu_seqlens on the host, as the reference's do)
            lengths = [128] * 32
            ptoks = torch.randint(0, cfg.vocab, (sum(lengths),), generator=gen).to(dev)
            model.prefill(ptoks, lengths)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(3):
                model.prefill(ptoks, lengths)
            torch.cuda.synchronize()
            pms = (time.perf_counter() - t0) * 1e3 / 3
            out["prefill B=32 x T=128 (packed)"] = {
                "ms": round(pms, 3), "tokens_per_s": round(4096 / pms * 1e3, 1),
                "reference_a100_ms": 61.0,
                "what": "24 layers, wall clock incl. host dispatch; reference README-EN.md:88-96"}
            log(f"prefill 32x128: {out['prefill B=32 x T=128 (packed)']}")
        del g, model
        torch.cuda.empty_cache()
    return out


def gdn_bench(pkg, dev):
    """Gated DeltaNet recurrence (the linear-attention mixer, 16 heads of
    128 x 128 fp32 state): decode graph-timed as algorithmic HBM GB/s (state
    read + written once, q/k/v/out, beta/g), sequential prefill as tokens/s."""
    gen = torch.Generator(device=dev).manual_seed(5)
    H, DK, DV = 16, 128, 128

    def qkv(T):
        q = torch.nn.functional.normalize(torch.randn(T, H, DK, device=dev, generator=gen), dim=-1)
        k = torch.nn.functional.normalize(torch.randn(T, H, DK, device=dev, generator=gen), dim=-1)
        v = torch.randn(T, H, DV, device=dev, generator=gen)
        beta = torch.sigmoid(torch.randn(T, H, device=dev, generator=gen))
        g = -torch.nn.functional.softplus(torch.randn(T, H, device=dev, generator=gen))
        return ((q * DK ** -0.5).to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16),
                beta, g)

    out = {}
    for B in (1, 32, 256):
        q, k, v, beta, g = qkv(B)
        state = torch.randn(B, H, DK, DV, device=dev, generator=gen) * 0.1
        nbytes = B * H * (2 * DK * DV * 4 + (2 * DK + 2 * DV) * 2 + 8)
        ms = time_graph_events(lambda: pkg.gdn_recurrent_decode(q, k, v, beta, g, state), 20)
        out[f"gdn_recurrent_decode B={B}"] = {
            "us": round(ms * 1e3, 2), "GB/s": round(nbytes / ms / 1e6, 1),
            "frac_of_hbm_peak": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4), "bytes": nbytes}
    # the whole decode mixer between the fused projection and out_proj
    for B in (1, 32):
        HD = H * DK
        fused = torch.randn(B, 4 * HD + 2 * H, device=dev, generator=gen).to(torch.bfloat16)
        cs = torch.randn(B, 4, 3 * HD, device=dev, generator=gen).to(torch.bfloat16)
        cw = (torch.randn(4, 3 * HD, device=dev, generator=gen) * 0.5).to(torch.bfloat16)
        a_log = torch.log(torch.rand(H, device=dev, generator=gen) * 15 + 1)
        dt = torch.randn(H, device=dev, generator=gen).to(torch.bfloat16)
        nw = 1 + 0.1 * torch.randn(DK, device=dev, generator=gen)
        state = torch.randn(B, H, DK, DV, device=dev, generator=gen) * 0.1
        ms_blk = time_graph_events(
            lambda: pkg.gdn_decode_block(fused, cs, cw, a_log, dt, nw, state), 20)
        ms_ops = time_graph_events(
            lambda: pkg.gdn_decode_ops(fused, cs, cw, a_log, dt, nw, state), 20)
        nbytes = B * H * 2 * DK * DV * 4 + B * (4 * HD + 2 * H) * 2 + B * 2 * 4 * 3 * HD * 2 \
            + B * HD * 2
        out[f"gdn_decode_block B={B}"] = {
            "us": round(ms_blk * 1e3, 2), "op_sequence_us": round(ms_ops * 1e3, 2),
            "GB/s": round(nbytes / ms_blk / 1e6, 1),
            "frac_of_hbm_peak": round(nbytes / ms_blk / 1e6 / HBM_PEAK_GBS, 4),
            "what": "conv4 decode + q/k norm + gates + recurrence + gated RMSNorm, one launch "
                    "vs the 4-op sequence"}
    for lengths in ([128] * 32, [4096]):
        T = sum(lengths)
        q, k, v, beta, g = qkv(T)
        cu = torch.tensor([0] + torch.tensor(lengths).cumsum(0).tolist(), dtype=torch.int32,
                          device=dev)
        # the op reads cu_seqlens[-1] on the host (reference assertion): not capturable
        ms = time_events(lambda: pkg.gdn_recurrent_prefill_sequential(q, k, v, beta, g, cu), 5)
        name = f"gdn_recurrent_prefill_sequential {len(lengths)} x {lengths[0]}"
        out[name] = {"us": round(ms * 1e3, 2), "tokens/s": round(T / ms * 1e3, 1),
                     "us_per_token_step": round(ms * 1e3 / max(lengths), 4)}
    # one long prompt through the chunk-64 WY form (the runner's route for a
    # single sequence of >= 2048 tokens), stage by stage and as the chain
    for T in (4096, 16384):
        q, k, v, beta, g = qkv(T)
        ms = time_events(lambda: pkg.call_gdn_recurrent_prefill_chunked_triton(q, k, v, beta, g), 5)
        w, u, G = pkg.gdn_chunk_prepare_wy(k, v, beta, g)
        delta, cs, _ = pkg.gdn_chunk_state(k, w, u, G)
        st = {"prepare_wy": time_events(lambda: pkg.gdn_chunk_prepare_wy(k, v, beta, g), 5),
              "state": time_events(lambda: pkg.gdn_chunk_state(k, w, u, G), 5),
              "output": time_events(lambda: pkg.gdn_chunk_output(q, k, delta, G, cs), 5)}
        r = {"us": round(ms * 1e3, 2), "tokens/s": round(T / ms * 1e3, 1),
             "stage_us": {n: round(x * 1e3, 2) for n, x in st.items()}}
        if T == 4096:
            r["vs_sequential"] = round(out["gdn_recurrent_prefill_sequential 1 x 4096"]["us"]
                                       / r["us"], 2)
        out[f"gdn_recurrent_prefill_chunked 1 x {T}"] = r
    for name, r in out.items():
        log(f"gdn {name}: {r}")
    return out


def elementwise_bench(pkg, dev):
    """Config 3 (32 x 128 tokens): partial RoPE of q and k, the K/V page scatter
    and the sigmoid gate pack, graph-timed, as algorithmic HBM GB/s (every byte
    the op must read and write once)."""
    gen = torch.Generator(device=dev).manual_seed(3)
    T, nseq = 4096, 32

    def rnd(*shape):
        return torch.randn(*shape, device=dev, generator=gen).to(torch.bfloat16)

    q, k, v = rnd(T, HQ, D), rnd(T, HKV, D), rnd(T, HKV, D)
    pos_ids = torch.arange(128, device=dev).repeat(nseq).view(1, T)
    inv = pkg.rope_inv_freq(64, 1e7, device=dev)
    cu = torch.arange(0, T + 1, 128, dtype=torch.int32, device=dev)
    pages_per_seq = 128 // PAGE + 1
    num_pages = nseq * pages_per_seq
    bt = torch.randperm(num_pages, device=dev, generator=gen).view(nseq, pages_per_seq)
    bt = bt.to(torch.int32).contiguous()
    kc = torch.zeros(num_pages, HKV, PAGE, D, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    x4, g4 = rnd(1, HQ, T, D), rnd(1, HQ, T, D)
    cases = {
        "partial_rope q [1,8,4096,256] (permuted view)":
            (lambda: pkg.partial_rope(q.permute(1, 0, 2).unsqueeze(0), pos_ids, inv, 64),
             2 * T * HQ * D * 2),
        "partial_rope k [1,2,4096,256] (permuted view)":
            (lambda: pkg.partial_rope(k.permute(1, 0, 2).unsqueeze(0), pos_ids, inv, 64),
             2 * T * HKV * D * 2),
        "paged_kv_fill_varlen 32 x 128 tokens":
            (lambda: pkg.paged_kv_fill_varlen(kc, vc, k.permute(1, 0, 2), v.permute(1, 0, 2),
                                              bt, cu, 128),
             4 * T * HKV * D * 2),
        "attention_gate_pack [1,8,4096,256]":
            (lambda: pkg.attention_gate_pack(x4, g4), 3 * T * HQ * D * 2),
    }
    out = {}
    for name, (fn, nbytes) in cases.items():
        ms = time_graph_events(fn, 20)
        out[name] = {"us": round(ms * 1e3, 2), "GB/s": round(nbytes / ms / 1e6, 1),
                     "frac_of_hbm_peak": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4),
                     "bytes": nbytes}
        log(f"elementwise {name}: {out[name]}")
    return out


def gemm_bench(pkg, dev):
    """wy_lib::gemm_2d on the attention block's projection shapes, graph-timed,
    next to torch.nn.functional.linear (hipBLASLt) on the same tensors.  Decode
    shapes are HBM-bound (bytes = weight + x + y), prefill shapes MFMA-bound."""
    gen = torch.Generator(device=dev).manual_seed(7)
    shapes = [("decode B=32 q/gate/k/v fused [5120,1024]", 32, 5120, 1024),
              ("decode B=32 o_proj [1024,2048]", 32, 1024, 2048),
              ("decode B=1 q/gate/k/v fused [5120,1024]", 1, 5120, 1024),
              ("prefill T=4096 q_proj [2048,1024]", 4096, 2048, 1024),
              ("prefill T=4096 k_proj [512,1024]", 4096, 512, 1024),
              ("prefill T=4096 o_proj [1024,2048]", 4096, 1024, 2048),
              ("prefill T=4096 down_proj [1024,3584]", 4096, 1024, 3584),
              ("prefill T=4096 GDN in_proj [8224,1024]", 4096, 8224, 1024),
              ("prefill T=16384 [6144,1024]", 16384, 6144, 1024)]
    out = {}
    for name, M, N, K in shapes:
        x = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
        wt = torch.randn(N, K, device=dev, generator=gen).to(torch.bfloat16)
        ms = time_graph_events(lambda: pkg.gemm_2d(x, wt), 20)
        ms_ref = time_graph_events(lambda: torch.nn.functional.linear(x, wt), 20)
        fl, by = 2 * M * N * K, 2 * (M * K + N * K + M * N)
        rec = {"M": M, "N": N, "K": K, "us": round(ms * 1e3, 2),
               "hipblaslt_us": round(ms_ref * 1e3, 2)}
        if M <= 64:
            rec["GB/s"] = round(by / ms / 1e6, 1)
            rec["frac_of_hbm_peak"] = round(by / ms / 1e6 / HBM_PEAK_GBS, 4)
        else:
            rec["TFLOP/s"] = round(fl / ms / 1e9, 1)
            rec["frac_of_mfma_peak"] = round(fl / ms / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4)
        out[name] = rec
        log(f"gemm {name}: {rec}")
        del x, wt
    # the MLP's gate/up projection with SwiGLU in the GEMM epilogue
    # (wy_lib::gate_up_swiglu) vs gemm_2d then swiglu, and hipBLASLt's GEMM
    for name, M in (("gate_up+SwiGLU decode B=32 [7168,1024]", 32),
                    ("gate_up+SwiGLU prefill T=4096 [7168,1024]", 4096)):
        I, K = 3584, 1024
        x = torch.randn(M, K, device=dev, generator=gen).to(torch.bfloat16)
        wt = (torch.randn(2 * I, K, device=dev, generator=gen) * 0.05).to(torch.bfloat16)
        ms = time_graph_events(lambda: pkg.gate_up_swiglu(x, wt), 20)

        def two_ops():
            gu = pkg.gemm_2d(x, wt)
            return pkg.swiglu(gu[:, :I], gu[:, I:])
        ms2 = time_graph_events(two_ops, 20)
        ms_ref = time_graph_events(lambda: torch.nn.functional.linear(x, wt), 20)
        rec = {"M": M, "I": I, "K": K, "us": round(ms * 1e3, 2),
               "gemm_then_swiglu_us": round(ms2 * 1e3, 2),
               "hipblaslt_gemm_only_us": round(ms_ref * 1e3, 2)}
        out[name] = rec
        log(f"gemm {name}: {rec}")
        del x, wt
    return out


def _timed_median(fn, budget_s, min_reps=3):
    """Median seconds of fn over repetitions filling about budget_s (at least
    min_reps), after one untimed call."""
    fn()
    ts = []
    t_end = time.perf_counter() + budget_s
    while len(ts) < min_reps or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return median(ts), len(ts)


def cpu_baseline(w, lens):
    """The CPU oracle (fp32 torch restatement of the same math, the build's own
    port) on the whole config-2 decode step of one layer: gather of every
    sequence's pages, softmax(q K^T / 16) V per KV group.  All host cores
    (torch.set_num_threads(os.cpu_count())), median of the repetitions that
    fill ~10 s."""
    from oracle import attention_oracle as orc

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    q, kc, vc, bt = w["q"].cpu(), w["kc"].cpu(), w["vc"].cpu(), w["bt"].cpu()
    dt, reps = _timed_median(lambda: orc.paged_decode(q, kc, vc, bt, lens), 10.0)
    gbs = split_kernel_bytes(lens) / dt / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"one layer's decode attention of all 32 config-2 sequences "
                      f"(sum L={sum(lens)}); median of {reps} reps: {dt*1e3:.1f} ms "
                      f"(GPU: one launch of the same step)",
            "ms_per_sample": round(dt * 1e3, 3)}


def cpu_baseline_prefill(dev):
    """The CPU oracle's varlen causal attention on the whole config-3 batch
    (32 x 128 tokens, the same seeded inputs as the GPU leg), all host cores,
    median of the repetitions that fill ~10 s; TFLOP/s over the causal FLOPs."""
    from oracle import attention_oracle as orc

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    lengths = [128] * 32
    q, k, v, cu = prefill_inputs(dev, lengths, seed=3)
    q, k, v, cu = q.cpu(), k.cpu(), v.cpu(), cu.cpu()
    dt, reps = _timed_median(lambda: orc.varlen_causal(q, k, v, cu), 10.0)
    tf = prefill_flops(lengths) / dt / 1e12
    return {"value": round(tf, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"config 3 whole (32 x 128 tokens, {prefill_flops(lengths)/1e9:.3f} "
                      f"GFLOP); median of {reps} reps: {dt*1e3:.1f} ms",
            "ms_per_sample": round(dt * 1e3, 3)}


if __name__ == "__main__":
    main()
