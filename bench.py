#!/usr/bin/env python3
"""KHQ decode-attention benchmark (config 3: 32K context, 16 layers, batch 1).

One step = one decode token through the 16 full-attention layers: per layer
one two-region KHQ attention step (32,640 compressed tokens + 128 raw ring
tokens, H_q 24 / H_kv 4, D 256) over a packed payload resident in HBM (a
separate 28.7 MB payload per layer, 460 MB in total, so the 256 MB last-level
cache cannot hold the working set).  The payload is seeded uniform-random
packed codes with outlier counts ~U[0,50] (--data compressed: the library's
own compression of N(0,1) K/V rows, ~28 outliers per K row).  Prints one JSON
line.

    python bench.py [--steps K] [--warmup W] [--no-cpu] [--data uniform|compressed]

value = microseconds per layer-step (lower is better), timed with HIP events
over exactly K steps.  roofline = the compressed-region kernel alone, timed
with HIP events on its launch stream, against 8 TB/s.  cpu_baseline = the
CPU oracle (C restatement of the reference kernels, OpenMP) on one layer-step
of the same workload on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "bonsai-mojo-1bit-optimization-t4-cuda_amd"))

H_Q, H_KV, D = 24, 4, 256
ROW_BYTES = 220
HBM_PEAK_GBS = 8000.0
RING = 256
KERNEL_NAMES = {"auto": "attn_ws_kernel (compressed region)",
                "portable": "attn_part_kernel<6> (compressed region)"}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=16)
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--win", type=int, default=128)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--kernel", choices=["auto", "portable"], default="auto",
                    help="compressed-region kernel (library default: auto)")
    ap.add_argument("--data", choices=["uniform", "compressed"], default="uniform",
                    help="payload: seeded uniform-random packed codes with outlier counts "
                         "~U[0,50] (the config's data, default) or the library's compression "
                         "of N(0,1) K/V rows")
    ap.add_argument("--config", choices=["c1", "c2", "c3", "c4", "c5"], default="c3",
                    help="c1: the uncompressed fp16 GQA baseline over 512 positions; c2: "
                         "the 512-token two-region step (384 compressed + 128 raw); "
                         "c3: the headline 32K-context step (default); c4: 32 ragged "
                         "sequences per layer-step in one batched call; c5: a 128-token "
                         "chunked-prefill step after 8,192 tokens")
    ap.add_argument("--counters-run", action="store_true",
                    help="profiling aid for rocprofv3 --pmc: a 256 MiB device copy (the "
                         "calibration kernel of known size), then the compressed-region kernel "
                         "on 4 C3 layers, 3 times; prints no JSON")
    ap.add_argument("--prewarm", type=float, default=0.5,
                    help="seconds of untimed steps before the warmup steps (GPU clock ramp)")
    ap.add_argument("--graph-batches", type=int, default=0,
                    help="profiling aid: after the eager timing, replay the captured C3 step "
                         "in this many batches of 10 (no warm replays) and print each batch's "
                         "us per layer-step to stderr")
    ap.add_argument("--no-configs", action="store_true",
                    help="default run only: skip the short runs of configs 1, 2, 4 and 5 "
                         "reported under 'configs'")
    ap.add_argument("--no-sweep", action="store_true",
                    help="skip the C3 sweep of the reference entry sequence at splits "
                         "1/8/32/64 (launch_khq_attn_fp16 + window + merge, and the split-K "
                         "reduce alone)")
    return ap.parse_args()


def main():
    args = parse()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only; --gpus must be 1", file=sys.stderr)
        sys.exit(2)
    import torch

    from khq import _lib, ops, synth

    _lib.call("khq_select_kernel", ["auto", "portable"].index(args.kernel))
    if args.config in ("c1", "c2"):
        return print(json.dumps(bench_small(args)), flush=True)
    if args.config == "c4":
        return print(json.dumps(bench_c4(args)), flush=True)
    if args.config == "c5":
        return print(json.dumps(bench_c5(args)), flush=True)
    if args.counters_run:
        return counters_run(args)
    from khq.centroids import synthetic_layer

    dev = "cuda"
    c_len = args.ctx - args.win
    win_len = args.win
    scale = 1.0 / 16.0
    layers = []
    for l in range(args.layers):
        lc = synthetic_layer(l, seed=1234)
        pay = ops.Payload(c_len * H_KV, dev)
        cents = ops.Centroids(lc, dev)
        if args.data == "compressed":
            synth.compressed_rows(pay, cents, seed=1000 + l)
        else:
            rows = synth.random_rows(c_len * H_KV, seed=1000 + l, device=dev)
            for k, v in rows.items():
                getattr(pay, k).copy_(v)
            del rows
        g = torch.Generator(device=dev)
        g.manual_seed(5000 + l)
        ring_k = torch.randn((RING, H_KV, D), generator=g, device=dev).half()
        ring_v = torch.randn((RING, H_KV, D), generator=g, device=dev).half()
        q = synth.q_gate(H_Q, seed=7000 + l, device=dev)
        out = torch.empty((H_Q, D), device=dev, dtype=torch.float16)
        layers.append(dict(lc=lc, cents=cents, pay=pay, ring_k=ring_k,
                           ring_v=ring_v, q=q, out=out))
    torch.cuda.synchronize()
    win_start = c_len % RING
    stream = torch.cuda.current_stream()

    def step():
        for L in layers:
            ops.attn_step(L["q"], L["pay"], L["cents"], L["ring_k"], L["ring_v"], L["out"],
                          H_q=H_Q, H_kv=H_KV, c_len=c_len, win_start=win_start, win_len=win_len,
                          ring_cap=RING, scale=scale)

    prewarm(step, args.prewarm)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms_total = e0.elapsed_time(e1)
    ms_per_step = ms_total / args.steps
    us_layer_step = ms_per_step * 1000.0 / args.layers

    # dominant kernel alone: compressed-region partials, HIP events on its stream
    n_launch = args.steps * args.layers

    def partials_step():
        for L in layers:
            ops.attn_partials(L["q"], L["pay"], L["cents"], H_q=H_Q, H_kv=H_KV, c_len=c_len,
                              scale=scale)
    partials_step()
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(args.steps):
        for L in layers:
            ops.attn_partials(L["q"], L["pay"], L["cents"], H_q=H_Q, H_kv=H_KV, c_len=c_len,
                              scale=scale)
    e1.record(stream)
    torch.cuda.synchronize()
    kern_us = e0.elapsed_time(e1) * 1000.0 / n_launch
    c_bytes = c_len * H_KV * ROW_BYTES
    step_bytes = c_bytes + win_len * H_KV * D * 2 * 2
    kern_gbs = c_bytes / (kern_us * 1e-6) / 1e9
    step_gbs = step_bytes / (us_layer_step * 1e-6) / 1e9

    # the box's own copy bandwidth (device-to-device, 1 GiB read + 1 GiB
    # written per copy), reported beside the vendor peak
    xa = torch.empty(1 << 28, device=dev, dtype=torch.float32)
    xb = torch.empty_like(xa)
    xb.copy_(xa)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(5):
        xb.copy_(xa)
    e1.record(stream)
    torch.cuda.synchronize()
    copy_gbs = 5 * 2 * xa.numel() * 4 / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del xa, xb

    traffic = {}
    tname = {"auto": "attn_ws_c3_traffic.json"}
    tpath = os.path.join(ROOT, "profiles", tname.get(args.kernel, "none"))
    if os.path.exists(tpath) and c_len == 32640:
        with open(tpath) as f:
            traffic = json.load(f)
    result = {
        "metric": "KHQ decode attn us/layer-step @32K ctx + achieved HBM GB/s (% of peak)",
        "value": round(us_layer_step, 3),
        "unit": "us/layer-step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "prewarm_s": args.prewarm,
        "dtype": "f16-mfma/f32-acc",
        "data": ("synthetic: N(0,1) K/V rows compressed by the library's KHQ compressor, "
                 "N(0,1) fp16 ring" if args.data == "compressed" else
                 "synthetic: seeded uniform-random packed codes, outlier count ~U[0,50], "
                 "N(0,1) fp16 ring"),
        "config": {
            "workload": f"C3: {args.layers} layers x ({c_len} compressed + {win_len} raw) tokens, "
                        f"batch 1, H_q {H_Q} / H_kv {H_KV}, D {D}, fused two-region step",
            "ctx": args.ctx, "layers": args.layers, "c_len": c_len, "win_len": win_len,
            "parallelism": "1 GPU",
        },
        "hbm_gbps": round(step_gbs, 1),
        "hbm_pct_peak": round(100.0 * step_gbs / HBM_PEAK_GBS, 2),
        "bytes_per_layer_step": step_bytes,
        "roofline": {
            "bound": "hbm",
            "kernel": KERNEL_NAMES[args.kernel],
            "achieved": round(kern_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(kern_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic.get("traffic_bytes_scaled"),
            "traffic_fetch_factor": traffic.get("fetch_factor"),
            "avg_kernel_us": round(kern_us, 3),
            "bytes_per_launch": c_bytes,
            "measured_copy_gbps": round(copy_gbs, 1),
        },
    }

    if args.data == "uniform":
        # the same kernel on the library's compression of N(0,1) K/V rows
        L0 = layers[0]
        upay = ops.Payload(c_len * H_KV, dev)
        synth.compressed_rows(upay, L0["cents"], seed=99)
        ops.attn_partials(L0["q"], upay, L0["cents"], H_q=H_Q, H_kv=H_KV, c_len=c_len,
                          scale=scale)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(args.steps):
            ops.attn_partials(L0["q"], upay, L0["cents"], H_q=H_Q, H_kv=H_KV, c_len=c_len,
                              scale=scale)
        e1.record(stream)
        torch.cuda.synchronize()
        result["roofline"]["avg_kernel_us_compressed_gaussian_rows"] = round(
            e0.elapsed_time(e1) * 1000.0 / args.steps, 3)
        del upay

    if args.graph_batches:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step()
        torch.cuda.synchronize()
        for b in range(args.graph_batches):
            e0.record(stream)
            for _ in range(10):
                g.replay()
            e1.record(stream)
            torch.cuda.synchronize()
            print(f"graph replay batch {b}: {e0.elapsed_time(e1) * 100.0 / args.layers:.2f} "
                  "us/layer-step", file=sys.stderr, flush=True)
        del g
    # the same fused step replayed from a HIP graph (launch overhead off the
    # host), checked bit for bit against the eager outputs
    result["graph_layer_step_us"] = round(graph_us(step, args.steps, layers) / args.layers, 3)

    if not args.no_sweep:
        # the reference's launch sequence per layer (ref:src/khq/runtime.mojo:554-613):
        # launch_khq_attn_fp16 (split-K partials into out_partial + reduce),
        # launch_khq_window_attn_fp16, launch_khq_merge_gate_fp16; and the
        # split-K reduce (khq_attn_reduce_kernel's counterpart) timed alone
        sweep, reduce_us = {}, {}
        ac = torch.empty((H_Q, D + 2), device=dev)
        aw = torch.empty((H_Q, D + 2), device=dev)
        ap_ = torch.empty((H_Q, 64, D + 2), device=dev)
        for sp in (1, 8, 32, 64):
            part = ap_[:, :sp].contiguous() if sp > 1 else None

            def ref_step():
                for L in layers:
                    ops.attn(L["q"], L["pay"], L["cents"], ac, c_len=c_len, H_q=H_Q, H_kv=H_KV,
                             scale=scale, num_splits=sp, out_partial=part)
                    ops.window_attn(L["q"], L["ring_k"], L["ring_v"], aw, win_start=win_start,
                                    win_len=win_len, ring_cap=RING, H_q=H_Q, H_kv=H_KV,
                                    scale=scale)
                    ops.merge_gate(ac, aw, L["q"], L["out"], H_q=H_Q, has_w=True)
            sweep[f"splits_{sp}"] = round(graph_us(ref_step, args.steps, layers) / args.layers, 3)
            if sp > 1:
                def red_step():
                    for _ in layers:
                        ops.attn_reduce(part, ac, num_queries=H_Q, num_splits=sp)
                reduce_us[f"splits_{sp}"] = round(graph_us(red_step, args.steps) / args.layers, 3)
        result["reference_entry_us_per_layer_step"] = sweep
        result["split_reduce_us"] = reduce_us

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(layers[0], c_len, win_len, win_start, scale,
                                              args.cpu_seconds)
    if not args.no_configs and args.layers == 16 and args.ctx == 32768:
        del layers
        torch.cuda.synchronize()
        result["configs"] = other_configs(args)
    print(json.dumps(result), flush=True)


def other_configs(args):
    """Short runs of the other configurations (2, 4
    and 5), each with its own roofline and CPU baseline, for the default
    benchmark line: 16 layers each, fewer steps, smaller CPU samples."""
    import copy

    out = {}
    drop = ("n_gpus", "higher_is_better", "scaling", "vs_baseline")
    for name, fn, steps, warm in (("c1", bench_small, 10, 2), ("c2", bench_small, 10, 2),
                                  ("c4", bench_c4, 10, 2), ("c5", bench_c5, 2, 1)):
        a = copy.copy(args)
        a.config, a.steps, a.warmup = name, min(args.steps, steps), min(args.warmup, warm)
        a.cpu_seconds = min(args.cpu_seconds, 3.0)
        t0 = time.perf_counter()
        r = fn(a)
        r = {k: v for k, v in r.items() if k not in drop}
        r["wall_s"] = round(time.perf_counter() - t0, 1)
        out[name] = r
    return out


def prewarm(fn, seconds):
    """Untimed work before the warmup steps: the GPU's clocks ramp up over the
    first tens of milliseconds of sustained load (replays of one graph went
    from 33.8 to 31.8 us per layer-step over their first ~30 calls)."""
    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        fn()
        torch.cuda.synchronize()


def graph_us(step, reps, layers=None):
    """GPU time of one call of step(), in us: step's launches captured once
    into a HIP graph (after an eager call that sizes the library workspace)
    and replayed reps times between HIP events, so host issue overhead is not
    counted; replays for 0.2 s first (clock ramp).  When layers is given,
    every layer's output after the last replay must equal the eager call's
    bit for bit."""
    import torch

    step()
    torch.cuda.synchronize()
    want = [L["out"].clone() for L in layers] if layers else []
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    prewarm(g.replay, 0.2)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    for L, w in zip(layers or [], want):
        if not torch.equal(L["out"], w):
            raise RuntimeError("graph replay differs from the eager step")
    return e0.elapsed_time(e1) * 1000.0 / reps


def counters_run(args):
    """Fixed dispatch sequence for hardware-counter passes: one 256 MiB copy
    (read 256 MiB, write 256 MiB: the scale of FETCH_SIZE / WRITE_SIZE), then
    khq_attn_partials_fp16 on 4 distinct C3 layers, 3 rounds (12 dispatches)."""
    import torch

    from khq import ops, synth
    from khq.centroids import synthetic_layer

    dev = "cuda"
    c_len = args.ctx - args.win
    x = torch.empty(64 << 20, device=dev)
    y = torch.empty_like(x)
    x.fill_(1.0)
    torch.cuda.synchronize()
    y.copy_(x)
    layers = []
    for l in range(4):
        lc = synthetic_layer(l, seed=1234)
        pay = ops.Payload(c_len * H_KV, dev)
        for k, v in synth.random_rows(c_len * H_KV, seed=1000 + l, device=dev).items():
            getattr(pay, k).copy_(v)
        layers.append((pay, ops.Centroids(lc, dev), synth.q_gate(H_Q, seed=7000 + l, device=dev)))
    torch.cuda.synchronize()
    for _ in range(3):
        for pay, cents, q in layers:
            ops.attn_partials(q, pay, cents, H_q=H_Q, H_kv=H_KV, c_len=c_len, scale=1.0 / 16.0)
    torch.cuda.synchronize()
    print("counters run done", file=sys.stderr)


def bench_c5(args):
    """Config 5: per layer, 8,192 tokens already appended (boundary 8,064),
    then one chunk of 128 tokens at positions 8,192..8,319 through
    khq_layer_prefill: ring writes, the compression event at the 128th append,
    decode of the newly compressed rows, MFMA attention of 127 queries over
    8,064 compressed + 129..255 raw tokens and of the last query over 8,192 +
    128.  Each timed step runs the chunk on 16 fresh layer states (one per
    layer); the dense attention kernel is also timed alone (MFMA roofline)."""
    import numpy as np
    import torch

    from khq import layer as KL
    from khq import ops, synth
    from khq.centroids import synthetic_layer

    dev = "cuda"
    n0, chunk, scale = 8192, 128, 1.0 / 16.0
    n_layers = args.layers
    g = torch.Generator(device=dev)
    g.manual_seed(1234)

    def toks(n):
        k = torch.randn((n, H_KV, D), generator=g, device=dev).half()
        pos = torch.arange(n, device=dev)
        return k, synth.rope_halfsplit(k.float(), pos).half(), \
            torch.randn((n, H_KV, D), generator=g, device=dev).half(), \
            torch.randn((n, H_Q, 2 * D), generator=g, device=dev).half()

    k, kr, v, q = toks(n0 + chunk)
    k_c, kr_c, v_c, q_c = (x[n0:].contiguous() for x in (k, kr, v, q))
    opt = KL.KhqOptions(splits=16, fused=True)
    scratch = torch.empty((chunk, H_Q, D), device=dev, dtype=torch.float16)

    def fresh_layers(n):
        out = []
        for l in range(n):
            L = KL.NativeKhqLayer(synthetic_layer(l % 16, seed=1234), H_q=H_Q, H_kv=H_KV,
                                  cap=n0 + 256, device=dev, options=opt)
            for i in range(0, n0, chunk):
                L.prefill(q[i:i + chunk], kr[i:i + chunk], v[i:i + chunk], k[i:i + chunk],
                          scratch, scale)
            out.append(L)
        torch.cuda.synchronize()
        return out

    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    out = torch.empty((chunk, H_Q, D), device=dev, dtype=torch.float16)
    import gc

    def run_chunk(layers):
        for L in layers:
            L.prefill(q_c, kr_c, v_c, k_c, out, scale)

    for _ in range(args.warmup):
        run_chunk(fresh_layers(n_layers))
    ms = []
    n_steps = min(args.steps, 5)  # each step needs 16 freshly prefilled layer states
    for _ in range(n_steps):
        layers = fresh_layers(n_layers)
        # the previous step's layers are destroyed here, outside the timed
        # region (a destroy synchronizes the device and frees its buffers)
        gc.collect()
        torch.cuda.synchronize()
        e0.record(stream)
        run_chunk(layers)
        e1.record(stream)
        torch.cuda.synchronize()
        ms.append(e0.elapsed_time(e1))
        del layers
    ms_step = float(np.mean(ms))
    us_layer = ms_step * 1000.0 / n_layers
    attended = sum((8064 + 129 + j) if j < 127 else 8192 + 128 for j in range(chunk))
    flops = 2 * 2 * H_Q * D * attended
    # the dense attention kernel alone: 127 queries over 8,064 + 255 keys
    n_k, n_q = 8064 + 255, 127
    ld = ops.vt_ld(n_k)
    kd = torch.randn((n_k, H_KV, D), generator=g, device=dev).half()
    vt = torch.randn((H_KV, D, ld), generator=g, device=dev).half()
    qd = q_c[:n_q].contiguous()
    od = torch.empty((n_q, H_Q, D), device=dev, dtype=torch.float16)
    run = lambda: ops.prefill_attn(qd, kd, vt, od, ld_vt=ld, n_k=n_k, n_q=n_q, vis0=8064 + 129,
                                   H_q=H_Q, H_kv=H_KV, scale=scale)
    run()
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(20):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    attn_us = e0.elapsed_time(e1) * 1000.0 / 20
    # the attention kernel alone (partials into the workspace, no merge)
    run_p = lambda: ops.prefill_attn_partials(qd, kd, vt, ld_vt=ld, n_k=n_k, n_q=n_q,
                                              vis0=8064 + 129, H_q=H_Q, H_kv=H_KV, scale=scale)
    run_p()
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(20):
        run_p()
    e1.record(stream)
    torch.cuda.synchronize()
    attn_only_us = e0.elapsed_time(e1) * 1000.0 / 20
    attn_flops = 2 * 2 * H_Q * D * sum(8064 + 129 + j for j in range(n_q))
    result = {
        "metric": "KHQ chunked-prefill us/layer-step (128 queries, 8K context) + MFMA TFLOP/s",
        "value": round(us_layer, 3),
        "unit": "us/layer-step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16-in/f32-acc",
        "timed_steps": n_steps,
        "step_us_per_layer": [round(x * 1000.0 / n_layers, 1) for x in ms],
        "data": "synthetic: N(0,1) fp16 tokens, compressed by the library",
        "config": {
            "workload": f"C5: {n_layers} layers x one 128-token chunk at positions 8192..8319 "
                        "(compression event at the last append)",
            "layers": n_layers, "chunk": chunk, "context": n0, "parallelism": "1 GPU",
        },
        "tflops_layer_step": round(flops / (us_layer * 1e-6) / 1e12, 2),
        "roofline": {
            "bound": "mfma",
            "kernel": "prefill_attn_rs_kernel (127 queries x 24 heads over 8,319 keys)",
            "achieved": round(attn_flops / (attn_only_us * 1e-6) / 1e12, 2),
            "peak": 2500.0,
            "unit": "TFLOP/s",
            "frac": round(attn_flops / (attn_only_us * 1e-6) / 1e12 / 2500.0, 4),
            "traffic": None,
            "avg_kernel_us": round(attn_only_us, 3),
            "flops_per_launch": attn_flops,
            "with_merge_us": round(attn_us, 3),
            "with_merge_tflops": round(attn_flops / (attn_us * 1e-6) / 1e12, 2),
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_c5(args.cpu_seconds)
    return result


def bench_small(args):
    """Configs 1 and 2, small and launch-bound (reported in µs, with HBM GB/s
    for the record).  C1: the uncompressed fp16 GQA decode baseline
    (launch_khq_gqa_attn_fp16) over 512 cached positions per layer.  C2: the
    fused two-region step with 384 compressed rows (seeded uniform-random
    codes) and 128 raw ring tokens per layer."""
    import torch

    from khq import ops, synth
    from khq.centroids import synthetic_layer

    dev = "cuda"
    scale = 1.0 / 16.0
    layers = []
    for l in range(args.layers):
        g = torch.Generator(device=dev)
        g.manual_seed(400000 + l)
        q = synth.q_gate(H_Q, seed=500000 + l, device=dev)
        out = torch.empty((H_Q, D), device=dev, dtype=torch.float16)
        if args.config == "c1":
            k = torch.randn((512, H_KV, D), generator=g, device=dev).half()
            v = torch.randn((512, H_KV, D), generator=g, device=dev).half()
            layers.append((q, k, v, out))
        else:
            cents = ops.Centroids(synthetic_layer(l, seed=1234), dev)
            pay = ops.Payload(384 * H_KV, dev)
            for kk, vv in synth.random_rows(384 * H_KV, seed=600000 + l, device=dev).items():
                getattr(pay, kk).copy_(vv)
            rk = torch.randn((RING, H_KV, D), generator=g, device=dev).half()
            rv = torch.randn((RING, H_KV, D), generator=g, device=dev).half()
            layers.append((q, pay, cents, rk, rv, out))

    def step():
        for L in layers:
            if args.config == "c1":
                q, k, v, out = L
                ops.gqa_attn(q, k, v, out, seq_len=512, H_q=H_Q, H_kv=H_KV, scale=scale,
                             check=False)
            else:
                q, pay, cents, rk, rv, out = L
                ops.attn_step(q, pay, cents, rk, rv, out, H_q=H_Q, H_kv=H_KV, c_len=384,
                              win_start=384 % RING, win_len=128, ring_cap=RING, scale=scale,
                              check=False)

    prewarm(step, min(args.prewarm, 0.2))
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / args.steps
    us_layer = ms_step * 1000.0 / args.layers
    # The same step captured once as a HIP graph and replayed (how a serving
    # loop issues these launch-bound steps); the replayed outputs must equal
    # the eager ones bit for bit before the figure is reported.
    ops.workspace_reserve(64 << 20)
    eager_out = [L[-1].clone() for L in layers]
    for L in layers:
        L[-1].zero_()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    graph.replay()
    torch.cuda.synchronize()
    same = all(torch.equal(a, L[-1]) for a, L in zip(eager_out, layers))
    prewarm(graph.replay, min(args.prewarm, 0.2))
    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(args.steps):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    us_layer_graph = e0.elapsed_time(e1) * 1000.0 / args.steps / args.layers if same else None
    if args.config == "c1":
        nbytes = 512 * H_KV * D * 2 * 2
        workload = f"C1: {args.layers} layers x 512 fp16 cached positions, H_q 24 / H_kv 4, D 256"
        metric = "uncompressed fp16 GQA decode baseline us/layer-step (512 ctx)"
    else:
        nbytes = 384 * H_KV * 220 + 128 * H_KV * D * 2 * 2
        workload = (f"C2: {args.layers} layers x (384 compressed + 128 raw) tokens, "
                    "fused two-region step")
        metric = "KHQ decode attn us/layer-step @512 ctx"
    gbs = nbytes / (us_layer * 1e-6) / 1e9
    result = {
        "metric": metric, "value": round(us_layer, 3), "unit": "us/layer-step", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f16-in/f32-acc" if args.config == "c1" else "f16-mfma/f32-acc",
        "data": "synthetic: N(0,1) fp16 K/V" if args.config == "c1" else
                "synthetic: seeded uniform-random packed codes, N(0,1) fp16 ring",
        "config": {"workload": workload, "layers": args.layers, "parallelism": "1 GPU"},
        "bytes_per_layer_step": nbytes,
        "roofline": {"bound": "hbm", "kernel": "whole layer-step (launch-bound)",
                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": None,
        "graph_replay": {"us_per_layer_step": None if us_layer_graph is None else
                         round(us_layer_graph, 3),
                         "outputs_equal_eager": same,
                         "note": "the 16-layer step captured as one HIP graph and replayed; "
                                 "value is the eager launch loop"},
    }
    if not args.no_cpu:
        if args.config == "c1":
            q, k, v, _ = layers[0]
            result["cpu_baseline"] = cpu_baseline_c1(q, k, v, scale, args.cpu_seconds)
        else:
            q, pay, cents, rk, rv, _ = layers[0]
            L0 = dict(pay=pay, lc=synthetic_layer(0, seed=1234), q=q, ring_k=rk, ring_v=rv)
            result["cpu_baseline"] = cpu_baseline(L0, 384, 128, 384 % RING, scale,
                                                  args.cpu_seconds)
    return result


def bench_c4(args):
    """Config 4: 32 independent sequences, contexts L_i ~ U[1024, 16384]
    (seeded), boundary_i = 128 floor((L_i - 128) / 128), window L_i - boundary_i
    raw tokens, one query token per sequence, all layers.  One layer-step = one
    khq_attn_step_batched_fp16 call over the 32 sequences; also timed: the same
    work as 32 single-sequence calls."""
    import numpy as np
    import torch

    from khq import ops, synth
    from khq.centroids import synthetic_layer

    dev = "cuda"
    n_seq = 32
    rng = np.random.default_rng(1234)
    lens = rng.integers(1024, 16385, n_seq)
    bounds = [128 * ((int(L) - 128) // 128) for L in lens]
    wins = [int(L) - b for L, b in zip(lens, bounds)]
    scale = 1.0 / 16.0
    layers = []
    for l in range(args.layers):
        cents = ops.Centroids(synthetic_layer(l, seed=1234), dev)
        seqs = []
        for i in range(n_seq):
            c_len, wl = bounds[i], wins[i]
            pay = ops.Payload(c_len * H_KV, dev)
            rows = synth.random_rows(c_len * H_KV, seed=100000 * l + i, device=dev)
            for k, v in rows.items():
                getattr(pay, k).copy_(v)
            del rows
            g = torch.Generator(device=dev)
            g.manual_seed(200000 * l + i)
            seqs.append(dict(q_gate=synth.q_gate(H_Q, seed=300000 * l + i, device=dev), pay=pay,
                             ring_k=torch.randn((RING, H_KV, D), generator=g, device=dev).half(),
                             ring_v=torch.randn((RING, H_KV, D), generator=g, device=dev).half(),
                             out=torch.empty((H_Q, D), device=dev, dtype=torch.float16),
                             c_len=c_len, win_start=c_len % RING, win_len=wl, ring_cap=RING))
        layers.append((cents, seqs))
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    per_step = {}

    def timed(fn):
        prewarm(fn, min(args.prewarm, 0.2))
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
        ev[0].record(stream)
        for i in range(args.steps):
            fn()
            ev[i + 1].record(stream)
        torch.cuda.synchronize()
        per_step[fn.__name__] = [round(ev[i].elapsed_time(ev[i + 1]) * 1000.0 / args.layers, 1)
                                 for i in range(args.steps)]
        return ev[0].elapsed_time(ev[-1]) / args.steps  # ms per step (all layers)

    def batched():
        for cents, seqs in layers:
            ops.attn_step_batched(seqs, cents, H_q=H_Q, H_kv=H_KV, scale=scale)

    def one_by_one():
        for cents, seqs in layers:
            for s in seqs:
                ops.attn_step(s["q_gate"], s["pay"], cents, s["ring_k"], s["ring_v"], s["out"],
                              H_q=H_Q, H_kv=H_KV, c_len=s["c_len"], win_start=s["win_start"],
                              win_len=s["win_len"], ring_cap=RING, scale=scale)

    ms_b = timed(batched)
    ms_s = timed(one_by_one)
    us_b = ms_b * 1000.0 / args.layers
    step_bytes = sum(b * H_KV * ROW_BYTES + w * H_KV * D * 2 * 2 for b, w in zip(bounds, wins))
    gbs = step_bytes / (us_b * 1e-6) / 1e9
    result = {
        "metric": "KHQ batched decode attn us/layer-step (32 ragged sequences)",
        "value": round(us_b, 3),
        "unit": "us/layer-step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_b, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16-mfma/f32-acc",
        "data": "synthetic: seeded uniform-random packed codes, outlier count ~U[0,50], "
                "N(0,1) fp16 rings",
        "config": {
            "workload": f"C4: {args.layers} layers x {n_seq} sequences, L ~ U[1024,16384] "
                        f"(sum {int(sum(lens))} tokens), one query token each",
            "layers": args.layers, "n_seq": n_seq, "tokens": int(sum(lens)),
            "parallelism": "1 GPU",
        },
        "hbm_gbps": round(gbs, 1),
        "hbm_pct_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "bytes_per_layer_step": step_bytes,
        "sequential_calls_us_per_layer_step": round(ms_s * 1000.0 / args.layers, 3),
        "per_step_us_per_layer_step": per_step["batched"],
        "roofline": {"bound": "hbm", "kernel": "whole batched layer-step (argument upload, "
                     "attn_ws_batched_kernel, step_finish_batched_kernel)",
                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        cents0, seqs0 = layers[0]
        result["cpu_baseline"] = cpu_baseline_c4(seqs0, synthetic_layer(0, seed=1234), scale,
                                                 args.cpu_seconds)
    return result


def cpu_baseline_c1(q, k, v, scale, budget_s):
    """Config 1's CPU path: the oracle's restatement of the host attention of
    ref:src/models/qwen3_5/attention.mojo:97-201 (fp32, softmax over 512
    positions, sigmoid gate), timed single-threaded and with OpenMP over query
    heads on the host's cores."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    qh, kh, vh = q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy()
    res = {}
    for threads in (1, max(1, min(16, os.cpu_count() or 1))):
        oracle.set_num_threads(threads)
        reps, t0 = 0, time.perf_counter()
        while True:
            oracle.gqa_host(qh, kh, vh, seq_len=512, H_q=H_Q, H_kv=H_KV, scale=scale)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget_s / 2 or reps >= 2000:
                break
        res[threads] = el / reps * 1e6
    nt = max(res)
    return {"value": round(res[nt], 1), "unit": "us/layer-step", "cores": nt,
            "single_thread_us": round(res[1], 1), "host_nproc": os.cpu_count(),
            "kind": "port",
            "sample": "layer 0 of the same workload (512 positions, 24/4 heads), repeated; "
                      "value with OpenMP over query heads, single_thread_us on one core"}


def _oracle_decode_step(oracle, rows, h, lc, q, rk, rv, c_len, win_start, win_len, scale):
    """One decode layer-step through the CPU oracle: compressed attention at
    the BONSAI_KHQ_SPLITS default, raw window, merge and gate."""
    from khq.layer import split_count

    _, ac, _ = oracle.attn(q, rows["kpay"], rows["vpay"], rows["vsm"], rows["kmask"],
                           rows["knorm"], rows["krn"], rows["vnorm"], rows["vrn"],
                           h["cents_k"], h["cents_v"], h["vq"], h["rotor_k"], h["rotor_v"],
                           h["d_k"], h["d_v"], num_queries=H_Q, num_heads=H_Q, L_q=1,
                           c_len=c_len, n_rep=H_Q // H_KV, scale=scale, alpha_k=lc.alpha_k,
                           alpha_v=lc.alpha_v, rope_base=1e7, start_pos=0,
                           num_splits=split_count(c_len, 16))
    _, aw = oracle.window_attn(q, rk, rv, win_start=win_start, win_len=win_len, ring_cap=RING,
                               H_q=H_Q, H_kv=H_KV, scale=scale)
    oracle.merge_gate(ac, aw, q, H_q=H_Q, has_w=True)


def _payload_np(pay, n_rows):
    import numpy as np

    rows = {k: getattr(pay, k)[:n_rows].cpu().numpy()
            for k in ("kmask", "kpay", "knorm", "krn", "vpay", "vnorm", "vrn", "vsm")}
    rows["kmask"] = rows["kmask"].view(np.uint32)
    return rows


def cpu_baseline_c4(seqs, lc, scale, budget_s):
    """Config 4's CPU path: the oracle's decode step per sequence (layer 0),
    sequences taken in order until the time budget is spent; the value is
    that time scaled to all 32 sequences by their compressed and raw bytes."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    threads = max(1, min(16, os.cpu_count() or 1))
    oracle.set_num_threads(threads)
    h = lc.fp16()

    def nbytes(s):
        return s["c_len"] * H_KV * ROW_BYTES + s["win_len"] * H_KV * D * 2 * 2

    done, el, t0 = 0, 0.0, time.perf_counter()
    for s in seqs:
        rows = _payload_np(s["pay"], s["c_len"] * H_KV)
        q = s["q_gate"].cpu().numpy()
        rk, rv = s["ring_k"].cpu().numpy(), s["ring_v"].cpu().numpy()
        t1 = time.perf_counter()
        _oracle_decode_step(oracle, rows, h, lc, q, rk, rv, s["c_len"], s["win_start"],
                            s["win_len"], scale)
        el += time.perf_counter() - t1
        done += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    frac = sum(nbytes(s) for s in seqs[:done]) / sum(nbytes(s) for s in seqs)
    return {"value": round(el / frac * 1e6, 1), "unit": "us/layer-step", "cores": threads,
            "host_nproc": os.cpu_count(), "kind": "port",
            "sample": f"{done} of the {len(seqs)} sequences of layer 0 through the oracle's "
                      f"decode step (OpenMP over query head x split), scaled to all "
                      f"{len(seqs)} by bytes ({100 * frac:.1f}% sampled)"}


def cpu_baseline_c5(budget_s):
    """Config 5's CPU path: the reference answers a chunk of queries one decode
    step at a time, so the oracle's decode step (8,064 compressed rows of
    seeded uniform-random codes plus the raw window, layer 0 constants) is
    timed for successive queries of the chunk until the budget is spent and
    scaled to the chunk's 128 queries (the compression event's own cost, 128
    rows once per chunk, is not counted)."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    from khq import ops, synth
    from khq.centroids import synthetic_layer

    threads = max(1, min(16, os.cpu_count() or 1))
    oracle.set_num_threads(threads)
    lc = synthetic_layer(0, seed=1234)
    h = lc.fp16()
    c_len = 8064
    rows = {k: v.numpy() for k, v in synth.random_rows(c_len * H_KV, seed=77, device="cpu").items()}
    rows["kmask"] = rows["kmask"].view(np.uint32)
    rng = np.random.default_rng(78)
    rk = rng.standard_normal((RING, H_KV, D)).astype(np.float16)
    rv = rng.standard_normal((RING, H_KV, D)).astype(np.float16)
    q = rng.standard_normal((H_Q, 2 * D)).astype(np.float16)
    done, t0 = 0, time.perf_counter()
    while True:
        j = done % 127
        _oracle_decode_step(oracle, rows, h, lc, q, rk, rv, c_len, c_len % RING, 129 + j, scale=1 / 16)
        done += 1
        el = time.perf_counter() - t0
        if el >= budget_s or done >= 128:
            break
    return {"value": round(el / done * 128 * 1e6, 1), "unit": "us/layer-step", "cores": threads,
            "host_nproc": os.cpu_count(), "kind": "port",
            "sample": f"{done} decode step(s) of the chunk's queries (8,064 compressed rows + "
                      f"129.. raw) through the oracle, scaled to 128 queries"}


def cpu_baseline(L, c_len, win_len, win_start, scale, budget_s):
    """Times the CPU oracle on one layer-step of the same workload (layer 0)."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    from khq.layer import split_count

    threads = max(1, min(16, os.cpu_count() or 1))
    oracle.set_num_threads(threads)
    pay = L["pay"]
    rows = {k: getattr(pay, k).cpu().numpy() for k in
            ("kmask", "kpay", "knorm", "krn", "vpay", "vnorm", "vrn", "vsm")}
    rows["kmask"] = rows["kmask"].view(np.uint32)
    h = L["lc"].fp16()
    q = L["q"].cpu().numpy()
    rk, rv = L["ring_k"].cpu().numpy(), L["ring_v"].cpu().numpy()
    n_sp = split_count(c_len, 16)  # BONSAI_KHQ_SPLITS default
    reps, t0 = 0, time.perf_counter()
    while True:
        _, ac, _ = oracle.attn(q, rows["kpay"], rows["vpay"], rows["vsm"], rows["kmask"],
                               rows["knorm"], rows["krn"], rows["vnorm"], rows["vrn"],
                               h["cents_k"], h["cents_v"], h["vq"], h["rotor_k"], h["rotor_v"],
                               h["d_k"], h["d_v"], num_queries=H_Q, num_heads=H_Q, L_q=1,
                               c_len=c_len, n_rep=H_Q // H_KV, scale=scale,
                               alpha_k=L["lc"].alpha_k, alpha_v=L["lc"].alpha_v,
                               rope_base=1e7, start_pos=0, num_splits=n_sp)
        _, aw = oracle.window_attn(q, rk, rv, win_start=win_start, win_len=win_len,
                                   ring_cap=RING, H_q=H_Q, H_kv=H_KV, scale=scale)
        oracle.merge_gate(ac, aw, q, H_q=H_Q, has_w=True)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 50:
            break
    return {"value": round(el / reps * 1e6, 1), "unit": "us/layer-step", "cores": threads,
            "host_nproc": os.cpu_count(), "kind": "port",
            "sample": f"{reps} layer-step(s) of layer 0 at the same shape "
                      f"({c_len} compressed + {win_len} raw, splits {n_sp}), OpenMP over "
                      f"(query head x split)"}


if __name__ == "__main__":
    main()
