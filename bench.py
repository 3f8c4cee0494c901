"""Benchmark of the AdaptiveIMI sparse-decode path on one MI355X.

Workload (BASELINE.json configs[1] attention path): 32 Llama-3-8B-shaped
layers (8 KV heads, 32 q heads, head_dim 128, bf16) at a 131072-token
context with the config-0 key/value distributions (synthetic), static window
32 + 64 tokens, IMI 2 x 64 centroids per subspace, 10 Lloyd iterations,
budget 0.1.  One step = the retrieval + gather + attention of every layer for
one decode token; the metric is decode steps/s per layer.

Prints ONE JSON line (rank 0).  Index-build time, per-kernel durations,
roofline and the CPU baseline are fields of the same line, and so are the
legs on other shapes: online index maintenance, the host tier, a configs[3]
and a configs[4] slice (two layers each) and the end-to-end model run.

`--workload config3` / `config4` run the same measurement on the other
single-GPU configurations of BASELINE.json (their parity cases are in the
tests): a 16-layer slice of a Qwen2.5-72B attention shape, batch 2 x 262144
tokens, 4-way IMI 4 x 32 centroids, a fixed budget of 4096 tokens; and 32
Llama-3-8B layers at 1,048,576 tokens, IMI 2 x 128 centroids, 20 Lloyd
iterations on a 65536-key sample then one full assignment, budget 0.02.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0  # MI355X HBM3E, vendor figure
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, vendor figure (no sparsity)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# BASELINE.json configurations that fit one GPU: layers, context, KV heads per
# sequence, query heads per KV head, centroids per subspace, Lloyd iterations,
# budget ratio (None: fixed_tokens), sequences, k-means sample (0: all keys)
WORKLOADS = {
    "config1": dict(layers=32, context=131072, kv_heads=8, groups=4, ks=(64, 64), iters=10, budget=0.1,
                    fixed_tokens=0, batch=1, sample=0),
    "config2": dict(layers=28, context=131072, kv_heads=4, groups=7, ks=(64, 64), iters=10, budget=0.1,
                    fixed_tokens=0, batch=4, sample=0, contexts=(32768, 65536, 98304, 131072)),
    "config3": dict(layers=16, context=262144, kv_heads=8, groups=8, ks=(32, 32, 32, 32), iters=10, budget=None,
                    fixed_tokens=4096, batch=2, sample=0),
    "config4": dict(layers=32, context=1048576, kv_heads=8, groups=4, ks=(128, 128), iters=20, budget=0.02,
                    fixed_tokens=0, batch=1, sample=65536),
}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--workload", choices=sorted(WORKLOADS), default="config1")
    p.add_argument("--layers", type=int, default=None)
    p.add_argument("--context", type=int, default=None)
    p.add_argument("--static-start", type=int, default=32)
    p.add_argument("--static-end", type=int, default=64)
    p.add_argument("--kv-heads", type=int, default=None)
    p.add_argument("--groups", type=int, default=None)
    p.add_argument("--k", type=int, default=None, help="centroids per subspace")
    p.add_argument("--iters", type=int, default=None)
    p.add_argument("--kmeans-init", choices=("first", "kmeans++"), default="first",
                   help="index-build seeding: the first k keys (as BASELINE.json specifies) or the reference's kmeans++")
    p.add_argument("--budget", type=float, default=None)
    p.add_argument("--cpu-baseline", type=int, default=1)
    p.add_argument("--cpu-seconds", type=float, default=40.0,
                   help="time bound of the CPU baseline leg (decode steps, then full index builds of layer 0)")
    p.add_argument("--no-graph", action="store_true")
    p.add_argument("--online-layers", type=int, default=4,
                   help="layers of the online-index-maintenance leg (async_update: batch 16, threshold 16, "
                        "512-token ring, 1024 decode keys); 0 skips it")
    p.add_argument("--host-tier-layers", type=int, default=2,
                   help="layers of the host-tier leg (lists in pinned host memory, GPU block cache of "
                        "round(n_centroids * 0.05) clusters x 2 pages); 0 skips it")
    p.add_argument("--config3-layers", type=int, default=2,
                   help="layers of the configs[3] leg (4-way 32^4 IMI, 2 x 8 KV heads at 262,144 tokens, GQA 8, "
                        "fixed 4,096-token budget): step and selection per layer; 0 skips it")
    p.add_argument("--config4-layers", type=int, default=2,
                   help="layers of the configs[4] leg (2 x 128 IMI at 1,048,576 tokens, 8 KV heads, GQA 4, "
                        "20 Lloyd iterations on a 65,536-key sample then one full assignment, budget 0.02): "
                        "index build, step and selection per layer; 0 skips it")
    p.add_argument("--e2e-layers", type=int, default=32,
                   help="end-to-end leg: a random-init Llama-3-8B-shaped model of this many layers prefills "
                        "--e2e-context tokens through the drop-in cache (index built on the side stream during "
                        "the prefill) and decodes --e2e-decode tokens greedily (0: skip; configs[1] only)")
    p.add_argument("--e2e-context", type=int, default=131072)
    p.add_argument("--e2e-decode", type=int, default=256)
    p.add_argument("--e2e-only", action="store_true", help="run only the end-to-end leg and print its JSON")
    p.add_argument("--copy-probe-mb", type=int, default=0,
                   help="run a device-to-device copy of this many MiB (3 times) before the timed region, as the "
                        "known-size reference for FETCH_SIZE / WRITE_SIZE counter runs")
    args = p.parse_args()
    w = dict(WORKLOADS[args.workload])
    w.setdefault("contexts", None)
    for name in ("layers", "context", "kv_heads", "groups", "iters", "budget"):
        if getattr(args, name) is not None:
            w[name] = getattr(args, name)
    if args.k is not None:
        w["ks"] = (args.k,) * len(w["ks"])
    for name, v in w.items():
        setattr(args, name, v)
    if args.workload != "config1":
        args.cpu_baseline = 0      # the CPU baseline is quoted on the default workload
        args.online_layers = 0
        args.host_tier_layers = 0
        args.config3_layers = 0
        args.config4_layers = 0
        if not args.e2e_only:
            args.e2e_layers = 0
    return args


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only (sharding over GPUs is a design, not "
                                   "code), so --gpus must be 1"}))
        sys.exit(2)
    import numpy as np
    import torch

    from adaptiveimi_amd import ops, synthetic
    from adaptiveimi_amd.sizing import decode_sizing

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.e2e_only:
        print(json.dumps({"e2e": e2e_leg(args)}), flush=True)
        return
    H, G, D, L = args.kv_heads * args.batch, args.groups, 128, args.layers   # H: KV heads of every sequence
    static_total = args.static_start + args.static_end
    T = args.context - static_total
    ks = tuple(args.ks)
    parts = len(ks)
    ncells = math.prod(ks)
    ratio = args.budget if args.budget is not None else args.fixed_tokens / T
    sz = decode_sizing(T, ratio, subspace_parts=parts, k_override=ks)
    if args.fixed_tokens:
        sz["max_tokens"] = args.fixed_tokens
        sz["buffer_pages"] = max(32, -(-args.fixed_tokens // sz["page_size"]))
    bud = ops.Budget(sz["nprobe"], sz["max_tokens"], sz["buffer_pages"])
    static_cap = static_total + 256
    static_len = static_total + 1   # one generated token in the steady zone
    log(f"[bench] {args.workload}: layers={L} context={args.context} T={T} heads={H} ks={ks} nprobe={bud.nprobe} "
        f"max_tokens={bud.max_tokens} buffer_pages={bud.buffer_pages}")

    # ---------------------------------------------------------- index build
    plans, build_ms = [], []
    start_ev = torch.cuda.Event(enable_timing=True)
    end_ev = torch.cuda.Event(enable_timing=True)
    keep_first = None
    head_tokens = H * T   # listed tokens over all KV heads (index-build roofline)
    if args.contexts:
        plans, build_ms, head_tokens = build_ragged(args, ks, static_total, static_cap, static_len, start_ev, end_ev)
    for layer in range(0 if args.contexts else L):
        keys, values = synthetic.make_kv(H, args.context, seed=1000 + layer, device="cuda")
        mid_k = keys[:, args.static_start:args.context - args.static_end]
        mid_v = values[:, args.static_start:args.context - args.static_end]
        steady_k = torch.zeros((H, static_cap, D), dtype=torch.bfloat16, device=dev)
        steady_v = torch.zeros_like(steady_k)
        steady_k[:, :args.static_start] = keys[:, :args.static_start]
        steady_k[:, args.static_start:static_total] = keys[:, args.context - args.static_end:]
        steady_v[:, :args.static_start] = values[:, :args.static_start]
        steady_v[:, args.static_start:static_total] = values[:, args.context - args.static_end:]
        steady_k[:, static_total] = keys[:, -1]
        steady_v[:, static_total] = values[:, -1]
        torch.cuda.synchronize()
        start_ev.record()
        if args.sample:
            cent, labels, _ = ops.kmeans_sampled(mid_k, list(ks), args.iters, args.sample, init=args.kmeans_init)
        else:
            cent, labels, _ = ops.kmeans(mid_k, list(ks), args.iters, init=args.kmeans_init)
        if parts == 4:   # selection over the occupied cells (compact ids)
            idx = ops.build_index(mid_k, mid_v, cent, labels, list(ks), compact=True, merged=False,
                                  n_centroids=min(T, ncells) + 1)
        else:
            idx = ops.build_index(mid_k, mid_v, cent, labels, list(ks), compact=False)
        end_ev.record()
        torch.cuda.synchronize()
        build_ms.append(start_ev.elapsed_time(end_ev))
        q = synthetic.make_queries(mid_k, G, seed=layer)[0]
        plan = ops.DecodePlan(cent, idx["cell_count"], idx["cell_offset"], ks, bud, idx["list_keys"],
                              idx["list_values"], steady_k, steady_v, G, query=q.contiguous(),
                              compact=idx if parts == 4 else None)
        plan.set_static_len(static_len)
        plans.append(plan)
        if layer == 0 and args.cpu_baseline:
            keep_first = dict(keys=mid_k.cpu(), values=mid_v.cpu(), cent=cent.cpu(), q=q.cpu(),
                              steady_k=steady_k.cpu(), steady_v=steady_v.cpu(), idx={k: v.cpu() for k, v in idx.items()})
        del keys, values, mid_k, mid_v, labels
        if layer % 8 == 7:
            log(f"[bench] built {layer + 1}/{L} layers, last build {build_ms[-1]:.2f} ms")
    torch.cuda.synchronize()

    if args.copy_probe_mb > 0:
        src = torch.empty(args.copy_probe_mb << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    def run_step():
        for p in plans:
            p.step()

    # -------------------------------------------------- graph of one step
    def capture(fn):
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        return g

    run_step()
    torch.cuda.synchronize()
    graph = None if args.no_graph else capture(run_step)

    def one_step():
        if graph is not None:
            graph.replay()
        else:
            run_step()

    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()
    t0.record()
    for _ in range(args.steps):
        one_step()
    t1.record()
    torch.cuda.synchronize()
    total_ms = t0.elapsed_time(t1)
    ms_per_step = total_ms / args.steps
    layer_steps_per_s = args.steps * L / (total_ms / 1e3)
    log(f"[bench] timed {args.steps} steps: {ms_per_step:.3f} ms/step ({ms_per_step / L * 1e3:.2f} us/layer)")

    # attended rows -> algorithmic bytes (K and V, bf16, 128 dims)
    rows = sum(int(p.selection["n_rows"].sum().item()) + H * static_len for p in plans)
    bytes_per_step = rows * 2 * D * 2
    bytes_per_layer = bytes_per_step / L

    # ------------------- per-launch durations: HIP events around graphs that
    # hold only one phase of every layer (back-to-back launches on one stream,
    # so host launch gaps do not enter); the selection the attention graph
    # reads is the one the last full step left in each plan's workspace.
    def per_launch_us(phase, reps):
        g = capture(lambda: [p.step(phases=phase) for p in plans])
        g.replay()
        torch.cuda.synchronize()
        t0.record()
        for _ in range(reps):
            g.replay()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) * 1e3 / (reps * L)

    reps = max(args.steps, 5)
    sel_us = per_launch_us(1, reps)
    att_us = per_launch_us(2, reps)      # split pass + merge
    split_us = per_launch_us(4, reps)    # attention_kernel alone (the kernel that moves the bytes)
    merge_us = per_launch_us(8, reps)    # merge_kernel alone
    achieved = bytes_per_layer / (split_us * 1e-6) / 1e9
    achieved_am = bytes_per_layer / (att_us * 1e-6) / 1e9
    step_gbps = bytes_per_layer / (ms_per_step / L * 1e-3) / 1e9
    log(f"[bench] per launch: select {sel_us:.2f} us, attention+merge {att_us:.2f} us "
        f"(attention_kernel {split_us:.2f} us, merge_kernel {merge_us:.2f} us)")

    online = None
    if args.online_layers > 0:
        online = online_update_leg(args, ks, bud, static_total, capture)
        log(f"[bench] online update: {online}")

    host_tier = None
    if args.host_tier_layers > 0:
        host_tier = host_tier_leg(args, ks, bud, static_total)
        log(f"[bench] host tier: {host_tier}")

    config3 = None
    if args.config3_layers > 0:
        config3 = config3_leg(args, capture)
        log(f"[bench] configs[3] leg: {config3}")

    config4 = None
    if args.config4_layers > 0:
        config4 = config4_leg(args, capture)
        log(f"[bench] configs[4] leg: {config4}")

    used_graph = graph is not None
    e2e = None
    if args.e2e_layers > 0:
        del plans, graph
        torch.cuda.empty_cache()
        try:
            e2e = e2e_leg(args)
        except (RuntimeError, ValueError) as exc:   # reported in the line; the decode-path figures stand
            e2e = {"error": f"{type(exc).__name__}: {exc}"[:300]}
        log(f"[bench] end-to-end leg: {e2e}")

    # ----------------------------------------------------- CPU baseline
    cpu = None
    if keep_first is not None:
        cpu = cpu_baseline(keep_first, ks, bud, static_len, args.cpu_seconds, args.iters)

    result = {
        "metric": "sparse-decode steps/s per layer @128k, budget 0.1; index-build ms; % HBM peak",
        "value": round(layer_steps_per_s, 1),
        "unit": "decode steps/s per layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (config-0 key/value distributions, seeded)",
        "config": {
            "workload": workload_name(args, L, H, G, ks),
            "layers": L, "context": args.context, "kv_heads": H, "q_heads": H * G, "static_window": static_total,
            "nprobe": bud.nprobe, "max_tokens": bud.max_tokens, "buffer_pages": bud.buffer_pages,
            "hip_graph": used_graph, "kmeans_init": args.kmeans_init,
        },
        "index_build_ms": {"per_layer_median": round(statistics.median(build_ms), 3),
                           "per_layer_min": round(min(build_ms), 3), "layers": L},
        "index_build_roofline": build_roofline(args, head_tokens, T, ks, statistics.median(build_ms)),
        "us_per_layer_step": round(ms_per_step / L * 1e3, 3),
        "attended_rows_per_layer": rows / L,
        "hbm_frac_step": round(step_gbps / HBM_PEAK_GBPS, 4),
        "kernels_us": {"select_kernel": round(sel_us, 2), "attention_kernel": round(split_us, 2),
                       "merge_kernel": round(merge_us, 2), "attention_kernel+merge_kernel": round(att_us, 2)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": measured_traffic(workload_name(args, L, H, G, ks)),
                     "kernel": "attention split pass: gather + GQA split-K attention (fixed_attention_kernel, "
                               "fixed row windows, at configs[1]; attention_kernel, row-balanced, elsewhere)",
                     "bytes_per_launch": int(bytes_per_layer),
                     "with_merge": {"achieved": round(achieved_am, 1), "frac": round(achieved_am / HBM_PEAK_GBPS, 4),
                                    "kernels": "attention_kernel + merge_kernel"}},
        "cpu_baseline": cpu,
        "online_update": online,
        "host_tier": host_tier,
        "config3": config3,
        "config4": config4,
        "e2e": e2e,
    }
    print(json.dumps(result), flush=True)


def workload_name(args, L, H, G, ks):
    imi = "x".join(str(k) for k in ks)
    budget = f"budget {args.budget}" if args.budget is not None else f"fixed budget {args.fixed_tokens} tokens"
    sample = f" on a {args.sample}-key sample + full assignment" if args.sample else ""
    if args.workload == "config1":
        head = f"configs[1] attention path: {L} Llama-3-8B layers"
    elif args.workload == "config2":
        head = (f"configs[2] attention path: {L} Qwen2.5-7B layers, ragged batch of {len(args.contexts)} sequences "
                f"({'/'.join(str(c) for c in args.contexts)} tokens) in one launch per layer")
    elif args.workload == "config3":
        head = f"configs[3] attention path: {L}-layer Qwen2.5-72B attention slice, batch {args.batch}"
    else:
        head = f"configs[4] attention path: {L} Llama-3-8B layers"
    return (f"{head} ({H} KV heads, GQA {G}, d128) at {args.context} tokens, IMI {imi}, {args.iters} Lloyd "
            f"iters{sample}, {budget}")


def e2e_leg(args):
    """End-to-end configs[1]: a random-init Llama-3-8B-shaped
    model (hidden 4096, 32 q / 8 KV heads, head_dim 128, FFN 14336, vocab
    128256, N(0, 0.02) bf16 weights, RMSNorm, rotate-half RoPE theta 500000)
    prefills a prompt of uniform random token ids and decodes greedily, with
    the drop-in cache driven as model_hub does (prefill.py:33-105: per layer
    prefill_update_kv_cache, prefill attention over the returned K / V, sync;
    base.py:324-350, 407-499: prepare_cache, then per layer
    decode_update_kv_cache + imi_decode_attn).  The cache takes the reference
    JSON's settings (config/Llama-3-8B-Instruct-Gradient-1048k.json: static
    32 + 64, pages_per_cluster 2, cache_ratio 0.05, budget 0.1, 32 buffer
    clusters, 20 Lloyd iterations, kmeans++ seeding) with BASELINE's IMI 2 x
    64, or at 1M tokens 2 x 128 on a 65536-key sample.  Each
    layer's index build runs on the cache's side stream while the following
    layers prefill.  The same prefill without the cache gives the build time
    the prefill does not hide.  Prefill attention is torch's flash SDPA (the
    reference uses flash_attn; out of this build's scope); the model's GEMMs
    are torch's."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    from adaptiveimi_amd import ops
    from adaptiveimi_amd.attn_hub.sparse_imi import imi_decode_attn
    from adaptiveimi_amd.cache_hub.adaptive_imi import adpimi_cache

    dev = torch.device("cuda:0")
    L, S, steps = args.e2e_layers, args.e2e_context, args.e2e_decode
    HID, HQ, HKV, D, FFN, VOC = 4096, 32, 8, 128, 14336, 128256
    eps, theta, chunk = 1e-5, 500000.0, 16384
    bf = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(7)

    def w(*shape):
        return torch.randn(shape, generator=g, device=dev, dtype=bf).mul_(0.02)

    embed, lm_head, norm = w(VOC, HID), w(VOC, HID), torch.ones(HID, dtype=bf, device=dev)
    layers = [dict(wqkv=w((HQ + 2 * HKV) * D, HID), wo=w(HID, HQ * D), w13=w(2 * FFN, HID), w2=w(HID, FFN),
                   ln1=torch.ones(HID, dtype=bf, device=dev), ln2=torch.ones(HID, dtype=bf, device=dev))
              for _ in range(L)]
    # RoPE angles of every position in fp64, kept as fp32 cos / sin tables
    inv = theta ** (-torch.arange(0, D // 2, dtype=torch.float64, device=dev) * 2.0 / D)
    ang = torch.arange(S + steps, dtype=torch.float64, device=dev)[:, None] * inv[None, :]
    cos_t, sin_t = ang.cos().float(), ang.sin().float()
    del ang

    def rms(x, wt):
        return F.rms_norm(x, (HID,), wt, eps)

    def rope(x, pos):   # x [n, heads, D], pos [n]
        c, s_ = cos_t[pos][:, None, :], sin_t[pos][:, None, :]
        x1, x2 = x[..., : D // 2].float(), x[..., D // 2:].float()
        return torch.cat([x1 * c - x2 * s_, x2 * c + x1 * s_], dim=-1).to(bf)

    def qkv_of(x, W, pos):
        n = x.shape[0]
        q = torch.empty((n, HQ, D), dtype=bf, device=dev)
        k = torch.empty((n, HKV, D), dtype=bf, device=dev)
        v = torch.empty((n, HKV, D), dtype=bf, device=dev)
        for s0 in range(0, n, chunk):
            e = min(n, s0 + chunk)
            t = rms(x[s0:e], W["ln1"]) @ W["wqkv"].t()
            q[s0:e] = rope(t[:, : HQ * D].view(e - s0, HQ, D), pos[s0:e])
            k[s0:e] = rope(t[:, HQ * D: (HQ + HKV) * D].view(e - s0, HKV, D), pos[s0:e])
            v[s0:e] = t[:, (HQ + HKV) * D:].view(e - s0, HKV, D)
        return q, k, v

    def mlp_(x, W):   # x += MLP(rms(x)), in token chunks
        for s0 in range(0, x.shape[0], chunk):
            e = min(x.shape[0], s0 + chunk)
            gu = rms(x[s0:e], W["ln2"]) @ W["w13"].t()
            x[s0:e] += (F.silu(gu[:, :FFN]) * gu[:, FFN:]) @ W["w2"].t()

    def logits_argmax(x):
        return (rms(x, norm) @ lm_head.t()).float().argmax(-1)

    def prefill(ids, cache, nl):
        n = ids.shape[0]
        pos = torch.arange(n, device=dev)
        x = embed[ids]
        for li in range(nl):
            W = layers[li]
            q, k, v = qkv_of(x, W, pos)
            kk, vv = k[None], v[None]                          # [1, S, H, D]
            if cache is not None:
                kk, vv = cache.prefill_update_kv_cache(q[None], kk, vv, li, 0)
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
                o = F.scaled_dot_product_attention(q.transpose(0, 1)[None].contiguous(),
                                                   kk.transpose(1, 2).contiguous(), vv.transpose(1, 2).contiguous(),
                                                   is_causal=True, enable_gqa=True)
            del q, k, v, kk, vv
            x += o[0].transpose(0, 1).reshape(n, HQ * D) @ W["wo"].t()
            del o
            if cache is not None:
                cache.sync(li, 0)
            mlp_(x, W)
        return logits_argmax(x[-1:])

    def decode(tok, pos, cache):
        x = embed[tok]
        for li, W in enumerate(layers):
            t = rms(x, W["ln1"]) @ W["wqkv"].t()
            q = rope(t[:, : HQ * D].view(1, HQ, D), pos)
            k = rope(t[:, HQ * D: (HQ + HKV) * D].view(1, HKV, D), pos)
            kk, vv = k.view(1, 1, HKV, D), t[:, (HQ + HKV) * D:].view(1, 1, HKV, D)
            cache.decode_update_kv_cache(kk, vv, li)
            o = imi_decode_attn(q.view(1, 1, HQ, D), kk, vv, li, cache)
            x = x + o.view(1, HQ * D) @ W["wo"].t()
            mlp_(x, W)
        return logits_argmax(x)

    four_m = S > 524288
    kcfg = {"k1": 128, "k2": 128, "sample_keys": 65536} if four_m else {"k1": 64, "k2": 64}
    kcfg.update(max_iters=20, tol=5e-4, early_stop_min_iter=20, early_stop_rel_tol=5e-4, init="kmeans++")
    ids = torch.randint(0, VOC, (S,), generator=g, device=dev)
    log(f"[e2e] {L} layers, {S}-token prompt, {steps} decode tokens; warm-up prefill of one layer")
    prefill(ids, None, 1)          # kernel selection / code loading of every prefill op
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    prefill(ids, None, L)
    torch.cuda.synchronize()
    plain_s = time.perf_counter() - t0
    log(f"[e2e] prefill without the index: {plain_s:.3f} s")
    torch.cuda.empty_cache()
    cache = adpimi_cache(valid_start=[0], layer_num=L, batch_size=1, max_length=S + steps, num_key_value_heads=HKV,
                         num_heads=HQ, head_dim=D, dtype=bf, layer_mapping={str(i): "cuda:0" for i in range(L)},
                         max_new_length=steps, input_length=S, static_pattern_start=32, static_pattern_end=64,
                         core=22, pages_per_cluster=2, retrieval_budget=0.02 if four_m else 0.1, cache_ratio=0.05,
                         buffer_cluster_num=32, prefill_bsz=1, num_gpus=1, model_size=8, subspace_parts=2,
                         runtime_config={"kmeans": kcfg})
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    tok = prefill(ids, cache, L)
    cache.prepare_cache()
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    log(f"[e2e] prefill with the index build: {prefill_s:.3f} s")
    # the same build alone (layer 0's listed keys and values as the input)
    lk0, lv0 = cache.list_keys[0][0, :, : cache.list_capacity], cache.list_values[0][0, :, : cache.list_capacity]
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    alone = []
    for _ in range(3):
        e0.record()
        km = dict(tol=5e-4, early_stop_min_iter=20, early_stop_rel_tol=5e-4, init="kmeans++")
        if four_m:
            cent, lab, _ = ops.kmeans_sampled(lk0, [kcfg["k1"], kcfg["k2"]], 20, kcfg["sample_keys"], **km)
        else:
            cent, lab, _ = ops.kmeans(lk0, [kcfg["k1"], kcfg["k2"]], 20, **km)
        ops.build_index(lk0, lv0, cent, lab, [kcfg["k1"], kcfg["k2"]], compact=False)
        e1.record()
        torch.cuda.synchronize()
        alone.append(e0.elapsed_time(e1))
    del lk0, lv0, cent, lab
    pos = torch.arange(S, S + steps, device=dev)
    out = [tok]
    t0 = time.perf_counter()
    for i in range(steps - 1):
        tok = decode(tok, pos[i:i + 1], cache)
        out.append(tok)
    torch.cuda.synchronize()
    decode_s = time.perf_counter() - t0
    ntok = steps - 1
    toks = torch.cat(out).tolist()
    res = {"model": "random-init Llama-3-8B shape (hidden 4096, 32 q / 8 KV heads, d128, FFN 14336, vocab 128256)",
           "layers": L, "context": S, "decode_tokens": steps, "imi": "2x128, 65536-key sample" if four_m else "2x64",
           "budget": 0.02 if four_m else 0.1, "kmeans": "kmeans++ seeding, 20 Lloyd iterations",
           "prefill_s": round(prefill_s, 3), "prefill_without_index_s": round(plain_s, 3),
           "exposed_index_build_ms_per_layer": round((prefill_s - plain_s) * 1e3 / L, 2),
           "index_build_alone_ms_per_layer": round(min(alone), 2),
           "decode_ms_per_token": round(decode_s * 1e3 / max(ntok, 1), 3),
           "decode_tokens_per_s": round(ntok / decode_s, 2) if ntok else None,
           "end2end_s": round(prefill_s + decode_s, 3), "nprobe": cache.nprobe,
           "max_tokens": cache.max_retrieval_tokens, "buffer_pages": cache.buffer_size,
           "first_tokens": toks[:8], "distinct_tokens": len(set(toks)),
           "clock": "host wall clock with device synchronisation around the prefill (index build included) and "
                    "around the decode loop (eager launches)"}
    del cache, layers, embed, lm_head
    torch.cuda.empty_cache()
    return res


def online_update_leg(args, ks, bud, static_total, capture):
    """The decode step with the reference's async update on (async_update.py:
    batch 16, threshold 16, 512-token delta ring) after 1024 generated keys,
    on the first online_layers layers (same seeds as the main run): time of
    imi_update_assign / imi_update_refresh per call, and the per-layer step
    with replaced centroids and delta rows against the same layers' plain
    step.  Decode keys are prompt keys drawn at random (a new token's key
    resembles the context's)."""
    import torch

    from adaptiveimi_amd import ops, synthetic

    dev = torch.device("cuda:0")
    H, G, D, NL = args.kv_heads, args.groups, 128, args.online_layers
    batch, thr, ring, gen = 16, 16, 512, 1024
    ncells = ks[0] * ks[1]
    static_cap = static_total + gen + 8
    static_len = static_total + gen
    exec_rows = bud.buffer_pages * bud.page_size + static_cap - static_len
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    plain, online, keep = [], [], []
    g = torch.Generator(device="cpu").manual_seed(11)
    for layer in range(NL):
        keys, values = synthetic.make_kv(H, args.context, seed=1000 + layer, device="cuda")
        mid_k = keys[:, args.static_start:args.context - args.static_end]
        mid_v = values[:, args.static_start:args.context - args.static_end]
        cent, labels, _ = ops.kmeans(mid_k, list(ks), args.iters)
        idx = ops.build_index(mid_k, mid_v, cent, labels, list(ks), compact=True, merged=True, n_centroids=ncells + 1)
        sk = torch.zeros((H, static_cap, D), dtype=torch.bfloat16, device=dev)
        sv = torch.zeros_like(sk)
        sk[:, :args.static_start] = keys[:, :args.static_start]
        sk[:, args.static_start:static_total] = keys[:, args.context - args.static_end:]
        sv[:, :static_total] = torch.cat([values[:, :args.static_start], values[:, args.context - args.static_end:]], 1)
        pick = torch.randint(0, mid_k.shape[1], (gen,), generator=g).to(dev)
        sk[:, static_total:static_len] = mid_k[:, pick]
        sv[:, static_total:static_len] = mid_v[:, pick]
        upd = ops.OnlineUpdate(idx["compact_centroids"], idx["compact_size"], idx["compact_gid"], idx["n_active"],
                               ncells, thr, ring, n_index=ncells, index_by_gid=True)
        for b in range(gen // batch):
            upd.assign(sk, static_total + b * batch, batch)
            upd.refresh(batch)
        q = synthetic.make_queries(mid_k, G, seed=layer)[0].contiguous()
        for lst, u in ((plain, None), (online, upd)):
            pl = ops.DecodePlan(cent, idx["cell_count"], idx["cell_offset"], ks, bud, idx["list_keys"],
                                idx["list_values"], sk, sv, G, query=q, update=u)
            pl.set_static_len(static_len)
            pl.set_exec_rows(exec_rows)
            lst.append(pl)
        keep.append((upd, idx, cent, sk, sv))
        del keys, values, labels
    def graph_us(fn, per):
        gr = capture(fn)
        for _ in range(3):
            gr.replay()
        torch.cuda.synchronize()
        ev0.record()
        for _ in range(20):
            gr.replay()
        ev1.record()
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) * 1e3 / (20 * per)

    res = {}
    for name, lst in (("plain", plain), ("online", online)):
        for p_ in lst:
            p_.step()
        res[name] = [round(graph_us(lambda: [p_.step(phases=ph) for p_ in lst], NL), 2) for ph in (3, 1, 2)]
    repl = sum(int(k[0].upd_n.sum().item()) for k in keep) / (NL * H)
    drows = sum(int(p_.selection["n_delta"].sum().item()) for p_ in online) / (NL * H)
    # the update kernels per call (graph replays: no host enqueue gaps); the
    # replays keep updating the state, which only changes what they time
    last = static_total + gen - batch
    assign_us = graph_us(lambda: [k[0].assign(k[3], last, batch) for k in keep], NL)
    refresh_us = graph_us(lambda: [k[0].refresh(batch) for k in keep], NL)
    return {"layers": NL, "decode_keys": gen, "batch": batch, "threshold": thr, "ring": ring,
            "assign_us": round(assign_us, 2), "refresh_us": round(refresh_us, 2),
            "us_per_layer_step": res["online"][0], "select_us": res["online"][1], "attention_merge_us": res["online"][2],
            "plain_us_per_layer_step": res["plain"][0], "plain_select_us": res["plain"][1],
            "plain_attention_merge_us": res["plain"][2],
            "replaced_cells_per_head": round(repl, 1), "delta_rows_per_head": round(drows, 1)}


def config3_leg(args, capture):
    """The configs[3] decode step (the reference's default 4-way IMI, 32^4
    cells, over a batch of 2 sequences x 8 KV heads at 262,144 tokens, GQA 8,
    fixed 4,096-token budget) on config3_layers layers: per layer-step time
    of the graphed step, and per launch of the selection alone (graph of the
    selection phase of every layer), as the main run times configs[1]."""
    import torch

    from adaptiveimi_amd import ops, synthetic
    from adaptiveimi_amd.sizing import decode_sizing

    w = WORKLOADS["config3"]
    dev = torch.device("cuda:0")
    H, G, D, NL = w["kv_heads"] * w["batch"], w["groups"], 128, args.config3_layers
    ks = tuple(w["ks"])
    static_total = args.static_start + args.static_end
    T = w["context"] - static_total
    sz = decode_sizing(T, w["fixed_tokens"] / T, subspace_parts=len(ks), k_override=ks)
    bud = ops.Budget(sz["nprobe"], w["fixed_tokens"], max(32, -(-w["fixed_tokens"] // sz["page_size"])))
    static_cap, static_len = static_total + 256, static_total + 1
    ncells = min(T, math.prod(ks))
    plans = []
    for layer in range(NL):
        keys, values = synthetic.make_kv(H, w["context"], seed=3000 + layer, device="cuda")
        mid_k = keys[:, args.static_start:w["context"] - args.static_end]
        mid_v = values[:, args.static_start:w["context"] - args.static_end]
        sk = torch.zeros((H, static_cap, D), dtype=torch.bfloat16, device=dev)
        sv = torch.zeros_like(sk)
        sk[:, :static_total] = torch.cat([keys[:, :args.static_start], keys[:, w["context"] - args.static_end:]], 1)
        sv[:, :static_total] = torch.cat([values[:, :args.static_start],
                                          values[:, w["context"] - args.static_end:]], 1)
        sk[:, static_total] = keys[:, -1]
        sv[:, static_total] = values[:, -1]
        cent, labels, _ = ops.kmeans(mid_k, list(ks), w["iters"], init=args.kmeans_init)
        idx = ops.build_index(mid_k, mid_v, cent, labels, list(ks), compact=True, merged=False,
                              n_centroids=ncells + 1)
        q = synthetic.make_queries(mid_k, G, seed=layer)[0]
        plan = ops.DecodePlan(cent, idx["cell_count"], idx["cell_offset"], ks, bud, idx["list_keys"],
                              idx["list_values"], sk, sv, G, query=q.contiguous(), compact=idx)
        plan.set_static_len(static_len)
        plans.append(plan)
        del keys, values, mid_k, mid_v, labels
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def per_layer_us(fn, reps):
        g = capture(fn)
        g.replay()
        torch.cuda.synchronize()
        ev0.record()
        for _ in range(reps):
            g.replay()
        ev1.record()
        torch.cuda.synchronize()
        return ev0.elapsed_time(ev1) * 1e3 / (reps * NL)

    reps = max(args.steps, 5)
    step_us = per_layer_us(lambda: [p.step() for p in plans], reps)
    sel_us = per_layer_us(lambda: [p.step(phases=1) for p in plans], reps)
    rows = sum(int(p.selection["n_rows"].sum().item()) for p in plans) / NL
    del plans
    torch.cuda.empty_cache()
    return {"layers": NL, "kv_heads": H, "q_heads": H * G, "context": w["context"], "ks": list(ks),
            "nprobe": bud.nprobe, "max_tokens": bud.max_tokens, "buffer_pages": bud.buffer_pages,
            "us_per_layer_step": round(step_us, 2), "select_us": round(sel_us, 2),
            "attended_rows_per_layer": rows,
            "clock": "HIP events around graphs of every layer's step (or its selection phase)"}


def config4_leg(args, capture):
    """The configs[4] index build and decode step (2 x 128 IMI over 8 KV heads
    at 1,048,576 tokens, GQA 4: 20 Lloyd iterations on an evenly strided
    65,536-key sample, then one assignment of every key, budget 0.02) on
    config4_layers layers: the build per layer on HIP events around it, and
    per layer-step times of graphs of every layer's step and of its
    selection and split-pass phases, as the main run times configs[1]."""
    import torch

    from adaptiveimi_amd import ops, synthetic
    from adaptiveimi_amd.sizing import decode_sizing

    w = WORKLOADS["config4"]
    dev = torch.device("cuda:0")
    H, G, D, NL = w["kv_heads"], w["groups"], 128, args.config4_layers
    ks = tuple(w["ks"])
    static_total = args.static_start + args.static_end
    T = w["context"] - static_total
    sz = decode_sizing(T, w["budget"], subspace_parts=len(ks), k_override=ks)
    bud = ops.Budget(sz["nprobe"], sz["max_tokens"], sz["buffer_pages"])
    static_cap, static_len = static_total + 256, static_total + 1
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    plans, build_ms = [], []
    for layer in range(NL):
        keys, values = synthetic.make_kv(H, w["context"], seed=4000 + layer, device="cuda")
        mid_k = keys[:, args.static_start:w["context"] - args.static_end]
        mid_v = values[:, args.static_start:w["context"] - args.static_end]
        sk = torch.zeros((H, static_cap, D), dtype=torch.bfloat16, device=dev)
        sv = torch.zeros_like(sk)
        sk[:, :static_total] = torch.cat([keys[:, :args.static_start], keys[:, w["context"] - args.static_end:]], 1)
        sv[:, :static_total] = torch.cat([values[:, :args.static_start],
                                          values[:, w["context"] - args.static_end:]], 1)
        sk[:, static_total] = keys[:, -1]
        sv[:, static_total] = values[:, -1]
        torch.cuda.synchronize()
        e0.record()
        cent, labels, _ = ops.kmeans_sampled(mid_k, list(ks), w["iters"], w["sample"], init=args.kmeans_init)
        idx = ops.build_index(mid_k, mid_v, cent, labels, list(ks), compact=False)
        e1.record()
        torch.cuda.synchronize()
        build_ms.append(e0.elapsed_time(e1))
        q = synthetic.make_queries(mid_k, G, seed=layer)[0]
        plan = ops.DecodePlan(cent, idx["cell_count"], idx["cell_offset"], ks, bud, idx["list_keys"],
                              idx["list_values"], sk, sv, G, query=q.contiguous())
        plan.set_static_len(static_len)
        plans.append(plan)
        del keys, values, mid_k, mid_v, labels
    torch.cuda.synchronize()

    def per_layer_us(fn, reps):
        g = capture(fn)
        g.replay()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / (reps * NL)

    reps = max(args.steps, 5)
    step_us = per_layer_us(lambda: [p.step() for p in plans], reps)
    sel_us = per_layer_us(lambda: [p.step(phases=1) for p in plans], reps)
    split_us = per_layer_us(lambda: [p.step(phases=4) for p in plans], reps)
    rows = sum(int(p.selection["n_rows"].sum().item()) + H * static_len for p in plans) / NL
    del plans
    torch.cuda.empty_cache()
    gbps = rows * 2 * D * 2 / (split_us * 1e-6) / 1e9
    return {"layers": NL, "kv_heads": H, "q_heads": H * G, "context": w["context"], "ks": list(ks),
            "kmeans": f"{w['iters']} Lloyd iterations on a {w['sample']}-key sample, then every key",
            "nprobe": bud.nprobe, "max_tokens": bud.max_tokens, "buffer_pages": bud.buffer_pages,
            "index_build_ms_per_layer": round(statistics.median(build_ms), 2),
            "us_per_layer_step": round(step_us, 2), "select_us": round(sel_us, 2),
            "split_pass_us": round(split_us, 2), "attended_rows_per_layer": rows,
            "split_pass_hbm_frac": round(gbps / 8000.0, 4),
            "clock": "HIP events around each build and around graphs of every layer's step (or one phase)"}


def host_tier_leg(args, ks, bud, static_total):
    """The decode step with the lists in pinned host memory and the
    reference's GPU block cache (wave_buffer_cpu_hotcold.cpp, sized as
    runtime.py:48-53 with the shipped configs' cache_ratio 0.05 and
    pages_per_cluster 2), on the first host_tier_layers layers (same seeds as
    the main run).  Host-synchronous like the reference's step (the selected
    cells go to the host), so it is timed on the host clock: the first step
    of each layer (every page a miss) and 10 steps with the same query after
    it (hits where the cache holds the cells)."""
    import time

    import torch

    from adaptiveimi_amd import ops, synthetic

    dev = torch.device("cuda:0")
    H, G, D, NL = args.kv_heads, args.groups, 128, args.host_tier_layers
    ncells = ks[0] * ks[1]
    cache_pages = ops.host_cache_pages(ncells + 1, bud.nprobe)
    static_cap = static_total + 8
    plans, cold, warm = [], [], []
    for layer in range(NL):
        keys, values = synthetic.make_kv(H, args.context, seed=1000 + layer, device="cuda")
        mid_k = keys[:, args.static_start:args.context - args.static_end]
        mid_v = values[:, args.static_start:args.context - args.static_end]
        cent, labels, _ = ops.kmeans(mid_k, list(ks), args.iters)
        idx = ops.build_index(mid_k, mid_v, cent, labels, list(ks), compact=False)
        sk = torch.zeros((H, static_cap, D), dtype=torch.bfloat16, device=dev)
        sv = torch.zeros_like(sk)
        sk[:, :args.static_start] = keys[:, :args.static_start]
        sk[:, args.static_start:static_total] = keys[:, args.context - args.static_end:]
        sv[:, :static_total] = torch.cat([values[:, :args.static_start], values[:, args.context - args.static_end:]], 1)
        q = synthetic.make_queries(mid_k, G, seed=layer)[0].contiguous()
        pl = ops.HostTierPlan(cent, idx["cell_count"], idx["cell_offset"], ks, bud, idx["list_keys"],
                              idx["list_values"], sk, sv, G, cache_pages=cache_pages)
        plans.append((pl, q, sk, sv, cent, idx["cell_count"], idx["cell_offset"]))
        del keys, values, mid_k, mid_v, labels, idx
    out = torch.empty((H * G, D), dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    hits = misses = mrows = 0
    for pl, q, *_ in plans:
        t0 = time.perf_counter()
        pl.step(q, out, static_total)
        torch.cuda.synchronize()
        cold.append((time.perf_counter() - t0) * 1e6)
        h0, m0, r0 = pl.hits, pl.misses, pl.miss_rows
        for _ in range(10):
            t0 = time.perf_counter()
            pl.step(q, out, static_total)
            torch.cuda.synchronize()
            warm.append((time.perf_counter() - t0) * 1e6)
        hits += pl.hits - h0
        misses += pl.misses - m0
        mrows += pl.miss_rows - r0
    warm_us = sorted(warm)[len(warm) // 2]
    miss_rows = mrows / (10 * NL)
    return {"layers": NL, "cache_pages": cache_pages, "buffer_pages": bud.buffer_pages,
            "cold_us_per_layer_step": round(sorted(cold)[len(cold) // 2], 1),
            "warm_us_per_layer_step": round(warm_us, 1),
            "warm_hit_block_fraction": round(hits / max(hits + misses, 1), 4),
            "warm_miss_rows_per_layer_step": round(miss_rows, 1),
            "warm_miss_gbps": round(miss_rows * 512 / (warm_us * 1e-6) / 1e9, 2),
            "clock": "host wall clock around each synchronous step"}


def measured_traffic(workload):
    """HBM bytes per split-pass launch from the committed counter
    summary of this exact workload (FETCH_SIZE + WRITE_SIZE per dispatch,
    each scaled by what the counter reads for a copy of known size), or
    None when no summary of this workload is committed."""
    f = ROOT / "profiles" / "fixed_attention_kernel_traffic_config1.md"
    if not f.exists():
        return None
    fields = {}
    for line in f.read_text().splitlines():
        if ":" in line and not line.startswith(("#", " ", "|")):
            k, v = line.split(":", 1)
            fields[k.strip()] = v.strip()
    if fields.get("workload") != workload or "traffic_bytes_per_launch" not in fields:
        return None
    return int(fields["traffic_bytes_per_launch"])


def build_ragged(args, ks, static_total, static_cap, static_len, start_ev, end_ev):
    """the KV heads of several sequences of different lengths in
    one launch per layer (sequence-major heads, each sequence's own token and
    page budget, the lists packed in one [B*H, max_len, D] buffer).  Returns
    the plans, the per-layer build times (every sequence's k-means and index)
    and the listed tokens over all heads."""
    import torch

    from adaptiveimi_amd import ops, synthetic
    from adaptiveimi_amd.sizing import decode_sizing

    dev = torch.device("cuda:0")
    Hs, G, D = args.kv_heads, args.groups, 128
    lens = [c - static_total for c in args.contexts]
    B = len(lens)
    buds = []
    for T in lens:
        sz = decode_sizing(T, args.budget, subspace_parts=len(ks), k_override=ks)
        buds.append(ops.Budget(sz["nprobe"], sz["max_tokens"], sz["buffer_pages"]))
    bud = ops.Budget.ragged(buds, Hs)
    log(f"[bench] ragged: sequences {list(args.contexts)}, per-sequence max_tokens {[b.max_tokens for b in buds]}, "
        f"buffer_pages {[b.buffer_pages for b in buds]}, nprobe {bud.nprobe}")
    plans, build_ms = [], []
    for layer in range(args.layers):
        lk = torch.zeros((B * Hs, max(lens), D), dtype=torch.bfloat16, device=dev)
        lv = torch.zeros_like(lk)
        sk = torch.zeros((B * Hs, static_cap, D), dtype=torch.bfloat16, device=dev)
        sv = torch.zeros_like(sk)
        cents, counts, offsets, qs, dur = [], [], [], [], 0.0
        for s_, ctx in enumerate(args.contexts):
            keys, values = synthetic.make_kv(Hs, ctx, seed=1000 + 97 * layer + s_, device="cuda")
            mid_k = keys[:, args.static_start:ctx - args.static_end]
            mid_v = values[:, args.static_start:ctx - args.static_end]
            hs = slice(s_ * Hs, (s_ + 1) * Hs)
            sk[hs, :args.static_start] = keys[:, :args.static_start]
            sk[hs, args.static_start:static_total] = keys[:, ctx - args.static_end:]
            sv[hs, :args.static_start] = values[:, :args.static_start]
            sv[hs, args.static_start:static_total] = values[:, ctx - args.static_end:]
            sk[hs, static_total] = keys[:, -1]
            sv[hs, static_total] = values[:, -1]
            torch.cuda.synchronize()
            start_ev.record()
            cent, labels, _ = ops.kmeans(mid_k, list(ks), args.iters)
            idx = ops.build_index(mid_k, mid_v, cent, labels, list(ks), compact=False, list_keys=lk[hs],
                                  list_values=lv[hs])
            end_ev.record()
            torch.cuda.synchronize()
            dur += start_ev.elapsed_time(end_ev)
            cents.append(cent)
            counts.append(idx["cell_count"])
            offsets.append(idx["cell_offset"])
            qs.append(synthetic.make_queries(mid_k, G, seed=layer * 10 + s_)[0])
            del keys, values, mid_k, mid_v, labels
        build_ms.append(dur)
        plan = ops.DecodePlan(torch.cat(cents), torch.cat(counts), torch.cat(offsets), ks, bud, lk, lv, sk, sv, G,
                              query=torch.cat(qs).contiguous())
        plan.set_static_len(static_len)
        plans.append(plan)
        if layer % 7 == 6:
            log(f"[bench] built {layer + 1}/{args.layers} layers, last build {build_ms[-1]:.2f} ms")
    return plans, build_ms, Hs * sum(lens)


def build_roofline(args, head_tokens, T, ks, build_ms):
    """Index-build fractions over the whole per-layer build (k-means +
    cell lists + K/V permutation, median wall time):
      E-step FLOPs = 2 T k D per Lloyd iteration per KV head (every key
        against the k centroids of each of the P subspaces of D/P dims), on
        the k-means sample for the iterations plus one full assignment when
        the build samples; against the dense bf16 MFMA peak (the E-step
        screens distances with bf16 MFMA and rechecks them in fp32);
      bytes >= the keys once plus the K/V permutation (read and write K
        and V), 5 T D 2 B per KV head; against the HBM peak."""
    D = 128
    k = max(ks)
    # per head: T listed tokens (head_tokens = their sum over the KV heads);
    # a sampled build iterates on min(sample, T) keys, then assigns all T
    heads = head_tokens / T
    n_it = min(args.sample, T) if args.sample else T
    flops = 2.0 * k * D * heads * (n_it * args.iters + (T if args.sample else 0))
    if args.contexts:
        flops = 2.0 * k * D * head_tokens * args.iters
    nbytes = 5.0 * D * 2 * head_tokens
    t = build_ms * 1e-3
    return {"estep_gflop": round(flops / 1e9, 2), "mfma_tflops": round(flops / t / 1e12, 2),
            "mfma_peak_tflops": MFMA_BF16_PEAK_TFLOPS, "mfma_frac": round(flops / t / 1e12 / MFMA_BF16_PEAK_TFLOPS, 5),
            "bytes_min": int(nbytes), "hbm_gbps": round(nbytes / t / 1e9, 1),
            "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBPS, 4),
            "basis": "whole build wall time per layer (median); E-step FLOPs 2*T*k*D per iteration per KV head"}


def cpu_build_layer(orc, kbits, vbits, ks, iters, cores):
    """The reference's CPU index build of one layer (kmeans_core.cpp:384-501,
    reorganize_core.cpp:18-311), restated by the oracle: bf16 -> fp32,
    subvector split, per-(head, subspace) Lloyd runs (first-k init, no early
    stop) on max_concurrent tasks of threads_per_phase OpenMP threads each
    (kmeans_core.cpp:433-443, cache.py:113-124), then the compaction and the
    stable K/V permutation per head."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    H, T, D = kbits.shape
    parts = len(ks)
    tasks = H * parts
    tpp = orc.reference_threads_per_phase(cores, H, parts)
    min_threads = max(1, min(max(1, cores // tasks), cores))
    max_conc = max(1, min(tasks, cores // min_threads))
    kf = orc.bf16_to_f32(kbits)
    sl = orc.subspace_slices(D, parts)
    subs = [[np.ascontiguousarray(kf[h][:, sl[p]]) for p in range(parts)] for h in range(H)]

    def run(hp):
        h, p = hp
        sub = subs[h][p]
        _, lab, _ = orc.lloyd(sub, sub[: ks[p]], iters, mstep_threads=tpp, estep_threads=tpp)
        return hp, lab

    labels = {}
    with ThreadPoolExecutor(max_conc) as ex:
        for hp, lab in ex.map(run, [(h, p) for h in range(H) for p in range(parts)]):
            labels[hp] = lab
    lists = []
    for h in range(H):
        r = orc.compact_reorg([labels[(h, p)] for p in range(parts)], ks)
        lists.append((kbits[h][r["perm"]], vbits[h][r["perm"]]))
    return lists, max_conc, tpp


def cpu_baseline(first, ks, bud, static_len, seconds, iters):
    """CPU baseline on the host cores (the oracle's C restatement of the
    reference's CPU path, OpenMP over every core in the affinity mask):
    decode steps of layer 0 in fp32 (median of >= 20), and the full index
    build of layer 0 (median of >= 5 runs when they fit the time bound)."""
    import numpy as np
    import torch

    from oracle import oracle as orc

    def bits(t):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)

    cores = len(os.sched_getaffinity(0))
    os.environ.setdefault("OMP_NUM_THREADS", str(cores))
    idx = first["idx"]
    H = first["keys"].shape[0]
    heads = []
    cent = first["cent"].numpy()
    cnt = idx["cell_count"].numpy()
    off = idx["cell_offset"].numpy()
    lk, lv = bits(idx["list_keys"]), bits(idx["list_values"])
    for h in range(H):
        gids = np.flatnonzero(cnt[h])
        offsets = np.concatenate([off[h][gids], [off[h][-1]]]).astype(np.int32)
        heads.append(dict(n_active=len(gids), offsets=offsets,
                          merged=orc.merged_centroids([cent[h, 0, :ks[0]], cent[h, 1, :ks[1]]], gids, ks)))
    n_c = ks[0] * ks[1] + 1
    q = bits(first["q"])
    base = orc.DecodeBaselineF32(heads, lk, lv, bits(first["steady_k"]), bits(first["steady_v"]), n_c)
    args = (static_len, bud.nprobe, bud.max_tokens, bud.buffer_pages)
    for _ in range(3):
        base.step(q, *args)
    dec = []
    t0 = time.perf_counter()
    while len(dec) < 20 or (time.perf_counter() - t0 < seconds * 0.3 and len(dec) < 200):
        t1 = time.perf_counter()
        base.step(q, *args)
        dec.append(time.perf_counter() - t1)
    dec_s = statistics.median(dec)
    kb, vb = bits(first["keys"]), bits(first["values"])
    build = []
    t0 = time.perf_counter()
    while len(build) < 5 and (len(build) == 0 or time.perf_counter() - t0 < seconds * 0.8):
        t1 = time.perf_counter()
        _, max_conc, tpp = cpu_build_layer(orc, kb, vb, ks, iters, cores)
        build.append(time.perf_counter() - t1)
    build_ms = statistics.median(build) * 1e3
    return {"value": round(1.0 / dec_s, 2), "unit": "decode steps/s per layer", "cores": cores, "kind": "port",
            "sample": f"layer 0 of the same workload: {len(dec)} decode steps ({H} KV heads, scores + selection + "
                      f"fp32 attention, AVX2 + OpenMP on {cores} cores, each K/V row read once for its "
                      f"{first['q'].shape[1]} query heads), median; {len(build)} full index builds of the "
                      f"layer ({H} heads x {len(ks)} subspaces, {iters} Lloyd iterations, {max_conc} concurrent "
                      f"runs x {tpp} threads as the reference splits them, compaction, K/V permutation), median",
            "decode_us_per_layer_median": round(dec_s * 1e6, 1), "decode_runs": len(dec),
            "index_build_ms_per_layer_median": round(build_ms, 1), "index_build_runs": len(build)}


if __name__ == "__main__":
    main()
