#!/usr/bin/env python3
"""Decode throughput of one GPT-OSS-120B-shaped MXFP4 MoE layer on one MI355X.

Workload: BASELINE config 2 -- hidden 2880, 128 experts, top-4 (softmax over
the selected), gate/up/down [128, 2880, 2880] MXFP4, clamped SwiGLU, batch 1.
A step is one token through router -> top-k -> 4 experts' gate/up/down
dequant-GEMVs -> weighted combine (nsx_moe_forward), on seeded synthetic
weights and activations already resident in HBM.

Weights of `--layers` independently seeded layers (1.7 GB of experts each)
rotate step by step and every step has its own token, so the expert bytes of
a step come from HBM rather than the 256 MB Infinity Cache. The K timed steps
run as one HIP graph (launch overhead as in a serving loop). Per-kernel
durations: `--profile-steps` further tokens, each with its own workspace, go
through the layer phase by phase (nsx_moe_phase); each phase is one HIP graph
of that kernel launched back to back over all those tokens, timed with HIP
events around its replay (an event pair around a single eager launch adds
several microseconds of marker latency). The phase outputs must equal the
full forward's.

Prints one JSON line (the driver's contract) with a `roofline` object for the
dominant kernel (the gate/up dequant-GEMV) and a `cpu_baseline` object: the
numpy restatement of the reference path (oracle/) on host cores, over a
bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E


def _parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=400)
    p.add_argument("--warmup", type=int, default=40)
    p.add_argument("--layers", type=int, default=6, help="rotating weight copies (1.7 GB each)")
    p.add_argument("--layout", choices=["t64", "gguf"], default="t64")
    p.add_argument("--profile-steps", type=int, default=96, help="tokens timed per phase graph")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--copy-probe-mib", type=int, default=0,
                   help="after the run, copy a buffer of this size 3 times (calibrates rocprofv3 byte counters)")
    return p.parse_args()


def _traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, scaled by a copy kernel of known size),
    or None when no such measurement is committed."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "pmc_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get("kernels", {}).get(kernel)
    except (OSError, ValueError):
        return None
    return None if rec is None else rec.get("traffic_bytes")


def _expert_bytes_per_token(cfg):
    """Algorithmic bytes of the expert GEMVs of one token (k experts): the
    quantized gate/up/down rows read once plus their fp32 biases."""
    gu = cfg.top_k * (cfg.expert_bytes("gate") + cfg.expert_bytes("up") + 2 * cfg.n_ff * 4)
    dn = cfg.top_k * (cfg.expert_bytes("down") + cfg.n_embd * 4)
    return gu, dn


def _cpu_baseline(cfg, t_cpu, X, budget_s, block_rows=512):
    """oracle.moe_gptoss (numpy restatement of model/gpt_oss.py:123-177 with
    compute/blockffn.py:146-231 block streaming) on host cores."""
    import numpy as np
    from oracle import moe as OM
    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    ncores = min(16, len(os.sched_getaffinity(0)))
    raw = {k: t_cpu[k] for k in ("gate", "up", "down")}
    bias = {k: t_cpu[k + "_b"] for k in ("gate", "up", "down")}
    ex = OM.ExpertSet(int(cfg.ggml_type), cfg.n_embd, cfg.n_ff, raw, bias)
    Wr, br = t_cpu["router_w"], t_cpu["router_b"]
    ctx = threadpool_limits(ncores) if threadpool_limits else None
    n = 0
    try:
        if ctx:
            ctx.__enter__()
        OM.moe_gptoss(X[:1], Wr, br, cfg.top_k, ex, block_rows=block_rows)  # warm-up
        t0 = time.perf_counter()
        while True:
            OM.moe_gptoss(X[n % len(X):n % len(X) + 1], Wr, br, cfg.top_k, ex, block_rows=block_rows)
            n += 1
            if time.perf_counter() - t0 >= budget_s:
                break
        dt = time.perf_counter() - t0
    finally:
        if ctx:
            ctx.__exit__(None, None, None)
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": ncores, "kind": "port",
            "sample": f"{n} decode tokens through one layer (oracle.moe_gptoss, numpy; dequant single-threaded, "
                      f"GEMV on BLAS with {ncores} threads; block_rows {block_rows}) in {dt:.1f} s"}


def main():
    args = _parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from nurostream_amd import _native as N
    from nurostream_amd import synth
    from nurostream_amd.compute.kernels import t64_pack_stacked
    from nurostream_amd.moe.fused import MoELayer

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    N.ensure_selftest(dev)
    cfg = synth.GPTOSS_120B
    T = 1
    K, W = args.steps, args.warmup
    n_layers = max(1, args.layers)

    layers, t_cpu = [], None
    for li in range(n_layers):
        t = synth.make_layer(cfg, seed=args.seed, device=dev, layer=li)
        if li == 0 and not args.no_cpu:
            t_cpu = {k: (None if v is None else v.float().cpu().numpy() if v.dtype != torch.uint8
                         else v.cpu().numpy()) for k, v in t.items()}
        if args.layout == "t64":
            mats = {k: t64_pack_stacked(t[k], cfg.ggml_type, cfg.n_expert, *cfg.rows_K(k))
                    for k in ("gate", "up", "down")}
            for k in ("gate", "up", "down"):
                t[k] = None
        else:
            mats = {k: t[k] for k in ("gate", "up", "down")}
        layers.append(MoELayer(ggml_type=cfg.ggml_type, n_expert=cfg.n_expert, top_k=cfg.top_k,
                               n_embd=cfg.n_embd, n_ff=cfg.n_ff, router_w=t["router_w"], router_b=t["router_b"],
                               gate=mats["gate"], up=mats["up"], down=mats["down"], gate_b=t["gate_b"],
                               up_b=t["up_b"], down_b=t["down_b"], layout=args.layout,
                               router_mode=cfg.router_mode, act=cfg.act))
        del t, mats
        torch.cuda.synchronize()
    torch.cuda.empty_cache()

    n_tok = W + K + args.profile_steps
    X = synth.activations(n_tok, cfg.n_embd, seed=args.seed + 1, device=dev)
    outs = torch.empty((n_tok, cfg.n_embd), dtype=torch.float32, device=dev)
    ids = torch.empty((n_tok, cfg.top_k), dtype=torch.int32, device=dev)
    wts = torch.empty((n_tok, cfg.top_k), dtype=torch.float32, device=dev)
    for lay in layers:
        lay.workspace(T)

    def step(i):
        lay = layers[i % n_layers]
        lay.forward(X[i:i + 1], out=outs[i:i + 1], ids=ids[i:i + 1], weights=wts[i:i + 1])

    # warm-up (eager), then capture the K timed steps (tokens W..W+K-1) as one graph
    for i in range(W):
        step(i)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for i in range(W, W + K):
                step(i)
    torch.cuda.synchronize()

    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    ev0.record()
    graph.replay()
    ev1.record()
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - t_wall
    ms_total = ev0.elapsed_time(ev1)
    ms_per_step = ms_total / K
    tok_s = K * T / (ms_total / 1e3)

    # per-kernel durations: R tokens, one workspace each, phase by phase; each
    # phase is a graph of R back-to-back launches of that phase's kernel
    P0 = W + K
    R = args.profile_steps
    toks = list(range(P0, P0 + R))
    wss = [layers[i % n_layers].new_workspace(T) for i in toks]
    graphs = []
    with torch.cuda.stream(stream):  # PHASE_COMBINE launches nothing: the down kernels combine
        for ph in (N.PHASE_ROUTER, N.PHASE_GATE_UP, N.PHASE_DOWN):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                for j, i in enumerate(toks):
                    layers[i % n_layers].phase(ph, X[i:i + 1], outs[i:i + 1], ids[i:i + 1], wts[i:i + 1], wss[j])
            graphs.append(g)
    torch.cuda.synchronize()
    for g in graphs:  # first replay: graph upload, untimed
        g.replay()
    torch.cuda.synchronize()
    phase_us = []
    for g in graphs:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        phase_us.append(e0.elapsed_time(e1) * 1e3 / R)
    ph_out = outs[P0:P0 + R].clone()
    for i in toks:
        step(i)
    torch.cuda.synchronize()
    if not torch.equal(ph_out, outs[P0:P0 + R]):
        raise RuntimeError("phase-by-phase outputs differ from nsx_moe_forward")

    gu_bytes, dn_bytes = _expert_bytes_per_token(cfg)
    gu_us = phase_us[1]
    achieved = gu_bytes / (gu_us * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": "moe_gu_kernel" if args.layout == "t64" else "moe_gu_raw_kernel",
                "bytes_per_launch": gu_bytes, "avg_us": round(gu_us, 3)}
    roofline["traffic"] = _traffic(roofline["kernel"])
    layer_bytes = cfg.layer_bytes_per_token()
    result = {
        "metric": "MoE-FFN decode tok/s (GPT-OSS-120B shape, MXFP4)",
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded MXFP4 experts, x~N(0,1)); weights resident in HBM",
        "config": {"workload": "gpt-oss-120b MoE layer, decode batch 1 (BASELINE config 2)",
                   "layout": args.layout, "rotating_layers": n_layers, "hidden": cfg.n_embd,
                   "experts": cfg.n_expert, "top_k": cfg.top_k, "graph": True},
        "layer_GBps": round(layer_bytes / (ms_per_step * 1e-3) / 1e9, 1),
        "kernel_us": {"router": round(phase_us[0], 3), "gate_up": round(phase_us[1], 3),
                     "down_combine": round(phase_us[2], 3)},
        "down_GBps": round(dn_bytes / (phase_us[2] * 1e-6) / 1e9, 1),
        "wall_s": round(wall_s, 4),
        "roofline": roofline,
    }
    if args.copy_probe_mib > 0:  # a plain copy of known size for the counter calibration
        n = args.copy_probe_mib << 18
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if not args.no_cpu:
        result["cpu_baseline"] = _cpu_baseline(cfg, t_cpu, X[:32].cpu().numpy(), args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
