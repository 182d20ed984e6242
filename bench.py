#!/usr/bin/env python3
"""MoE expert-path throughput on one MI355X (default: GPT-OSS-120B decode).

Default workload (the driver's line): one GPT-OSS-120B-shaped MXFP4 MoE layer
at decode batch 1 -- hidden 2880, 128 experts, top-4 (softmax over the
selected), gate/up/down [128, 2880, 2880] MXFP4, clamped SwiGLU. A step is
one token through router -> top-k -> 4 experts' gate/up/down dequant-GEMVs ->
weighted combine (nsx_moe_forward), on seeded synthetic weights and
activations already resident in HBM.

Weights of `--layers` independently seeded layers (1.7 GB of experts each)
rotate step by step and every step has its own tokens, so the expert bytes of
a step come from HBM rather than the 256 MB Infinity Cache. The K timed steps
are captured as one HIP graph (launch overhead as in a serving loop); after
one untimed replay, `--replays` replays run back to back with a HIP event
between each two, and `ms_per_step` is the median replay over K (the fastest
and slowest are in `timing`). Per-kernel
durations: `--profile-steps` further steps, each with its own workspace, go
through the layer phase by phase (nsx_moe_phase); each phase is one HIP graph
of that phase launched back to back over all those steps, timed with HIP
events around its replay (an event pair around a single eager launch adds
several microseconds of marker latency). The phase outputs must equal the
full forward's.

Other workloads (`--workload`, one JSON line each, for the design notes):
  gptoss-t128   BASELINE config 3: T=128 tokens per step, Zipf(1.1) expert
                popularity, grouped dispatch (sort by expert, grouped MFMA)
  qwen3-t1      BASELINE config 4: Qwen3-235B-shaped Q4_K layer (GGUF rows), T=1
  qwen3-t32     the same at T=32
  stack-t1      BASELINE config 5: 36 GPT-OSS layers resident (61 GB),
                x <- x + moe_l(rms_norm(x)) per layer, T=1
  stack-t8      the same at T=8
  stack-t1-host25, stack-t8-host25
                BASELINE config 5b: the same stack with a seeded 25% of the
                512-row expert blocks in pinned host RAM, staged per step
                (eager: one host synchronisation per layer for the routing)
  q4_0-gemv     BASELINE config 1: the fused Q4_0 dequant-GEMV (nsx_fused_gemv,
                T=1) over a 4096 x 4096 Q4_0 matrix, 64 distinct weight copies
                rotating so the bytes come from HBM; CPU baseline: the
                reference's CPU stream_linear (512-row blocks, dequantize
                then x @ w.T in torch)
  lmhead-q6k    the fused raw-GGUF GEMV (nsx_fused_gemv) at T=1 over a
                Qwen3-235B-shaped Q6_K LM head, 151936 x 4096 (the Q6_K
                tensor of Q4_K_M files); two weight copies alternate
  lmhead-q8     the same over a GPT-OSS-120B-shaped Q8_0 LM head,
                201088 x 2880
  gptoss-token  a whole GPT-OSS-120B decode token as one HIP graph: token
                embedding, 36 x (rms_norm, q/k/v, YaRN rotary + KV append,
                sink attention, o-proj, MoE FFN), output norm, LM head, with
                `--context` positions already in the KV cache (synthetic);
                dense tensors Q8_0, experts MXFP4 t64 slabs, all in HBM
  disk-stream   expert weights from a GGUF file on the box's disk: one
                GPT-OSS-120B-shaped layer's MXFP4 expert tensors (1.7 GB)
                are written, then read into HBM in 512-row blocks by the
                native reader (O_DIRECT, then buffered), and decode tokens
                run through the layer with every expert block streamed from
                the file (DiskSource + BlockPrefetcher + stream_expert_ffn)

Prints one JSON line (the driver's contract) with a `roofline` object for the
dominant kernel (the gate/up dequant-GEMV) and a `cpu_baseline` object: the
reference's torch CPU path restated under oracle/, on the host cores, over a
bounded sample of the same workload.

The default run also measures the other BASELINE configs, each at its own
default steps and with a short CPU baseline, and adds them to the same line
under "configs" (compact: ms_per_step, value, spread, roofline kernel /
bytes / avg_us / frac, cpu_baseline): "1" (q4_0-gemv), "3" (gptoss-t128),
"4_t1" / "4_t32" (qwen3-t1 / -t32), "5_t1" / "5_t8" (one resident 36-layer
stack at T=1 and T=8) and "5b_t1" (the 25%-host stack at T=1: the kernels
reading host tiles over PCIe, and under "prefetch" the same stack staging its
host blocks through BlockPrefetcher at depth 4). `--configs none` skips them.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
PCIE_PEAK_GBS = 64.0  # PCIe Gen5 x16, one direction
WORKLOADS = ("gptoss-decode", "gptoss-t128", "qwen3-t1", "qwen3-t32", "stack-t1", "stack-t8", "stack-t1-host25",
             "stack-t8-host25", "q4_0-gemv", "lmhead-q6k", "lmhead-q8", "disk-stream", "gptoss-token")

# per workload: (config name, T, steps, warmup, rotating layers or stack depth, profile steps)
_DEFAULTS = {
    "gptoss-decode": ("GPTOSS_120B", 1, 400, 40, 6, 96),
    "gptoss-t128": ("GPTOSS_120B", 128, 40, 5, 4, 8),
    "qwen3-t1": ("QWEN3_235B", 1, 300, 30, 4, 64),
    "qwen3-t32": ("QWEN3_235B", 32, 60, 6, 4, 8),
    "stack-t1": ("GPTOSS_120B", 1, 40, 4, 36, 0),
    "stack-t8": ("GPTOSS_120B", 8, 20, 2, 36, 0),
    "stack-t1-host25": ("GPTOSS_120B", 1, 20, 3, 36, 0),
    "stack-t8-host25": ("GPTOSS_120B", 8, 10, 2, 36, 0),
    "q4_0-gemv": ("Q4_0", 1, 400, 40, 64, 0),
    "lmhead-q6k": ("Q6_K", 1, 200, 20, 2, 0),
    "lmhead-q8": ("Q8_0", 1, 200, 20, 2, 0),
    "disk-stream": ("GPTOSS_120B", 1, 12, 2, 1, 0),
    "gptoss-token": ("GPTOSS_120B", 1, 200, 20, 36, 0),
}
# GEMV shapes: (rows, K, what); the LM heads' rows are the vocabulary
_LMHEAD = {"q4_0-gemv": (4096, 4096, "dense 4096x4096 (BASELINE config 1)"),
           "lmhead-q6k": (151936, 4096, "qwen3-235b-a22b"), "lmhead-q8": (201088, 2880, "gpt-oss-120b")}


def _parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--workload", choices=WORKLOADS, default="gptoss-decode")
    p.add_argument("--steps", type=int, default=None, help="timed steps (default per workload)")
    p.add_argument("--warmup", type=int, default=None, help="untimed steps (default per workload)")
    p.add_argument("--layers", type=int, default=None, help="rotating weight copies, or the stack depth")
    p.add_argument("--layout", choices=["t64", "gguf"], default="t64")
    p.add_argument("--dispatch", choices=["auto", "pairs", "grouped", "mfma"], default="auto")
    p.add_argument("--profile-steps", type=int, default=None, help="steps timed per phase graph")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-probe", action="store_true", help="skip the HBM read-bandwidth probe")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--host-mode", choices=("read", "stage", "prefetch"), default="read",
                   help="config 5b: kernels read pinned host tiles over PCIe (read), or they are DMA-staged per "
                        "layer all at once (stage) or through BlockPrefetcher at depth 4 (prefetch)")
    p.add_argument("--context", type=int, default=1024,
                   help="gptoss-token: positions already in the KV cache when the timed tokens start")
    p.add_argument("--copy-probe-mib", type=int, default=0,
                   help="after the run, copy a buffer of this size 3 times (calibrates rocprofv3 byte counters)")
    p.add_argument("--decode-chain", choices=("on", "off"), default="on",
                   help="stack workloads at T=1: the decode chain (no router launch after the first layer) or the "
                        "folded-norm path (a router launch per layer)")
    p.add_argument("--replays", type=int, default=20,
                   help="timed replays of the captured steps (after one untimed replay); the median is reported")
    p.add_argument("--configs", choices=("all", "none"), default="all",
                   help="default workload only: also measure BASELINE configs 1, 3, 4, 5 and 5b (compact results "
                        "under 'configs'), each at its own default steps")
    p.add_argument("--sub-cpu-seconds", type=float, default=3.0,
                   help="budget of each sub-config's CPU baseline sample")
    return p.parse_args()


def csrc_digest():
    """sha256 (first 16 hex digits) over the library's HIP sources, in name
    order: the code a committed counter measurement was taken on."""
    import hashlib
    d = os.path.join(os.path.dirname(os.path.abspath(__file__)), "nurostream_amd", "csrc")
    h = hashlib.sha256()
    for name in sorted(os.listdir(d)):
        if name.endswith((".hip", ".h")):
            with open(os.path.join(d, name), "rb") as f:
                h.update(name.encode() + b"\0" + f.read())
    return h.hexdigest()[:16]


def _traffic(kernel, workload):
    """HBM bytes per launch of `kernel` in `workload` from the committed
    rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE, scaled by a copy kernel
    of known size, written by bench_pmc.py), or None when there is no such
    measurement or it was taken on other kernel sources than the ones built
    now. A name without template arguments matches the workload's one
    instantiation of that kernel."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "pmc_traffic.json")
    try:
        with open(path) as f:
            doc = json.load(f)
    except (OSError, ValueError):
        return None
    if doc.get("csrc_digest") != csrc_digest():
        return None
    kernels = doc.get("workloads", {}).get(workload, {}).get("kernels", {})
    rec = kernels.get(kernel)
    if rec is None:
        same = [v for k, v in kernels.items() if k.split("<")[0] == kernel.split("<")[0]]
        rec = same[0] if len(same) == 1 else None
    return None if rec is None else rec.get("traffic_bytes")


def _cpu_env():
    """(threads for the CPU baseline = every core this process may run on, CPU model)."""
    n = len(os.sched_getaffinity(0))
    model = "?"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return n, model


def _median_cpu(fn, warmup=3, runs=5):
    """Median wall seconds of `runs` calls of fn after `warmup` untimed calls."""
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2], ts


class _Threads:
    """torch's CPU thread count set to n inside the block, restored after."""

    def __init__(self, torch, n):
        self.torch, self.n = torch, n

    def __enter__(self):
        self.prev = self.torch.get_num_threads()
        self.torch.set_num_threads(self.n)

    def __exit__(self, *exc):
        self.torch.set_num_threads(self.prev)


def _cpu_baseline_layer(torch, cfg, t_cpu, h, budget_s, block_rows=512, n_layers=1):
    """The reference's CPU torch path for one MoE layer (oracle.torch_path:
    router, then per chosen expert in ascending id stream_linear windows of
    block_rows rows -- dequantize, x @ w.T -- activation and the weighted
    combine) on the host cores, over the step's T tokens h. When the step's
    experts would take more than about budget_s / 8 per run, a sample of the
    chosen experts is timed and scaled to all of them. n_layers > 1 scales
    one layer to a stack of identical cost."""
    from oracle import torch_path as TP
    n, model = _cpu_env()
    raw = {k: torch.from_numpy(t_cpu[k]) for k in ("gate", "up", "down")}
    bias = {k: torch.from_numpy(t_cpu[k + "_b"]) for k in ("gate", "up", "down")} if cfg.bias else {}
    ex = TP.Experts(int(cfg.ggml_type), cfg.n_embd, cfg.n_ff, raw, bias)
    Wr = torch.from_numpy(t_cpu["router_w"]).float()
    br = torch.from_numpy(t_cpu["router_b"]).float() if t_cpu.get("router_b") is not None else None
    act = TP.clamped_swiglu if cfg.act == "clamped_swiglu" else TP.silu_mul
    h = torch.as_tensor(h).float().reshape(-1, cfg.n_embd).contiguous()
    T = h.shape[0]

    def route():
        if cfg.router_mode == "gptoss":
            return TP.route_gptoss(h, Wr, br, cfg.top_k)
        return TP.route_qwen3(h, Wr, cfg.top_k)

    with _Threads(torch, n):
        ids, w = route()
        chosen = torch.unique(ids).tolist()
        t0 = time.perf_counter()
        TP.moe_layer(h, ids, w, ex, act, block_rows, experts=chosen[:1])
        per_expert = time.perf_counter() - t0
        n_sample = max(1, min(len(chosen), int(budget_s / 8 / max(per_expert, 1e-6))))
        sample = chosen[:n_sample]
        t_route, _ = _median_cpu(route)
        t_exp, runs = _median_cpu(lambda: TP.moe_layer(h, ids, w, ex, act, block_rows, experts=sample))
    step_s = n_layers * (t_route + t_exp * len(chosen) / n_sample)
    what = (f"{'all ' if n_sample == len(chosen) else ''}{n_sample} of the step's {len(chosen)} distinct experts"
            + ("" if n_sample == len(chosen) else " (time scaled to all of them)"))
    return {"value": round(T / step_s, 4), "unit": "tok/s", "cores": n, "kind": "port",
            "cpu_model": model, "ms_per_step": round(step_s * 1e3, 2),
            "sample": f"{T} token(s) through {'one layer' if n_layers == 1 else f'layer 0 (x{n_layers} layers)'}: "
                      f"router, {what}; oracle.torch_path ({block_rows}-row blocks: dequantize, x @ w.T, fp32), "
                      f"{n} threads, median of {len(runs)} after 3 warm-ups"}


def _cpu_baseline_gemv(torch, raw_cpu, t, x, rows, K, budget_s, block_rows=512, unit="tok/s", nbytes=None):
    """stream_linear's CPU branch (oracle.torch_path.stream_linear: per
    block_rows-row block dequantize then x @ w.T in fp32) over the matrix, or
    over a leading row sample of it scaled to every row when a full pass would
    take more than about budget_s / 8."""
    from oracle import torch_path as TP
    n, model = _cpu_env()
    rb = TP.row_bytes(int(t), K)
    raw = torch.from_numpy(raw_cpu)
    xt = torch.as_tensor(x).float().reshape(1, K)
    with _Threads(torch, n):
        probe = min(rows, 4 * block_rows)
        t0 = time.perf_counter()
        TP.stream_linear(raw[:probe * rb], int(t), xt, probe, K, block_rows)
        per_row = (time.perf_counter() - t0) / probe
        n_rows = min(rows, max(block_rows, int(budget_s / 8 / max(per_row, 1e-12)) // block_rows * block_rows))
        med, runs = _median_cpu(lambda: TP.stream_linear(raw[:n_rows * rb], int(t), xt, n_rows, K, block_rows))
    pass_s = med * rows / n_rows
    value = 1.0 / pass_s if unit == "tok/s" else nbytes / pass_s / 1e9
    return {"value": round(value, 4 if unit == "tok/s" else 2), "unit": unit, "cores": n, "kind": "port",
            "cpu_model": model, "ms_per_pass": round(pass_s * 1e3, 3),
            "sample": f"{'the whole' if n_rows == rows else f'the first {n_rows} rows of the'} {rows} x {K} matrix"
                      + ("" if n_rows == rows else " (scaled to every row)")
                      + f", T=1; oracle.torch_path.stream_linear ({block_rows}-row blocks: dequantize, x @ w.T, fp32), "
                      f"{n} threads, median of {len(runs)} after 3 warm-ups"}


def _build_layer(torch, synth, cfg, li, args, dev, zipf, keep_cpu):
    from nurostream_amd.compute.kernels import t64_pack_stacked
    from nurostream_amd.moe.fused import MoELayer
    if zipf:
        t, c = synth.make_zipf_layer(cfg, seed=args.seed, device=dev, layer=li)
    else:
        t, c = synth.make_layer(cfg, seed=args.seed, device=dev, layer=li), None
    t_cpu = None
    if keep_cpu:
        t_cpu = {k: (None if v is None else v.float().cpu().numpy() if v.dtype != torch.uint8
                     else v.cpu().numpy()) for k, v in t.items()}
    layout = args.layout if cfg.ggml_type == synth.GGMLType.MXFP4 else "gguf"
    if layout == "t64":
        mats = {k: t64_pack_stacked(t[k], cfg.ggml_type, cfg.n_expert, *cfg.rows_K(k)) for k in ("gate", "up", "down")}
    else:
        mats = {k: t[k] for k in ("gate", "up", "down")}
    layer = MoELayer(ggml_type=cfg.ggml_type, n_expert=cfg.n_expert, top_k=cfg.top_k, n_embd=cfg.n_embd,
                     n_ff=cfg.n_ff, router_w=t["router_w"], router_b=t["router_b"], gate=mats["gate"],
                     up=mats["up"], down=mats["down"], gate_b=t["gate_b"], up_b=t["up_b"], down_b=t["down_b"],
                     layout=layout, router_mode=cfg.router_mode, act=cfg.act, dispatch=args.dispatch)
    return layer, t_cpu, c, layout


class _Timed:
    """Replays of a captured run of K steps: `ms` is the median replay in ms,
    `lo` / `hi` the fastest and slowest, `n` the number timed."""

    def __init__(self, times, wall_s, stream, K):
        ts = sorted(times)
        self.ms, self.lo, self.hi, self.n = ts[len(ts) // 2], ts[0], ts[-1], len(ts)
        self.wall_s, self.stream, self.K = wall_s, stream, K

    def spread(self):
        """[fastest, median, slowest] ms per step over the timed replays."""
        return [round(v / self.K, 5) for v in (self.lo, self.ms, self.hi)]


def _graph_time(torch, run_steps, W, K, replays=20):
    """Eager warm-up steps 0..W-1, then steps W..W+K-1 captured as one graph.
    One untimed replay (the graph's upload), then `replays` replays queued back
    to back on the capture stream with a HIP event between each two, so every
    replay has its own interval and the host runs ahead of the GPU: a _Timed."""
    run_steps(range(W))
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            run_steps(range(W, W + K))
    torch.cuda.synchronize()
    n = max(1, replays)
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    with torch.cuda.stream(stream):
        graph.replay()  # upload + first run, untimed
        torch.cuda.synchronize()
        t_wall = time.perf_counter()
        evs[0].record(stream)
        for i in range(n):
            graph.replay()
            evs[i + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    return _Timed([evs[i].elapsed_time(evs[i + 1]) for i in range(n)], wall, stream, K)


def _expert_bytes(cfg, n_experts):
    """Algorithmic bytes of the gate/up and of the down products of n_experts
    distinct experts: quantized rows read once plus fp32 bias rows."""
    b = 4 if cfg.bias else 0
    gu = n_experts * (cfg.expert_bytes("gate") + cfg.expert_bytes("up") + 2 * cfg.n_ff * b)
    dn = n_experts * (cfg.expert_bytes("down") + cfg.n_embd * b)
    return gu, dn


_METRIC = {"gptoss-decode": "MoE-FFN decode tok/s (GPT-OSS-120B shape, MXFP4)",
           "gptoss-t128": "MoE-FFN prefill-chunk tok/s (GPT-OSS-120B shape, MXFP4, T=128, Zipf 1.1)",
           "qwen3-t1": "MoE-FFN decode tok/s (Qwen3-235B-A22B shape, Q4_K)",
           "qwen3-t32": "MoE-FFN batch-32 tok/s (Qwen3-235B-A22B shape, Q4_K)"}
_WORKLOAD = {"gptoss-decode": "gpt-oss-120b MoE layer, decode batch 1 (BASELINE config 2)",
             "gptoss-t128": "gpt-oss-120b MoE layer, T=128, Zipf(1.1) routing (BASELINE config 3)",
             "qwen3-t1": "qwen3-235b-a22b MoE layer, decode batch 1 (BASELINE config 4)",
             "qwen3-t32": "qwen3-235b-a22b MoE layer, batch 32 (BASELINE config 4)"}


def _dtype_label(cfg, layout, mq):
    """The arithmetic the expert kernels run."""
    if layout == "t64":
        return "mxfp4 weights x 4-term e4m3 activation split, block-scaled MFMA, fp32 accumulate"
    if mq:
        return "q4_k codes as exact f16 (sc*q) x 2-term f16 activation split (f16 MFMA, fp32 accumulate)"
    if cfg.ggml_type.name == "Q4_K":
        return ("q4_k codes x 2-term int8 activation split per 16 elements (v_dot4 int8, exact integer sums), "
                "fp32 scales and accumulate")
    return f"{cfg.ggml_type.name.lower()} weights dequantized in registers x fp32 activations, fp32 accumulate"


def _read_probe(torch, N, dev):
    """Same-box HBM read bandwidth (nsx_read_probe) beside the 8 TB/s peak, at
    the sizes of config 2's two expert launches: 35,343,360 bytes (gate/up)
    and 17,671,680 bytes (down), each over several grids, and 1 GiB. Each
    figure is a graph of back-to-back launches over distinct regions of a 2 GiB
    buffer (more than the 256 MB Infinity Cache between reuses), timed with HIP
    events around its replay on the launching stream; the best grid counts."""
    lib = N.load()
    buf = torch.empty(2 << 30, dtype=torch.uint8, device=dev)
    buf.fill_(1)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    stream = torch.cuda.Stream()

    def timed(nbytes, wgs, threads):
        n = max(2, min(48, (2 << 30) // nbytes))
        regions = [(i % n) * nbytes for i in range(n)]
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream), torch.cuda.graph(g, stream=stream):
            for off in regions:
                N.check(lib.nsx_read_probe(buf.data_ptr() + off, nbytes, wgs, threads, sink.data_ptr(),
                                           stream.cuda_stream), "read_probe")
        with torch.cuda.stream(stream):
            g.replay()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            g.replay()
            e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / len(regions)
        return round(nbytes / (us * 1e-6) / 1e9, 1)

    grids = ((180, 1024), (256, 1024), (512, 1024), (1024, 256), (2048, 256), (4096, 256))
    gu = [timed(35343360, w, t) for w, t in grids]
    dn = [timed(17671680, w, t) for w, t in grids]
    big = [timed(1 << 30, w, t) for w, t in ((4096, 1024), (16384, 256))]
    del buf
    torch.cuda.empty_cache()
    return {"35MB_GBps": max(gu), "35MB_expert_grid_GBps": gu[0], "17.7MB_GBps": max(dn), "1GiB_GBps": max(big)}


def layer_workload(args, torch, N, synth, dev):
    name = args.workload
    cfg_name, T, K0, W0, L0, R0 = _DEFAULTS[name]
    cfg = getattr(synth, cfg_name)
    K = args.steps if args.steps is not None else K0
    W = args.warmup if args.warmup is not None else W0
    n_layers = max(1, args.layers if args.layers is not None else L0)
    R = args.profile_steps if args.profile_steps is not None else R0
    zipf = name == "gptoss-t128"
    default = name == "gptoss-decode"

    layers, t_cpu, zipf_c, layout = [], None, None, None
    for li in range(n_layers):
        keep = li == 0 and not args.no_cpu
        lay, tc, c, layout = _build_layer(torch, synth, cfg, li, args, dev, zipf, keep)
        layers.append(lay)
        t_cpu = tc if tc is not None else t_cpu
        zipf_c = c if c is not None else zipf_c
        torch.cuda.synchronize()
    torch.cuda.empty_cache()

    n_steps = W + K + R
    X = synth.activations(n_steps * T, cfg.n_embd, seed=args.seed + 1, device=dev).view(n_steps, T, cfg.n_embd)
    outs = torch.empty((n_steps, T, cfg.n_embd), dtype=torch.float32, device=dev)
    ids = torch.empty((n_steps, T, cfg.top_k), dtype=torch.int32, device=dev)
    wts = torch.empty((n_steps, T, cfg.top_k), dtype=torch.float32, device=dev)
    for lay in layers:
        lay.workspace(T)

    def run_steps(rng):
        for i in rng:
            layers[i % n_layers].forward(X[i], out=outs[i], ids=ids[i], weights=wts[i])

    tm = _graph_time(torch, run_steps, W, K, args.replays)
    ms_total, wall_s, stream = tm.ms, tm.wall_s, tm.stream
    ms_per_step = ms_total / K
    tok_s = K * T / (ms_total / 1e3)

    # per-phase durations: R further steps, one workspace each. Which kernels a phase runs follows the
    # library's dispatch rule (moe.hip use_grouped / use_mq): t64 layers group from 3 tokens (or on request);
    # stacked aligned Q4_K layers take the matrix-core kernels from 104 (token, expert) pairs (or on request).
    q4k = layout == "gguf" and cfg.ggml_type == synth.GGMLType.Q4_K
    mq = q4k and (args.dispatch == "mfma" or (args.dispatch == "auto" and T * cfg.top_k >= 104))
    grouped = mq or (args.dispatch == "grouped" and (layout == "t64" or q4k)) or (
        layout == "t64" and args.dispatch == "auto" and T >= 3)
    # (per pair, the down kernel combines: the combine phase launches nothing and is not captured)
    phases = (N.PHASE_ROUTER, N.PHASE_GATE_UP, N.PHASE_DOWN) + ((N.PHASE_COMBINE,) if grouped else ())
    phase_us = {}
    if R > 0:
        P0 = W + K
        steps = list(range(P0, P0 + R))
        wss = [layers[i % n_layers].new_workspace(T) for i in steps]
        graphs = []
        with torch.cuda.stream(stream):
            for ph in phases:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=stream):
                    for j, i in enumerate(steps):
                        layers[i % n_layers].phase(ph, X[i], outs[i], ids[i], wts[i], wss[j])
                graphs.append(g)
        torch.cuda.synchronize()
        for g in graphs:  # first replay: graph upload, untimed
            g.replay()
        torch.cuda.synchronize()
        for ph, g in zip(phases, graphs):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            g.replay()
            e1.record()
            torch.cuda.synchronize()
            phase_us[ph] = e0.elapsed_time(e1) * 1e3 / R
        ph_out = outs[P0:P0 + R].clone()
        run_steps(steps)
        torch.cuda.synchronize()
        if not torch.equal(ph_out, outs[P0:P0 + R]):
            raise RuntimeError("phase-by-phase outputs differ from nsx_moe_forward")

    # distinct experts per step: the expert bytes a step must read at least once
    ids_cpu = ids[W:W + K + R].cpu()
    distinct = [len(torch.unique(ids_cpu[s])) for s in range(ids_cpu.shape[0])]
    mean_distinct = sum(distinct) / len(distinct)
    # the gate/up kernel and every kernel the timed gate/up phase launches
    if layout == "t64":
        gu_kernel = "moe_gu_grouped_kernel" if grouped else "moe_gu_kernel"
        gu_phase = ["moe_sort_kernel", gu_kernel] if grouped else [gu_kernel]
    elif q4k:  # stacked 16-byte aligned Q4_K experts take the Q4_K kernels
        gu_kernel = "moe_q4k_mfma_kernel<true>" if mq else (
            "moe_gu_q4k_grouped_kernel" if grouped else "moe_gu_q4k_kernel")
        gu_phase = (["moe_sort_kernel", "mq_terms_kernel", gu_kernel] if mq
                    else ["moe_sort_kernel", gu_kernel] if grouped else [gu_kernel])
    else:
        gu_kernel = f"moe_gu_raw_kernel<{int(cfg.ggml_type)}>"
        gu_phase = [gu_kernel]
    gu_bytes, dn_bytes = _expert_bytes(cfg, mean_distinct)
    roofline = None
    if R > 0:
        kname, kbytes, kus = gu_kernel, gu_bytes, phase_us[N.PHASE_GATE_UP]
        achieved = kbytes / (kus * 1e-6) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": _traffic(kname, name),
                    "kernel": kname, "bytes_per_launch": int(kbytes), "avg_us": round(kus, 3),
                    "timing": f"graph of {R} gate/up phases, each its own tokens and workspace"}
        if len(gu_phase) > 1:
            roofline["note"] = "avg_us is the whole gate/up phase: " + " + ".join(gu_phase)
    step_bytes = sum(_expert_bytes(cfg, mean_distinct))
    kernel_us = None
    if R > 0:
        kernel_us = {"router": round(phase_us[N.PHASE_ROUTER], 3), "gate_up": round(phase_us[N.PHASE_GATE_UP], 3),
                     "down": round(phase_us[N.PHASE_DOWN], 3)}
        if grouped:
            kernel_us["combine"] = round(phase_us[N.PHASE_COMBINE], 3)
    result = {
        "metric": _METRIC[name],
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": _dtype_label(cfg, layout, mq),
        "data": f"synthetic (seeded {cfg.ggml_type.name} experts, x~N(0,1)); weights resident in HBM",
        "config": {"workload": _WORKLOAD[name], "tokens_per_step": T, "layout": layout, "dispatch": args.dispatch,
                   "rotating_layers": n_layers, "hidden": cfg.n_embd, "experts": cfg.n_expert, "top_k": cfg.top_k,
                   "graph": True},
        "distinct_experts_per_step": round(mean_distinct, 2),
        "expert_GBps": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 1),
        "kernel_us": kernel_us,
        "timing": {"replays": tm.n, "ms_per_step_min_med_max": tm.spread(), "wall_s": round(wall_s, 4)},
        "roofline": roofline,
    }
    if zipf:
        counts = torch.bincount(ids_cpu.reshape(-1).long(), minlength=cfg.n_expert).tolist()
        result["zipf"] = {"s": 1.1, "c": round(zipf_c, 5), "top8_counts": sorted(counts, reverse=True)[:8],
                          "experts_never_chosen": sum(1 for c in counts if c == 0)}
    result["cpu_baseline"] = None if args.no_cpu else _cpu_baseline_layer(
        torch, cfg, t_cpu, X[0].cpu(), args.cpu_seconds)
    if default and not args.no_probe:
        probe = result["hbm_read_probe"] = _read_probe(torch, N, dev)
        if roofline is not None:
            roofline["frac_of_probe"] = round(roofline["achieved"] / probe["35MB_GBps"], 4)
        if kernel_us is not None:  # the down kernel against the same-size read
            dn_gbs = dn_bytes / (kernel_us["down"] * 1e-6) / 1e9
            kernel_us["down_frac"] = round(dn_gbs / HBM_PEAK_GBS, 4)
            kernel_us["down_frac_of_probe"] = round(dn_gbs / probe["17.7MB_GBps"], 4)
    return result


def build_stack(args, torch, synth, dev, name):
    """The config-5 stack (resident) or config-5b stack (25% of the 512-row
    blocks in pinned host RAM, host mode args.host_mode) for workload `name`."""
    from nurostream_amd.model.gpt_oss import GptOssFFNStack, GptOssHostStreamedStack
    cfg = getattr(synth, _DEFAULTS[name][0])
    n_layers = args.layers if args.layers is not None else _DEFAULTS[name][4]
    if name.endswith("host25"):
        stack = GptOssHostStreamedStack.synthetic(cfg, n_layers, seed=args.seed, device=dev, host_fraction=0.25,
                                                  block_rows=512, dispatch=args.dispatch, mode=args.host_mode,
                                                  depth=4)
    else:
        stack = GptOssFFNStack.synthetic(cfg, n_layers, seed=args.seed, device=dev, layout=args.layout,
                                         dispatch=args.dispatch)
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return stack


def stack_workload(args, torch, N, synth, dev, stack=None, cpu_cache=None):
    """36 resident layers chained x <- x + moe_l(rms_norm(x));
    5b (`*-host25`): 25% of the blocks in pinned host RAM, reached as
    args.host_mode says ("read": the kernels read them over PCIe, one graph per
    step; "stage" / "prefetch": copied into staging slots per layer, all at once
    or through BlockPrefetcher at depth 4, eager with one host sync per layer).
    `stack` reuses a stack built by build_stack; `cpu_cache` (a dict) keeps the
    CPU baseline's per-layer time between calls on the same layer shape."""
    name = args.workload
    cfg_name, T, K0, W0, L0, _ = _DEFAULTS[name]
    cfg = getattr(synth, cfg_name)
    K = args.steps if args.steps is not None else K0
    W = args.warmup if args.warmup is not None else W0
    streamed = name.endswith("host25")
    if stack is None:
        stack = build_stack(args, torch, synth, dev, name)
    elif streamed:
        stack.set_mode(args.host_mode)
    stack.decode_chain = args.decode_chain == "on"
    n_layers = len(stack.layers)
    n_steps = W + K
    X = synth.activations(n_steps * T, cfg.n_embd, seed=args.seed + 1, device=dev).view(n_steps, T, cfg.n_embd)
    Y = torch.empty_like(X)

    def run_steps(rng):
        for i in rng:
            stack(X[i], out=Y[i])

    staged = streamed and args.host_mode != "read"
    tm = None
    if staged:  # host synchronisations inside a step: timed eagerly, an event pair per step
        run_steps(range(W))
        torch.cuda.synchronize()
        b0 = stack.bytes_from_host
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(K + 1)]
        t_wall = time.perf_counter()
        evs[0].record()
        for j, i in enumerate(range(W, W + K)):
            stack(X[i], out=Y[i])
            evs[j + 1].record()
        torch.cuda.synchronize()
        wall_s = time.perf_counter() - t_wall
        per = sorted(evs[j].elapsed_time(evs[j + 1]) for j in range(K))
        ms_total = per[len(per) // 2] * K  # the median step
        spread = [round(per[0], 5), round(per[len(per) // 2], 5), round(per[-1], 5)]
        host_bytes_step = (stack.bytes_from_host - b0) / K
    else:
        tm = _graph_time(torch, run_steps, W, K, args.replays)
        ms_total, wall_s, stream = tm.ms, tm.wall_s, tm.stream
        spread = tm.spread()
    ids, _ = stack.last_routing(T)
    ids_cpu = ids.cpu()
    roofline = None
    if not staged:
        # the dominant kernel in place: every layer's gate/up phase again, over the workspace the last step left
        # (logits and activation terms of that step), as one graph timed with HIP events on its stream
        h_b, y_b, ids_b, wts_b = stack._buffers(T)
        g = torch.cuda.CUDAGraph()
        # one token runs as a decode chain: layers 1.. launch moe_gu_chain_kernel, which reads the router shares
        # the last step left (the chain's own gate/up launch, alone)
        chain = T == 1 and stack.decode_chain and stack._chain_ok()
        timed_layers = list(range(1, n_layers)) if chain else list(range(n_layers))
        x_b = Y[W + K - 1].clone()
        with torch.cuda.stream(stream), torch.cuda.graph(g, stream=stream):
            for li in timed_layers:
                layer = stack.layers[li]
                if chain:
                    layer.chain_t1(x_b, stack.norm_weights[li], stack.cfg.rms_eps, stack._share, None, None, None,
                                   y_b, ids_b[li], wts_b[li], phases=N.CHAIN_GATE_UP)
                else:
                    layer.phase(N.PHASE_GATE_UP, h_b, y_b, ids_b[li], wts_b[li], layer.workspace(T))
        gts = []
        with torch.cuda.stream(stream):
            g.replay()  # upload, untimed
            for _ in range(5):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                g.replay()
                e1.record(stream)
                gts.append((e0, e1))
        torch.cuda.synchronize()
        gt = sorted(a.elapsed_time(b) for a, b in gts)
        gu_us = gt[len(gt) // 2] * 1e3 / len(timed_layers)
        per_layer = [len(torch.unique(ids_cpu[li])) for li in range(n_layers)]
        gu_bytes = sum(_expert_bytes(cfg, d)[0] for d in per_layer) / n_layers
        grouped = args.dispatch == "grouped" or (args.dispatch == "auto" and T >= 3)
        # (a gate/up phase launched on its own sorts in moe_sort_kernel, so the grouped phase runs the <false> kernel;
        # the stack's forward, which also runs the router, takes <true>)
        kname = ("moe_gu_chain_kernel" if chain else "moe_gu_grouped_kernel<false>" if grouped else "moe_gu_kernel")
        achieved = gu_bytes / (gu_us * 1e-6) / 1e9
        step_alg = sum(sum(_expert_bytes(cfg, d)) for d in per_layer)
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": _traffic(kname, name),
                    "kernel": kname, "bytes_per_launch": int(gu_bytes), "avg_us": round(gu_us, 3),
                    "timing": f"median of 5 replays of a graph of {len(timed_layers)} layers' gate/up launches",
                    "step_frac": round(step_alg / (ms_total / K * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        if grouped:
            roofline["note"] = "avg_us is the whole gate/up phase: moe_sort_kernel + moe_gu_grouped_kernel"
    cpu = None
    if not args.no_cpu:
        key = (cfg_name, T)
        cpu = None if cpu_cache is None else cpu_cache.get(key)
        if cpu is None:
            t0 = synth.make_layer(cfg, seed=args.seed, device=dev, layer=0)
            t_cpu = {k: (None if v is None else v.float().cpu().numpy() if v.dtype != torch.uint8
                         else v.cpu().numpy()) for k, v in t0.items()}
            del t0
            torch.cuda.empty_cache()
            cpu = _cpu_baseline_layer(torch, cfg, t_cpu, X[0].cpu(), args.cpu_seconds, n_layers=n_layers)
            if cpu_cache is not None:
                cpu_cache[key] = cpu
    if streamed and not staged:  # the kernels read the host tiles themselves: bytes of the last step's routing
        host_bytes_step = stack.host_bytes_of_routing(ids_cpu)
    distinct = [len(torch.unique(ids_cpu[li])) for li in range(n_layers)]
    mean_distinct = sum(distinct) / len(distinct)
    ms_per_step = ms_total / K
    step_bytes = n_layers * sum(_expert_bytes(cfg, mean_distinct))
    extra = {}
    if streamed:
        host_gb = sum(st.host_bytes for st in stack.stores) / 1e9
        pcie = host_bytes_step / (ms_per_step * 1e-3) / 1e9
        extra = {"host_resident_GB": round(host_gb, 2), "host_bytes_per_step": int(host_bytes_step),
                 "pcie_GBps": round(pcie, 1), "pcie_frac": round(pcie / PCIE_PEAK_GBS, 4),
                 "host_mode": args.host_mode,
                 "note": {"stage": "PCIe-inclusive: every host block of the chosen experts DMA-copied per layer at "
                                   "once over 4 copy streams; eager, one host sync per layer",
                          "prefetch": "PCIe-inclusive: host blocks through BlockPrefetcher (depth 4, 512-row blocks, "
                                      "arena of 5 blocks), DMA copies on side streams into staging slots; eager, one "
                                      "host sync per layer",
                          "read": "PCIe-inclusive: the kernels read pinned host tiles over PCIe; one graph per step, "
                                  "no host sync; host bytes from the last step's routing"}[args.host_mode]}
        if args.host_mode == "prefetch":
            extra["prefetch"] = stack.prefetch_stats()
        # a step reading 25% of its expert bytes from pinned host RAM is PCIe-bound: its roofline is the link's
        roofline = {"bound": "pcie", "achieved": round(pcie, 1), "peak": PCIE_PEAK_GBS, "unit": "GB/s",
                    "frac": round(pcie / PCIE_PEAK_GBS, 4), "traffic": None,
                    "kernel": f"whole step ({args.host_mode}: host blocks over PCIe)",
                    "bytes_per_launch": int(host_bytes_step), "avg_us": round(ms_per_step * 1e3, 1),
                    "timing": "the step's host bytes over its median time; peak = PCIe Gen5 x16, one direction"}
    return {
        "metric": f"MoE-FFN stack tok/s ({n_layers} GPT-OSS-120B-shaped MXFP4 layers, T={T}"
                  + (", 25% of blocks from pinned host RAM)" if streamed else ")"),
        "value": round(K * T / (ms_total / 1e3), 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": _dtype_label(cfg, "t64", False),
        "data": "synthetic (seeded MXFP4 experts per layer, x~N(0,1)); all expert slabs resident in HBM",
        "config": {"workload": f"gpt-oss-120b FFN stack, {n_layers} layers, T={T} (BASELINE config "
                               + ("5b)" if streamed else "5)"),
                   "tokens_per_step": T, "layers": n_layers, "layout": args.layout, "dispatch": args.dispatch,
                   "graph": not staged, "chain": "x <- x + moe_l(rms_norm(x)), unit norm weight, eps 1e-5",
                   "decode_chain": bool(T == 1 and not staged and stack.decode_chain and stack._chain_ok())},
        "resident_GB": round(n_layers * cfg.n_expert * sum(cfg.expert_bytes(k) for k in ("gate", "up", "down"))
                             / 1e9 - extra.get("host_resident_GB", 0.0), 2),
        **extra,
        "distinct_experts_per_layer": round(mean_distinct, 2),
        "expert_GBps": round(step_bytes / (ms_per_step * 1e-3) / 1e9, 1),
        "roofline_tok_s": round(T / (step_bytes / (HBM_PEAK_GBS * 1e9)), 1),
        "timing": {"replays" if tm else "steps": tm.n if tm else K, "ms_per_step_min_med_max": spread,
                   "wall_s": round(wall_s, 4)},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }


def gemv_workload(args, torch, N, synth, dev):
    """One token through a raw GGUF matrix per step (nsx_fused_gemv, T=1): BASELINE config 1's
    Q4_0 4096 x 4096 GEMV, or an LM-head-shaped matrix."""
    name = args.workload
    fmt_name, T, K0, W0, L0, _ = _DEFAULTS[name]
    rows, K, model = _LMHEAD[name]
    K_steps = args.steps if args.steps is not None else K0
    W = args.warmup if args.warmup is not None else W0
    n_copies = max(1, args.layers if args.layers is not None else L0)
    t = getattr(synth.GGMLType, fmt_name)
    raws = [synth.matrix_bytes(t, rows, K, synth.generator(synth.layer_seed(args.seed, i), dev), dev)
            for i in range(n_copies)]
    nbytes = raws[0].numel()
    xs = synth.activations(W + K_steps, K, seed=args.seed + 1, device=dev)
    ys = torch.empty((W + K_steps, rows), dtype=torch.float32, device=dev)
    lib = N.load()

    def run_steps(rng):
        s = N.stream_ptr(dev)
        for i in rng:
            N.check(lib.nsx_fused_gemv(int(t), raws[i % n_copies].data_ptr(), rows, K, xs[i].data_ptr(), N.DT_F32,
                                       1, ys[i].data_ptr(), s), "fused_gemv")

    tm = _graph_time(torch, run_steps, W, K_steps, args.replays)
    ms, wall_s = tm.ms, tm.wall_s
    us = ms * 1e3 / K_steps
    # parity spot check of the timed outputs against the oracle (a row block)
    from oracle import quant as OQ
    rb = OQ.row_bytes(int(t), K)
    i = W + K_steps - 1
    raw_i = raws[i % n_copies][:512 * rb].cpu().numpy()
    ref = OQ.gemv(raw_i, int(t), xs[i:i + 1].cpu().numpy(), 512, K, f64=True)[0]
    got = ys[i, :512].cpu().numpy()
    import numpy as np
    err = float(np.max(np.abs(got - ref)) / max(1e-30, float(np.max(np.abs(ref)))))
    if err > 1e-3:
        raise RuntimeError(f"{name}: timed outputs differ from the oracle (max rel err {err:.3g})")
    # algorithmic bytes per launch: the quantized matrix, x and y in fp32 (9,469,952 B at config 1)
    alg_bytes = nbytes + 4 * K + 4 * rows
    config1 = name == "q4_0-gemv"
    cpu = None
    if not args.no_cpu:
        cpu = _cpu_baseline_gemv(torch, raws[0].cpu().numpy(), t, xs[0:1].cpu(), rows, K, args.cpu_seconds,
                                 unit="GB/s" if config1 else "tok/s", nbytes=alg_bytes)
    achieved = alg_bytes / (us * 1e-6) / 1e9
    kname = f"gemv_raw_kernel<{int(t)}, 1, true>"
    out = {
        "metric": (f"{fmt_name} dequant-GEMV HBM GB/s ({rows}x{K}, T=1, fused GEMV)" if config1 else
                   f"LM-head decode tok/s ({model} shape, {fmt_name} raw GGUF rows, fused GEMV)"),
        "value": round(achieved, 1) if config1 else round(1e6 / us, 1), "unit": "GB/s" if config1 else "tok/s",
        "n_gpus": 1, "steps": K_steps, "warmup": W,
        "ms_per_step": round(us * 1e-3, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": f"{fmt_name.lower()} weights dequantized in registers x fp32 activations, fp32 accumulate",
        "data": "synthetic",
        "config": {"workload": (f"{model}, {fmt_name}, T=1 ({n_copies} rotating weight copies, "
                                f"{n_copies * nbytes / 1e6:.0f} MB)" if config1 else
                                f"{model} LM head {rows} x {K} {fmt_name}, T=1 ({n_copies} alternating copies)"),
                   "rows": rows, "K": K, "T": 1, "graph": True},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": _traffic(kname, name),
                     "kernel": kname, "bytes_per_launch": alg_bytes, "avg_us": round(us, 3),
                     "timing": f"HIP events around a graph of {K_steps} launches on the launching stream"},
        "parity_max_rel_err": err,
        "timing": {"replays": tm.n, "ms_per_step_min_med_max": tm.spread(), "wall_s": round(wall_s, 4)},
        "cpu_baseline": cpu,
    }
    return out


def _fs_of(path):
    """(mount point, file system type) holding `path`, from /proc/mounts."""
    best = ("", "?")
    try:
        with open("/proc/mounts") as f:
            for line in f:
                parts = line.split()
                if len(parts) >= 3 and str(path).startswith(parts[1]) and len(parts[1]) >= len(best[0]):
                    best = (parts[1], parts[2])
    except OSError:
        pass
    return best


def disk_workload(args, torch, N, synth, dev):
    """Expert blocks from a GGUF on disk into HBM: the reader's raw rate, then decode tokens."""
    import shutil
    import tempfile
    import numpy as np
    from nurostream_amd.compute.blockffn import BlockPrefetcher, stream_expert_ffn
    from nurostream_amd.format.gguf import GGUFWriter, row_geometry, tensor_info
    from nurostream_amd.io.arena import Arena
    from nurostream_amd.io.reader import DiskReader
    from nurostream_amd.io.stream import DiskSource
    from oracle import moe as OM
    from oracle import quant as OQ
    cfg = synth.GPTOSS_120B
    K_steps = args.steps if args.steps is not None else _DEFAULTS["disk-stream"][2]
    W = args.warmup if args.warmup is not None else _DEFAULTS["disk-stream"][3]
    block_rows = 512
    tmp = tempfile.mkdtemp(prefix="nsx_disk_", dir=os.environ.get("NSX_DISK_DIR") or None)
    path = os.path.join(tmp, "layer.gguf")
    try:
        t = synth.make_layer(cfg, seed=args.seed, device="cpu")
        gw = GGUFWriter(path, "gpt-oss")
        names = {}
        for kind in ("gate", "up", "down"):
            rows, K = cfg.rows_K(kind)
            nm = f"blk.0.ffn_{kind}_exps.weight"
            gw.add_tensor(nm, (cfg.n_expert, rows, K), synth.GGMLType.MXFP4, t[kind].numpy())
            gw.add_tensor(f"blk.0.ffn_{kind}_exps.bias", (cfg.n_expert, rows), synth.GGMLType.F32,
                          t[kind + "_b"].reshape(-1).numpy().view(np.uint8))
            names[kind] = nm
        gw.write()
        del gw
        mount, fstype = _fs_of(os.path.realpath(path))
        src0 = DiskSource(path, Arena(1 << 30), n_workers=1, device="cpu")
        infos = {k: src0.gguf.tensors[names[k]] for k in names}
        spans = []
        for info in infos.values():
            n_rows, _, rb = row_geometry(info)
            off = src0.gguf.file_offset(info)
            spans += [(off + r0 * rb, min(block_rows, n_rows - r0) * rb) for r0 in range(0, n_rows, block_rows)]
        src0.close()
        total = sum(n for _, n in spans)

        def raw_rate(direct):
            with DiskReader(path, n_workers=16, device=dev, direct=direct) as r:
                window, futs, t0 = 64, [], time.perf_counter()
                for span in spans:
                    futs.append(r.submit(*span))
                    if len(futs) >= window:
                        r.wait(futs.pop(0))
                for f in futs:
                    r.wait(f)
                torch.cuda.synchronize()
                dt = time.perf_counter() - t0
                return {"GBps": round(total / dt / 1e9, 3), "seconds": round(dt, 3), "direct": r.direct,
                        "blocks": len(spans), "bytes": total}

        rates = {"o_direct": raw_rate(True), "buffered": raw_rate(False)}

        # decode tokens through the layer, every expert block from the file
        src = DiskSource(path, Arena(256 << 20), n_workers=16, device=dev)
        xs = synth.activations(W + K_steps, cfg.n_embd, seed=args.seed + 7, device="cpu")
        rng = np.random.default_rng(args.seed)

        def act_t(g, u):
            gc = torch.clamp(g, max=7.0)
            uc = torch.clamp(u, -7.0, 7.0)
            return (uc + 1) * (gc * torch.sigmoid(1.702 * gc))

        def step(i):
            experts = sorted(rng.choice(cfg.n_expert, cfg.top_k, replace=False).tolist())
            plan = [(names[k], e * r, (e + 1) * r) for e in experts
                    for k, r in (("gate", cfg.n_ff), ("up", cfg.n_ff), ("down", cfg.n_embd))]
            x = xs[i:i + 1].to(dev)
            with BlockPrefetcher(src, plan, block_rows=block_rows, depth=24) as pf:
                ys = [stream_expert_ffn(src, "blk.0.", e, x, cfg.n_ff, cfg.n_embd, act_t, block_rows=block_rows,
                                        device=dev, bias=True, lookahead=2, prefetcher=pf) for e in experts]
            return experts, ys

        for i in range(W):
            step(i)
        torch.cuda.synchronize()
        st0 = src.stats
        t0 = time.perf_counter()
        last = None
        for i in range(W, W + K_steps):
            last = (i, step(i))
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        st1 = src.stats
        # parity of the last token's expert outputs against the oracle
        i, (experts, ys) = last
        ex = OM.ExpertSet(OQ.MXFP4, cfg.n_embd, cfg.n_ff, {k: t[k].numpy() for k in ("gate", "up", "down")},
                          {k: t[k + "_b"].numpy() for k in ("gate", "up", "down")})
        err = 0.0
        for e, y in zip(experts, ys):
            ref = OM.expert_ffn(ex, e, xs[i:i + 1].numpy(), lambda g, u: OM.clamped_swiglu(g, u),
                                block_rows=block_rows)
            err = max(err, float(np.max(np.abs(y.cpu().numpy() - ref)) / max(1e-30, float(np.max(np.abs(ref))))))
        if err > 1e-3:
            raise RuntimeError(f"disk-stream: expert outputs differ from the oracle (max rel err {err:.3g})")
        direct = src.reader.direct
        src.close()
        tok_bytes = cfg.top_k * sum(cfg.expert_bytes(k) for k in ("gate", "up", "down"))
        ms = dt * 1e3 / K_steps
        return {
            "metric": "MoE-FFN decode tok/s with every expert block read from disk (GPT-OSS-120B shape, MXFP4)",
            "value": round(K_steps / dt, 3), "unit": "tok/s", "n_gpus": 1, "steps": K_steps, "warmup": W,
            "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "mxfp4 weights x fp32 activations", "data": "synthetic (a GGUF written to the box's disk)",
            "config": {"workload": "gpt-oss-120b MoE layer experts from a GGUF file on disk, T=1, 512-row blocks",
                       "block_rows": block_rows, "prefetch_depth": 24, "n_workers": 16, "file_bytes":
                       os.path.getsize(path), "fs": fstype, "mount": mount, "o_direct": direct},
            "expert_bytes_per_token": tok_bytes,
            "disk_GBps_during_decode": round((st1.bytes_read - st0.bytes_read) / dt / 1e9, 3),
            "reader_raw": rates,
            "stall_seconds": round(st1.stall_seconds - st0.stall_seconds, 4),
            "parity_max_rel_err": err,
            "roofline": None,
            "cpu_baseline": None,
        }
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


class _ModelIndex:
    """A GGUF-like index (tensors + metadata) for a model built in memory."""

    def __init__(self, tensors, metadata):
        self.tensors, self.metadata = tensors, metadata

    def arch(self):
        return "gpt-oss"

    def cfg(self, suffix, default=None):
        return self.metadata.get(f"gpt-oss.{suffix}", default)


def token_workload(args, torch, N, synth, dev):
    """One GPT-OSS-120B decode token (every layer's attention and MoE FFN, LM head) per graph replay."""
    import math
    from nurostream_amd.format.gguf import GGMLType, tensor_info
    from nurostream_amd.io.arena import Arena
    from nurostream_amd.io.source import HostSource
    from nurostream_amd.model.decode import DeviceKV
    from nurostream_amd.model.gpt_oss import GptOssDecodeGraph, GptOssFFNStack, GptOssModel, MoEModelConfig
    from nurostream_amd.residency.cache import TieredCache
    cfg = synth.GPTOSS_120B
    K_steps = args.steps if args.steps is not None else _DEFAULTS["gptoss-token"][2]
    W = args.warmup if args.warmup is not None else _DEFAULTS["gptoss-token"][3]
    n_layers = args.layers if args.layers is not None else _DEFAULTS["gptoss-token"][4]
    n_head, n_kv, hd, vocab, window = 64, 8, 64, 201088, 128
    ctx0 = max(0, int(args.context))
    meta = {"gpt-oss.embedding_length": cfg.n_embd, "gpt-oss.block_count": n_layers,
            "gpt-oss.attention.head_count": n_head, "gpt-oss.attention.head_count_kv": n_kv,
            "gpt-oss.attention.key_length": hd, "gpt-oss.rope.freq_base": 150000.0,
            "gpt-oss.context_length": 131072, "gpt-oss.attention.sliding_window": window,
            "gpt-oss.rope.scaling.factor": 32.0, "gpt-oss.rope.scaling.original_context_length": 4096,
            "gpt-oss.rope.scaling.yarn_beta_fast": 32.0, "gpt-oss.rope.scaling.yarn_beta_slow": 1.0}
    g = synth.generator(synth.layer_seed(args.seed, 999), dev)
    infos, tensors = {}, {}

    def add(name, shape, dtype, data):
        infos[name] = tensor_info(name, shape, dtype)
        tensors[name] = (infos[name], data.reshape(-1).view(torch.uint8))

    def q8(rows, K):
        return synth.matrix_bytes(GGMLType.Q8_0, rows, K, g, dev, d_std=0.02)

    def f32(n, scale=0.1, base=0.0):
        return (torch.randn(n, generator=g, device=dev) * scale + base).float()

    add("token_embd.weight", (vocab, cfg.n_embd), GGMLType.Q8_0, q8(vocab, cfg.n_embd))
    add("output.weight", (vocab, cfg.n_embd), GGMLType.Q8_0, q8(vocab, cfg.n_embd))
    add("output_norm.weight", (cfg.n_embd,), GGMLType.F32, f32(cfg.n_embd, 0.05, 1.0))
    for li in range(n_layers):
        p = f"blk.{li}."
        add(p + "attn_norm.weight", (cfg.n_embd,), GGMLType.F32, f32(cfg.n_embd, 0.05, 1.0))
        add(p + "post_attention_norm.weight", (cfg.n_embd,), GGMLType.F32, f32(cfg.n_embd, 0.05, 1.0))
        for nm, rows, K in (("attn_q", n_head * hd, cfg.n_embd), ("attn_k", n_kv * hd, cfg.n_embd),
                            ("attn_v", n_kv * hd, cfg.n_embd), ("attn_output", cfg.n_embd, n_head * hd)):
            add(p + nm + ".weight", (rows, K), GGMLType.Q8_0, q8(rows, K))
            add(p + nm + ".bias", (rows,), GGMLType.F32, f32(rows))
        add(p + "attn_sinks.weight", (n_head,), GGMLType.F32, f32(n_head, 1.0))
    src = HostSource(tensors, Arena(1 << 30), device=dev, pin=False)
    src.gguf = _ModelIndex(infos, meta)
    cache = TieredCache(src, device=dev, vram_budget=1 << 40)
    for name in infos:
        assert cache.admit_vram(name), name
    dense_bytes = sum(i.nbytes for i in infos.values())
    mcfg = MoEModelConfig(n_layer=n_layers, n_embd=cfg.n_embd, n_expert=cfg.n_expert, n_expert_used=cfg.top_k,
                          n_ffn_expert=cfg.n_ff, rms_eps=1e-5)
    model = GptOssModel(cache, mcfg, dev)
    stack = GptOssFFNStack.synthetic(cfg, n_layers, seed=args.seed, device=dev)
    model._fused = dict(enumerate(stack.layers))
    del tensors
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    acfg = model.attn_config()
    kv = DeviceKV(n_layers, acfg, ctx0 + W + K_steps + 2, dev)
    for t in (*kv.k, *kv.v):  # a synthetic history of ctx0 positions
        t[:, :ctx0].normal_(0.0, 0.5, generator=g)
    kv.pos.fill_(ctx0)
    kv.length = ctx0
    graph = GptOssDecodeGraph(model, kv)
    toks = torch.randint(0, vocab, (W + K_steps,), generator=torch.Generator().manual_seed(args.seed)).tolist()
    for i in range(W):
        graph.step(toks[i], record=False)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_wall = time.perf_counter()
    ev0.record()
    for i in range(W, W + K_steps):
        logits = graph.step(toks[i], record=False)
    ev1.record()
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - t_wall
    ms = ev0.elapsed_time(ev1) / K_steps
    if not bool(torch.isfinite(logits).all()):
        raise RuntimeError("gptoss-token: non-finite logits")
    # bytes a token must read: 4 experts per layer (+ router, biases), attention weights, the KV history
    # (full-attention odd layers read every position, sliding even layers the last 128), the LM head
    ctx_mid = ctx0 + W + K_steps // 2
    full_layers, sliding_layers = n_layers // 2, n_layers - n_layers // 2
    kv_bytes = (full_layers * (ctx_mid + 1) + sliding_layers * min(window, ctx_mid + 1)) * n_kv * hd * 4 * 2
    attn_bytes = sum(i.nbytes for n, i in infos.items() if n.startswith("blk."))
    token_bytes = n_layers * cfg.layer_bytes_per_token() + attn_bytes + infos["output.weight"].nbytes + kv_bytes
    achieved = token_bytes / (ms * 1e-3) / 1e9
    return {
        "metric": "GPT-OSS-120B decode tok/s, whole token on the device as one graph (T=1)",
        "value": round(1e3 / ms, 1), "unit": "tok/s", "n_gpus": 1, "steps": K_steps, "warmup": W,
        "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "mxfp4 experts, q8_0 dense weights, fp32 activations and KV", "data": "synthetic",
        "config": {"workload": f"gpt-oss-120b decode token, {n_layers} layers, {ctx0} positions in the KV cache",
                   "n_layers": n_layers, "context": ctx0, "n_head": n_head, "n_kv": n_kv, "head_dim": hd,
                   "vocab": vocab, "sliding_window": window, "dense_type": "Q8_0",
                   "dense_bytes": dense_bytes, "kv_cache_bytes": kv.nbytes()},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "whole token",
                     "algorithmic_bytes": int(token_bytes)},
        "wall_s": round(wall_s, 4),
        "cpu_baseline": None,
    }


_SUBCONFIGS = (("1", "q4_0-gemv"), ("3", "gptoss-t128"), ("4_t1", "qwen3-t1"), ("4_t32", "qwen3-t32"),
               ("5_t1", "stack-t1"), ("5_t8", "stack-t8"), ("5b_t1", "stack-t1-host25"))


def _compact(r):
    """The figures of one workload's line that the sub-config summary keeps."""
    lo, _, hi = r["timing"]["ms_per_step_min_med_max"]
    out = {"ms_per_step": r["ms_per_step"], "value": r["value"], "unit": r["unit"], "spread": [lo, hi]}
    rf = r.get("roofline")
    if rf:
        out["roofline"] = {"kernel": rf["kernel"], "bytes_per_launch": rf.get("bytes_per_launch"),
                           "avg_us": rf.get("avg_us"), "frac": rf["frac"]}
        if rf.get("traffic") and rf.get("bytes_per_launch"):
            out["roofline"]["traffic_x"] = round(rf["traffic"] / rf["bytes_per_launch"], 3)
    cb = r.get("cpu_baseline")
    if cb:
        out["cpu_baseline"] = {"value": cb["value"], "cores": cb["cores"],
                               "ms_per_step": cb.get("ms_per_step", cb.get("ms_per_pass"))}
    for k in ("distinct_experts_per_step", "distinct_experts_per_layer", "pcie_GBps", "pcie_frac"):
        if k in r:
            out[k] = r[k]
    return out


def run_configs(args, torch, N, synth, dev):
    """BASELINE configs 1, 3, 4 (T=1, 32), 5 (T=1, 8) and 5b (T=1: the kernels
    reading the host blocks over PCIe, and the blocks staged through
    BlockPrefetcher at depth 4), each at its workload's default steps, with a
    short CPU baseline: {key: compact result}."""
    import copy
    import gc

    def sub(workload, **kw):
        a = copy.copy(args)
        a.workload, a.steps, a.warmup, a.layers, a.profile_steps = workload, None, None, None, None
        a.cpu_seconds, a.no_probe, a.copy_probe_mib = args.sub_cpu_seconds, True, 0
        for k, v in kw.items():
            setattr(a, k, v)
        return a

    def free():
        gc.collect()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()

    t0 = time.perf_counter()
    out = {}
    for key, wl in _SUBCONFIGS[:4]:
        r = (gemv_workload if wl == "q4_0-gemv" else layer_workload)(sub(wl), torch, N, synth, dev)
        out[key] = _compact(r)
        del r
        free()
    cache = {}
    stack = build_stack(sub("stack-t1"), torch, synth, dev, "stack-t1")
    for key, wl in _SUBCONFIGS[4:6]:
        out[key] = _compact(stack_workload(sub(wl), torch, N, synth, dev, stack=stack, cpu_cache=cache))
    del stack
    free()
    hs = build_stack(sub("stack-t1-host25", host_mode="read"), torch, synth, dev, "stack-t1-host25")
    r = _compact(stack_workload(sub("stack-t1-host25", host_mode="read"), torch, N, synth, dev, stack=hs,
                                cpu_cache=cache))
    pf = stack_workload(sub("stack-t1-host25", host_mode="prefetch"), torch, N, synth, dev, stack=hs,
                        cpu_cache=cache)
    lo, _, hi = pf["timing"]["ms_per_step_min_med_max"]
    r["prefetch"] = {"ms_per_step": pf["ms_per_step"], "value": pf["value"], "pcie_GBps": pf["pcie_GBps"],
                     "pcie_frac": pf["pcie_frac"], "spread": [lo, hi], "hits": pf["prefetch"]["hits"],
                     "blocks": pf["prefetch"]["blocks"]}
    out["5b_t1"] = r
    del hs, pf
    free()
    out["wall_s"] = round(time.perf_counter() - t0, 1)
    return out


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

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    N.ensure_selftest(dev)
    if args.workload.startswith("stack"):
        result = stack_workload(args, torch, N, synth, dev)
    elif args.workload.startswith("lmhead") or args.workload == "q4_0-gemv":
        result = gemv_workload(args, torch, N, synth, dev)
    elif args.workload == "disk-stream":
        result = disk_workload(args, torch, N, synth, dev)
    elif args.workload == "gptoss-token":
        result = token_workload(args, torch, N, synth, dev)
    else:
        result = layer_workload(args, torch, N, synth, dev)
        if args.workload == "gptoss-decode" and args.configs == "all":
            result["configs"] = run_configs(args, torch, N, synth, dev)
    if args.copy_probe_mib > 0:  # a plain copy of known size for the counter calibration
        n = args.copy_probe_mib << 18
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    print(json.dumps(result, separators=(",", ":")), flush=True)


if __name__ == "__main__":
    main()
