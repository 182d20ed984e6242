#!/usr/bin/env python3
"""rocprofv3 counter passes over bench.py workloads -> profiles/pmc_traffic.json
and profiles/pmc_counters.md.

    python bench_pmc.py [--workloads gptoss-decode,gptoss-t128,...] [--raw DIR]

Run on the GPU box from the repository root, after building the library.
This process never touches the GPU: every pass is a child process,
`rocprofv3 <pass> -- python3 bench.py --workload W --configs none --no-cpu
--no-probe --copy-probe-mib 256 --replays 3`, run from /tmp with TMPDIR=/tmp
and a time limit of its own. The passes, each its own run (rocprofv3 does
not split counters over runs):

  trace   --kernel-trace --stats: average duration per kernel
  fetch   --pmc FETCH_SIZE  (KiB the L2 read from memory, per dispatch)
  write   --pmc WRITE_SIZE  (KiB the L2 wrote to memory, per dispatch)
  sq      --pmc SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_VALU_MFMA_MOPS_F6F4
          SQ_INSTS_VALU_MFMA_MOPS_F16 SQ_INSTS_VMEM_RD SQ_INSTS_LDS
          SQ_LDS_BANK_CONFLICT SQ_WAVES GRBM_GUI_ACTIVE
  util    --pmc MfmaUtil VALUBusy  (rocprofv3's derived metrics:
          100 * sum(SQ_VALU_MFMA_BUSY_CYCLES) / (max(GRBM_GUI_ACTIVE) * SIMDs),
          100 * sum(SQ_ACTIVE_INST_VALU) / CUs / max(GRBM_GUI_ACTIVE))
  mfma    --pmc SQ_INSTS_VALU_MFMA_F6F4 SQ_INSTS_VALU_MFMA_F8
          SQ_INSTS_VALU_MFMA_I8 SQ_INSTS_VALU_MFMA_F32
          SQ_INSTS_VALU_MFMA_MOPS_F8 SQ_INSTS_VALU_MFMA_MOPS_I8
          SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CU_CYCLES GRBM_GUI_ACTIVE
          (MFMA instructions by operand type -- the block-scaled FP4 x FP8
          MFMA counts as F6F4 or F8 by its operand formats -- and the
          matrix cores' busy cycles against the CUs' busy cycles)

Every bench run ends with a plain 256 MiB device copy; its FETCH_SIZE and
WRITE_SIZE against the 262,144 KiB it moves give the factors that turn the
byte counters into bytes (on gfx950 FETCH_SIZE reads half of a copy's bytes,
WRITE_SIZE all of them). Traffic per launch = fetch KiB * 1024 * fetch factor
+ write KiB * 1024 * write factor, averaged over the kernel's dispatches in
that workload.

The JSON records the digest of nurostream_amd/csrc the counters were taken
on (bench.csrc_digest); bench.py reports `roofline.traffic` only while the
sources still have that digest.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import subprocess
import sys
import time
from collections import defaultdict

ROOT = os.path.dirname(os.path.abspath(__file__))
PASSES = {
    "trace": ["--kernel-trace", "--stats"],
    "fetch": ["--pmc", "FETCH_SIZE"],
    "write": ["--pmc", "WRITE_SIZE"],
    "sq": ["--pmc", "SQ_INSTS_VALU", "SQ_INSTS_MFMA", "SQ_INSTS_VALU_MFMA_MOPS_F6F4", "SQ_INSTS_VALU_MFMA_MOPS_F16",
           "SQ_INSTS_VMEM_RD", "SQ_INSTS_LDS", "SQ_LDS_BANK_CONFLICT", "SQ_WAVES", "GRBM_GUI_ACTIVE"],
    "util": ["--pmc", "MfmaUtil", "VALUBusy"],
    "mfma": ["--pmc", "SQ_INSTS_VALU_MFMA_F6F4", "SQ_INSTS_VALU_MFMA_F8", "SQ_INSTS_VALU_MFMA_I8",
             "SQ_INSTS_VALU_MFMA_F32", "SQ_INSTS_VALU_MFMA_MOPS_F8", "SQ_INSTS_VALU_MFMA_MOPS_I8",
             "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CU_CYCLES", "GRBM_GUI_ACTIVE"],
}
DEFAULT_WORKLOADS = ("gptoss-decode", "gptoss-t128", "qwen3-t1", "qwen3-t32", "q4_0-gemv", "stack-t1", "stack-t8")
# the stacks launch ~110 kernels a step: fewer steps keep the dispatches under counter collection few
STEPS = {"stack-t1": ["--steps", "4", "--warmup", "1"], "stack-t8": ["--steps", "2", "--warmup", "1"]}
COPY_KIB = 262144.0  # the 256 MiB calibration copy reads and writes this many KiB
COPY_KERNEL = "copyBuffer"


def kernel_base(name: str) -> str:
    """A demangled kernel name without its return type and parameter list
    ('void moe_gu_grouped_kernel<false>(MoeDev)' -> 'moe_gu_grouped_kernel<false>')."""
    name = name.strip()
    if name.startswith("void "):
        name = name[5:]
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            return name[:i].strip()
    return name


def run_pass(workload: str, pas: str, raw: str, timeout: int) -> str:
    out = os.path.join(raw, f"{workload}_{pas}")
    os.makedirs(out, exist_ok=True)
    cmd = ["rocprofv3", *PASSES[pas], "--output-format", "csv", "-d", out, "-o", "p", "--",
           sys.executable, os.path.join(ROOT, "bench.py"), "--workload", workload, "--configs", "none", "--no-cpu",
           "--no-probe", "--copy-probe-mib", "256", "--replays", "3", *STEPS.get(workload, [])]
    env = dict(os.environ, TMPDIR="/tmp")
    print(f"[pmc] {workload} {pas}: {' '.join(cmd)}", flush=True)
    t0 = time.time()
    with open(os.path.join(out, "run.log"), "w") as log:
        res = subprocess.run(cmd, cwd="/tmp", env=env, stdout=log, stderr=subprocess.STDOUT, timeout=timeout)
    if res.returncode not in (0, 139) or not glob.glob(os.path.join(out, "**", "*.csv"), recursive=True):
        # (rocprofv3 may end with 139 after a complete run; its CSV files then exist)
        raise RuntimeError(f"{workload} {pas}: rocprofv3 exited {res.returncode}; see {out}/run.log")
    print(f"[pmc] {workload} {pas}: done in {time.time() - t0:.1f} s", flush=True)
    return out


def read_counters(out: str):
    """({kernel: {counter: (mean over dispatches, dispatches)}}, the mean of
    each counter over the last three COPY_KERNEL dispatches -- the calibration
    copies at the end of the run) from a --pmc pass."""
    acc = defaultdict(list)
    copies = defaultdict(list)
    for fn in glob.glob(os.path.join(out, "**", "*counter_collection.csv"), recursive=True):
        with open(fn) as f:
            for i, r in enumerate(csv.DictReader(f)):
                k, c, v = kernel_base(r["Kernel_Name"]), r["Counter_Name"], float(r["Counter_Value"])
                acc[(k, c)].append(v)
                if COPY_KERNEL in k:
                    copies[c].append((int(r.get("Dispatch_Id") or i), v))
    res = defaultdict(dict)
    for (k, c), v in acc.items():
        res[k][c] = (sum(v) / len(v), len(v))
    calib = {c: sum(v for _, v in sorted(lst)[-3:]) / len(sorted(lst)[-3:]) for c, lst in copies.items()}
    return res, calib


def read_stats(out: str) -> dict:
    """{kernel: (average ns, calls)} from a --kernel-trace --stats pass."""
    res = {}
    for fn in glob.glob(os.path.join(out, "**", "*kernel_stats.csv"), recursive=True):
        with open(fn) as f:
            for r in csv.DictReader(f):
                res[kernel_base(r["Name"])] = (float(r["AverageNs"]), int(r["Calls"]))
    return res


def main() -> None:
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--workloads", default=",".join(DEFAULT_WORKLOADS))
    p.add_argument("--raw", default="/tmp/nsx_pmc", help="rocprofv3 output folder")
    p.add_argument("--json", default=os.path.join(ROOT, "profiles", "pmc_traffic.json"))
    p.add_argument("--md", default=os.path.join(ROOT, "profiles", "pmc_counters.md"))
    p.add_argument("--timeout", type=int, default=150, help="seconds per pass")
    p.add_argument("--merge", action="store_true",
                   help="keep the workloads already in --json when it was made on the same sources (a sweep over "
                        "several runs)")
    args = p.parse_args()
    sys.path.insert(0, ROOT)
    from bench import csrc_digest

    doc = {"csrc_digest": csrc_digest(), "bench_args": "--configs none --no-cpu --no-probe --copy-probe-mib 256 "
           "--replays 3 (each workload's default steps; " + "; ".join(f"{w}: {' '.join(a)}" for w, a in STEPS.items())
           + ")", "passes": {k: " ".join(v) for k, v in PASSES.items()},
           "workloads": {}}
    if args.merge and os.path.exists(args.json):
        with open(args.json) as f:
            old = json.load(f)
        if old.get("csrc_digest") == doc["csrc_digest"] and old.get("passes") == doc["passes"]:
            doc["workloads"] = old.get("workloads", {})
        else:
            print(f"[pmc] {args.json} was made on other sources or passes: starting afresh", flush=True)
    for w in args.workloads.split(","):
        got = {pas: run_pass(w, pas, args.raw, args.timeout) for pas in PASSES}
        stats = read_stats(got["trace"])
        cnt, calib = {}, {}
        for pas in ("fetch", "write", "sq", "util", "mfma"):
            cnt[pas], calib[pas] = read_counters(got[pas])
        if "FETCH_SIZE" not in calib["fetch"] or "WRITE_SIZE" not in calib["write"]:
            raise RuntimeError(f"{w}: no {COPY_KERNEL} dispatch to calibrate the byte counters")
        ff = COPY_KIB / calib["fetch"]["FETCH_SIZE"]
        wf = COPY_KIB / calib["write"]["WRITE_SIZE"]
        kernels = {}
        for k in sorted(set(cnt["fetch"]) | set(stats)):
            if COPY_KERNEL in k or k.startswith("__amd") or "at::" in k or "elementwise" in k.lower():
                continue
            rec = {}
            if k in stats:
                rec["avg_us"], rec["calls"] = round(stats[k][0] / 1e3, 3), stats[k][1]
            f, wr = cnt["fetch"].get(k, {}).get("FETCH_SIZE"), cnt["write"].get(k, {}).get("WRITE_SIZE")
            if f and wr:
                rec["fetch_kib"], rec["write_kib"], rec["dispatches"] = round(f[0], 2), round(wr[0], 2), f[1]
                rec["traffic_bytes"] = int(f[0] * 1024 * ff + wr[0] * 1024 * wf)
            for c, (v, _) in sorted(cnt["sq"].get(k, {}).items()):
                rec[c] = round(v, 1)
            for c, (v, _) in sorted(cnt["util"].get(k, {}).items()):
                rec[c] = round(v, 3)
            for c, (v, _) in sorted(cnt["mfma"].get(k, {}).items()):
                rec["mfma_pass." + c if c in rec else c] = round(v, 1)
            kernels[k] = rec
        doc["workloads"][w] = {"fetch_factor": round(ff, 5), "write_factor": round(wf, 5), "kernels": kernels}
        with open(args.json, "w") as f:  # after every workload, so a later failure keeps what was measured
            json.dump(doc, f, indent=1)
    write_md(doc, args.md)
    print(f"[pmc] wrote {args.json} and {args.md}", flush=True)


def write_md(doc: dict, path: str) -> None:
    lines = ["# rocprofv3 counters per kernel and workload",
             "",
             f"Made by `python bench_pmc.py` (sources digest {doc['csrc_digest']}): for each workload, six rocprofv3 "
             f"runs of `bench.py --workload W {doc['bench_args']}`, one per pass:",
             ""]
    lines += [f"- {k}: `rocprofv3 {v} --output-format csv -- python3 bench.py ...`" for k, v in doc["passes"].items()]
    lines += ["",
              "traffic x = (FETCH_SIZE x fetch factor + WRITE_SIZE x write factor) per dispatch over the kernel's "
              "algorithmic bytes where bench.py states them (the factors from the run's own 256 MiB copy). "
              "MfmaUtil and VALUBusy are rocprofv3's derived metrics (percent of the kernel's active cycles; they "
              "are taken with counters attached, so durations there run long).",
              ""]
    for w, rec in doc["workloads"].items():
        lines += [f"## {w}", "", f"fetch factor {rec['fetch_factor']}, write factor {rec['write_factor']}", "",
                  "| kernel | calls | avg us | traffic MB | VALU instr | MFMA instr | F6F4 / F8 / I8 / F32 MFMA instr "
                  "| MFMA busy / CU busy cycles | MfmaUtil % | VALUBusy % |",
                  "|---|---|---|---|---|---|---|---|---|---|"]
        for k, r in sorted(rec["kernels"].items(), key=lambda kv: -kv[1].get("avg_us", 0) * kv[1].get("calls", 0)):
            tb = r.get("traffic_bytes")
            mix = " / ".join(str(r.get(f"SQ_INSTS_VALU_MFMA_{t}", "")) for t in ("F6F4", "F8", "I8", "F32"))
            mb, cb = r.get("SQ_VALU_MFMA_BUSY_CYCLES"), r.get("SQ_BUSY_CU_CYCLES")
            busy = f"{mb:.0f} / {cb:.0f}" if mb is not None and cb else ""
            lines.append(f"| `{k}` | {r.get('calls', '')} | {r.get('avg_us', '')} | "
                         f"{'' if tb is None else round(tb / 1e6, 2)} | {r.get('SQ_INSTS_VALU', '')} | "
                         f"{r.get('SQ_INSTS_MFMA', '')} | {mix} | {busy} | "
                         f"{r.get('MfmaUtil', '')} | {r.get('VALUBusy', '')} |")
        lines.append("")
    with open(path, "w") as f:
        f.write("\n".join(lines))


if __name__ == "__main__":
    main()
