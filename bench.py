#!/usr/bin/env python3
"""Benchmark of the block-sparse causal attention forward on one MI355X.

Metric (the reference's headline, docs/OPTIMIZATION_JOURNAL.md:16, README.md:9): geometric mean
over the three sparsity families (sliding window w=8, global prefix 4 + local 4, retrieval
diagonal + previous + 14 seeded blocks) of the median forward latency at B=2, H=16, T=8192,
D=128, fp16, plus the fraction of dense fp16 MFMA peak counting only active 128x128 blocks
(4·128^3 FLOP each).

A step is one forward call of each family on synthetic inputs already resident in HBM. Every
call is bracketed by HIP events on the launch stream; the per-family median gives the latency.

    python bench.py [--steps K] [--warmup W] [--cpu-heads N | --no-cpu]

Prints one JSON line.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time

import numpy as np
import torch

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

from usagi_amd import block_sparse_attn_fwd  # noqa: E402
from usagi_amd import patterns as P  # noqa: E402

METRIC = "geomean fwd ms @B2 H16 T8192 D128 over 3 sparsity families; % fp16 MFMA peak"
PEAK_FP16_TFLOPS = 2516.6  # MI355X dense fp16 MFMA, published
FLOP_PER_BLOCK = 4 * 128 ** 3
TRAFFIC_FILE = os.path.join(REPO, "profiles", "bsa_fwd_hbm_traffic_b2h16t8192.txt")


def geomean(xs):
    return float(math.exp(sum(math.log(x) for x in xs) / len(xs)))


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def read_traffic():
    """HBM bytes per launch of the kernel per family, from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, calibrated against a copy kernel), or None."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    out = {}
    with open(TRAFFIC_FILE) as f:
        for line in f:
            m = re.match(r"^traffic_bytes_per_launch\s+(\w+)\s+([0-9.eE+]+)", line.strip())
            if m:
                out[m.group(1)] = float(m.group(2))
    return out or None


def cpu_baseline(fams, inputs, n_heads: int):
    """The C port of the reference CSR walk (oracle/bsa_ref.c, OpenMP) on a bounded sample of
    heads (b = 0, h < n_heads) of each family, projected to the full workload by active
    blocks."""
    from oracle import c_ref

    q, k, v = inputs
    qs, ks, vs = (x[:1, :n_heads].float().numpy() for x in (q, k, v))
    per = {}
    for name, (rp, ci) in fams.items():
        rps, cis = rp[:1, :n_heads], ci[:1, :n_heads]
        t0 = time.perf_counter()
        c_ref.fwd(qs, ks, vs, rps, cis)
        dt = time.perf_counter() - t0
        per[name] = dt * 1e3 * P.active_blocks(rp) / P.active_blocks(rps)
    cores = int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)
    return {
        "value": round(geomean(list(per.values())), 3),
        "unit": "ms",
        "cores": cores,
        "kind": "port",
        "sample": (f"oracle/bsa_ref.c (C restatement of the reference CSR walk, fp32, OpenMP) on "
                   f"heads b=0,h<{n_heads} of each family, projected to B2 H16 T8192 by active "
                   f"blocks; host CPU: {cpu_model()}"),
        "per_family_ms": {k2: round(v2, 3) for k2, v2 in per.items()},
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-heads", type=int, default=4)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--seed", type=int, default=P.INPUT_SEED)
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="before the warmup, run one device copy of this many MiB (the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this path has no multi-GPU mode "
              "(B*H head sharding needs no exchange; see the design notes). Use --gpus 1.",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    wl = P.workloads()
    B, H, T, D = 2, 16, 8192, 128
    inputs = P.make_qkv(B, H, T, seed=args.seed)
    q, k, v = (x.to(dev) for x in inputs)
    fams = {}
    dev_csr = {}
    for name in P.FAMILIES:
        rp, ci = wl[name].csr()
        fams[name] = (rp, ci)
        dev_csr[name] = (torch.from_numpy(rp).to(dev), torch.from_numpy(ci).to(dev))

    if args.calib_copy_mib:
        n = args.calib_copy_mib * (1 << 20) // 4
        src = torch.ones(n, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    def call(name):
        rp, ci = dev_csr[name]
        return block_sparse_attn_fwd(q, k, v, rp, ci, None)

    for _ in range(args.warmup):
        for name in P.FAMILIES:
            call(name)
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream(dev)
    ev = {n: [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(args.steps)] for n in P.FAMILIES}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        for name in P.FAMILIES:
            a, b = ev[name][s]
            a.record(stream)
            call(name)
            b.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    fam_out = {}
    medians, means, flops = [], [], []
    for name in P.FAMILIES:
        ts = [a.elapsed_time(b) for a, b in ev[name]]
        med = float(np.median(ts))
        mean = float(np.mean(ts))
        fl = P.active_blocks(fams[name][0]) * FLOP_PER_BLOCK
        medians.append(med)
        means.append(mean)
        flops.append(fl)
        fam_out[name] = {
            "median_ms": round(med, 4),
            "mean_ms": round(mean, 4),
            "active_blocks": P.active_blocks(fams[name][0]),
            "tflops": round(fl / med / 1e9, 1),
            "frac_peak": round(fl / med / 1e9 / PEAK_FP16_TFLOPS, 4),
        }

    value = geomean(medians)
    achieved = sum(flops) / sum(means) / 1e9  # TFLOP/s: mean FLOP per launch / mean duration
    traffic = read_traffic()
    roofline = {
        "bound": "mfma",
        "achieved": round(achieved, 1),
        "peak": PEAK_FP16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / PEAK_FP16_TFLOPS, 4),
        "traffic": (round(sum(traffic[n] for n in P.FAMILIES) / len(P.FAMILIES))
                    if traffic and all(n in traffic for n in P.FAMILIES) else None),
        "kernel": "bsa_fwd_kernel<fp16>",
        "avg_launch_ms": round(sum(means) / len(means), 4),
        "algorithmic_flop_per_launch": int(sum(flops) / len(flops)),
        "geomean_frac_peak": round(geomean([f["frac_peak"] for f in fam_out.values()]), 4),
    }

    out = {
        "metric": METRIC,
        "value": round(value, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1e3 / args.steps, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {
            "workload": "block-sparse causal attention fwd, B2 H16 T8192 D128 fp16, "
                        "3 families: sliding w8 / global 4 + local 4 / retrieval diag+prev+14",
            "B": B, "H": H, "T": T, "D": D, "block": 128,
            "families": fam_out,
            "input_seed": args.seed,
            "pattern_seed": P.PATTERN_SEED,
        },
        "roofline": roofline,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(fams, inputs, args.cpu_heads)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
