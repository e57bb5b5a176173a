#!/usr/bin/env python3
"""Benchmark of the block-sparse causal attention forward on one MI355X.

Metric (the reference's headline, docs/OPTIMIZATION_JOURNAL.md:16, README.md:9): geometric mean
over the three sparsity families (sliding window w=8, global prefix 4 + local 4, retrieval
diagonal + previous + 14 seeded blocks) of the median forward latency at B=2, H=16, T=8192,
D=128, fp16, plus the fraction of dense fp16 MFMA peak counting only active 128x128 blocks
(4·128^3 FLOP each).

A step is one forward call of each family on synthetic inputs already resident in HBM. Every
call is bracketed by HIP events on the launch stream; the per-family median gives the latency.

    python bench.py [--steps K] [--warmup W] [--min-warmup-s S] [--cpu-heads N | --no-cpu]

The warmup is W steps plus, if needed, more whole steps until S seconds have passed (reported as
warmup_extra_steps): from idle the GPU takes tens of ms of sustained load to reach steady clocks.

Prints one JSON line. Besides the contract fields: per family launch_ms (mean per-call event time
of the timed steps, the roofline's launch duration) and burst_ms (back-to-back bursts, after the
timed steps); config.analytic_rows (the analytic window path against the CSR path on the sliding
and global families); config.other_workloads (the long-context mixed workload, outside the
geomean); cpu_baseline (PyTorch CPU dense-masked attention on the host, with the C walk beside
it). --pmc-summary turns rocprofv3 counter runs into per-family traffic and derived figures.
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

from usagi_amd import block_sparse_attn_fwd, block_sparse_attn_fwd_window  # noqa: E402
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


def cpu_baseline(fams, inputs, n_heads: int, c_heads: int):
    """The reference math as PyTorch CPU fp32 dense-masked attention (oracle/torch_dense.py) on
    the host cores, per family over heads b < B, h < n_heads (all heads by default: the full
    workload), projected to B2 H16 by head count when fewer heads are run. The C restatement of
    the reference's blockwise CSR walk (oracle/bsa_ref.c, OpenMP) is timed beside it on c_heads
    heads and projected by active blocks."""
    from oracle import c_ref, torch_dense

    q, k, v = inputs
    B, H = q.shape[:2]
    cores = torch.get_num_threads()
    heads = [(b, h) for b in range(B) for h in range(min(n_heads, H))]
    per, per_c = {}, {}
    for name, (rp, ci) in fams.items():
        rpt, cit = torch.from_numpy(rp), torch.from_numpy(ci)
        t0 = time.perf_counter()
        torch_dense.dense_masked(q, k, v, rpt, cit, heads=heads)
        per[name] = (time.perf_counter() - t0) * 1e3 * (B * H) / len(heads)
        if c_heads:
            qs, ks, vs = (x[:1, :c_heads].float().numpy() for x in (q, k, v))
            rps, cis = rp[:1, :c_heads], ci[:1, :c_heads]
            t0 = time.perf_counter()
            c_ref.fwd(qs, ks, vs, rps, cis)
            per_c[name] = ((time.perf_counter() - t0) * 1e3 * P.active_blocks(rp)
                           / P.active_blocks(rps))
    sample = ("all B2 H16 heads of each family (the full workload)" if len(heads) == B * H else
              f"heads b<{B}, h<{n_heads} of each family, projected to B2 H16 by head count")
    out = {
        "value": round(geomean(list(per.values())), 3),
        "unit": "ms",
        "cores": cores,
        "kind": "port",
        "sample": (f"PyTorch CPU fp32 dense-masked attention (oracle/torch_dense.py: block mask "
                   f"from the CSR, causal, query slabs of 1024 rows against keys up to the slab "
                   f"end) on {sample}; geomean over the 3 families of one run each; host CPU: "
                   f"{cpu_model()}, {cores} threads"),
        "per_family_ms": {k2: round(v2, 3) for k2, v2 in per.items()},
    }
    if per_c:
        out["blockwise_c_port"] = {
            "value": round(geomean(list(per_c.values())), 3),
            "unit": "ms",
            "sample": (f"oracle/bsa_ref.c (the reference's CSR walk in C, fp32, OpenMP) on heads "
                       f"b=0, h<{c_heads}, projected by active blocks"),
            "per_family_ms": {k2: round(v2, 3) for k2, v2 in per_c.items()},
        }
    return out


KERNEL = "bsa_fwd_dma_kernel"


def pmc_summary(paths, calib_mib: int) -> int:
    """Per-family averages of rocprofv3 --pmc counters for the attention kernel.

    Dispatches of the kernel come in family order (sliding, global, retrieval) on every warmup
    and timed step, so dispatch i belongs to FAMILIES[i % 3]. The calibration kernel is the
    last dispatch before the first attention dispatch (the elementwise -in of
    --calib-copy-mib MiB, which reads and writes exactly that many bytes); FETCH_SIZE and
    WRITE_SIZE (KiB) are each scaled by (known KiB / counter KiB) of that kernel.

    When a pass also ran with --kernel-trace, its run_kernel_trace.csv (next to the counter
    file) gives each dispatch's duration, and run_agent_info.csv the part's XCD and SIMD
    counts; the derived lines then put the counters against time: the shader clock
    (GRBM_GUI_ACTIVE is summed over the XCDs), MFMA busy share, TFLOP/s on active blocks and
    the fraction of the MFMA peak at that clock, HBM GB/s and the LDS bank-conflict rate.
    """
    import csv

    if not calib_mib:
        print("--pmc-summary needs the --calib-copy-mib value of the profiled run", file=sys.stderr)
        return 2
    known_kib = calib_mib * 1024.0
    sums: dict = {}
    durs: dict = {}
    calib: dict = {}
    calib_name = None
    n_xcc, n_simd = 8, 1024
    for path in paths:
        with open(path) as f:
            rows = list(csv.DictReader(f))
        by_disp: dict = {}
        for r in rows:
            d = int(r["Dispatch_Id"])
            by_disp.setdefault(d, {"name": r["Kernel_Name"], "ctr": {}})
            c = by_disp[d]["ctr"]
            c[r["Counter_Name"]] = c.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        trace = path.replace("counter_collection", "kernel_trace")
        dur_of: dict = {}
        if trace != path and os.path.exists(trace):
            with open(trace) as f:
                for r in csv.DictReader(f):
                    dur_of[int(r["Dispatch_Id"])] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
        agent = path.replace("counter_collection", "agent_info")
        if agent != path and os.path.exists(agent):
            with open(agent) as f:
                for r in csv.DictReader(f):
                    if r.get("Name", "").startswith("gfx"):
                        n_xcc, n_simd = int(r["Num_Xcc"]), int(r["Simd_Count"])
        order = sorted(by_disp)
        first = next(i for i, d in enumerate(order) if KERNEL in by_disp[order[i]]["name"])
        if first > 0:
            cal = by_disp[order[first - 1]]
            calib_name = cal["name"]
            calib.update(cal["ctr"])
        i = 0
        for d in order[first:]:
            e = by_disp[d]
            if KERNEL not in e["name"]:
                continue
            fam = P.FAMILIES[i % len(P.FAMILIES)]
            i += 1
            for cname, val in e["ctr"].items():
                s = sums.setdefault(fam, {}).setdefault(cname, [0.0, 0])
                s[0] += val
                s[1] += 1
            if d in dur_of:
                t = durs.setdefault(fam, [0.0, 0])
                t[0] += dur_of[d]
                t[1] += 1
    print(f"kernel {KERNEL}; calibration kernel: {calib_name}")
    for cname, val in sorted(calib.items()):
        print(f"calibration {cname} {val:.1f}")
    factor = {}
    for cname in ("FETCH_SIZE", "WRITE_SIZE"):
        if calib.get(cname):
            factor[cname] = known_kib / calib[cname]
            print(f"scale {cname} {factor[cname]:.4f}  (known {known_kib:.0f} KiB / counter "
                  f"{calib[cname]:.1f} KiB)")
    wl = P.workloads()
    for fam in P.FAMILIES:
        if fam not in sums:
            continue
        avg = {cname: tot / n for cname, (tot, n) in sums[fam].items()}
        for cname, (tot, n) in sorted(sums[fam].items()):
            print(f"avg {fam} {cname} {tot / n:.1f}  (over {n} dispatches)")
        traffic = None
        if factor.keys() == {"FETCH_SIZE", "WRITE_SIZE"} and \
                {"FETCH_SIZE", "WRITE_SIZE"} <= avg.keys():
            fk = avg["FETCH_SIZE"] * factor["FETCH_SIZE"]
            wk = avg["WRITE_SIZE"] * factor["WRITE_SIZE"]
            traffic = (fk + wk) * 1024
            print(f"traffic_bytes_per_launch {fam} {traffic:.0f}  "
                  f"(read {fk * 1024:.0f} + write {wk * 1024:.0f})")
        if fam not in durs:
            continue
        dur_ns = durs[fam][0] / durs[fam][1]
        flop = P.active_blocks(wl[fam].csr()[0]) * 4 * P.BLOCK ** 3
        tflops = flop / dur_ns / 1e3
        print(f"derived {fam} duration_us {dur_ns / 1e3:.1f}  (kernel trace of the counter passes, "
              f"{durs[fam][1]} dispatches)  tflops_active {tflops:.1f}")
        if avg.get("GRBM_GUI_ACTIVE"):
            cyc = avg["GRBM_GUI_ACTIVE"] / n_xcc
            ghz = cyc / dur_ns
            peak_at_clock = ghz * 1e9 * n_simd * 1024 / 1e12  # 1024 fp16 FLOP/clk per SIMD
            print(f"derived {fam} clock_ghz {ghz:.3f}  (GRBM_GUI_ACTIVE / {n_xcc} XCDs / duration)  "
                  f"mfma_peak_at_clock_tflops {peak_at_clock:.0f}  "
                  f"frac_of_peak_at_clock {tflops / peak_at_clock:.3f}")
            if avg.get("SQ_VALU_MFMA_BUSY_CYCLES") is not None:
                print(f"derived {fam} mfma_busy {avg['SQ_VALU_MFMA_BUSY_CYCLES'] / (cyc * n_simd):.3f}  "
                      f"(SQ_VALU_MFMA_BUSY_CYCLES / ({n_simd} SIMDs x cycles))")
        if avg.get("SQ_VALU_MFMA_COEXEC_CYCLES") is not None and avg.get("SQ_VALU_MFMA_BUSY_CYCLES"):
            print(f"derived {fam} valu_coexec_share_of_mfma_busy "
                  f"{avg['SQ_VALU_MFMA_COEXEC_CYCLES'] / avg['SQ_VALU_MFMA_BUSY_CYCLES']:.3f}")
        if avg.get("SQ_LDS_IDX_ACTIVE") and "SQ_LDS_BANK_CONFLICT" in avg:
            print(f"derived {fam} lds_bank_conflict_rate "
                  f"{avg['SQ_LDS_BANK_CONFLICT'] / avg['SQ_LDS_IDX_ACTIVE']:.4f}  "
                  f"(SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE)")
        if traffic is not None:
            print(f"derived {fam} hbm_gbs {traffic / dur_ns:.0f}")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=150)
    ap.add_argument("--burst", type=int, default=10,
                    help="calls per event pair of the back-to-back bursts timed after the timed "
                         "steps (burst_ms, informational)")
    ap.add_argument("--burst-reps", type=int, default=5)
    ap.add_argument("--min-warmup-s", type=float, default=0.3,
                    help="keep warming up (whole steps) until this much wall time has passed: the "
                         "GPU needs a few tens of ms of sustained load to reach its steady clocks, "
                         "and the first calls after idle run up to 20%% slower")
    ap.add_argument("--cpu-heads", type=int, default=16,
                    help="heads per batch entry timed by the CPU baseline (16 = all)")
    ap.add_argument("--cpu-c-heads", type=int, default=4,
                    help="heads timed by the C blockwise port beside it (0 = skip)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--seed", type=int, default=P.INPUT_SEED)
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="before the warmup, run one elementwise kernel (out = -in, fp32) that "
                         "reads and writes this many MiB: the known-size kernel that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    ap.add_argument("--pmc-summary", nargs="+", metavar="CSV",
                    help="summarise rocprofv3 --pmc counter_collection.csv files of a run of "
                         "this script (made with --calib-copy-mib) and exit; no GPU is used")
    args = ap.parse_args()

    if args.pmc_summary:
        return pmc_summary(args.pmc_summary, args.calib_copy_mib)

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
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst

    def call(name):
        rp, ci = dev_csr[name]
        return block_sparse_attn_fwd(q, k, v, rp, ci, None)

    for _ in range(args.warmup):
        for name in P.FAMILIES:
            call(name)
    torch.cuda.synchronize()
    extra = 0
    t_w = time.perf_counter()
    while time.perf_counter() - t_w < args.min_warmup_s and args.min_warmup_s > 0:
        for _ in range(10):
            for name in P.FAMILIES:
                call(name)
            extra += 1
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

    # Kernel launch duration for the roofline: the mean per-call event time of the timed steps,
    # per family, on the launch stream. It includes each call's event packets and dispatch gap
    # (a few us over the kernel's own duration), so it is, if anything, long. Back-to-back bursts
    # of --burst calls are timed after the timed region too (burst_ms, per call): sustained load
    # without gaps lowers the clock, so they run a few percent slower still.
    launch_ms = {}
    for name in P.FAMILIES:
        launch_ms[name] = float(np.mean([a.elapsed_time(b) for a, b in ev[name]]))
        fam_out[name]["launch_ms"] = round(launch_ms[name], 4)
    mean_launch = sum(launch_ms.values()) / len(launch_ms)
    burst = {n: [] for n in P.FAMILIES}
    for _ in range(args.burst_reps):
        for name in P.FAMILIES:
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for _ in range(args.burst):
                call(name)
            b.record(stream)
            burst[name].append((a, b))
    torch.cuda.synchronize()
    for name in P.FAMILIES:
        fam_out[name]["burst_ms"] = round(
            float(np.mean([a.elapsed_time(b) / args.burst for a, b in burst[name]])), 4)

    # Analytic rows (no CSR, block_sparse_attn_fwd_window) for the families that are a window or
    # a window plus a global prefix, call by call against the CSR path for a like-for-like ratio.
    analytic = {}
    for name in P.FAMILIES:
        ex = wl[name].extra
        if "window" not in ex:
            continue
        ev_w = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                for _ in range(args.steps)]
        ev_c = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                for _ in range(args.steps)]
        for s in range(args.steps):
            a, b = ev_w[s]
            a.record(stream)
            block_sparse_attn_fwd_window(q, k, v, ex["window"], ex["n_global"])
            b.record(stream)
            a, b = ev_c[s]
            a.record(stream)
            call(name)
            b.record(stream)
        torch.cuda.synchronize()
        mw = float(np.median([a.elapsed_time(b) for a, b in ev_w]))
        mc = float(np.median([a.elapsed_time(b) for a, b in ev_c]))
        analytic[name] = {"window": ex["window"], "n_global": ex["n_global"],
                          "median_ms": round(mw, 4), "csr_median_ms": round(mc, 4),
                          "ratio_to_csr": round(mw / mc, 4)}
    # The long-context mixed workload (B1 H16 T16384, rows of 1-26 blocks varying by head): a
    # parity configuration, timed here for information only (not part of the geomean).
    others = {}
    mw = wl["mixed"]
    mq, mk, mv = (x.to(dev) for x in P.make_qkv(mw.B, mw.H, mw.T, seed=args.seed))
    mrp, mci = mw.csr()
    mrpd, mcid = torch.from_numpy(mrp).to(dev), torch.from_numpy(mci).to(dev)
    for _ in range(5):
        block_sparse_attn_fwd(mq, mk, mv, mrpd, mcid, None)
    ev_m = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in range(args.steps)]
    for a, b in ev_m:
        a.record(stream)
        block_sparse_attn_fwd(mq, mk, mv, mrpd, mcid, None)
        b.record(stream)
    torch.cuda.synchronize()
    mmed = float(np.median([a.elapsed_time(b) for a, b in ev_m]))
    mfl = P.active_blocks(mrp) * FLOP_PER_BLOCK
    others["mixed"] = {"B": mw.B, "H": mw.H, "T": mw.T, "active_blocks": P.active_blocks(mrp),
                      "median_ms": round(mmed, 4), "tflops": round(mfl / mmed / 1e9, 1),
                      "frac_peak": round(mfl / mmed / 1e9 / PEAK_FP16_TFLOPS, 4)}
    del mq, mk, mv

    achieved = (sum(flops) / len(flops)) / mean_launch / 1e9  # TFLOP/s: mean FLOP / mean duration
    traffic = read_traffic()
    roofline = {
        "bound": "mfma",
        "achieved": round(achieved, 1),
        "peak": PEAK_FP16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / PEAK_FP16_TFLOPS, 4),
        "traffic": (round(sum(traffic[n] for n in P.FAMILIES) / len(P.FAMILIES))
                    if traffic and all(n in traffic for n in P.FAMILIES) else None),
        "kernel": "bsa_fwd_dma_kernel",
        "avg_launch_ms": round(mean_launch, 4),
        "avg_launch_timing": ("HIP events around each call of the timed steps on the launch "
                              "stream: mean per family, then mean over the families (event "
                              "packets and dispatch gap included)"),
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
        "warmup_extra_steps": extra,
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
            "latency_timing": "HIP events around each call on the launch stream; median over "
                              "the timed steps per family",
            "analytic_rows": analytic,
            "other_workloads": others,
            "input_seed": args.seed,
            "pattern_seed": P.PATTERN_SEED,
        },
        "roofline": roofline,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(fams, inputs, args.cpu_heads, args.cpu_c_heads)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
