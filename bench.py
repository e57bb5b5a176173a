#!/usr/bin/env python3
"""Benchmark of the block-sparse causal attention forward on one MI355X.

Metric (the reference's headline, docs/OPTIMIZATION_JOURNAL.md:16, README.md:9): geometric mean
over the three sparsity families (sliding window w=8, global prefix 4 + local 4, retrieval
diagonal + previous + 14 seeded blocks) of the median forward latency at B=2, H=16, T=8192,
D=128, fp16, plus the fraction of dense fp16 MFMA peak counting only active 128x128 blocks
(4·128^3 FLOP each).

A step is one forward call of each family on synthetic inputs already resident in HBM. Every
call is bracketed by HIP events on the launch stream. The K timed steps are split into
--repeats consecutive groups; a family's latency is the median over the groups of its median
within each group (the reference's protocol of comparing medians over repeated runs,
docs/OPTIMIZATION_JOURNAL.md:135, 189-190).

    python bench.py [--steps K] [--warmup W] [--repeats R] [--min-warmup-s S] [--no-cpu]

The warmup is W steps plus, if needed, more whole steps until S seconds have passed (reported as
warmup_extra_steps): from idle the GPU takes tens of ms of sustained load to reach steady clocks.

Prints one JSON line. Besides the contract fields: per family launch_ms (the roofline's launch
duration: the mean kernel duration over a second block of the same steps, right after the timed
ones, from events attached to each kernel dispatch itself; a call's latency adds a few us of
launch gap and event packets to it) and, after that, burst_ms (back-to-back bursts);
config.full_seq_variant (seq_lens None, the kernel with the length masks compiled out, against
seq_lens of all T); config.window_routing (the shim runs the window-shaped sliding and global
CSRs on the analytic-row kernel: that against the CSR walk on the same tensors);
config.csr_first_call (a call with CSR tensors the shim has not seen against a cached one, host
wall time); config.reference_conditions (bf16 inputs, and bf16 with variable seq_lens, as the reference was
scored); config.other_workloads (the long-context mixed workload, with and without the work
plan; sliding w2, whose short rows run the pipelined kernel, against the two-phase kernel);
config.power_context (the sliding family on all-zero inputs, which keep the part at its top
clock, and a dense fp16 GEMM on random inputs on the same box); cpu_baseline (PyTorch CPU dense-masked attention on the host, median of 3, with the C
walk beside it). profile.family_dispatches counts the kernel dispatches of the warmup and timed
steps, which --pmc-summary and --trace-summary attribute to the families when given the JSON of
a profiled run.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import subprocess
import sys
import time

import numpy as np
import torch

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

from usagi_amd import _native, submission  # noqa: E402
from usagi_amd import block_sparse_attn_fwd  # noqa: E402
from usagi_amd import patterns as P  # noqa: E402

METRIC = "geomean fwd ms @B2 H16 T8192 D128 over 3 sparsity families; % fp16 MFMA peak"
PEAK_FP16_TFLOPS = 2516.6  # MI355X dense fp16 MFMA, published
PEAK_SCLK_MHZ = 2400  # the shader clock the published peak is quoted at
FLOP_PER_BLOCK = 4 * 128 ** 3
# v_mfma_f32_16x16x32 the kernel issues for a diagonal block: 304 of a full block's 512 (each wave
# skips the 16-key tiles above each of its two 16-row query tiles in Q·K^T and the 32-key steps
# above its rows in P·V).
DIAG_MFMA_SHARE = 304 / 512
TRAFFIC_FILE = os.path.join(REPO, "profiles", "bsa_fwd_hbm_traffic_b2h16t8192.txt")
REF_SEQ_LENS = [8192, 5000]  # variable sequence lengths for the reference-condition lines


def geomean(xs):
    return float(math.exp(sum(math.log(x) for x in xs) / len(xs)))


def cpu_model() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
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


def executed_flop(row_ptr) -> int:
    """FLOP of the MFMAs the kernel issues: full blocks, and 304/512 of one per diagonal."""
    n_diag = int(np.prod(row_ptr.shape[:-1])) * (row_ptr.shape[-1] - 1)
    return int((P.active_blocks(row_ptr) - n_diag * (1 - DIAG_MFMA_SHARE)) * FLOP_PER_BLOCK)


def cpu_baseline(fams, inputs, n_heads: int, c_heads: int, runs: int):
    """The reference math as PyTorch CPU fp32 dense-masked attention (oracle/torch_dense.py) on
    the host cores, per family over heads b < B, h < n_heads (all heads by default: the full
    workload), projected to B2 H16 by head count when fewer heads are run; the median of `runs`
    runs per family. The C restatement of the reference's blockwise CSR walk (oracle/bsa_ref.c,
    OpenMP) is timed beside it on c_heads heads, once, projected by active blocks."""
    from oracle import c_ref, torch_dense

    q, k, v = inputs
    B, H = q.shape[:2]
    threads = torch.get_num_threads()
    heads = [(b, h) for b in range(B) for h in range(min(n_heads, H))]
    per, per_c, spread = {}, {}, {}
    for name, (rp, ci) in fams.items():
        rpt, cit = torch.from_numpy(rp), torch.from_numpy(ci)
        ts = []
        for _ in range(runs):
            t0 = time.perf_counter()
            torch_dense.dense_masked(q, k, v, rpt, cit, heads=heads)
            ts.append((time.perf_counter() - t0) * 1e3 * (B * H) / len(heads))
        per[name] = float(np.median(ts))
        spread[name] = [round(x, 1) for x in ts]
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
        "cores": threads,
        "kind": "port",
        "sample": (f"PyTorch CPU fp32 dense-masked attention (oracle/torch_dense.py: block mask "
                   f"from the CSR, causal, query slabs of 1024 rows against keys up to the slab "
                   f"end) on {sample}; per family the median of {runs} runs, then the geomean "
                   f"over the 3 families; {threads} threads (the process's thread budget; "
                   f"os.cpu_count() = {os.cpu_count()}); host CPU: {cpu_model()}"),
        "per_family_ms": {k2: round(v2, 3) for k2, v2 in per.items()},
        "per_family_runs_ms": spread,
        "os_cpu_count": os.cpu_count(),
    }
    if per_c:
        out["blockwise_c_port"] = {
            "value": round(geomean(list(per_c.values())), 3),
            "unit": "ms",
            "sample": (f"oracle/bsa_ref.c (the reference's CSR walk in C, fp32, OpenMP) on heads "
                       f"b=0, h<{c_heads}, projected by active blocks, one run"),
            "per_family_ms": {k2: round(v2, 3) for k2, v2 in per_c.items()},
        }
    return out


KERNEL = "bsa_fwd_dma_kernel"
CALIB_KERNEL = "neg"


def pmc_summary(paths, calib_mib: int, bench_json) -> int:
    """Per-family averages of rocprofv3 --pmc counters for the attention kernel.

    The first profile.family_dispatches dispatches of the kernel (read from the JSON line the
    profiled bench run printed, --bench-json: one file per counter CSV, in the same order, or
    one file for all of them) are its warmup and timed steps, issued in family
    order (sliding, global, retrieval) every step, so dispatch i of them belongs to
    FAMILIES[i % 3]; later dispatches (bursts, the other lines of the bench) are left out. The
    calibration kernel is the elementwise negation of --calib-copy-mib MiB (it reads and writes
    exactly that many bytes); FETCH_SIZE and WRITE_SIZE (KiB) are each scaled by (known KiB /
    counter KiB) of that kernel.

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
    if not bench_json or len(bench_json) not in (1, len(paths)):
        print("--pmc-summary needs --bench-json: the JSON line of each profiled run (one file per "
              "counter CSV, or one for all)", file=sys.stderr)
        return 2
    n_fams = []
    for jp in bench_json:
        with open(jp) as f:
            line = [x for x in f.read().splitlines() if x.startswith("{")][-1]
        n_fams.append(int(json.loads(line)["profile"]["family_dispatches"]))
    if len(n_fams) == 1:
        n_fams = n_fams * len(paths)
    known_kib = calib_mib * 1024.0
    sums: dict = {}
    durs: dict = {}
    calib: dict = {}
    calib_name = None
    n_xcc, n_simd = 8, 1024
    for path, n_fam in zip(paths, n_fams):
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
        cal = [d for d in order if CALIB_KERNEL in by_disp[d]["name"]
               and KERNEL not in by_disp[d]["name"]]
        if cal:
            calib_name = by_disp[cal[0]]["name"]
            calib.update(by_disp[cal[0]]["ctr"])
        att = [d for d in order if KERNEL in by_disp[d]["name"]]
        if len(att) < n_fam:
            print(f"{path}: {len(att)} kernel dispatches, fewer than the {n_fam} of the warmup and "
                  f"timed steps", file=sys.stderr)
            return 2
        for i, d in enumerate(att[:n_fam]):
            fam = P.FAMILIES[i % len(P.FAMILIES)]
            for cname, val in by_disp[d]["ctr"].items():
                s = sums.setdefault(fam, {}).setdefault(cname, [0.0, 0])
                s[0] += val
                s[1] += 1
            if d in dur_of:
                t = durs.setdefault(fam, [0.0, 0])
                t[0] += dur_of[d]
                t[1] += 1
    print(f"kernel {KERNEL}: the first {'/'.join(str(n) for n in n_fams)} dispatches of the "
          f"passes (their warmup and timed steps); calibration kernel: {calib_name}")
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
        flop = P.active_blocks(wl[fam].csr()[0]) * FLOP_PER_BLOCK
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


def trace_summary(trace_csv: str, bench_json: str) -> int:
    """Per-family kernel durations from a rocprofv3 --kernel-trace of a run of this script.

    The kernel's dispatches are taken in order: the first profile.family_dispatches are the
    warmup and timed steps (family FAMILIES[i % 3] for dispatch i), the timed ones being the last
    3 x steps of them; the next profile.kernel_timing_dispatches repeat the timed steps with
    events attached to each dispatch (the launch_ms of the JSON line). Prints both blocks beside
    the JSON line's figures."""
    import csv

    with open(bench_json) as f:
        line = [x for x in f.read().splitlines() if x.startswith("{")][-1]
    bj = json.loads(line)
    n_fam = int(bj["profile"]["family_dispatches"])
    n_kt = int(bj["profile"]["kernel_timing_dispatches"])
    steps = int(bj["steps"])
    fams = bj["config"]["families"]
    with open(trace_csv) as f:
        rows = [r for r in csv.DictReader(f) if KERNEL in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    if len(rows) < n_fam + n_kt:
        print(f"{trace_csv}: {len(rows)} kernel dispatches, fewer than {n_fam + n_kt}", file=sys.stderr)
        return 2
    dur = [int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in rows]
    nf = len(FAM_ORDER)
    blocks = (("timed per-call dispatches", n_fam - nf * steps, n_fam, "median_ms",
               "call latency"),
              ("kernel-timing dispatches (events attached to each dispatch)", n_fam,
               n_fam + n_kt, "launch_ms", "launch_ms"))
    for title, lo, hi, key, what in blocks:
        print(f"## {title}: kernel dispatches {lo} .. {hi - 1} of the run, ns")
        means = []
        for fi, fam in enumerate(FAM_ORDER):
            d = np.array([dur[i] for i in range(lo, hi) if (i - lo) % nf == fi])
            means.append(d.mean())
            ref = fams[fam][key] * 1e6
            print(f"{fam:10s} n={len(d)} mean={d.mean():.0f} median={np.median(d):.0f} "
                  f"min={d.min()} max={d.max()}   bench {key} {ref:.0f} ({what} "
                  f"{ref - np.median(d):+.0f} ns over the kernel's median)")
        print(f"all three  mean of family means {np.mean(means):.0f}")
    names = sorted({r["Kernel_Name"] for r in rows[:n_fam]})
    print("kernels of the timed steps: " + "; ".join(names))
    return 0


FAM_ORDER = P.FAMILIES


def sclk_under_load(fn, seconds: float = 0.8):
    """Median of the shader clock rocm-smi reports (MHz) while fn runs back to back, or None
    when rocm-smi is not there."""
    import threading

    samples = []

    def sample():
        time.sleep(seconds / 3)
        for _ in range(2):
            try:
                r = subprocess.run(["rocm-smi", "--showclocks"], capture_output=True, text=True,
                                   timeout=10)
                m = re.search(r"sclk[^\n]*\((\d+)\s*Mhz\)", r.stdout, re.I)
                if m:
                    samples.append(int(m.group(1)))
            except (OSError, subprocess.SubprocessError):
                pass
            time.sleep(seconds / 4)

    th = threading.Thread(target=sample)
    th.start()
    t0 = time.perf_counter()
    while th.is_alive() or time.perf_counter() - t0 < seconds:
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
    th.join()
    return int(np.median(samples)) if samples else None


def event_pair():
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def time_calls(fns, n, stream):
    """n rounds of calling every fn once, each call between its own events; returns the
    per-call times (ms) per fn."""
    ev = [[event_pair() for _ in range(n)] for _ in fns]
    for s in range(n):
        for i, fn in enumerate(fns):
            a, b = ev[i][s]
            a.record(stream)
            fn()
            b.record(stream)
    torch.cuda.synchronize()
    return [[a.elapsed_time(b) for a, b in e] for e in ev]


def warm(fns, seconds):
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            for fn in fns:
                fn()
        torch.cuda.synchronize()


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=150)
    ap.add_argument("--repeats", type=int, default=5,
                    help="groups the timed steps are split into (median of the group medians)")
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
    ap.add_argument("--cpu-runs", type=int, default=3, help="CPU baseline runs per family (median)")
    ap.add_argument("--cpu-c-heads", type=int, default=4,
                    help="heads timed by the C blockwise port beside it (0 = skip)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the informational lines after the timed steps")
    ap.add_argument("--seed", type=int, default=P.INPUT_SEED)
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="before the warmup, run one elementwise kernel (out = -in, fp32) that "
                         "reads and writes this many MiB: the known-size kernel that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    ap.add_argument("--pmc-summary", nargs="+", metavar="CSV",
                    help="summarise rocprofv3 --pmc counter_collection.csv files of a run of "
                         "this script (made with --calib-copy-mib) and exit; no GPU is used")
    ap.add_argument("--bench-json", nargs="+",
                    help="with --pmc-summary / --trace-summary: the JSON output of each "
                         "profiled run")
    ap.add_argument("--trace-summary", metavar="CSV",
                    help="summarise the run_kernel_trace.csv of a rocprofv3 --kernel-trace run of "
                         "this script per family (needs --bench-json) and exit; no GPU is used")
    args = ap.parse_args()

    if args.pmc_summary:
        return pmc_summary(args.pmc_summary, args.calib_copy_mib, args.bench_json)
    if args.trace_summary:
        if not args.bench_json:
            print("--trace-summary needs --bench-json", file=sys.stderr)
            return 2
        return trace_summary(args.trace_summary, args.bench_json[0])

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
    # Everything the lines after the timed steps use is built here, before the GPU warms up.
    mw = wl["mixed"]
    mixed = None
    if not args.no_extra:
        mq, mk, mv = (x.to(dev) for x in P.make_qkv(mw.B, mw.H, mw.T, seed=args.seed))
        mrp, mci = mw.csr()
        mixed = (mq, mk, mv, mrp, torch.from_numpy(mrp).to(dev), torch.from_numpy(mci).to(dev))
        qb16, kb16, vb16 = (x.to(torch.bfloat16) for x in (q, k, v))
        srp, sci = P.sliding_csr(B, H, T, 2)
        srpd, scid = (torch.from_numpy(x).to(dev) for x in (srp, sci))
        qz, kz, vz = (torch.zeros_like(x) for x in (q, k, v))
        gen = torch.Generator(device=dev).manual_seed(args.seed)
        ga = torch.randn((8192, 8192), device=dev, dtype=torch.float16, generator=gen)
        gb = torch.randn((8192, 8192), device=dev, dtype=torch.float16, generator=gen)
        gc = torch.empty((8192, 8192), device=dev, dtype=torch.float16)
    full_sl = torch.full((B,), T, dtype=torch.int32, device=dev)
    ref_sl = torch.tensor(REF_SEQ_LENS, dtype=torch.int32, device=dev)

    if args.calib_copy_mib:
        n = args.calib_copy_mib * (1 << 20) // 4
        src = torch.ones(n, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst

    def call(name, qq=q, kk=k, vv=v, sl=None):
        rp, ci = dev_csr[name]
        return block_sparse_attn_fwd(qq, kk, vv, rp, ci, sl)

    step_fns = [(lambda n=name: call(n)) for name in P.FAMILIES]
    for _ in range(args.warmup):
        for fn in step_fns:
            fn()
    torch.cuda.synchronize()
    extra = 0
    t_w = time.perf_counter()
    while time.perf_counter() - t_w < args.min_warmup_s and args.min_warmup_s > 0:
        for _ in range(10):
            for fn in step_fns:
                fn()
            extra += 1
        torch.cuda.synchronize()

    stream = torch.cuda.current_stream(dev)
    ev = {n: [event_pair() for _ in range(args.steps)] for n in P.FAMILIES}
    # Events attached to each kernel dispatch (usagi_bsa_time_next_launch) time the kernel
    # itself, without the launch gap and event packets that events around a call include. They
    # add a few us to the call around them, so they are used in a second block of the same
    # steps right after the timed ones, never in the timed steps.
    kev = {n: [event_pair() for _ in range(args.steps)] for n in P.FAMILIES}
    for pairs in kev.values():
        for a, b in pairs:  # torch creates its events at their first record
            a.record(stream)
            b.record(stream)
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
    for s in range(args.steps):
        for name in P.FAMILIES:
            ka, kb = kev[name][s]
            _native.time_next_launch(ka.cuda_event, kb.cuda_event)
            call(name)
    torch.cuda.synchronize()

    groups = max(1, min(args.repeats, args.steps))
    bounds = np.linspace(0, args.steps, groups + 1).astype(int)
    fam_out = {}
    medians, flops, exec_flops = [], [], []
    launch_ms = {}
    for name in P.FAMILIES:
        ts = np.array([a.elapsed_time(b) for a, b in ev[name]])
        kts = np.array([a.elapsed_time(b) for a, b in kev[name]])
        group_meds = [float(np.median(ts[bounds[g]:bounds[g + 1]])) for g in range(groups)]
        med = float(np.median(group_meds))
        fl = P.active_blocks(fams[name][0]) * FLOP_PER_BLOCK
        efl = executed_flop(fams[name][0])
        medians.append(med)
        flops.append(fl)
        exec_flops.append(efl)
        launch_ms[name] = float(np.mean(kts))
        fam_out[name] = {
            "median_ms": round(med, 4),
            "group_medians_ms": [round(x, 4) for x in group_meds],
            "median_all_steps_ms": round(float(np.median(ts)), 4),
            "mean_ms": round(float(np.mean(ts)), 4),
            "launch_ms": round(launch_ms[name], 4),
            "kernel_median_ms": round(float(np.median(kts)), 4),
            "active_blocks": P.active_blocks(fams[name][0]),
            "tflops": round(fl / med / 1e9, 1),
            "frac_peak": round(fl / med / 1e9 / PEAK_FP16_TFLOPS, 4),
            "executed_mfma_tflops": round(efl / med / 1e9, 1),
        }
    value = geomean(medians)
    mean_launch = sum(launch_ms.values()) / len(launch_ms)

    extra_cfg = {}
    if not args.no_extra:
        # Back-to-back bursts: sustained load without gaps lowers the clock a little further.
        burst = {n: [] for n in P.FAMILIES}
        for _ in range(args.burst_reps):
            for name in P.FAMILIES:
                a, b = event_pair()
                a.record(stream)
                for _ in range(args.burst):
                    call(name)
                b.record(stream)
                burst[name].append((a, b))
        torch.cuda.synchronize()
        for name in P.FAMILIES:
            fam_out[name]["burst_ms"] = round(
                float(np.mean([a.elapsed_time(b) / args.burst for a, b in burst[name]])), 4)

        # seq_lens None runs the variant with every length mask compiled out; seq_lens of all T
        # runs the masked one on the same work. Call by call, alternating.
        full_seq = {}
        for name in P.FAMILIES:
            t_none, t_full = time_calls([lambda n=name: call(n),
                                         lambda n=name: call(n, sl=full_sl)], args.steps, stream)
            mn, mf = float(np.median(t_none)), float(np.median(t_full))
            full_seq[name] = {"seq_lens_none_ms": round(mn, 4), "seq_lens_all_T_ms": round(mf, 4),
                              "ratio_none_to_all_T": round(mn / mf, 4)}
        extra_cfg["full_seq_variant"] = full_seq

        # Window-shaped CSRs: the shim runs them on the analytic-row kernel (no CSR reads); the
        # CSR walk on the same tensors, straight through the C ABI, beside it.
        analytic = {}
        for name in P.FAMILIES:
            rp_d, ci_d = dev_csr[name]
            route = submission._csr_entry(rp_d, ci_d, B, H, T // 128, dev, False).window
            if route is None:
                continue
            o_w = torch.empty_like(q)
            l_w = torch.empty((B, H, T), device=dev, dtype=torch.float32)

            def csr_walk(rp_d=rp_d, ci_d=ci_d, o_w=o_w, l_w=l_w):
                _native.fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), rp_d.data_ptr(),
                            ci_d.data_ptr(), None, o_w.data_ptr(), l_w.data_ptr(), B, H, T, D,
                            ci_d.shape[-1], _native.FP16, None, 0, stream.cuda_stream)

            t_s, t_c = time_calls([lambda n=name: call(n), csr_walk], args.steps, stream)
            ms_, mc = float(np.median(t_s)), float(np.median(t_c))
            analytic[name] = {"window": route[0], "n_global": route[1],
                              "shim_median_ms": round(ms_, 4), "csr_walk_median_ms": round(mc, 4),
                              "ratio_shim_to_csr_walk": round(ms_ / mc, 4)}
        extra_cfg["window_routing"] = analytic

        # A CSR the shim has not seen: the first call copies it to the host (a device
        # synchronisation), checks its rows, looks for a window pattern and plans the work
        # order. Timed end to end on the host (synchronised before and after) for fresh tensors
        # holding the same CSR, against the same for a call whose CSR is cached.
        first = {}
        for name in P.FAMILIES:
            rp_d, ci_d = dev_csr[name]
            t_new, t_unchecked, t_hit = [], [], []
            for _ in range(5):
                for validate, ts_ in ((True, t_new), (False, t_unchecked)):
                    fresh = (rp_d.clone(), ci_d.clone())
                    torch.cuda.synchronize()
                    submission.VALIDATE_CSR = validate
                    try:
                        t0 = time.perf_counter()
                        block_sparse_attn_fwd(q, k, v, fresh[0], fresh[1], None)
                        torch.cuda.synchronize()
                        ts_.append((time.perf_counter() - t0) * 1e3)
                    finally:
                        submission.VALIDATE_CSR = True
                t0 = time.perf_counter()
                call(name)
                torch.cuda.synchronize()
                t_hit.append((time.perf_counter() - t0) * 1e3)
            first[name] = {"first_call_ms": round(float(np.median(t_new)), 4),
                           "first_call_unchecked_ms": round(float(np.median(t_unchecked)), 4),
                           "cached_call_ms": round(float(np.median(t_hit)), 4)}
        submission.clear_csr_cache()
        first["note"] = ("host wall time of one call, synchronised before and after, median of "
                         "5: first_call_ms with freshly cloned CSR tensors (cache miss: host copy, "
                         "check, window pattern and plan before the launch), "
                         "first_call_unchecked_ms the same with USAGI_BSA_VALIDATE=0 (no check, no "
                         "synchronisation: the CSR walk launches at once and the host copy "
                         "follows it on the stream), cached_call_ms with the bench's own CSR "
                         "tensors (cache hit)")
        extra_cfg["csr_first_call"] = first

        # The reference was scored on bf16 inputs with variable sequence lengths
        # (docs/OPTIMIZATION_JOURNAL.md:14-16): the same three families that way.
        ref = {}
        for label, sl in (("bf16", None), (f"bf16_seq_lens_{REF_SEQ_LENS[0]}_{REF_SEQ_LENS[1]}", ref_sl)):
            fns = [(lambda n=name, s=sl: call(n, qb16, kb16, vb16, s)) for name in P.FAMILIES]
            warm(fns, args.min_warmup_s)
            ts = time_calls(fns, args.steps, stream)
            meds = {n: float(np.median(t)) for n, t in zip(P.FAMILIES, ts)}
            ref[label] = {"median_ms": {n: round(m, 4) for n, m in meds.items()},
                          "geomean_ms": round(geomean(list(meds.values())), 4)}
            if sl is None:
                ref[label]["frac_peak"] = {
                    n: round(P.active_blocks(fams[n][0]) * FLOP_PER_BLOCK / m / 1e9
                             / PEAK_FP16_TFLOPS, 4) for n, m in meds.items()}
                ref[label]["ratio_to_fp16"] = round(
                    ref[label]["geomean_ms"] / geomean(medians), 4)
        ref["note"] = ("bf16 q/k/v/O with fp16 P·V; the seq_lens line cuts batch 1 at "
                       f"{REF_SEQ_LENS[1]} tokens (the active-block FLOP count is not reduced)")
        extra_cfg["reference_conditions"] = ref

        # The long-context mixed workload (B1 H16 T16384, rows of 1-26 blocks varying by head):
        # a parity configuration, timed for information (outside the geomean), with the work
        # plan the shim makes for it and without one (the kernel's built-in order).
        mq, mk, mv, mrp, mrpd, mcid = mixed
        G = mw.B * mw.H * mw.nqb
        m_out = torch.empty_like(mq)
        m_lse = torch.empty((mw.B, mw.H, mw.T), device=dev, dtype=torch.float32)

        def mixed_builtin():
            _native.fwd(mq.data_ptr(), mk.data_ptr(), mv.data_ptr(), mrpd.data_ptr(),
                        mcid.data_ptr(), None, m_out.data_ptr(), m_lse.data_ptr(), mw.B, mw.H,
                        mw.T, D, mcid.shape[-1], _native.FP16, None, 0, stream.cuda_stream)

        mfns = [lambda: block_sparse_attn_fwd(mq, mk, mv, mrpd, mcid, None), mixed_builtin]
        warm(mfns, args.min_warmup_s)
        t_plan, t_builtin = time_calls(mfns, args.steps, stream)
        mp, mb = float(np.median(t_plan)), float(np.median(t_builtin))
        mfl = P.active_blocks(mrp) * FLOP_PER_BLOCK
        sched = _native.plan_host(mrp, mw.B, mw.H, mw.nqb)
        extra_cfg["other_workloads"] = {"mixed": {
            "B": mw.B, "H": mw.H, "T": mw.T, "active_blocks": P.active_blocks(mrp),
            "median_ms": round(mp, 4), "tflops": round(mfl / mp / 1e9, 1),
            "frac_peak": round(mfl / mp / 1e9 / PEAK_FP16_TFLOPS, 4),
            "work_plan_slots": None if sched is None else int(len(sched)), "items": G,
            "builtin_order_median_ms": round(mb, 4),
            "ratio_plan_to_builtin": round(mp / mb, 4)}}
        del mixed, mq, mk, mv

        # Short rows (sliding w2 on the same tensors): the pipelined kernel, which the library
        # picks for rows of at most 4 blocks, against the two-phase kernel on the same calls.
        sfn = [lambda: block_sparse_attn_fwd(q, k, v, srpd, scid, None)]
        short = {}
        prev = os.environ.get("USAGI_BSA_PIPE")
        try:
            for label, mode in (("pipelined", "1"), ("two_phase", "0")):
                os.environ["USAGI_BSA_PIPE"] = mode
                warm(sfn, args.min_warmup_s)
                short[label] = float(np.median(time_calls(sfn, args.steps, stream)[0]))
        finally:
            if prev is None:
                os.environ.pop("USAGI_BSA_PIPE", None)
            else:
                os.environ["USAGI_BSA_PIPE"] = prev
        sfl = P.active_blocks(srp) * FLOP_PER_BLOCK
        extra_cfg["other_workloads"]["sliding_w2"] = {
            "B": B, "H": H, "T": T, "active_blocks": P.active_blocks(srp),
            "median_ms": round(short["pipelined"], 4),
            "frac_peak": round(sfl / short["pipelined"] / 1e9 / PEAK_FP16_TFLOPS, 4),
            "two_phase_kernel_median_ms": round(short["two_phase"], 4),
            "ratio_pipelined_to_two_phase": round(short["pipelined"] / short["two_phase"], 4)}

        # Power context: the sliding family on all-zero inputs (no operand bits toggle, the part
        # keeps its top clock), and a dense fp16 GEMM on random inputs (torch.matmul, 8192^3),
        # both on this box right after the timed steps.
        zfn = [lambda: block_sparse_attn_fwd(qz, kz, vz, *dev_csr["sliding"], None)]
        warm(zfn, args.min_warmup_s)
        zero_ms = float(np.median(time_calls(zfn, args.steps, stream)[0]))
        clk_zero = sclk_under_load(zfn[0])
        clk_random = sclk_under_load(lambda: call("sliding"))
        del qz, kz, vz
        gfn = [lambda: torch.matmul(ga, gb, out=gc)]
        warm(gfn, args.min_warmup_s)
        gemm_ms = float(np.median(time_calls(gfn, args.steps, stream)[0]))
        gemm_tflops = 2.0 * 8192 ** 3 / gemm_ms / 1e9
        clk_gemm = sclk_under_load(gfn[0])
        del ga, gb, gc
        extra_cfg["power_context"] = {
            "sliding_zero_inputs_ms": round(zero_ms, 4),
            "sliding_random_inputs_ms": round(fam_out["sliding"]["median_ms"], 4),
            "ratio_random_to_zero": round(fam_out["sliding"]["median_ms"] / zero_ms, 4),
            "sclk_mhz_sliding_random_inputs": clk_random,
            "sclk_mhz_sliding_zero_inputs": clk_zero,
            # the fraction of the MFMA peak at the clock the part held (peak quoted at 2.4 GHz)
            "sliding_frac_peak_at_sclk": (round(fam_out["sliding"]["frac_peak"] * PEAK_SCLK_MHZ
                                                / clk_random, 4) if clk_random else None),
            "dense_fp16_gemm_tflops": round(gemm_tflops, 1),
            "dense_fp16_gemm_frac_peak": round(gemm_tflops / PEAK_FP16_TFLOPS, 4),
            "sclk_mhz_dense_fp16_gemm": clk_gemm,
            "note": ("call medians on the same box after the timed steps; all-zero inputs keep "
                     "the part at its top clock, random fp16 inputs make it throttle, which "
                     "holds a dense GEMM below the 2.4 GHz peak as well; sclk as rocm-smi "
                     "reports it while the sliding family, or the GEMM, runs back to back")}

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
        "avg_launch_timing": ("HIP events attached to each kernel dispatch (hipExtLaunchKernel via "
                              "usagi_bsa_time_next_launch) over a block of the same steps run "
                              "right after the timed ones: the kernel's own duration, mean per "
                              "family, then mean over the families"),
        "algorithmic_flop_per_launch": int(sum(flops) / len(flops)),
        "geomean_frac_peak": round(geomean([f["frac_peak"] for f in fam_out.values()]), 4),
        "executed_mfma_flop_per_launch": int(sum(exec_flops) / len(exec_flops)),
        "executed_mfma_frac": round((sum(exec_flops) / len(exec_flops)) / mean_launch / 1e9
                                    / PEAK_FP16_TFLOPS, 4),
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
            "latency_timing": (f"HIP events around each call on the launch stream; the timed "
                               f"steps split into {groups} consecutive groups, per family the "
                               f"median over the groups of the median within each group"),
            **extra_cfg,
            "input_seed": args.seed,
            "pattern_seed": P.PATTERN_SEED,
        },
        "roofline": roofline,
        "profile": {"family_dispatches": (args.warmup + extra + args.steps) * len(P.FAMILIES),
                    "kernel_timing_dispatches": args.steps * len(P.FAMILIES),
                    "order": list(P.FAMILIES)},
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(fams, inputs, args.cpu_heads, args.cpu_c_heads,
                                           args.cpu_runs)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
