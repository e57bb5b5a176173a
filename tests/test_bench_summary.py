"""bench.py --pmc-summary on synthetic rocprofv3 CSVs with known answers (CPU only).

The counter values are chosen so every derived figure has a closed form: a calibration kernel
that reads half its known size in FETCH_SIZE (scale 2) and all of it in WRITE_SIZE (scale 1), then
the warmup and timed steps (one attention dispatch per family each, with fixed per-family
counters and durations), then dispatches that must not be counted: a runtime copy kernel, bursts
of one family, the analytic-row and mixed-workload calls (the same kernel name) with counters
far off. The bench JSON of the run says how many dispatches the steps made.
"""
import json
import csv
import os
import subprocess
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)

from usagi_amd import patterns as P  # noqa: E402

KERNEL = "(anonymous namespace)::bsa_fwd_dma_kernel((anonymous namespace)::Args)"
CALIB = "vectorized_elementwise_kernel<neg>"


STEPS = 4  # warmup + timed steps in the synthetic run: 12 family dispatches
MFMA = {"sliding": 3768320.0, "global": 3768320.0, "retrieval": 7208960.0}


def _write(dirpath, with_trace=True):
    ctr = os.path.join(dirpath, "run_counter_collection.csv")
    fields = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    rows = []
    trace = []
    calib_kib = 256 * 1024
    rows += [(1, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 1.0), (1, "__amd_rocclr_copyBuffer", "WRITE_SIZE", 1.0)]
    rows += [(2, CALIB, "FETCH_SIZE", calib_kib / 2), (2, CALIB, "WRITE_SIZE", calib_kib),
             (2, CALIB, "GRBM_GUI_ACTIVE", 1000.0), (2, CALIB, "SQ_VALU_MFMA_BUSY_CYCLES", 0.0),
             (2, CALIB, "SQ_LDS_BANK_CONFLICT", 0.0), (2, CALIB, "SQ_LDS_IDX_ACTIVE", 1.0),
             (2, CALIB, "SQ_INSTS_MFMA", 0.0)]
    trace.append((2, CALIB, 0, 5000))
    d = 3
    for step in range(STEPS):
        for fam in P.FAMILIES:
            # 8 XCDs x 200000 cycles in 100 us -> 2.0 GHz; MFMA busy half of 1024 SIMDs x 200000
            rows += [(d, KERNEL, "FETCH_SIZE", 100000.0), (d, KERNEL, "WRITE_SIZE", 50000.0),
                     (d, KERNEL, "GRBM_GUI_ACTIVE", 8 * 200000.0),
                     (d, KERNEL, "SQ_VALU_MFMA_BUSY_CYCLES", 0.5 * 1024 * 200000.0),
                     (d, KERNEL, "SQ_LDS_BANK_CONFLICT", 10.0), (d, KERNEL, "SQ_LDS_IDX_ACTIVE", 1000.0),
                     (d, KERNEL, "SQ_INSTS_MFMA", MFMA[fam])]
            trace.append((d, KERNEL, 10_000_000 * d, 10_000_000 * d + 100_000))
            d += 1
            if step == 0 and fam == "sliding":
                rows += [(d, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 9.0)]  # a runtime copy
                d += 1
    for _ in range(7):  # bursts / analytic rows / mixed: same kernel name, other counters
        rows += [(d, KERNEL, "FETCH_SIZE", 1e9), (d, KERNEL, "WRITE_SIZE", 1e9),
                 (d, KERNEL, "GRBM_GUI_ACTIVE", 1.0), (d, KERNEL, "SQ_VALU_MFMA_BUSY_CYCLES", 1.0),
                 (d, KERNEL, "SQ_LDS_BANK_CONFLICT", 999.0), (d, KERNEL, "SQ_LDS_IDX_ACTIVE", 1000.0),
                 (d, KERNEL, "SQ_INSTS_MFMA", 1.0)]
        trace.append((d, KERNEL, 10_000_000 * d, 10_000_000 * d + 7))
        d += 1
    with open(ctr, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(fields)
        w.writerows(rows)
    if with_trace:
        with open(os.path.join(dirpath, "run_kernel_trace.csv"), "w", newline="") as f:
            w = csv.writer(f)
            w.writerow(["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"])
            w.writerows(trace)
        with open(os.path.join(dirpath, "run_agent_info.csv"), "w", newline="") as f:
            w = csv.writer(f)
            w.writerow(["Name", "Num_Xcc", "Simd_Count", "Cu_Count"])
            w.writerow(["gfx950", 8, 1024, 256])
    with open(os.path.join(dirpath, "bench.json"), "w") as f:
        f.write("some stderr line\n" + json.dumps(
            {"profile": {"family_dispatches": 3 * STEPS, "order": list(P.FAMILIES)}}) + "\n")
    return ctr


def _run(ctr, steps_json=True):
    cmd = [sys.executable, os.path.join(REPO, "bench.py"), "--pmc-summary", ctr,
           "--calib-copy-mib", "256"]
    if steps_json:
        cmd += ["--bench-json", os.path.join(os.path.dirname(ctr), "bench.json")]
    out = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    return out.stdout


def _field(text, key, fam, name):
    for line in text.splitlines():
        parts = line.split()
        if len(parts) >= 4 and parts[0] == key and parts[1] == fam:
            for a, b in zip(parts[2:], parts[3:]):
                if a == name:
                    return float(b)
    raise AssertionError(f"{key} {fam} {name} missing in:\n{text}")


def test_traffic_scaled_by_the_calibration_kernel(tmp_path):
    text = _run(_write(str(tmp_path), with_trace=False))
    for fam in P.FAMILIES:
        # (100000 KiB x 2 + 50000 KiB x 1) x 1024
        line = next(l for l in text.splitlines() if l.startswith(f"traffic_bytes_per_launch {fam} "))
        assert float(line.split()[2]) == pytest.approx(250000 * 1024)
    assert "derived" not in text  # no kernel trace: no time-based figures


def test_derived_figures_against_closed_forms(tmp_path):
    text = _run(_write(str(tmp_path)))
    wl = P.workloads()
    for fam in P.FAMILIES:
        assert _field(text, "derived", fam, "duration_us") == pytest.approx(100.0)
        flop = P.active_blocks(wl[fam].csr()[0]) * 4 * 128 ** 3
        tf = _field(text, "derived", fam, "tflops_active")
        assert tf == pytest.approx(flop / 100e-6 / 1e12, rel=1e-3)
        assert _field(text, "derived", fam, "clock_ghz") == pytest.approx(2.0)
        # peak at 2.0 GHz: 1024 SIMDs x 1024 FLOP/clk
        assert _field(text, "derived", fam, "mfma_peak_at_clock_tflops") == pytest.approx(2097, abs=1)
        assert _field(text, "derived", fam, "frac_of_peak_at_clock") == pytest.approx(
            tf / (2.0e9 * 1024 * 1024 / 1e12), abs=1e-3)
        assert _field(text, "derived", fam, "mfma_busy") == pytest.approx(0.5)
        assert _field(text, "derived", fam, "lds_bank_conflict_rate") == pytest.approx(0.01)
        assert _field(text, "derived", fam, "hbm_gbs") == pytest.approx(250000 * 1024 / 100e3, rel=1e-3)


def test_only_the_step_dispatches_are_attributed(tmp_path):
    """Each family's average is over exactly its STEPS step dispatches: the bursts, analytic
    and mixed calls after them (FETCH_SIZE 1e9) and the runtime copies are left out, so the
    MFMA instruction count per family is exact."""
    text = _run(_write(str(tmp_path)))
    for fam in P.FAMILIES:
        line = next(l for l in text.splitlines() if l.startswith(f"avg {fam} SQ_INSTS_MFMA "))
        assert float(line.split()[3]) == MFMA[fam] and f"(over {STEPS} dispatches)" in line
        line = next(l for l in text.splitlines() if l.startswith(f"avg {fam} FETCH_SIZE "))
        assert float(line.split()[3]) == 100000.0


def test_summary_needs_the_bench_json(tmp_path):
    ctr = _write(str(tmp_path))
    out = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--pmc-summary", ctr,
                          "--calib-copy-mib", "256"], capture_output=True, text=True, timeout=300)
    assert out.returncode == 2 and "--bench-json" in out.stderr


def test_more_than_one_gpu_exits_with_a_message():
    out = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=300)
    assert out.returncode == 2
    assert "one GPU" in out.stderr and not out.stdout.strip()


def test_trace_summary_splits_timed_and_kernel_timing_dispatches(tmp_path):
    """bench.py --trace-summary: 2 warmup + 3 timed steps, then 3 kernel-timing steps, then
    dispatches that must be left out. Family f's timed dispatches last 100 + 10 f us (step 0, 1:
    far off), its kernel-timing ones 200 + 10 f us."""
    steps, warm = 3, 2
    trace = [(1, "__amd_rocclr_copyBuffer", 0, 5)]
    d = 2
    for s in range(warm + steps + steps):
        for fi, _ in enumerate(P.FAMILIES):
            if s < warm:
                us = 999
            elif s < warm + steps:
                us = 100 + 10 * fi
            else:
                us = 200 + 10 * fi
            trace.append((d, KERNEL, 1_000_000_000 * d, 1_000_000_000 * d + us * 1000))
            d += 1
    for _ in range(5):
        trace.append((d, KERNEL, 1_000_000_000 * d, 1_000_000_000 * d + 7))
        d += 1
    csv_path = os.path.join(str(tmp_path), "run_kernel_trace.csv")
    with open(csv_path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writerows(trace)
    fams = {fam: {"median_ms": (105 + 10 * fi) / 1e3, "launch_ms": (200 + 10 * fi) / 1e3}
            for fi, fam in enumerate(P.FAMILIES)}
    bj = os.path.join(str(tmp_path), "bench.json")
    with open(bj, "w") as f:
        f.write(json.dumps({"steps": steps, "config": {"families": fams},
                            "profile": {"family_dispatches": 3 * (warm + steps),
                                        "kernel_timing_dispatches": 3 * steps}}) + "\n")
    out = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--trace-summary",
                          csv_path, "--bench-json", bj], capture_output=True, text=True,
                         timeout=300)
    assert out.returncode == 0, out.stderr
    blocks = out.stdout.split("## ")[1:]
    assert len(blocks) == 2
    for block, base in zip(blocks, (100, 200)):
        for fi, fam in enumerate(P.FAMILIES):
            line = next(l for l in block.splitlines() if l.startswith(fam))
            assert f"n={steps} " in line and f"median={(base + 10 * fi) * 1000} " in line, line
    assert "(call latency +5000 ns" in blocks[0]
    assert "mean of family means 210000" in blocks[1]
