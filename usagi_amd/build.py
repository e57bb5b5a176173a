"""Ahead-of-time build of the gfx950 HIP library (replaces the reference's Triton JIT warm-up,
kernels/v7_blockptr_warpspec.py:195-247: nothing is compiled at run time here).

    python -m usagi_amd.build            # builds usagi_amd/lib/libusagi_bsa.so
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
INCLUDE_DIR = os.path.join(REPO_DIR, "include")
CSRC_DIR = os.path.join(PKG_DIR, "csrc")
# The kernels and their launch ABI (HIP), and the host-only validator and work planner.
SRCS = [os.path.join(CSRC_DIR, "bsa_fwd.hip"), os.path.join(CSRC_DIR, "bsa_plan.cpp")]
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libusagi_bsa.so")
ARCH = "gfx950"


def hipcc_path() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (looked at $HIPCC, /opt/rocm/bin/hipcc, PATH)")


def hipcc_command(srcs: list[str] | None = None, out: str = LIB_PATH,
                  extra: list[str] | None = None) -> list[str]:
    return [
        hipcc_path(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        # Packed FP32 VALU forms are kept out of the device code.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", INCLUDE_DIR,
        "-I", CSRC_DIR,
        *(extra or []),
        *(srcs or SRCS),
        "-o", out,
    ]


def generate_asm() -> str:
    """Write csrc/bsa_pipe_asm.inc (the pipelined kernel's work item as inline assembly) from its
    generator, csrc/gen_bsa_pipe.py; returns its path."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("gen_bsa_pipe", os.path.join(CSRC_DIR, "gen_bsa_pipe.py"))
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    return gen.write()


def build(verbose: bool = False) -> str:
    """Generate the pipelined kernel's assembly, then compile the HIP source into an in-tree
    shared library; returns its path."""
    generate_asm()
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB_PATH + ".tmp"
    cmd = hipcc_command(out=tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
