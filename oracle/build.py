"""Build recipe for the C restatement (TEST INFRASTRUCTURE ONLY).

    python -m oracle.build          # -> oracle/_build/libbsa_ref.so
    python -m oracle.build --asan   # -> oracle/_build/libbsa_ref_asan.so (ASan + UBSan)

The reference itself is Python + Triton (kernels/*.py): there is no C/C++ source of it to
compile, so nothing is built into oracle/_ref/.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "bsa_ref.c")
OUT_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(OUT_DIR, "libbsa_ref.so")
LIB_ASAN = os.path.join(OUT_DIR, "libbsa_ref_asan.so")


def build(asan: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    out = LIB_ASAN if asan else LIB
    flags = ["-O3", "-march=x86-64-v3", "-fopenmp"]
    if asan:
        flags = ["-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined"]
    cmd = ["gcc", "-std=c11", "-shared", "-fPIC", *flags, SRC, "-o", out + ".tmp", "-lm"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed:\n{res.stdout}\n{res.stderr}")
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    print(build(asan="--asan" in sys.argv))
