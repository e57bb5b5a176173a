"""Checks on the gfx950 assembly of usagi_amd/csrc/bsa_fwd.hip (compiled here with hipcc, no GPU
needed), for properties that neither parity nor timing would show until they went wrong:

- M0 is written only right before an LDS DMA: in bsa_fwd_dma_kernel by the DMA statement
  (dma_16b), each write immediately followed by its global_load_lds_dwordx4; in the pipelined
  kernel's generated assembly by an s_add_u32 that sets the sub-tile's LDS base for its two
  DMAs. No other instruction reads M0. The compiler does not preserve M0 across an asm
  statement that lists it as clobbered, so this is what keeps the DMA safe.
- No kernel spills registers or uses scratch memory (a spill would silently cost several
  percent; every instantiation is sized to fit 2 workgroups per CU).
- No packed-FP32 VALU instruction is emitted.
- gen_bsa_pipe.py, which the build runs to write bsa_pipe_asm.inc, is deterministic.
"""

from __future__ import annotations

import re
import subprocess

import pytest

from usagi_amd import build as B



def _have_hipcc() -> bool:
    try:
        B.hipcc_path()
        return True
    except RuntimeError:
        return False


pytestmark = pytest.mark.skipif(not _have_hipcc(), reason="hipcc not available")


@pytest.fixture(scope="module")
def asm(tmp_path_factory) -> str:
    B.generate_asm()
    out = str(tmp_path_factory.mktemp("isa") / "bsa_fwd.s")
    cmd = [c for c in B.hipcc_command(srcs=[B.SRCS[0]], out=out) if c not in ("-shared", "-fPIC")]
    cmd[1:1] = ["--offload-device-only", "-S"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    with open(out) as f:
        return f.read()


def _instructions(text: str) -> list[str]:
    lines = []
    for ln in text.splitlines():
        ln = ln.split(";")[0].strip()
        if ln and not ln.startswith(".") and not ln.endswith(":"):
            lines.append(ln)
    return lines


def _kernels(text: str) -> dict[str, list[str]]:
    """Kernel symbol -> its instructions."""
    out: dict[str, list[str]] = {}
    name = None
    for ln in text.splitlines():
        m = re.match(r"^(_Z\w*bsa_fwd_\w+):", ln)
        if m:
            name = m.group(1)
            out[name] = []
            continue
        if name is None:
            continue
        out[name] += _instructions(ln)
        if "s_endpgm" in ln and "pipe" not in name:
            name = None
    return out


def test_m0_only_feeds_the_dma(asm):
    kernels = _kernels(asm)
    assert len(kernels) == 16, list(kernels)
    n_dma = 0
    for name, ins in kernels.items():
        pipe = "pipe" in name
        for i, ln in enumerate(ins):
            op = ln.split()[0]
            if op == "global_load_lds_dwordx4":
                if pipe:
                    # s_add_u32 m0, ...; s_nop 0; DMA; DMA (the sub-tile's two pieces)
                    j = i - 1 if ins[i - 1] == "s_nop 0" else i - 2
                    assert ins[j] == "s_nop 0" and ins[j - 1].startswith("s_add_u32 m0, s"), ins[j - 1:i + 1]
                else:
                    assert ins[i - 2].startswith("s_mov_b32 m0, s") and ins[i - 1] == "s_nop 0", ins[i - 2:i + 1]
                n_dma += 1
            elif re.search(r"\bm0\b", ln):
                if pipe:
                    assert re.fullmatch(r"s_add_u32 m0, s\d+, \d+", ln), ln
                    assert ins[i + 1] == "s_nop 0" and ins[i + 2].startswith("global_load_lds_dwordx4"), ln
                    assert ins[i + 3].startswith("global_load_lds_dwordx4"), ln
                else:
                    assert re.fullmatch(r"s_mov_b32 m0, s\d+", ln), ln
                    assert ins[i + 1] == "s_nop 0" and ins[i + 2].startswith("global_load_lds_dwordx4"), ln
            # instructions that read M0 implicitly
            assert not re.match(r"(s_sendmsg|s_movrel|v_movrel|ds_gws|v_interp|buffer_load_\w+ .*lds)", ln), ln
            assert not op.endswith("_addtid_b32"), ln
    assert n_dma > 0


def test_no_spills_no_scratch(asm):
    names = re.findall(r"\.name:\s+(_Z\w*bsa_fwd\w*)", asm)
    # bsa_fwd_dma_kernel: 2 dtypes x 3 row sources x with/without seq_lens; the pipelined kernel:
    # 2 dtypes x CSR and analytic rows
    assert len(names) == 16, names
    for key in ("vgpr_spill_count", "sgpr_spill_count", "private_segment_fixed_size"):
        vals = [int(v) for v in re.findall(rf"\.{key}:\s+(\d+)", asm)]
        assert len(vals) >= 16 and all(v == 0 for v in vals), (key, vals)
    vgprs = [int(v) for v in re.findall(r"\.vgpr_count:\s+(\d+)", asm)]
    assert vgprs and max(vgprs) <= 256, vgprs  # 2 waves per SIMD


def test_no_packed_fp32(asm):
    assert not re.search(r"v_pk_(add|mul|fma|mov)_f32", asm)


def test_pipelined_kernel_fits_two_workgroups_per_cu(asm):
    """VGPRs (rounded to 8) plus AGPRs within the 256 of two waves per SIMD."""
    for m in re.finditer(r"\.agpr_count:\s+(\d+).*?\.name:\s+(\S+).*?\.vgpr_count:\s+(\d+)", asm, re.S):
        agpr, name, total = int(m.group(1)), m.group(2), int(m.group(3))
        if "pipe" in name:
            assert agpr == 64 and total <= 256, (name, agpr, total)


def test_generated_assembly_is_deterministic():
    """The build writes bsa_pipe_asm.inc from gen_bsa_pipe.py; two runs give the same text."""
    import os
    import sys

    path = B.generate_asm()
    first = open(path).read()
    gen = os.path.join(os.path.dirname(B.SRCS[0]), "gen_bsa_pipe.py")
    res = subprocess.run([sys.executable, gen, "--check"], capture_output=True, text=True)
    assert res.returncode == 0 and open(path).read() == first
