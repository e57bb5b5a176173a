"""The C ABI library: loads, exports what include/usagi_bsa.h declares, rejects bad arguments
before touching the GPU; and the submission shim's host-side checks. No GPU compute here."""

from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch

import usagi_amd
from usagi_amd import _native
from usagi_amd.build import INCLUDE_DIR, LIB_PATH

HEADER = os.path.join(INCLUDE_DIR, "usagi_bsa.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(usagi_bsa_\w+)\s*\(", text, re.M)))


def test_library_is_built_in_tree():
    assert os.path.exists(LIB_PATH), "run `python -m usagi_amd.build` (or __graft_entry__.build())"
    assert os.path.dirname(LIB_PATH).endswith(os.path.join("usagi_amd", "lib"))


def test_exports_every_declared_symbol():
    lib = ctypes.CDLL(LIB_PATH)
    names = declared_functions()
    assert set(names) == set(_native.EXPORTED_SYMBOLS), names
    for name in names:
        assert hasattr(lib, name), name


def test_version_and_empty_error():
    assert _native.version().startswith("usagi_bsa ") and "gfx950" in _native.version()


def _fwd(generic=False, **over):
    args = dict(q=1, k=1, v=1, rp=1, ci=1, sl=None, o=1, lse=None, B=1, H=1, T=128, D=128,
                nnz=1, dtype=0, sched=None, slots=0, stream=None)
    args.update(over)
    lib = _native.load()
    f = lib.usagi_bsa_fwd_generic if generic else lib.usagi_bsa_fwd
    p = lambda x: None if x is None else ctypes.c_void_p(x)  # noqa: E731
    return f(p(args["q"]), p(args["k"]), p(args["v"]), p(args["rp"]), p(args["ci"]),
             p(args["sl"]), p(args["o"]), p(args["lse"]), args["B"], args["H"], args["T"],
             args["D"], args["nnz"], args["dtype"], p(args["sched"]), args["slots"],
             p(args["stream"]))


@pytest.mark.parametrize("generic", [False, True])
@pytest.mark.parametrize("over,code", [
    (dict(q=None), -1), (dict(o=None), -1), (dict(rp=None), -1),
    (dict(dtype=7), -2), (dict(D=64), -3), (dict(T=100), -4), (dict(T=0), -4),
    (dict(B=0), -1), (dict(H=-1), -1), (dict(nnz=-1), -1), (dict(ci=None, nnz=3), -1),
    # a plan must cover at least every item (here 1) and at most USAGI_BSA_PLAN_CAP(1) = 10 slots
    (dict(sched=1, slots=0), -1), (dict(sched=1, slots=11), -1),
])
def test_argument_errors_are_reported_before_any_launch(over, code, generic):
    assert _fwd(generic=generic, **over) == code
    assert _native.last_error()


def _fwd_window(**over):
    args = dict(q=1, k=1, v=1, window=8, g=0, sl=None, o=1, lse=None, B=1, H=1, T=128, D=128,
                dtype=0, stream=None)
    args.update(over)
    lib = _native.load()
    p = lambda x: None if x is None else ctypes.c_void_p(x)  # noqa: E731
    return lib.usagi_bsa_fwd_window(p(args["q"]), p(args["k"]), p(args["v"]), args["window"],
                                    args["g"], p(args["sl"]), p(args["o"]), p(args["lse"]),
                                    args["B"], args["H"], args["T"], args["D"], args["dtype"],
                                    p(args["stream"]))


@pytest.mark.parametrize("over,code", [
    (dict(q=None), -1), (dict(o=None), -1), (dict(window=0), -1), (dict(g=-1), -1),
    (dict(dtype=7), -2), (dict(D=64), -3), (dict(T=100), -4), (dict(B=0), -1),
])
def test_window_argument_errors_are_reported_before_any_launch(over, code):
    assert _fwd_window(**over) == code
    assert _native.last_error()


def test_shim_rejects_host_tensors_and_bad_shapes():
    q = torch.zeros(1, 1, 128, 128, dtype=torch.float16)
    rp = torch.tensor([[[0, 1]]], dtype=torch.int32)
    ci = torch.tensor([[[0]]], dtype=torch.int32)
    with pytest.raises(ValueError, match="GPU"):
        usagi_amd.block_sparse_attn_fwd(q, q, q, rp, ci, None)
    with pytest.raises((TypeError, ValueError)):
        usagi_amd.block_sparse_attn_fwd(q.float(), q.float(), q.float(), rp, ci, None)
    with pytest.raises(TypeError):
        usagi_amd.block_sparse_attn_fwd(q.numpy(), q, q, rp, ci, None)
    with pytest.raises(ValueError, match="GPU"):
        usagi_amd.block_sparse_attn_fwd_window(q, q, q, 8)


def test_setup_on_cpu_device_returns_none_like_the_reference():
    class Spec:
        t_max = 1024

    assert usagi_amd.setup([Spec()], "cpu", usagi_amd.VARIANT_MANIFEST) is None
    assert usagi_amd.VARIANT_MANIFEST == [{"name": "default"}]
    assert usagi_amd.BLOCK_SIZE == 128 and usagi_amd.HEAD_DIM == 128


def test_check_csr_null_and_sizes():
    lib = _native.load()
    assert lib.usagi_bsa_check_csr(None, None, None, 1, 1, 1, 0) == -1
    rp = np.array([0, 1], np.int32)
    ci = np.array([0], np.int32)
    assert lib.usagi_bsa_check_csr(rp.ctypes.data, ci.ctypes.data, None, 1, 1, 1, 1) == 0


def test_setup_off_gpu_needs_no_library(monkeypatch, tmp_path):
    """Like the reference (v7:202-203), setup returns None for a non-GPU device or no specs
    without touching the library; on a GPU device a missing library is reported."""
    class Spec:
        t_max = 1024

    monkeypatch.setattr(_native, "LIB_PATH", str(tmp_path / "missing.so"))
    monkeypatch.setattr(_native, "_lib", None)
    assert usagi_amd.setup([Spec()], "cpu", usagi_amd.VARIANT_MANIFEST) is None
    assert usagi_amd.setup([], "cuda", usagi_amd.VARIANT_MANIFEST) is None
    with pytest.raises(RuntimeError, match="missing"):
        usagi_amd.setup([Spec()], "cuda", usagi_amd.VARIANT_MANIFEST)
