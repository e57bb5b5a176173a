"""ctypes wrapper of the C restatement oracle/bsa_ref.c — TEST INFRASTRUCTURE ONLY."""

from __future__ import annotations

import ctypes
import os

import numpy as np

from .build import LIB

_lib = None


def load(path: str = LIB) -> ctypes.CDLL:
    global _lib
    if _lib is not None and path == LIB:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} missing; run `python -m oracle.build`")
    lib = ctypes.CDLL(path)
    p = ctypes.c_void_p
    i32 = ctypes.c_int32
    lib.oracle_bsa_fwd.argtypes = [p, p, p, p, p, p, p, p, i32, i32, i32, i32, i32, i32, i32]
    lib.oracle_bsa_fwd.restype = ctypes.c_int
    if path == LIB:
        _lib = lib
    return lib


def fwd(q, k, v, row_ptr, col_idx, seq_lens=None, round_p_fp16: bool = True, lib=None,
        generic: bool = False):
    """q/k/v: float arrays [B,H,T,D] (any float dtype; converted to fp32). Returns (O, LSE).
    generic: the order-free walk of kernels/v1_baseline.py:360-406 instead of v7's."""
    lib = lib or load()
    qn = np.ascontiguousarray(q, dtype=np.float32)
    kn = np.ascontiguousarray(k, dtype=np.float32)
    vn = np.ascontiguousarray(v, dtype=np.float32)
    B, H, T, D = qn.shape
    rp = np.ascontiguousarray(row_ptr, dtype=np.int32)
    ci = np.ascontiguousarray(col_idx, dtype=np.int32)
    max_nnz = ci.shape[-1]
    sl = None if seq_lens is None else np.ascontiguousarray(seq_lens, dtype=np.int32)
    out = np.empty_like(qn)
    lse = np.empty((B, H, T), dtype=np.float32)
    rc = lib.oracle_bsa_fwd(qn.ctypes.data, kn.ctypes.data, vn.ctypes.data, rp.ctypes.data,
                            ci.ctypes.data if max_nnz else None,
                            sl.ctypes.data if sl is not None else None,
                            out.ctypes.data, lse.ctypes.data, B, H, T, D, max_nnz,
                            1 if round_p_fp16 else 0, 1 if generic else 0)
    if rc != 0:
        raise ValueError(f"oracle_bsa_fwd rejected its arguments (rc={rc})")
    return out, lse
