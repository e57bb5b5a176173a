"""ctypes binding of libusagi_bsa.so (declarations in include/usagi_bsa.h).

torch is imported first so that the library binds to the HIP runtime torch already loaded
(one runtime per process). There is no fallback: a missing library raises.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load: shares torch's HIP runtime)

from .build import LIB_PATH

FP16 = 0
BF16 = 1

EXPORTED_SYMBOLS = (
    "usagi_bsa_fwd",
    "usagi_bsa_fwd_generic",
    "usagi_bsa_fwd_window",
    "usagi_bsa_check_csr",
    "usagi_bsa_plan",
    "usagi_bsa_time_next_launch",
    "usagi_bsa_version",
    "usagi_bsa_last_error",
)

_lib = None


class NativeError(RuntimeError):
    """A nonzero status from the C ABI."""

    def __init__(self, code: int, message: str):
        super().__init__(f"usagi_bsa error {code}: {message}")
        self.code = code


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"native library {LIB_PATH} is missing; build it with `python -m usagi_amd.build`"
        )
    lib = ctypes.CDLL(LIB_PATH)
    p = ctypes.c_void_p
    i32 = ctypes.c_int32
    fwd_args = [p, p, p, p, p, p, p, p, i32, i32, i32, i32, i32, i32, p, i32, p]
    lib.usagi_bsa_fwd.argtypes = fwd_args
    lib.usagi_bsa_fwd.restype = ctypes.c_int
    lib.usagi_bsa_fwd_generic.argtypes = fwd_args
    lib.usagi_bsa_fwd_generic.restype = ctypes.c_int
    lib.usagi_bsa_fwd_window.argtypes = [p, p, p, i32, i32, p, p, p, i32, i32, i32, i32, i32, p]
    lib.usagi_bsa_fwd_window.restype = ctypes.c_int
    lib.usagi_bsa_check_csr.argtypes = [p, p, p, i32, i32, i32, i32]
    lib.usagi_bsa_check_csr.restype = ctypes.c_int
    lib.usagi_bsa_plan.argtypes = [p, i32, i32, i32, i32, p, i32]
    lib.usagi_bsa_plan.restype = ctypes.c_int
    lib.usagi_bsa_time_next_launch.argtypes = [p, p]
    lib.usagi_bsa_time_next_launch.restype = ctypes.c_int
    lib.usagi_bsa_version.argtypes = []
    lib.usagi_bsa_version.restype = ctypes.c_char_p
    lib.usagi_bsa_last_error.argtypes = []
    lib.usagi_bsa_last_error.restype = ctypes.c_char_p
    _lib = lib
    return lib


def last_error() -> str:
    return load().usagi_bsa_last_error().decode()


def version() -> str:
    return load().usagi_bsa_version().decode()


def check(code: int) -> None:
    if code != 0:
        raise NativeError(code, last_error())


def fwd(q_ptr, k_ptr, v_ptr, row_ptr_ptr, col_idx_ptr, seq_lens_ptr, out_ptr, lse_ptr,
        batch, heads, seq_len, head_dim, max_nnz, dtype, sched_ptr, n_slots, stream,
        generic: bool = False) -> None:
    lib = load()
    f = lib.usagi_bsa_fwd_generic if generic else lib.usagi_bsa_fwd
    check(f(q_ptr, k_ptr, v_ptr, row_ptr_ptr, col_idx_ptr, seq_lens_ptr, out_ptr, lse_ptr, batch,
            heads, seq_len, head_dim, max_nnz, dtype, sched_ptr, n_slots, stream))


def fwd_window(q_ptr, k_ptr, v_ptr, window, n_global, seq_lens_ptr, out_ptr, lse_ptr,
               batch, heads, seq_len, head_dim, dtype, stream) -> None:
    check(load().usagi_bsa_fwd_window(q_ptr, k_ptr, v_ptr, window, n_global, seq_lens_ptr,
                                      out_ptr, lse_ptr, batch, heads, seq_len, head_dim, dtype,
                                      stream))


def time_next_launch(start_event, stop_event) -> None:
    """Attach two hipEvent_t handles (ints, e.g. torch.cuda.Event(enable_timing=True).cuda_event
    of events recorded once already) to this thread's next forward launch: they then time the
    kernel itself."""
    check(load().usagi_bsa_time_next_launch(start_event or None, stop_event or None))


def plan_cap(n_items: int) -> int:
    """USAGI_BSA_PLAN_CAP of include/usagi_bsa.h."""
    return 2 * n_items + 8


def plan_host(row_ptr, batch: int, heads: int, nqb: int, generic: bool = False):
    """Work plan over a host (numpy) row_ptr: an int32 slot -> item array, or None when the
    kernel's built-in order is already balanced."""
    import numpy as np

    rp = np.ascontiguousarray(row_ptr, dtype=np.int32)
    cap = plan_cap(batch * heads * nqb)
    sched = np.empty(cap, dtype=np.int32)
    n = load().usagi_bsa_plan(rp.ctypes.data, batch, heads, nqb, 1 if generic else 0,
                              sched.ctypes.data, cap)
    if n < 0:
        raise NativeError(n, last_error())
    return sched[:n].copy() if n else None


def check_csr_host(row_ptr, col_idx, batch: int, heads: int, nqb: int, max_nnz: int,
                   seq_lens=None) -> None:
    """Validate host (numpy int32, C-contiguous) CSR arrays through the C validator; with
    seq_lens (host, [batch]) the rows of query blocks at or past seq_len are not checked."""
    import numpy as np

    rp = np.ascontiguousarray(row_ptr, dtype=np.int32)
    ci = np.ascontiguousarray(col_idx, dtype=np.int32)
    sl = None if seq_lens is None else np.ascontiguousarray(seq_lens, dtype=np.int32).reshape(-1)
    if sl is not None and sl.size != batch:
        raise ValueError(f"seq_lens must hold {batch} values, got {sl.size}")
    code = load().usagi_bsa_check_csr(rp.ctypes.data, ci.ctypes.data if ci.size else None,
                                      None if sl is None else sl.ctypes.data,
                                      batch, heads, nqb, max_nnz)
    if code != 0:
        raise ValueError(f"malformed CSR: {last_error()}")
