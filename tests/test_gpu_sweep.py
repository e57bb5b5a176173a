"""Seeded sweep over every entry point on the GPU against the fp32 C walk: the default walk (rows
of 0-100 entries, around the 64-entry column chunk), the generic walk (rows with repeats, missing
or misplaced diagonals, empty rows), analytic window rows, and a work plan forced onto any CSR;
fp16 and bf16, with and without seq_lens. Tolerance as in test_gpu_parity.py: atol = rtol = 2e-3
(plus half a bf16 ulp for bf16 O)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import c_ref
from tests._helpers import assert_close
from usagi_amd import _native, block_sparse_attn_fwd, block_sparse_attn_fwd_generic
from usagi_amd import block_sparse_attn_fwd_window
from usagi_amd import patterns as P

pytestmark = pytest.mark.gpu

DEV = "cuda"
ENTRIES = ["default", "generic", "window", "plan"]


def case_inputs(seed):
    rng = np.random.default_rng(7000 + seed)
    entry = ENTRIES[seed % 4]
    B = int(rng.integers(1, 3))
    H = int(rng.choice([1, 2, 3, 4, 8, 16]))
    nqb = int(rng.integers(1, 40))
    nqb = max(1, min(nqb, 1200 // (B * H)))
    T = 128 * nqb
    dtype = torch.bfloat16 if (seed // 4) % 3 == 2 else torch.float16
    sl = None
    if (seed // 4) % 2:
        sl = [int(x) for x in rng.integers(0, T + 1, size=B)]
    extra = {}
    if entry == "window":
        extra = {"w": int(rng.integers(1, 20)), "g": int(rng.integers(0, 6))}
        g, w = extra["g"], extra["w"]
        rp, ci = P.global_csr(B, H, T, g, w) if g else P.sliding_csr(B, H, T, w)
    elif entry == "generic":
        def row(b, h, i):
            r = [int(x) for x in rng.integers(0, nqb, size=int(rng.integers(0, min(70, nqb + 3))))]
            if rng.random() < 0.7:
                r.insert(int(rng.integers(0, len(r) + 1)), i)
            return r
        rp, ci = P.make_csr(B, H, T, row)
    else:
        target = int(rng.choice([8, 63, 64, 65, 66, 100]))

        def row(b, h, i):
            n = min(i, int(rng.integers(0, target + 1)))
            return sorted(int(x) for x in rng.choice(i, size=n, replace=False)) + [i]
        rp, ci = P.make_csr(B, H, T, row)
    q, k, v = P.make_qkv(B, H, T, seed=8000 + seed, dtype=dtype)
    return entry, B, H, T, dtype, sl, rp, ci, q, k, v, extra


@pytest.mark.parametrize("seed", range(48))
def test_sweep_vs_fp32_walk(seed):
    entry, B, H, T, dtype, sl, rp, ci, q, k, v, extra = case_inputs(seed)
    nqb = T // 128
    print(f"case sweep seed={seed} {entry} B{B} H{H} T{T} {dtype} seq_lens={sl}", flush=True)
    dq, dk, dv = (x.to(DEV) for x in (q, k, v))
    drp, dci = torch.from_numpy(rp).to(DEV), torch.from_numpy(ci).to(DEV)
    dsl = None if sl is None else torch.tensor(sl, dtype=torch.int32, device=DEV)
    if entry == "window":
        o, lse = block_sparse_attn_fwd_window(dq, dk, dv, extra["w"], extra["g"], dsl)
    elif entry == "plan":
        sched = _native.plan_host(rp, B, H, nqb)
        if sched is None:  # any plan is valid: the items in reverse, padded to a multiple of 8
            n = B * H * nqb
            sched = np.full((n + 7) // 8 * 8, -1, np.int32)
            sched[:n] = np.arange(n)[::-1]
        dsched = torch.from_numpy(sched).to(DEV)
        o = torch.empty_like(dq)
        lse = torch.empty((B, H, T), device=DEV, dtype=torch.float32)
        _native.fwd(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), drp.data_ptr(), dci.data_ptr(),
                    None if dsl is None else dsl.data_ptr(), o.data_ptr(), lse.data_ptr(),
                    B, H, T, 128, ci.shape[-1],
                    _native.BF16 if dtype == torch.bfloat16 else _native.FP16,
                    dsched.data_ptr(), len(sched), torch.cuda.current_stream().cuda_stream)
    else:
        fn = block_sparse_attn_fwd_generic if entry == "generic" else block_sparse_attn_fwd
        o, lse = fn(dq, dk, dv, drp, dci, dsl)
    torch.cuda.synchronize()
    oo, ol = c_ref.fwd(q.float().numpy(), k.float().numpy(), v.float().numpy(), rp, ci,
                       None if sl is None else np.asarray(sl, np.int32), round_p_fp16=False,
                       generic=entry == "generic")
    rtol = 2e-3 + (2.0 ** -9 if dtype == torch.bfloat16 else 0.0)
    assert_close(o.float().cpu().numpy(), oo, rtol=rtol)
    assert_close(lse.cpu().numpy(), ol, what="LSE")
