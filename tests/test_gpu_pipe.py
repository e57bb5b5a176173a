"""The pipelined kernel (bsa_fwd_pipe_kernel) on the GPU parity cases it can run.

The library picks it by itself for short rows only (no seq_lens, CSR or analytic rows averaging
at most 4 key blocks); USAGI_BSA_PIPE=1 makes it take every such call, so the parity tests of
the default walk and of the window path run again on it here, in fp16 and bf16 (cases with
seq_lens still run on bsa_fwd_dma_kernel). Left out are the tests whose point is bitwise equality
with the other kernel (the generic walk, the seq_lens variant): the two kernels round
differently within the parity tolerance (the row sum of P in fp32 here, from fp16 pairs there).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import bsa_oracle
from tests import test_gpu_parity as gp
from tests import test_gpu_walks as gw
from tests._helpers import assert_close
from usagi_amd import patterns as P

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _pipelined(monkeypatch):
    monkeypatch.setenv("USAGI_BSA_PIPE", "1")


# the default walk and the window path again, on the pipelined kernel
full_inputs = gp.full_inputs
test_plumbing_vs_dense_oracle = gp.test_plumbing_vs_dense_oracle
test_full_size_every_head_vs_fp32_walk = gp.test_full_size_every_head_vs_fp32_walk
test_full_size_rows_in_any_order_before_the_diagonal = gp.test_full_size_rows_in_any_order_before_the_diagonal
test_random_csr = gp.test_random_csr
test_bf16_inputs = gp.test_bf16_inputs
test_bf16_full_size_every_head_vs_fp32_walk = gp.test_bf16_full_size_every_head_vs_fp32_walk
test_bf16_running_max_growth = gp.test_bf16_running_max_growth
test_window_path_bf16 = gp.test_window_path_bf16
test_golden_fixtures = gp.test_golden_fixtures
test_full_size_deterministic = gp.test_full_size_deterministic
test_full_size_linear_in_v = gp.test_full_size_linear_in_v
test_full_size_constant_v = gp.test_full_size_constant_v
test_full_size_head_permutation = gp.test_full_size_head_permutation
test_rows_longer_than_64_blocks = gp.test_rows_longer_than_64_blocks
test_long_sequence = gp.test_long_sequence
test_single_and_two_block_sequences = gp.test_single_and_two_block_sequences
test_running_max_growth_takes_the_rescale_path = gp.test_running_max_growth_takes_the_rescale_path
test_sharp_softmax = gp.test_sharp_softmax
test_window_path_equals_csr_path_bitwise = gp.test_window_path_equals_csr_path_bitwise
test_shim_routes_window_shaped_csr_to_the_analytic_rows = gp.test_shim_routes_window_shaped_csr_to_the_analytic_rows
test_shim_keeps_a_near_window_csr_on_the_csr_walk = gp.test_shim_keeps_a_near_window_csr_on_the_csr_walk
test_window_path_vs_dense_oracle = gp.test_window_path_vs_dense_oracle
test_randomised_shapes_patterns_and_dtypes = gp.test_randomised_shapes_patterns_and_dtypes
test_empty_rows_take_the_implicit_diagonal = gp.test_empty_rows_take_the_implicit_diagonal
test_many_heads_single_block = gp.test_many_heads_single_block
test_plan_gives_bitwise_the_same_result = gw.test_plan_gives_bitwise_the_same_result
test_default_walk_rejects_a_row_whose_diagonal_is_not_last = gw.test_default_walk_rejects_a_row_whose_diagonal_is_not_last
test_timing_hook_times_the_kernel_itself = gw.test_timing_hook_times_the_kernel_itself
test_unchecked_csr_is_planned_without_a_synchronisation = gw.test_unchecked_csr_is_planned_without_a_synchronisation
test_planned_csr_launched_from_other_streams = gw.test_planned_csr_launched_from_other_streams


def _csr_walk_with(mode, monkeypatch, q, k, v, rp, ci):
    if mode is None:
        monkeypatch.delenv("USAGI_BSA_PIPE", raising=False)
    else:
        monkeypatch.setenv("USAGI_BSA_PIPE", mode)
    return gp.run_csr_walk(q, k, v, rp, ci)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("w", [1, 2, 4])
def test_short_rows_choose_the_pipelined_kernel(monkeypatch, w, dtype):
    """Sliding windows of up to 4 blocks: the automatic choice gives bitwise the pipelined
    kernel's result, and both kernels agree with the dense oracle."""
    B, H, T = 1, 4, 2048
    rp, ci = P.sliding_csr(B, H, T, w)
    q, k, v = P.make_qkv(B, H, T, seed=30 + w)
    q, k, v = (x.to(dtype) for x in (q, k, v))
    rtol = gp.BF16_RTOL if dtype == torch.bfloat16 else None
    print(f"case short rows sliding w{w} {dtype}", flush=True)
    o_auto, l_auto = _csr_walk_with(None, monkeypatch, q, k, v, rp, ci)
    o_pipe, l_pipe = _csr_walk_with("1", monkeypatch, q, k, v, rp, ci)
    o_dma, l_dma = _csr_walk_with("0", monkeypatch, q, k, v, rp, ci)
    assert np.array_equal(o_auto, o_pipe) and np.array_equal(l_auto, l_pipe)
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp, ci)
    for o, lse in ((o_pipe, l_pipe), (o_dma, l_dma)):
        if rtol is None:
            assert_close(o, oo)
        else:
            assert_close(o, oo, rtol=rtol)
        assert_close(lse, ol, what="LSE")


def test_longer_rows_keep_the_dma_kernel(monkeypatch):
    """Rows of 8 blocks: the automatic choice gives bitwise bsa_fwd_dma_kernel's result."""
    B, H, T = 1, 4, 2048
    rp, ci = P.sliding_csr(B, H, T, 8)
    q, k, v = P.make_qkv(B, H, T, seed=41)
    print("case longer rows sliding w8", flush=True)
    o_auto, l_auto = _csr_walk_with(None, monkeypatch, q, k, v, rp, ci)
    o_dma, l_dma = _csr_walk_with("0", monkeypatch, q, k, v, rp, ci)
    assert np.array_equal(o_auto, o_dma) and np.array_equal(l_auto, l_dma)


@pytest.mark.parametrize("w,g", [(1, 0), (2, 1), (3, 1), (1, 3)])
def test_short_window_rows_vs_dense_oracle(monkeypatch, w, g):
    """Analytic rows of at most 4 blocks (chosen automatically) against the dense oracle, with
    the CSR walk of the same pattern bitwise equal."""
    monkeypatch.delenv("USAGI_BSA_PIPE", raising=False)
    B, H, T = 2, 3, 1024
    q, k, v = P.make_qkv(B, H, T, seed=50 + 4 * w + g)
    rp, ci = P.global_csr(B, H, T, g, w)
    print(f"case short window rows w{w} g{g}", flush=True)
    o_win, l_win = gp.run_gpu_window(q, k, v, w, g)
    o_csr, l_csr = gp.run_csr_walk(q, k, v, rp, ci)
    assert np.array_equal(o_win, o_csr) and np.array_equal(l_win, l_csr)
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp, ci)
    assert_close(o_win, oo)
    assert_close(l_win, ol, what="LSE")


def test_without_lse_output():
    """A null LSE pointer: O is the same, nothing else is written."""
    from usagi_amd import _native

    B, H, T = 1, 8, 1024
    rp, ci = P.sliding_csr(B, H, T, 3)
    q, k, v = P.make_qkv(B, H, T, seed=60)
    print("case no LSE", flush=True)
    o_ref, _ = gp.run_csr_walk(q, k, v, rp, ci)
    dq, dk, dv = (x.to("cuda") for x in (q, k, v))
    drp = torch.from_numpy(np.ascontiguousarray(rp, dtype=np.int32)).to("cuda")
    dci = torch.from_numpy(np.ascontiguousarray(ci, dtype=np.int32)).to("cuda")
    o = torch.empty_like(dq)
    _native.fwd(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), drp.data_ptr(), dci.data_ptr(), None,
                o.data_ptr(), None, B, H, T, 128, ci.shape[-1], _native.FP16, None, 0,
                torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert np.array_equal(o.float().cpu().numpy(), o_ref)


# Each off-diagonal block's P is computed with the running max and accepted while its row sum
# stays <= 2^12: tiles 0-2 are checked at the end of the pass that computed them, tile 3 just
# before its P·V. Scores of some keys of key block 0 far above the rest (x6: P would overflow
# fp16 without the exact-max path, leaving NaN in O) pick which check fails and where:
#   keys 96-127 (tile 3 only) with rows [0, qb-1, qb]: the tile-3 check inside the loop
#   keys 96-127 with rows [0, qb]: the tile-3 check in the last pass
#   keys 0-95 with rows [0, qb]: the tiles-0-2 check of the last loop iteration
#   keys 0-127 with rows [0, qb-2, qb-1, qb]: the tiles-0-2 check with blocks still ahead
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("keys,window", [((96, 128), 2), ((96, 128), 1), ((0, 96), 1),
                                         ((0, 128), 3)])
def test_speculation_fallbacks(keys, window, dtype):
    B, H, T = 1, 2, 1024
    rp, ci = P.global_csr(B, H, T, 1, window)
    q, k, v = P.make_qkv(B, H, T, seed=70 + window)
    k = k.clone()
    k[:, :, keys[0]:keys[1]] *= 6.0
    q, k, v = (x.to(dtype) for x in (q, k, v))
    print(f"case fallback keys {keys} window {window} {dtype}", flush=True)
    o, lse = gp.run_csr_walk(q, k, v, rp, ci)
    assert np.isfinite(o).all()
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp, ci)
    if dtype == torch.bfloat16:
        assert_close(o, oo, rtol=gp.BF16_RTOL)
    else:
        assert_close(o, oo)
    assert_close(lse, ol, what="LSE")
