"""Pattern generators, CSR validators (Python and the C ABI's usagi_bsa_check_csr). No GPU."""

from __future__ import annotations

import numpy as np
import pytest

from usagi_amd import _native
from usagi_amd import patterns as P

# Active 128x128 blocks of each workload (the diagonal counts as a full block).
EXPECTED_ACTIVE = {"plumbing": 104, "sliding": 15488, "global": 15488, "retrieval": 28928,
                   "mixed": 36223}


@pytest.mark.parametrize("name", list(EXPECTED_ACTIVE))
def test_workload_active_blocks_and_validity(name):
    w = P.workloads()[name]
    rp, ci = w.csr()
    assert rp.dtype == np.int32 and ci.dtype == np.int32
    assert rp.shape == (w.B, w.H, w.nqb + 1)
    assert P.active_blocks(rp) == EXPECTED_ACTIVE[name]
    P.validate_csr(rp, ci, w.T)
    _native.check_csr_host(rp, ci, w.B, w.H, w.nqb, ci.shape[-1])


def test_family_rows():
    assert P.sliding_row(0, 8) == [0]
    assert P.sliding_row(9, 8) == list(range(2, 10))
    assert P.global_row(2, 4, 4) == [0, 1, 2]
    assert P.global_row(10, 4, 4) == [0, 1, 2, 3, 7, 8, 9, 10]
    for i in range(64):
        r = P.retrieval_row(i, 14, 1234, 1, 3)
        assert r == sorted(set(r)) and r[-1] == i
        assert len(r) == (1 if i == 0 else 2 + min(14, i - 1))
        assert r == P.retrieval_row(i, 14, 1234, 1, 3)  # deterministic per (seed, b, h, i)
    assert P.retrieval_row(40, 14, 1234, 0, 0) != P.retrieval_row(40, 14, 1234, 0, 1)


def analytic_row(i, w, g):
    """The analytic rows of the window path, as the kernel walks them: the global blocks below
    the window (min(g, lo) of them), then the window lo .. i (lo = max(0, i - w + 1))."""
    lo = max(0, i - w + 1)
    return list(range(min(g, lo))) + list(range(lo, i + 1))


def test_analytic_rows_equal_the_csr_rows():
    # min(g, lo) rather than min(g, i + 1): global blocks inside the window are not repeated
    for w in (1, 2, 3, 4, 8, 100):
        for g in (0, 1, 2, 4, 100):
            for i in range(0, 70):
                assert analytic_row(i, w, g) == P.global_row(i, g, w), (i, w, g)
    wl = P.workloads()
    for name in ("sliding", "global"):
        ex = wl[name].extra
        rp, ci = wl[name].csr()
        for qb in range(wl[name].nqb):
            row = list(ci[0, 0, rp[0, 0, qb]:rp[0, 0, qb + 1]])
            assert row == analytic_row(qb, ex["window"], ex["n_global"])


def test_mixed_heads():
    rp, ci = P.workloads()["mixed"].csr()
    per_head = [int(rp[0, h, -1]) for h in range(16)]
    assert per_head[:6] == [1928] * 6 and per_head[6:11] == [1928] * 5
    assert per_head[11:] == [3003] * 5


def _broken(kind):
    rp, ci = P.sliding_csr(1, 2, 512, 3)
    rp, ci = rp.copy(), ci.copy()
    if kind == "duplicate":
        ci[0, 1, rp[0, 1, 3] + 1] = ci[0, 1, rp[0, 1, 3]]
    elif kind == "diagonal_in_the_middle":
        ci[0, 1, rp[0, 1, 3] + 1:rp[0, 1, 4]] = ci[0, 1, rp[0, 1, 3] + 1:rp[0, 1, 4]][::-1]
    elif kind == "negative_block":
        ci[0, 1, rp[0, 1, 3]] = -1
    elif kind == "no_diagonal_last":
        ci[0, 0, rp[0, 0, 2] - 1] = 0
    elif kind == "future_block":
        ci[0, 0, rp[0, 0, 1] - 1] = 3
    elif kind == "empty_row":
        rp[0, 0, 1:] = np.concatenate([[0], rp[0, 0, 2:] - 1])
        ci[0, 0, :-1] = ci[0, 0, 1:]
    elif kind == "row_ptr_start":
        rp[0, 1, 0] = 1
    elif kind == "row_ptr_overflow":
        rp[0, 1, -1] = ci.shape[-1] + 1
    return rp, ci


@pytest.mark.parametrize("kind", ["duplicate", "diagonal_in_the_middle", "negative_block",
                                  "no_diagonal_last", "future_block", "empty_row",
                                  "row_ptr_start", "row_ptr_overflow"])
def test_validators_reject_malformed_csr(kind):
    rp, ci = _broken(kind)
    with pytest.raises(ValueError):
        P.validate_csr(rp, ci, 512)
    with pytest.raises(ValueError, match="malformed CSR"):
        _native.check_csr_host(rp, ci, 1, 2, 4, ci.shape[-1])


def test_validators_accept_rows_in_any_order_before_the_diagonal():
    """The walk does not depend on the order of the entries before the diagonal."""
    rp, ci = P.global_csr(1, 2, 1024, 2, 3)
    ci = ci.copy()
    rng = np.random.default_rng(0)
    for h in range(2):
        for i in range(8):
            a, b = rp[0, h, i], rp[0, h, i + 1] - 1
            ci[0, h, a:b] = rng.permutation(ci[0, h, a:b])
    P.validate_csr(rp, ci, 1024)
    _native.check_csr_host(rp, ci, 1, 2, 8, ci.shape[-1])


@pytest.mark.parametrize("seed", range(6))
def test_validators_agree_on_random_csr(seed):
    rng = np.random.default_rng(seed)
    T = 128 * int(rng.integers(1, 9))
    rp, ci = P.random_csr(2, 2, T, float(rng.uniform(0, 1)), seed)
    P.validate_csr(rp, ci, T)
    _native.check_csr_host(rp, ci, 2, 2, T // 128, ci.shape[-1])


def test_make_qkv_is_deterministic_fp16():
    import torch

    a = P.make_qkv(1, 2, 256, seed=3)
    b = P.make_qkv(1, 2, 256, seed=3)
    assert all(x.dtype == torch.float16 and x.shape == (1, 2, 256, 128) for x in a)
    assert all(torch.equal(x, y) for x, y in zip(a, b))
