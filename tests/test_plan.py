"""The host-side work planner (usagi_bsa_plan) and the submission shim's per-CSR cache.
No GPU: the planner runs on host arrays, and the cache is exercised with CPU tensors."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from usagi_amd import _native, submission
from usagi_amd import patterns as P

XCDS = 8
OVERHEAD = 1.5  # the planner's per-item fixed cost, in key blocks


def item_costs(rp, generic=False):
    n = np.diff(rp.reshape(-1, rp.shape[-1]).astype(np.int64), axis=-1).clip(min=0)
    blocks = n if generic else np.maximum(n - 1, 0) + 1
    return (blocks + OVERHEAD).reshape(-1)  # item b*H*nqb + h*nqb + qb


def builtin_order(bh_count, nqb):
    """The kernel's built-in slot -> item order (restated from its description: head-major
    per XCD, each head's query blocks from the last one down, when B*H is a multiple of 8;
    otherwise query blocks from the last one down with b*h fastest)."""
    out = []
    for s in range(bh_count * nqb):
        if bh_count % XCDS == 0:
            x, j = s % XCDS, s // XCDS
            hl, r = divmod(j, nqb)
            out.append((x + XCDS * hl) * nqb + (nqb - 1 - r))
        else:
            r, bh = divmod(s, bh_count)
            out.append(bh * nqb + (nqb - 1 - r))
    return np.array(out)


def xcd_loads(order, cost):
    load = np.zeros(XCDS)
    for s, it in enumerate(order):
        if it >= 0:
            load[s % XCDS] += cost[it]
    return load


def check_plan(sched, cost, n_items, tol):
    assert len(sched) % XCDS == 0 and n_items <= len(sched) <= _native.plan_cap(n_items)
    real = sched[sched >= 0]
    assert np.array_equal(np.sort(real), np.arange(n_items)), "every item exactly once"
    assert np.all(sched[sched < 0] == -1)
    load = xcd_loads(sched, cost)
    assert load.max() <= (1 + tol) * load.mean(), load
    # within each XCD: longest rows first, and idle slots only after its last item
    for x in range(XCDS):
        q = sched[x::XCDS]
        items = q[q >= 0]
        assert np.all(q[len(items):] == -1)
        c = cost[items]
        assert np.all(np.diff(c) <= 0)
    return load


@pytest.mark.parametrize("name", ["sliding", "global", "retrieval"])
def test_uniform_families_keep_the_builtin_order(name):
    w = P.workloads()[name]
    rp, _ = w.csr()
    cost = item_costs(rp)
    load = xcd_loads(builtin_order(w.B * w.H, w.nqb), cost)
    assert load.max() <= 1.02 * load.mean()
    assert _native.plan_host(rp, w.B, w.H, w.nqb) is None


def test_mixed_workload_is_planned_evenly_over_the_xcds():
    w = P.workloads()["mixed"]
    rp, _ = w.csr()
    cost = item_costs(rp)
    G = w.B * w.H * w.nqb
    before = xcd_loads(builtin_order(w.B * w.H, w.nqb), cost)
    assert before.max() > 1.05 * before.mean()  # heads x and x + 8 per XCD: unequal pairs
    sched = _native.plan_host(rp, w.B, w.H, w.nqb)
    assert sched is not None
    check_plan(sched, cost, G, tol=0.01)
    # each XCD walks a contiguous run of heads (about 2.3 heads' work each: at most 4 heads,
    # the outer two partly), so few heads' K/V tiles are live in its L2 at a time
    for x in range(XCDS):
        items = sched[x::XCDS]
        heads = sorted(set((items[items >= 0] // w.nqb).tolist()))
        assert heads == list(range(heads[0], heads[-1] + 1)) and len(heads) <= 4, heads


def test_heads_not_a_multiple_of_eight():
    B, H, T = 1, 5, 4096
    rows = lambda b, h, i: P.sliding_row(i, 2 + 6 * h)  # noqa: E731  windows 2 .. 26
    rp, _ = P.make_csr(B, H, T, rows)
    cost = item_costs(rp)
    sched = _native.plan_host(rp, B, H, T // 128)
    assert sched is not None
    check_plan(sched, cost, B * H * (T // 128), tol=0.02)


def test_extreme_skew_falls_back_to_equal_counts():
    """One head of full causal rows among heads of diagonal-only rows: equal-cost runs of the
    head sequence would need more idle slots than the budget allows, so the planner deals
    items longest first in a snake order instead (equal counts per XCD)."""
    B, H, T = 1, 8, 16384
    rows = lambda b, h, i: list(range(i + 1)) if h == 0 else [i]  # noqa: E731
    rp, _ = P.make_csr(B, H, T, rows)
    cost = item_costs(rp)
    G = B * H * (T // 128)
    sched = _native.plan_host(rp, B, H, T // 128)
    assert sched is not None
    load = check_plan(sched, cost, G, tol=0.05)
    counts = [int((sched[x::XCDS] >= 0).sum()) for x in range(XCDS)]
    assert max(counts) - min(counts) <= 1 and len(sched) == G
    assert load.max() < xcd_loads(builtin_order(H, T // 128), cost).max()


def test_generic_plans_count_no_implicit_diagonal():
    """In the generic walk an empty row costs only the item overhead."""
    B, H, T = 1, 8, 2048
    rows = lambda b, h, i: list(range(i + 1)) if h < 4 else []  # noqa: E731
    rp, _ = P.make_csr(B, H, T, rows)
    cost = item_costs(rp, generic=True)
    assert cost[4 * 16] == OVERHEAD
    sched = _native.plan_host(rp, B, H, 16, generic=True)
    assert sched is not None
    check_plan(sched, cost, B * H * 16, tol=0.05)


def test_plan_argument_errors():
    rp = np.zeros((1, 1, 3), np.int32)
    lib = _native.load()
    sched = np.empty(4, np.int32)
    assert lib.usagi_bsa_plan(rp.ctypes.data, 1, 1, 2, 0, sched.ctypes.data, 4) == -1  # cap < 12
    assert "sched_cap" in _native.last_error()
    assert lib.usagi_bsa_plan(None, 1, 1, 2, 0, sched.ctypes.data, 12) == -1


# ------------------------------------------------------------------------------ the CSR cache


def _cpu_entry(rp, ci, generic=False):
    B, H, n1 = rp.shape
    return submission._csr_entry(rp, ci, B, H, n1 - 1, torch.device("cpu"), generic)


def test_cache_checks_each_csr_once_and_rechecks_after_a_change():
    submission.clear_csr_cache()
    rp, ci = (torch.from_numpy(x) for x in P.sliding_csr(1, 2, 512, 3))
    e1 = _cpu_entry(rp, ci)
    assert _cpu_entry(rp, ci) is e1  # same objects, unchanged: no second check
    ci[0, 0, 0] = 1  # in place (torch bumps the version counter): row 0 loses its diagonal
    with pytest.raises(ValueError, match="malformed CSR"):
        _cpu_entry(rp, ci)
    ci[0, 0, 0] = 0
    e2 = _cpu_entry(rp, ci)
    assert e2 is not e1


def test_cache_does_not_trust_a_new_tensor_at_an_old_address():
    submission.clear_csr_cache()
    rp, ci = (torch.from_numpy(x) for x in P.sliding_csr(1, 1, 256, 2))
    e1 = _cpu_entry(rp, ci)
    view = ci.view(ci.shape)  # another tensor object over the same memory, same version
    assert _cpu_entry(rp, view) is not e1


def test_generic_rows_are_not_checked_but_planned():
    submission.clear_csr_cache()
    rp = torch.tensor([[[0, 0, 3]]], dtype=torch.int32)  # empty row, then [1, 1, 0]
    ci = torch.tensor([[[1, 1, 0]]], dtype=torch.int32)
    e = _cpu_entry(rp, ci, generic=True)
    assert e.sched is None or e.n_slots >= 2
    with pytest.raises(ValueError):
        _cpu_entry(rp, ci, generic=False)


def test_cache_is_bounded():
    submission.clear_csr_cache()
    keep = []
    for _ in range(submission._CSR_CACHE_SIZE + 5):
        rp, ci = (torch.from_numpy(x) for x in P.sliding_csr(1, 1, 256, 1))
        keep.append((rp, ci))
        _cpu_entry(rp, ci)
    assert len(submission._csr_cache) == submission._CSR_CACHE_SIZE
    submission.clear_csr_cache()


# ------------------------------------------------------------------------------ seq_lens, inference


def test_rows_past_seq_len_are_not_checked():
    """Rows of query blocks starting at or past seq_len are never read by the walk (v7:63-67),
    so the C check, the Python validator and the shim's cache accept them in any state."""
    submission.clear_csr_cache()
    rp = np.array([[[0, 1, 3, 3, 3]]], np.int32)  # nqb = 4; rows 2 and 3 empty
    ci = np.array([[[0, 0, 1]]], np.int32)
    for sl in ([256], [129]):
        _native.check_csr_host(rp, ci, 1, 1, 4, 3, seq_lens=np.array(sl, np.int32))
        P.validate_csr(rp, ci, 512, seq_lens=sl)
    for sl in (None, [257], [512]):
        with pytest.raises(ValueError, match="empty"):
            _native.check_csr_host(rp, ci, 1, 1, 4, 3,
                                   seq_lens=None if sl is None else np.array(sl, np.int32))
        with pytest.raises(ValueError, match="empty"):
            P.validate_csr(rp, ci, 512, seq_lens=sl)
    # no rows read at all: row_ptr may even start elsewhere
    _native.check_csr_host(rp + 5, ci, 1, 1, 4, 3, seq_lens=np.array([0], np.int32))

    trp, tci = torch.from_numpy(rp), torch.from_numpy(ci)
    sl_t = torch.tensor([256], dtype=torch.int32)
    e = submission._csr_entry(trp, tci, 1, 1, 4, torch.device("cpu"), False, sl_t)
    assert submission._csr_entry(trp, tci, 1, 1, 4, torch.device("cpu"), False, sl_t) is e
    with pytest.raises(ValueError, match="empty"):  # longer sequences read the empty rows
        submission._csr_entry(trp, tci, 1, 1, 4, torch.device("cpu"), False, [512])
    with pytest.raises(ValueError, match="empty"):
        submission._csr_entry(trp, tci, 1, 1, 4, torch.device("cpu"), False, None)
    assert submission._csr_entry(trp, tci, 1, 1, 4, torch.device("cpu"), False, [200]) is not e
    submission.clear_csr_cache()


def test_inference_mode_csr_is_cached():
    """Inference tensors carry no version counter; their CSR is checked once and then reused."""
    submission.clear_csr_cache()
    with torch.inference_mode():
        rp, ci = (torch.from_numpy(x).clone() for x in P.sliding_csr(1, 2, 512, 3))
    assert rp.is_inference()
    e = _cpu_entry(rp, ci)
    assert _cpu_entry(rp, ci) is e
    submission.clear_csr_cache()


# ------------------------------------------------------------------------------ window patterns


def _pattern(rp, ci):
    return submission.window_pattern(rp.reshape(-1, rp.shape[-1]), ci.reshape(rp.shape[0] *
                                     rp.shape[1], -1), rp.shape[-1] - 1)


@pytest.mark.parametrize("name,want", [("plumbing", (4, 0)), ("sliding", (8, 0)),
                                       ("global", (4, 4)), ("retrieval", None),
                                       ("mixed", None)])
def test_window_pattern_of_the_workloads(name, want):
    rp, ci = P.workloads()[name].csr()
    assert _pattern(rp, ci) == want


@pytest.mark.parametrize("nqb", [1, 2, 5, 16, 64])
@pytest.mark.parametrize("w", [1, 2, 3, 8, 70])
@pytest.mark.parametrize("g", [0, 1, 4, 9])
def test_window_pattern_reads_back_an_equivalent_pattern(nqb, w, g):
    """Whatever (window, n_global) it reads off, the CSR of that pattern is the same arrays."""
    T = 128 * nqb
    rp, ci = P.global_csr(2, 3, T, g, w) if g else P.sliding_csr(2, 3, T, w)
    got = _pattern(rp, ci)
    assert got is not None
    w2, g2 = got
    rp2, ci2 = P.global_csr(2, 3, T, g2, w2) if g2 else P.sliding_csr(2, 3, T, w2)
    assert np.array_equal(rp, rp2) and np.array_equal(ci, ci2[..., :ci.shape[-1]])


def test_window_pattern_rejects_near_misses():
    B, H, T = 2, 3, 2048
    rp, ci = P.sliding_csr(B, H, T, 4)
    assert _pattern(rp, ci) == (4, 0)
    drop = lambda b, h, i: [x for x in P.sliding_row(i, 4) if not (h == 2 and i == 9 and x == 7)]  # noqa: E731,E501
    assert _pattern(*P.make_csr(B, H, T, drop)) is None
    other_head = lambda b, h, i: P.sliding_row(i, 5 if (b, h) == (1, 1) else 4)  # noqa: E731
    assert _pattern(*P.make_csr(B, H, T, other_head)) is None
    desc = lambda b, h, i: sorted(P.sliding_row(i, 4)[:-1], reverse=True) + [i]  # noqa: E731
    assert _pattern(*P.make_csr(B, H, T, desc)) is None  # same blocks, another order
    extra = lambda b, h, i: P.global_row(i, 1, 4) if i == 15 else P.sliding_row(i, 4)  # noqa: E731
    assert _pattern(*P.make_csr(B, H, T, extra)) is None
    # padding past the last row's end does not matter
    ci_pad = np.concatenate([ci, np.full(ci.shape[:-1] + (5,), 77, np.int32)], axis=-1)
    assert _pattern(rp, ci_pad) == (4, 0)
