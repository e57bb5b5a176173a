"""Property-based tests (hypothesis) of the host-side CSR check and work planner over arbitrary
rows, on the CPU. The seeded tests in test_patterns.py and test_plan.py cover the workloads; these
search the space of row shapes for a counterexample."""

from __future__ import annotations

import numpy as np
import pytest
from hypothesis import HealthCheck, event, given, settings
from hypothesis import strategies as st

from tests.test_plan import XCDS, builtin_order, item_costs, xcd_loads
from usagi_amd import _native
from usagi_amd import patterns as P

SETTINGS = settings(max_examples=80, deadline=None,
                    suppress_health_check=[HealthCheck.too_slow, HealthCheck.data_too_large])


@st.composite
def csr_rows(draw, max_nqb=6):
    """B, H, nqb and one row (list of key blocks) per (b, h, qb): every row well formed (blocks
    below the diagonal in any order, then the diagonal), or one row replaced by an arbitrary
    list, or every row arbitrary."""
    B = draw(st.integers(1, 2))
    H = draw(st.integers(1, 3))
    nqb = draw(st.integers(1, max_nqb))
    mode = draw(st.sampled_from(["valid", "valid", "one_bad", "arbitrary"]))
    arbitrary = st.lists(st.integers(-1, nqb), max_size=nqb + 2)

    def good_row(qb):
        below = draw(st.permutations(sorted(draw(st.sets(st.integers(0, max(qb - 1, 0)), max_size=qb)))))
        return [c for c in below if c < qb] + [qb]

    rows = [[[draw(arbitrary) if mode == "arbitrary" else good_row(i) for i in range(nqb)]
             for _ in range(H)] for _ in range(B)]
    if mode == "one_bad":
        b, h, i = draw(st.integers(0, B - 1)), draw(st.integers(0, H - 1)), draw(st.integers(0, nqb - 1))
        rows[b][h][i] = draw(arbitrary)
    return B, H, nqb, rows


def well_formed(row, qb):
    """The precondition of the implicit-diagonal walk (kernels/v7_blockptr_warpspec.py:83-136):
    the row is non-empty, ends with its diagonal, and lists distinct blocks below it before."""
    return (len(row) > 0 and row[-1] == qb and len(set(row[:-1])) == len(row) - 1
            and all(0 <= c < qb for c in row[:-1]))


@SETTINGS
@given(csr_rows())
def test_c_and_python_checks_agree_with_the_rule(case):
    B, H, nqb, rows = case
    rp, ci = P.make_csr(B, H, 128 * nqb, lambda b, h, i: rows[b][h][i])
    expect_ok = all(well_formed(rows[b][h][i], i) for b in range(B) for h in range(H) for i in range(nqb))
    try:
        P.validate_csr(rp, ci, 128 * nqb)
        py_ok = True
    except ValueError:
        py_ok = False
    try:
        _native.check_csr_host(rp, ci, B, H, nqb, ci.shape[-1])
        c_ok = True
    except ValueError:
        c_ok = False
    assert py_ok == c_ok == expect_ok
    event("well formed" if expect_ok else "malformed")


@st.composite
def row_lengths(draw):
    """row_ptr for B*H heads of nqb query blocks with arbitrary (skewed) row lengths."""
    B = draw(st.integers(1, 2))
    H = draw(st.sampled_from([1, 3, 4, 8, 12, 16]))
    nqb = draw(st.integers(1, 24))
    generic = draw(st.booleans())
    lo = 0 if generic else 1
    per_head = draw(st.lists(st.integers(lo, 40), min_size=B * H, max_size=B * H))
    jitter = draw(st.integers(0, 6))
    rng = np.random.default_rng(draw(st.integers(0, 2**31 - 1)))
    rp = np.zeros((B, H, nqb + 1), dtype=np.int32)
    for k in range(B * H):
        n = np.clip(per_head[k] + rng.integers(-jitter, jitter + 1, size=nqb), lo, None)
        rp.reshape(B * H, nqb + 1)[k, 1:] = np.cumsum(n)
    return B, H, nqb, generic, rp


@SETTINGS
@given(row_lengths())
def test_plan_is_a_balanced_permutation(case):
    B, H, nqb, generic, rp = case
    n_items = B * H * nqb
    cost = item_costs(rp, generic)
    sched = _native.plan_host(rp, B, H, nqb, generic)
    if sched is None:
        # The planner keeps the built-in order only when it is already balanced.
        load = xcd_loads(builtin_order(B * H, nqb), cost)
        assert load.max() <= 1.02 * load.mean() + 1e-9
        event("built-in order kept")
        return
    event("planned")
    assert len(sched) % XCDS == 0 and n_items <= len(sched) <= _native.plan_cap(n_items)
    real = sched[sched >= 0]
    assert np.array_equal(np.sort(real), np.arange(n_items)), "every item exactly once"
    assert np.all(sched[sched < 0] == -1)
    load = xcd_loads(sched, cost)
    assert load.max() <= load.mean() + 2 * cost.max() + 1e-9, (load, cost.max())
    for x in range(XCDS):
        q = sched[x::XCDS]
        items = q[q >= 0]
        assert np.all(q[len(items):] == -1), "idle slots only after an XCD's last item"
        assert np.all(np.diff(cost[items]) <= 0), "longest rows first within an XCD"


@pytest.mark.parametrize("generic", [False, True])
def test_planner_keeps_a_balanced_order_and_replaces_a_skewed_one(generic):
    """Both outcomes on fixed rows: equal rows keep the built-in order, three heads of five
    times the length get a plan."""
    uniform = np.tile(np.arange(0, 8 * 4, 4, dtype=np.int32), (1, 8, 1))[:, :, :8]
    rp = np.zeros((1, 8, 8), dtype=np.int32)
    rp[..., :] = uniform
    assert _native.plan_host(rp, 1, 8, 7, generic) is None
    skew = rp.copy()
    skew[0, :3] *= 5
    assert _native.plan_host(skew, 1, 8, 7, generic) is not None
