"""Shared helpers for the test suite."""

from __future__ import annotations

import numpy as np

ATOL = 2e-3  # atol = rtol = 2e-3 against fp32 dense-masked attention
RTOL = 2e-3


def assert_close(got, want, atol=ATOL, rtol=RTOL, what="O"):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    inf_w = np.isinf(want)
    assert np.array_equal(np.isinf(got), inf_w), f"{what}: -inf positions differ"
    assert np.array_equal(got[inf_w], want[inf_w]), f"{what}: inf signs differ"
    g = got[~inf_w]
    w = want[~inf_w]
    assert np.all(np.isfinite(g)), f"{what}: non-finite values"
    err = np.abs(g - w)
    bad = err > atol + rtol * np.abs(w)
    if bad.any():
        i = int(np.argmax(err - (atol + rtol * np.abs(w))))
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} elements out of tolerance; "
                             f"max abs err {err.max():.3e}; worst got {g[i]!r} want {w[i]!r}")
