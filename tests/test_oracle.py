"""Pins of the CPU oracle (no GPU).

The reference has no tests or golden vectors of its own (its correctness lived in an external
challenge harness), so the oracle is pinned by checks that do not restate its formula:
  * the golden fixtures of tests/golden/ (fp64 brute force over explicitly enumerated key sets);
  * torch.nn.functional.scaled_dot_product_attention for a full lower-triangular CSR (plain
    causal attention) and for a diagonal-only CSR (causal attention inside each 128 block);
  * closed forms: V constant -> O constant; Q = 0 -> O = mean of the visible V rows; query row 0
    attends only key 0 -> O = V[0], LSE = q0·k0/sqrt(128); LSE = logsumexp of the visible
    scaled scores; a seq_len cut gives O = 0 / LSE = -inf past it;
  * the reference's own walk restated twice (numpy blockwise_v7, C bsa_ref.c) agreeing with the
    dense-masked oracle;
  * planted mistakes (oracle._mutation) that each of these checks must reject.
The generic walk (blockwise_v1 and the C walk with generic=True) is pinned by its own fixture
(golden_generic_t384.npz: fp64 over key multisets), by agreeing with the dense-masked oracle on
rows in any order with or without their diagonal, and by duplicating every entry (O unchanged,
LSE + ln 2). The PyTorch CPU oracle (oracle/torch_dense.py, the timed CPU baseline) is pinned by
the fixtures and by agreeing with bsa_oracle.dense_masked.
"""

from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from oracle import bsa_oracle as O
from oracle import c_ref, torch_dense
from tests._helpers import assert_close
from usagi_amd import patterns as P

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _rand_qkv(B, H, T, seed, dtype=np.float16):
    rng = np.random.default_rng(seed)
    return tuple(rng.standard_normal((B, H, T, 128)).astype(dtype) for _ in range(3))


@pytest.fixture(scope="module", autouse=True)
def _c_oracle_built():
    if not os.path.exists(c_ref.LIB):
        from oracle.build import build

        build()


# ------------------------------------------------------------------------------ golden


@pytest.mark.parametrize("name", ["golden_families_t512.npz", "golden_seqlens_t256.npz"])
@pytest.mark.parametrize("impl", ["dense", "dense64", "blockwise", "c"])
def test_oracle_matches_golden(name, impl):
    g = np.load(os.path.join(GOLDEN, name))
    args = (g["q"], g["k"], g["v"], g["row_ptr"], g["col_idx"], g["seq_lens"])
    if impl == "dense":
        o, lse = O.dense_masked(*args)
        tol = 2e-5
    elif impl == "dense64":
        o, lse = O.dense_masked(*args, dtype=np.float64)
        tol = 1e-6
    elif impl == "blockwise":
        o, lse = O.blockwise_v7(*args)
        tol = 2e-3  # P is rounded to fp16 before P·V, as in the reference
    else:
        o, lse = c_ref.fwd(*[a.astype(np.float32) if a.dtype == np.float16 else a for a in args])
        tol = 2e-3
    assert_close(o, g["out"], atol=tol, rtol=tol)
    assert_close(lse, g["lse"], atol=tol, rtol=tol, what="LSE")


# ------------------------------------------------------------------------------ library routines


def _sdpa(q, k, v, mask):
    qt, kt, vt = (torch.from_numpy(x.astype(np.float64)) for x in (q, k, v))
    return torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask).numpy()


def test_full_lower_triangular_csr_is_causal_sdpa():
    B, H, T = 1, 2, 512
    nqb = T // 128
    rp, ci = P.make_csr(B, H, T, lambda b, h, i: list(range(i + 1)))
    q, k, v = _rand_qkv(B, H, T, 1)
    o, _ = O.dense_masked(q, k, v, rp, ci, dtype=np.float64)
    causal = torch.ones(T, T, dtype=torch.bool).tril()
    ref = _sdpa(q, k, v, causal)
    assert np.abs(o - ref).max() < 1e-10
    assert nqb == 4


def test_diagonal_only_csr_is_blockwise_causal_sdpa():
    B, H, T = 1, 2, 384
    rp, ci = P.make_csr(B, H, T, lambda b, h, i: [i])
    q, k, v = _rand_qkv(B, H, T, 2)
    o, _ = O.dense_masked(q, k, v, rp, ci, dtype=np.float64)
    t = torch.arange(T)
    mask = (t[None, :] <= t[:, None]) & (t[None, :] // 128 == t[:, None] // 128)
    ref = _sdpa(q, k, v, mask)
    assert np.abs(o - ref).max() < 1e-10


# ------------------------------------------------------------------------------ closed forms


def test_constant_v_gives_constant_output():
    B, H, T = 1, 2, 512
    rp, ci = P.retrieval_csr(B, H, T, 2, 5)
    q, k, _ = _rand_qkv(B, H, T, 3)
    v = np.full((B, H, T, 128), 0.625, np.float16)
    o, _ = O.dense_masked(q, k, v, rp, ci)
    assert np.abs(o - 0.625).max() < 1e-6


def test_zero_q_gives_mean_of_visible_rows():
    B, H, T = 1, 1, 384
    w = 2
    rp, ci = P.sliding_csr(B, H, T, w)
    _, k, v = _rand_qkv(B, H, T, 4)
    q = np.zeros_like(k)
    o, lse = O.dense_masked(q, k, v, rp, ci, dtype=np.float64)
    vd = v.astype(np.float64)[0, 0]
    for t in (0, 5, 127, 128, 200, 383):
        lo = max(0, t // 128 - w + 1) * 128
        visible = vd[lo:t + 1]
        assert np.abs(o[0, 0, t] - visible.mean(axis=0)).max() < 1e-12
        assert abs(lse[0, 0, t] - math.log(t + 1 - lo)) < 1e-12


def test_first_query_row_attends_only_key_zero():
    B, H, T = 2, 2, 256
    rp, ci = P.global_csr(B, H, T, 1, 2)
    q, k, v = _rand_qkv(B, H, T, 5)
    o, lse = O.dense_masked(q, k, v, rp, ci, dtype=np.float64)
    for b in range(B):
        for h in range(H):
            assert np.abs(o[b, h, 0] - v[b, h, 0].astype(np.float64)).max() < 1e-12
            s00 = float(q[b, h, 0].astype(np.float64) @ k[b, h, 0].astype(np.float64)) / math.sqrt(128)
            assert abs(lse[b, h, 0] - s00) < 1e-12


def test_lse_is_logsumexp_of_visible_scores():
    from scipy.special import logsumexp

    B, H, T = 1, 1, 512
    rp, ci = P.random_csr(B, H, T, 0.5, 9)
    q, k, v = _rand_qkv(B, H, T, 6)
    _, lse = O.dense_masked(q, k, v, rp, ci, dtype=np.float64)
    rows = P.csr_rows(rp, ci, 0, 0)
    qd, kd = q[0, 0].astype(np.float64), k[0, 0].astype(np.float64)
    for t in (0, 130, 255, 300, 511):
        qb = t // 128
        keys = [s for kb in rows[qb] for s in range(kb * 128, (kb + 1) * 128) if s <= t]
        ref = logsumexp(kd[keys] @ qd[t] / math.sqrt(128))
        assert abs(lse[0, 0, t] - ref) < 1e-10


def test_seq_len_cut():
    B, H, T = 2, 1, 384
    rp, ci = P.sliding_csr(B, H, T, 3)
    q, k, v = _rand_qkv(B, H, T, 7)
    o, lse = O.dense_masked(q, k, v, rp, ci, np.array([384, 140]))
    assert np.all(o[1, 0, 140:] == 0) and np.all(np.isneginf(lse[1, 0, 140:]))
    assert np.all(np.isfinite(lse[1, 0, :140])) and np.all(np.isfinite(lse[0]))
    # rows before the cut only see keys before the cut: identical to a run on truncated data
    o2, _ = O.dense_masked(q, k, v, rp, ci, np.array([384, 384]))
    assert np.abs(o[1, 0, :140] - o2[1, 0, :140]).max() < 1e-6


# ------------------------------------------------------------------------------ restatements


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_blockwise_and_c_restatements_match_dense(seed):
    rng = np.random.default_rng(seed)
    B, H = 2, 2
    T = 128 * int(rng.integers(1, 6))
    rp, ci = P.random_csr(B, H, T, float(rng.uniform(0.1, 0.9)), seed)
    q, k, v = _rand_qkv(B, H, T, 20 + seed)
    sl = np.array([T, int(rng.integers(1, T + 1))])
    od, ld = O.dense_masked(q, k, v, rp, ci, sl)
    ob, lb = O.blockwise_v7(q, k, v, rp, ci, sl)
    oc, lc = c_ref.fwd(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), rp, ci, sl)
    assert_close(ob, od)
    assert_close(lb, ld, what="LSE")
    assert_close(oc, ob, atol=1e-4, rtol=1e-4)
    assert_close(lc, lb, atol=1e-5, rtol=1e-5, what="LSE")


def test_off_diagonal_order_does_not_matter():
    B, H, T = 1, 1, 768
    rp, ci = P.random_csr(B, H, T, 0.7, 3)
    q, k, v = _rand_qkv(B, H, T, 8)
    ci2 = ci.copy()
    rng = np.random.default_rng(0)
    for i in range(T // 128):
        a, b = rp[0, 0, i], rp[0, 0, i + 1] - 1  # keep the diagonal last
        ci2[0, 0, a:b] = rng.permutation(ci2[0, 0, a:b])
    o1, l1 = O.blockwise_v7(q, k, v, rp, ci)
    o2, l2 = O.blockwise_v7(q, k, v, rp, ci2)
    # Equal up to the fp16 rounding of P, which depends on the running max at each block.
    assert_close(o2, o1, atol=5e-4, rtol=5e-4)
    assert_close(l2, l1, atol=1e-5, rtol=1e-5, what="LSE")


# ------------------------------------------------------------------------------ planted mistakes


@pytest.mark.parametrize("mutation", O.MUTATIONS)
def test_pins_reject_planted_mistakes(mutation):
    """Each planted mistake in the oracle must fail at least one of the pins above."""
    g = np.load(os.path.join(GOLDEN, "golden_families_t512.npz"))
    args = (g["q"], g["k"], g["v"], g["row_ptr"], g["col_idx"], g["seq_lens"])
    o, lse = O.dense_masked(*args, _mutation=mutation)
    caught_golden = not (np.allclose(o, g["out"], atol=2e-5, rtol=2e-5)
                         and np.allclose(lse, g["lse"], atol=2e-5, rtol=2e-5))
    # the closed form at query row 0 alone
    s00 = float(g["q"][0, 0, 0].astype(np.float64) @ g["k"][0, 0, 0].astype(np.float64)) / math.sqrt(128)
    caught_row0 = (abs(lse[0, 0, 0] - s00) > 1e-4
                   or np.abs(o[0, 0, 0] - g["v"][0, 0, 0].astype(np.float64)).max() > 1e-4)
    assert caught_golden, mutation
    if mutation in ("scale_1_over_d", "mask_transposed", "k_for_v"):
        assert caught_row0, mutation


# ------------------------------------------------------------------------------ C restatement under ASan


def test_c_restatement_under_address_sanitizer(tmp_path):
    import subprocess
    import sys

    from oracle.build import build

    lib = build(asan=True)
    libasan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True,
                             text=True).stdout.strip()
    code = f"""
import numpy as np, sys
sys.path.insert(0, {repr(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))})
from oracle import c_ref, torch_dense
from usagi_amd import patterns as P
rp, ci = P.random_csr(2, 2, 384, 0.6, 1)
rng = np.random.default_rng(0)
q, k, v = (rng.standard_normal((2, 2, 384, 128)).astype(np.float32) for _ in range(3))
o, l = c_ref.fwd(q, k, v, rp, ci, np.array([384, 200]), lib=c_ref.load({repr(lib)}))
assert np.isfinite(o).all()
print("ok")
"""
    env = dict(os.environ, LD_PRELOAD=libasan, ASAN_OPTIONS="detect_leaks=0")
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env,
                         timeout=600)
    assert res.returncode == 0 and "ok" in res.stdout, res.stderr[-2000:]


# ------------------------------------------------------------------------------ PyTorch CPU oracle


@pytest.mark.parametrize("name", ["golden_families_t512.npz", "golden_seqlens_t256.npz"])
def test_torch_dense_matches_golden(name):
    g = np.load(os.path.join(GOLDEN, name))
    q, k, v = (torch.from_numpy(g[x]) for x in ("q", "k", "v"))
    o, lse = torch_dense.dense_masked(q, k, v, torch.from_numpy(g["row_ptr"]),
                                      torch.from_numpy(g["col_idx"]), g["seq_lens"])
    assert_close(o.numpy(), g["out"], atol=2e-5, rtol=2e-5)
    assert_close(lse.numpy(), g["lse"], atol=2e-5, rtol=2e-5, what="LSE")


def test_torch_dense_matches_numpy_dense_on_a_head_subset():
    B, H, T = 2, 3, 1280  # two query slabs of 1024 rows, the second one partial
    rp, ci = P.retrieval_csr(B, H, T, 4, 8)
    q, k, v = P.make_qkv(B, H, T, seed=60)
    heads = [(0, 2), (1, 0)]
    sl = np.array([T, 1000])
    o, lse = torch_dense.dense_masked(q, k, v, torch.from_numpy(rp), torch.from_numpy(ci), sl,
                                      heads=heads)
    od, ld = O.dense_masked(q, k, v, rp, ci, sl, heads=heads)
    for b, h in heads:
        assert_close(o[b, h].numpy(), od[b, h], atol=1e-5, rtol=1e-5)
        assert_close(lse[b, h].numpy(), ld[b, h], atol=1e-5, rtol=1e-5, what="LSE")
    assert torch.isnan(o[0, 0]).all()  # heads outside the subset stay NaN


# ------------------------------------------------------------------------------ generic walk (v1)


def _golden_generic():
    g = np.load(os.path.join(GOLDEN, "golden_generic_t384.npz"))
    return g, (g["q"], g["k"], g["v"], g["row_ptr"], g["col_idx"], g["seq_lens"])


@pytest.mark.parametrize("impl", ["blockwise", "blockwise_fp32", "c"])
def test_generic_walk_matches_golden(impl):
    g, args = _golden_generic()
    if impl == "blockwise":
        o, lse = O.blockwise_v1(*args)
        tol = 2e-3  # P rounded to fp16 before P·V, as in the reference (v1:395)
    elif impl == "blockwise_fp32":
        o, lse = O.blockwise_v1(*args, round_p_fp16=False)
        tol = 2e-5
    else:
        o, lse = c_ref.fwd(*[a.astype(np.float32) if a.dtype == np.float16 else a for a in args],
                           generic=True)
        tol = 2e-3
    assert_close(o, g["out"], atol=tol, rtol=tol)
    assert_close(lse, g["lse"], atol=tol, rtol=tol, what="LSE")


def test_generic_golden_covers_its_cases():
    g, _ = _golden_generic()
    # head 1, qb 0 is an empty row: O = 0, LSE = -inf for every row of it
    assert np.all(g["out"][:, 1, :128] == 0) and np.all(np.isneginf(g["lse"][:, 1, :128]))
    # batch 1 has seq_len 200: query block 2 is cut entirely
    assert np.all(g["out"][1, :, 256:] == 0) and np.all(np.isneginf(g["lse"][1, :, 256:]))
    assert np.all(np.isfinite(g["lse"][0, 0]))


@pytest.mark.parametrize("mutation", O.V1_MUTATIONS)
def test_generic_pins_reject_planted_mistakes(mutation):
    g, args = _golden_generic()
    o, lse = O.blockwise_v1(*args, round_p_fp16=False, _mutation=mutation)
    assert not (np.allclose(o, g["out"], atol=2e-3, rtol=2e-3)
                and np.allclose(lse, g["lse"], atol=2e-3, rtol=2e-3)), mutation


def _shuffled_rows(rp, ci, seed, drop_diag_every=0):
    """Every row permuted (diagonal anywhere); with drop_diag_every = n, every n-th row loses
    its diagonal. Returns a new (row_ptr, col_idx)."""
    rng = np.random.default_rng(seed)
    B, H, n1 = rp.shape
    rows = []
    for b in range(B):
        rows.append([])
        for h in range(H):
            rr = []
            for i in range(n1 - 1):
                r = [int(x) for x in ci[b, h, rp[b, h, i]:rp[b, h, i + 1]]]
                if drop_diag_every and i % drop_diag_every == 1:
                    r = [x for x in r if x != i]
                rr.append([int(x) for x in rng.permutation(r)])
            rows[b].append(rr)
    return P.rows_to_csr(rows)


@pytest.mark.parametrize("seed", [0, 1])
def test_generic_walk_equals_dense_on_rows_in_any_order(seed):
    """Rows of distinct blocks at or below the query block, in any order, with or without
    their diagonal: the generic walk is the dense block mask ∧ causal ∧ seq_len attention."""
    B, H, T = 2, 2, 640
    rp, ci = P.random_csr(B, H, T, 0.6, 30 + seed)
    rp2, ci2 = _shuffled_rows(rp, ci, seed, drop_diag_every=3)
    q, k, v = _rand_qkv(B, H, T, 40 + seed)
    sl = np.array([T, 333])
    od, ld = O.dense_masked(q, k, v, rp2, ci2, sl)
    ob, lb = O.blockwise_v1(q, k, v, rp2, ci2, sl)
    oc, lc = c_ref.fwd(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), rp2, ci2,
                       sl, generic=True)
    assert_close(ob, od)
    assert_close(lb, ld, what="LSE")
    assert_close(oc, ob, atol=1e-4, rtol=1e-4)
    assert_close(lc, lb, atol=1e-5, rtol=1e-5, what="LSE")
    # the v7 walk agrees where its precondition holds (every row ends with its diagonal)
    o7, l7 = O.blockwise_v7(q, k, v, rp, ci, sl)
    o1, l1 = O.blockwise_v1(q, k, v, rp, ci, sl)
    assert_close(o1, o7, atol=5e-4, rtol=5e-4)
    assert_close(l1, l7, atol=1e-5, rtol=1e-5, what="LSE")


def test_generic_walk_duplicated_entries_add_ln2():
    """Listing every entry twice doubles every weight: O is unchanged, LSE grows by ln 2."""
    B, H, T = 1, 2, 512
    rp, ci = P.random_csr(B, H, T, 0.5, 5)
    rows = [[[r + r for r in P.csr_rows(rp, ci, b, h)] for h in range(H)] for b in range(B)]
    rp2, ci2 = P.rows_to_csr(rows)
    q, k, v = _rand_qkv(B, H, T, 9)
    o1, l1 = O.blockwise_v1(q, k, v, rp, ci, round_p_fp16=False)
    o2, l2 = O.blockwise_v1(q, k, v, rp2, ci2, round_p_fp16=False)
    assert_close(o2, o1, atol=1e-5, rtol=1e-5)
    assert_close(l2 - math.log(2.0), l1, atol=1e-5, rtol=1e-5, what="LSE")
    oc, lc = c_ref.fwd(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), rp2, ci2,
                       round_p_fp16=False, generic=True)
    assert_close(oc, o2, atol=1e-5, rtol=1e-5)
    assert_close(lc, l2, atol=1e-5, rtol=1e-5, what="LSE")
