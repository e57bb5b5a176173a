"""GPU tests of the generic CSR walk (block_sparse_attn_fwd_generic, kernels/v1_baseline.py:
331-406), the work plan, the seq_lens-free kernel variant and the CSR check of the default walk.
Parity as in test_gpu_parity.py: atol = rtol = 2e-3 against fp32 attention (the C walk in fp32
with generic=True for the generic rows, pinned by the CPU suite to its own fp64 fixture)."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import c_ref
from tests._helpers import assert_close
from usagi_amd import _native, block_sparse_attn_fwd, block_sparse_attn_fwd_generic
from usagi_amd import block_sparse_attn_fwd_window
from usagi_amd import patterns as P
from usagi_amd import submission

pytestmark = pytest.mark.gpu

DEV = "cuda"
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
BF16_RTOL = 2e-3 + 2.0 ** -9  # O stored in bf16 (half an ulp, 2^-9 relative) on top of 2e-3


def _dev(x):
    if isinstance(x, torch.Tensor):
        return x.to(DEV)
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def run(fn, q, k, v, rp, ci, sl=None):
    dsl = None if sl is None else torch.as_tensor(np.asarray(sl, dtype=np.int32)).to(DEV)
    o, lse = fn(_dev(q), _dev(k), _dev(v), _dev(rp), _dev(ci), dsl)
    torch.cuda.synchronize()
    return o.float().cpu().numpy(), lse.cpu().numpy()


def c_generic(q, k, v, rp, ci, sl=None):
    qs, ks, vs = (x.float().numpy() for x in (q, k, v))
    return c_ref.fwd(qs, ks, vs, rp, ci, None if sl is None else np.asarray(sl, np.int32),
                     round_p_fp16=False, generic=True)


def messy_csr(B, H, T, seed, max_len=None):
    """Rows for the generic walk: random length (empty rows included), entries drawn from the
    whole sequence (blocks above the diagonal too), repeats allowed, the diagonal anywhere or
    missing, random order."""
    rng = np.random.default_rng(seed)
    nqb = T // 128
    max_len = max_len or nqb + 3

    def row(b, h, i):
        n = int(rng.integers(0, max_len + 1))
        r = [int(x) for x in rng.integers(0, nqb, size=n)]
        if rng.random() < 0.6:
            r.insert(int(rng.integers(0, len(r) + 1)), i)
        return r

    return P.make_csr(B, H, T, row)


def test_generic_golden_fixture():
    g = np.load(os.path.join(GOLDEN, "golden_generic_t384.npz"))
    q, k, v = (torch.from_numpy(g[x]) for x in ("q", "k", "v"))
    print("case generic golden", flush=True)
    o, lse = run(block_sparse_attn_fwd_generic, q, k, v, g["row_ptr"], g["col_idx"], g["seq_lens"])
    assert_close(o, g["out"])
    assert_close(lse, g["lse"], what="LSE")


@pytest.mark.parametrize("seed", range(8))
def test_generic_messy_rows_vs_fp32_walk(seed):
    rng = np.random.default_rng(900 + seed)
    B, H = int(rng.integers(1, 3)), int(rng.integers(1, 5))
    T = 128 * int(rng.integers(1, 13))
    dtype = torch.bfloat16 if seed % 3 == 2 else torch.float16
    sl = None
    if seed % 2:
        sl = [int(x) for x in rng.integers(0, T + 1, size=B)]
    rp, ci = messy_csr(B, H, T, seed)
    q, k, v = P.make_qkv(B, H, T, seed=910 + seed, dtype=dtype)
    print(f"case generic messy seed={seed} B{B} H{H} T{T} {dtype} seq_lens={sl}", flush=True)
    o, lse = run(block_sparse_attn_fwd_generic, q, k, v, rp, ci, sl)
    oo, ol = c_generic(q, k, v, rp, ci, sl)
    assert_close(o, oo, rtol=BF16_RTOL if dtype == torch.bfloat16 else 2e-3)
    assert_close(lse, ol, what="LSE")


def test_generic_rows_longer_than_64_entries():
    """Rows of 70-140 entries: the diagonal search and the entry after it cross the 64-entry
    chunks of the column list."""
    B, H, T = 1, 2, 128 * 48
    rng = np.random.default_rng(5)

    def row(b, h, i):
        r = [int(x) for x in rng.integers(0, i + 1, size=int(rng.integers(70, 140)))]
        r[int(rng.integers(64, len(r)))] = i  # the first diagonal sits past entry 63
        return [x if x != i else max(i - 1, 0) for x in r[:64]] + r[64:]

    rp, ci = P.make_csr(B, H, T, row)
    q, k, v = P.make_qkv(B, H, T, seed=6)
    print("case generic long rows", flush=True)
    o, lse = run(block_sparse_attn_fwd_generic, q, k, v, rp, ci)
    oo, ol = c_generic(q, k, v, rp, ci)
    assert_close(o, oo)
    assert_close(lse, ol, what="LSE")


@pytest.mark.parametrize("name", ["sliding", "retrieval"])
def test_generic_walk_equals_default_walk_bitwise(name):
    """Rows that end with their diagonal are walked in the same order by both: the diagonal
    first, then the entries before it."""
    w = P.workloads()[name]
    rp, ci = w.csr()
    q, k, v = P.make_qkv(w.B, w.H, w.T, seed=12)
    print(f"case generic == default {name}", flush=True)
    o1, l1 = run(block_sparse_attn_fwd, q, k, v, rp, ci)
    o2, l2 = run(block_sparse_attn_fwd_generic, q, k, v, rp, ci)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)


def test_generic_out_of_range_entries_are_clamped():
    """Entries below 0 or past the last block read block 0 / the last block (memory safety; the
    reference would read outside K/V)."""
    B, H, T = 1, 2, 512
    rp, ci = P.make_csr(B, H, T, lambda b, h, i: [-7, i, 99])
    rp2, ci2 = P.make_csr(B, H, T, lambda b, h, i: [0, i, 3])
    q, k, v = P.make_qkv(B, H, T, seed=13)
    print("case generic clamped entries", flush=True)
    o1, l1 = run(block_sparse_attn_fwd_generic, q, k, v, rp, ci)
    o2, l2 = run(block_sparse_attn_fwd_generic, q, k, v, rp2, ci2)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)


# ------------------------------------------------------------------------------ work plan


def _launch(q, k, v, rp, ci, sched, n_slots, generic=False):
    """Straight through the C ABI, so the plan can be left out."""
    B, H, T, D = q.shape
    o = torch.empty_like(q)
    lse = torch.empty((B, H, T), device=DEV, dtype=torch.float32)
    stream = torch.cuda.current_stream().cuda_stream
    _native.fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), rp.data_ptr(), ci.data_ptr(), None,
                o.data_ptr(), lse.data_ptr(), B, H, T, D, ci.shape[-1], _native.FP16,
                None if sched is None else sched.data_ptr(), n_slots, stream, generic=generic)
    torch.cuda.synchronize()
    return o, lse


@pytest.mark.parametrize("generic", [False, True])
def test_plan_gives_bitwise_the_same_result(generic):
    w = P.workloads()["mixed"]
    rp, ci = w.csr()
    sched = _native.plan_host(rp, w.B, w.H, w.nqb, generic)
    assert sched is not None and len(sched) > w.B * w.H * w.nqb  # idle slots included
    q, k, v = (x.to(DEV) for x in P.make_qkv(w.B, w.H, w.T, seed=14))
    drp, dci = _dev(rp), _dev(ci)
    print(f"case plan generic={generic}", flush=True)
    o1, l1 = _launch(q, k, v, drp, dci, None, 0, generic)
    o2, l2 = _launch(q, k, v, drp, dci, _dev(sched), len(sched), generic)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    # and the shim picks the plan up by itself
    fn = block_sparse_attn_fwd_generic if generic else block_sparse_attn_fwd
    o3, l3 = fn(q, k, v, drp, dci, None)
    torch.cuda.synchronize()
    assert torch.equal(o1, o3) and torch.equal(l1, l3)


# ------------------------------------------------------------------------------ seq_lens-free variant


def test_without_seq_lens_equals_seq_lens_of_t_bitwise():
    """seq_lens None runs the variant with the length masks compiled out; seq_lens all T runs
    the masked one. Every row is valid in both, so the results agree bit for bit."""
    w = P.workloads()["sliding"]
    rp, ci = w.csr()
    q, k, v = (x.to(DEV) for x in P.make_qkv(w.B, w.H, w.T, seed=15))
    drp, dci = _dev(rp), _dev(ci)
    full = torch.full((w.B,), w.T, dtype=torch.int32, device=DEV)
    print("case seq_lens None vs T", flush=True)
    for fn in (block_sparse_attn_fwd, block_sparse_attn_fwd_generic):
        o1, l1 = fn(q, k, v, drp, dci, None)
        o2, l2 = fn(q, k, v, drp, dci, full)
        torch.cuda.synchronize()
        assert torch.equal(o1, o2) and torch.equal(l1, l2)
    o1, l1 = block_sparse_attn_fwd_window(q, k, v, 8, 0, None)
    o2, l2 = block_sparse_attn_fwd_window(q, k, v, 8, 0, full)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


# ------------------------------------------------------------------------------ CSR check


def test_default_walk_rejects_a_row_whose_diagonal_is_not_last():
    """The reference's walk would attend the future tokens of such a row (its last entry is
    taken as the diagonal); the shim raises instead, before any launch."""
    submission.clear_csr_cache()
    B, H, T = 1, 2, 512
    rp, ci = P.make_csr(B, H, T, lambda b, h, i: [i, 0] if i == 2 else list(range(i + 1)))
    q, k, v = P.make_qkv(B, H, T, seed=16)
    print("case CSR check", flush=True)
    with pytest.raises(ValueError, match="not the diagonal"):
        run(block_sparse_attn_fwd, q, k, v, rp, ci)
    # the generic walk defines that row: entries 2 (causally masked) and 0
    o, lse = run(block_sparse_attn_fwd_generic, q, k, v, rp, ci)
    oo, ol = c_generic(q, k, v, rp, ci)
    assert_close(o, oo)
    assert_close(lse, ol, what="LSE")


# ------------------------------------------------------------------------------ timing hook


def test_timing_hook_times_the_kernel_itself():
    """usagi_bsa_time_next_launch attaches events to the next dispatch: their elapsed time is
    positive and within the events recorded around the call, the result is unchanged, and the
    setting is used by that one launch only."""
    w = P.workloads()["sliding"]
    rp, ci = w.csr()
    q, k, v = (x.to(DEV) for x in P.make_qkv(w.B, w.H, w.T, seed=17))
    drp, dci = _dev(rp), _dev(ci)
    st = torch.cuda.current_stream()
    o1, l1 = block_sparse_attn_fwd(q, k, v, drp, dci, None)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    for e in ev:
        e.record(st)
    torch.cuda.synchronize()
    print("case timing hook", flush=True)
    ev[0].record(st)
    _native.time_next_launch(ev[1].cuda_event, ev[2].cuda_event)
    o2, l2 = block_sparse_attn_fwd(q, k, v, drp, dci, None)
    ev[3].record(st)
    o3, l3 = block_sparse_attn_fwd(q, k, v, drp, dci, None)  # no events attached any more
    torch.cuda.synchronize()
    kernel_ms = ev[1].elapsed_time(ev[2])
    call_ms = ev[0].elapsed_time(ev[3])
    assert 0.0 < kernel_ms <= call_ms, (kernel_ms, call_ms)
    assert torch.equal(o1, o2) and torch.equal(l1, l2) and torch.equal(o1, o3)


def test_timing_hook_is_used_up_by_a_rejected_call():
    """A forward call that rejects its arguments still uses up the events set before it, so they
    never attach to a later, unrelated launch."""
    w = P.workloads()["sliding"]
    rp, ci = w.csr()
    q, k, v = (x.to(DEV) for x in P.make_qkv(w.B, w.H, w.T, seed=18))
    drp, dci = _dev(rp), _dev(ci)
    st = torch.cuda.current_stream()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    for e in ev:
        e.record(st)
    torch.cuda.synchronize()
    before = ev[0].elapsed_time(ev[1])
    print("case timing hook after a rejected call", flush=True)
    _native.time_next_launch(ev[0].cuda_event, ev[1].cuda_event)
    with pytest.raises(_native.NativeError):
        _native.fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), drp.data_ptr(), dci.data_ptr(),
                    None, q.data_ptr(), None, w.B, w.H, w.T, 64, ci.shape[-1], _native.FP16,
                    None, 0, st.cuda_stream)  # head_dim 64: rejected before any launch
    block_sparse_attn_fwd(q, k, v, drp, dci, None)
    torch.cuda.synchronize()
    assert ev[0].elapsed_time(ev[1]) == before


@pytest.mark.parametrize("name", ["mixed", "sliding"])
def test_unchecked_csr_is_planned_without_a_synchronisation(monkeypatch, name):
    """With the check off, the first call launches the CSR walk in the built-in order at once
    and copies the CSR to the host behind it; a later call picks the copy up and switches to
    the work plan (mixed) or the analytic rows (sliding). Every call gives the same bits."""
    monkeypatch.setattr(submission, "VALIDATE_CSR", False)
    submission.clear_csr_cache()
    w = P.workloads()[name]
    rp, ci = w.csr()
    q, k, v = (x.to(DEV) for x in P.make_qkv(w.B, w.H, w.T, seed=19))
    drp, dci = _dev(rp), _dev(ci)
    print(f"case unchecked CSR {name}", flush=True)
    o1, l1 = block_sparse_attn_fwd(q, k, v, drp, dci, None)
    (entry,) = submission._csr_cache.values()
    assert entry.pending is not None and entry.sched is None and entry.window is None
    torch.cuda.synchronize()
    o2, l2 = block_sparse_attn_fwd(q, k, v, drp, dci, None)
    assert entry.pending is None
    if name == "mixed":
        assert entry.sched is not None and entry.n_slots > w.B * w.H * w.nqb
    else:
        assert entry.window == (8, 0)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    submission.clear_csr_cache()


@pytest.mark.parametrize("validate", [True, False])
def test_planned_csr_launched_from_other_streams(monkeypatch, validate):
    """A work plan copied on one stream is used by launches on others (they wait for an
    asynchronous copy and keep its memory alive): every stream gives the same bits."""
    monkeypatch.setattr(submission, "VALIDATE_CSR", validate)
    submission.clear_csr_cache()
    w = P.workloads()["mixed"]
    rp, ci = w.csr()
    q, k, v = (x.to(DEV) for x in P.make_qkv(w.B, w.H, w.T, seed=20))
    drp, dci = _dev(rp), _dev(ci)
    print(f"case plan across streams validate={validate}", flush=True)
    o0, l0 = block_sparse_attn_fwd(q, k, v, drp, dci, None)
    torch.cuda.synchronize()
    outs = []
    for _ in range(2):
        s2 = torch.cuda.Stream()
        with torch.cuda.stream(s2):
            outs.append(block_sparse_attn_fwd(q, k, v, drp, dci, None))
        outs.append(block_sparse_attn_fwd(q, k, v, drp, dci, None))
    torch.cuda.synchronize()
    (entry,) = submission._csr_cache.values()
    assert entry.sched is not None and entry.pending is None
    for o, l in outs:
        assert torch.equal(o, o0) and torch.equal(l, l0)
    submission.clear_csr_cache()
