"""GPU parity: the HIP kernel through the C ABI against the CPU oracle.

Tolerance: atol = rtol = 2e-3 against fp32 dense-masked attention: the numpy dense oracle at
small sizes, and at the full sizes the C restatement of the reference walk in fp32 (P not
rounded to fp16), which the CPU suite pins to the dense oracle, over every head.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import bsa_oracle, c_ref
from tests._helpers import assert_close
from usagi_amd import block_sparse_attn_fwd
from usagi_amd import patterns as P

pytestmark = pytest.mark.gpu

DEV = "cuda"


def run_gpu(q, k, v, rp, ci, sl=None):
    dq, dk, dv = (x.to(DEV) for x in (q, k, v))
    drp = torch.from_numpy(np.ascontiguousarray(rp)).to(DEV)
    dci = torch.from_numpy(np.ascontiguousarray(ci)).to(DEV)
    dsl = None if sl is None else torch.as_tensor(np.asarray(sl, dtype=np.int32)).to(DEV)
    o, lse = block_sparse_attn_fwd(dq, dk, dv, drp, dci, dsl)
    torch.cuda.synchronize()
    return o.float().cpu().numpy(), lse.cpu().numpy()


def run_csr_walk(q, k, v, rp, ci, sl=None):
    """The CSR walk straight through the C ABI (the shim would run a window-shaped CSR on the
    analytic-row kernel instead)."""
    from usagi_amd import _native

    dq, dk, dv = (x.to(DEV) for x in (q, k, v))
    B, H, T, D = dq.shape
    drp = torch.from_numpy(np.ascontiguousarray(rp, dtype=np.int32)).to(DEV)
    dci = torch.from_numpy(np.ascontiguousarray(ci, dtype=np.int32)).to(DEV)
    dsl = None if sl is None else torch.as_tensor(np.asarray(sl, dtype=np.int32)).to(DEV)
    o = torch.empty_like(dq)
    lse = torch.empty((B, H, T), device=DEV, dtype=torch.float32)
    _native.fwd(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), drp.data_ptr(), dci.data_ptr(),
                None if dsl is None else dsl.data_ptr(), o.data_ptr(), lse.data_ptr(), B, H, T,
                D, ci.shape[-1], _native.BF16 if dq.dtype == torch.bfloat16 else _native.FP16,
                None, 0, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return o.float().cpu().numpy(), lse.cpu().numpy()


def c_oracle(q, k, v, rp, ci, sl=None, generic=False):
    """The fp32 walk over every head (OpenMP), as float32 numpy (O, LSE)."""
    qs, ks, vs = (x.float().numpy() for x in (q, k, v))
    return c_ref.fwd(qs, ks, vs, rp, ci, None if sl is None else np.asarray(sl, np.int32),
                     round_p_fp16=False, generic=generic)


def test_plumbing_vs_dense_oracle():
    w = P.workloads()["plumbing"]
    rp, ci = w.csr()
    q, k, v = P.make_qkv(w.B, w.H, w.T, seed=1)
    print(f"case plumbing B{w.B} H{w.H} T{w.T}", flush=True)
    o, lse = run_gpu(q, k, v, rp, ci)
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp, ci)
    assert_close(o, oo)
    assert_close(lse, ol, what="LSE")


@pytest.mark.parametrize("name", ["sliding", "global", "retrieval", "mixed"])
def test_full_size_every_head_vs_fp32_walk(name):
    w = P.workloads()[name]
    rp, ci = w.csr()
    q, k, v = P.make_qkv(w.B, w.H, w.T, seed=2)
    print(f"case {name} B{w.B} H{w.H} T{w.T}", flush=True)
    o, lse = run_gpu(q, k, v, rp, ci)
    oo, ol = c_oracle(q, k, v, rp, ci)
    assert_close(o, oo)
    assert_close(lse, ol, what="LSE")


def test_full_size_seq_lens_cut():
    """Global family at B2 H16 T8192 with seq_lens [8192, 5000]: batch 1 cuts inside query
    block 39 (5000 = 39 * 128 + 8) and drops blocks 40..63."""
    w = P.workloads()["global"]
    rp, ci = w.csr()
    q, k, v = P.make_qkv(w.B, w.H, w.T, seed=8)
    sl = [8192, 5000]
    print(f"case global seq_lens={sl}", flush=True)
    o, lse = run_gpu(q, k, v, rp, ci, sl)
    oo, ol = c_oracle(q, k, v, rp, ci, sl)
    assert_close(o, oo)
    assert_close(lse, ol, what="LSE")
    assert np.all(o[1, :, 5000:] == 0) and np.all(np.isneginf(lse[1, :, 5000:]))


def test_full_size_rows_in_any_order_before_the_diagonal():
    """Retrieval rows with the entries before the diagonal shuffled (diagonal kept last): the
    default walk accepts them and the result matches the fp32 walk of the sorted rows."""
    w = P.workloads()["retrieval"]
    rp, ci = w.csr()
    ci2 = ci.copy()
    rng = np.random.default_rng(3)
    for b in range(w.B):
        for h in range(w.H):
            for i in range(w.nqb):
                a, e = rp[b, h, i], rp[b, h, i + 1] - 1
                ci2[b, h, a:e] = rng.permutation(ci2[b, h, a:e])
    q, k, v = P.make_qkv(w.B, w.H, w.T, seed=9)
    print("case shuffled retrieval rows", flush=True)
    o, lse = run_gpu(q, k, v, rp, ci2)
    oo, ol = c_oracle(q, k, v, rp, ci)
    assert_close(o, oo)
    assert_close(lse, ol, what="LSE")


@pytest.mark.parametrize("seq_lens", [[1024, 700], [128, 1], [0, 1000], [1024, 1023]])
def test_seq_lens_masking(seq_lens):
    B, H, T = 2, 2, 1024
    rp, ci = P.global_csr(B, H, T, 2, 3)
    q, k, v = P.make_qkv(B, H, T, seed=3)
    print(f"case seq_lens {seq_lens}", flush=True)
    o, lse = run_gpu(q, k, v, rp, ci, seq_lens)
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp, ci, np.array(seq_lens))
    assert_close(o, oo)
    assert_close(lse, ol, what="LSE")


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_random_csr(seed):
    rng = np.random.default_rng(seed)
    B, H = int(rng.integers(1, 3)), int(rng.integers(1, 4))
    T = 128 * int(rng.integers(1, 9))
    density = float(rng.uniform(0.0, 1.0))
    rp, ci = P.random_csr(B, H, T, density, seed)
    q, k, v = P.make_qkv(B, H, T, seed=10 + seed)
    print(f"case random seed={seed} B{B} H{H} T{T} density={density:.2f}", flush=True)
    o, lse = run_gpu(q, k, v, rp, ci)
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp, ci)
    assert_close(o, oo)
    assert_close(lse, ol, what="LSE")


# O is stored in bf16 for bf16 inputs: its rounding (up to half an ulp, 2^-9 relative) comes on
# top of the 2e-3 budget, so rtol = 2e-3 + 2^-9. LSE is fp32 and keeps atol = rtol = 2e-3.
BF16_RTOL = 2e-3 + 2.0 ** -9


def test_bf16_inputs():
    B, H, T = 1, 2, 1024
    rp, ci = P.retrieval_csr(B, H, T, 5, 7)
    q, k, v = P.make_qkv(B, H, T, seed=4, dtype=torch.bfloat16)
    print("case bf16", flush=True)
    o, lse = run_gpu(q, k, v, rp, ci)
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp, ci)
    assert_close(o, oo, rtol=BF16_RTOL)
    assert_close(lse, ol, what="LSE")


@pytest.mark.parametrize("name", ["sliding", "global", "retrieval", "mixed"])
def test_bf16_full_size_every_head_vs_fp32_walk(name):
    """bf16 inputs at the full sizes against the fp32 walk over every head."""
    w = P.workloads()[name]
    rp, ci = w.csr()
    q, k, v = P.make_qkv(w.B, w.H, w.T, seed=7, dtype=torch.bfloat16)
    print(f"case bf16 {name} B{w.B} H{w.H} T{w.T}", flush=True)
    o, lse = run_gpu(q, k, v, rp, ci)
    oo, ol = c_oracle(q, k, v, rp, ci)
    assert_close(o, oo, rtol=BF16_RTOL)
    assert_close(lse, ol, what="LSE")


# ------------------------------------------------------------------------------ golden fixtures

import os  # noqa: E402

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("name", ["golden_families_t512.npz", "golden_seqlens_t256.npz"])
def test_golden_fixtures(name):
    g = np.load(os.path.join(GOLDEN, name))
    q, k, v = (torch.from_numpy(g[x]) for x in ("q", "k", "v"))
    print(f"case golden {name}", flush=True)
    o, lse = run_gpu(q, k, v, g["row_ptr"], g["col_idx"], g["seq_lens"])
    assert_close(o, g["out"])
    assert_close(lse, g["lse"], what="LSE")


# ------------------------------------------------------------------------------ full-size properties


@pytest.fixture(scope="module")
def full_inputs():
    B, H, T = 2, 16, 8192
    q, k, v = (x.to(DEV) for x in P.make_qkv(B, H, T, seed=5))
    return q, k, v


def _dev_csr(name):
    rp, ci = P.workloads()[name].csr()
    return torch.from_numpy(rp).to(DEV), torch.from_numpy(ci).to(DEV)


@pytest.mark.parametrize("name", ["sliding", "retrieval"])
def test_full_size_deterministic(full_inputs, name):
    q, k, v = full_inputs
    rp, ci = _dev_csr(name)
    print(f"case determinism {name}", flush=True)
    o1, l1 = block_sparse_attn_fwd(q, k, v, rp, ci, None)
    o2, l2 = block_sparse_attn_fwd(q, k, v, rp, ci, None)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


@pytest.mark.parametrize("name", ["global", "retrieval"])
def test_full_size_linear_in_v(full_inputs, name):
    """O(2V) = 2 O(V): P is unchanged and scaling by 2 is exact in fp16 and fp32."""
    q, k, v = full_inputs
    rp, ci = _dev_csr(name)
    print(f"case linearity {name}", flush=True)
    o1, l1 = block_sparse_attn_fwd(q, k, v, rp, ci, None)
    o2, l2 = block_sparse_attn_fwd(q, k, v * 2, rp, ci, None)
    torch.cuda.synchronize()
    assert torch.equal(l1, l2)
    assert (o2.float() - 2 * o1.float()).abs().max().item() <= 2.0 ** -23


def test_full_size_constant_v(full_inputs):
    q, k, _ = full_inputs
    rp, ci = _dev_csr("sliding")
    v = torch.full_like(q, 0.3125)
    print("case constant V", flush=True)
    o, lse = block_sparse_attn_fwd(q, k, v, rp, ci, None)
    torch.cuda.synchronize()
    assert (o.float() - 0.3125).abs().max().item() <= 2e-3 * 0.3125
    assert torch.isfinite(lse).all()


def test_full_size_head_permutation(full_inputs):
    """Swapping the data and patterns of two (b, h) pairs swaps their outputs bit for bit."""
    q, k, v = full_inputs
    rp, ci = P.workloads()["retrieval"].csr()
    print("case head permutation", flush=True)
    o1, l1 = block_sparse_attn_fwd(q, k, v, torch.from_numpy(rp).to(DEV),
                                   torch.from_numpy(ci).to(DEV), None)
    perm = lambda x: torch.stack([x[1].flip(0), x[0].flip(0)])  # noqa: E731  (b, h) -> (1-b, H-1-h)
    rp2 = np.ascontiguousarray(np.stack([rp[1][::-1], rp[0][::-1]]))
    ci2 = np.ascontiguousarray(np.stack([ci[1][::-1], ci[0][::-1]]))
    o2, l2 = block_sparse_attn_fwd(perm(q).contiguous(), perm(k).contiguous(), perm(v).contiguous(),
                                   torch.from_numpy(rp2).to(DEV), torch.from_numpy(ci2).to(DEV), None)
    torch.cuda.synchronize()
    assert torch.equal(perm(o1), o2) and torch.equal(perm(l1), l2)


# ------------------------------------------------------------------------------ edge cases


def test_rows_longer_than_64_blocks():
    """Rows of up to ~90 key blocks exercise the chunked column-index reload."""
    B, H, T = 1, 2, 128 * 96
    rp, ci = P.random_csr(B, H, T, 0.92, 21)
    assert int(np.diff(rp, axis=-1).max()) > 64
    q, k, v = P.make_qkv(B, H, T, seed=22)
    print(f"case long rows T{T} max row {int(np.diff(rp, axis=-1).max())}", flush=True)
    o, lse = run_gpu(q, k, v, rp, ci)
    for h in range(H):
        oo, ol = c_ref.fwd(q[:, h:h + 1].float().numpy(), k[:, h:h + 1].float().numpy(),
                           v[:, h:h + 1].float().numpy(), rp[:, h:h + 1], ci[:, h:h + 1])
        assert_close(o[:, h:h + 1], oo, what=f"O[h={h}]")
        assert_close(lse[:, h:h + 1], ol, what=f"LSE[h={h}]")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_long_sequence(dtype):
    """T = 32768 (256 query blocks): a global prefix, a window and random far blocks, rows of
    up to 80 entries (past the 64-entry column chunk), seq_lens cutting inside a block; every
    head against the fp32 walk."""
    B, H, T = 1, 2, 128 * 256
    rng = np.random.default_rng(31)

    def row(b, h, i):
        near = set(range(max(0, i - 7), i)) | set(range(min(4, i)))
        far = rng.choice(i, size=min(i, 80 - 1 - len(near)), replace=False) if i > 100 else []
        return sorted(near | {int(x) for x in far}) + [i]

    rp, ci = P.make_csr(B, H, T, row)
    assert int(np.diff(rp, axis=-1).max()) > 64
    sl = [30000]
    q, k, v = P.make_qkv(B, H, T, seed=32, dtype=dtype)
    print(f"case long sequence T{T} {dtype} max row {int(np.diff(rp, axis=-1).max())}", flush=True)
    o, lse = run_gpu(q, k, v, rp, ci, sl)
    oo, ol = c_oracle(q, k, v, rp, ci, sl)
    rtol = 2e-3 + (2.0 ** -9 if dtype == torch.bfloat16 else 0.0)  # bf16 O: half an ulp more
    assert_close(o, oo, rtol=rtol)
    assert_close(lse, ol, what="LSE")
    assert np.all(o[:, :, 30000:] == 0) and np.all(np.isneginf(lse[:, :, 30000:]))


def test_int64_csr_noncontiguous_inputs_and_list_seq_lens():
    B, H, T = 2, 3, 640
    rp, ci = P.retrieval_csr(B, H, T, 3, 4)
    q, k, v = P.make_qkv(B, H, T, seed=23)
    print("case int64 csr / non-contiguous", flush=True)
    # non-contiguous views of the same values: [B, T, H, D] storage transposed to [B, H, T, D]
    qt, kt, vt = (x.transpose(1, 2).contiguous().to(DEV).transpose(1, 2) for x in (q, k, v))
    assert not qt.is_contiguous()
    o, lse = block_sparse_attn_fwd(qt, kt, vt, torch.from_numpy(rp.astype(np.int64)).to(DEV),
                                   torch.from_numpy(ci.astype(np.int64)).to(DEV), [640, 300])
    torch.cuda.synchronize()
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp, ci, np.array([640, 300]))
    assert_close(o.float().cpu().numpy(), oo)
    assert_close(lse.cpu().numpy(), ol, what="LSE")


@pytest.mark.parametrize("T", [128, 256])
def test_single_and_two_block_sequences(T):
    B, H = 3, 2
    rp, ci = P.sliding_csr(B, H, T, 2)
    q, k, v = P.make_qkv(B, H, T, seed=T)
    print(f"case T={T}", flush=True)
    o, lse = run_gpu(q, k, v, rp, ci, [T, T // 2, 1])
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp, ci, np.array([T, T // 2, 1]))
    assert_close(o, oo)
    assert_close(lse, ol, what="LSE")


def test_setup_warms_up():
    import usagi_amd

    class Spec:
        def __init__(self, t):
            self.t_max = t

    print("case setup", flush=True)
    assert usagi_amd.setup([Spec(1024), Spec(8192), Spec(1024)], "cuda", usagi_amd.VARIANT_MANIFEST) is None


# ------------------------------------------------------------------------------ running-max growth


def _growth_inputs(seed):
    """Scores of key block 0 far above the diagonal block's: the running max taken on the
    diagonal (processed first) is then exceeded by far more than the fp16 range of P in a later
    block, which must take the exact-max rescale path. Also a case with every score sharpened."""
    B, H, T = 1, 2, 768
    rp, ci = P.global_csr(B, H, T, 1, 2)  # every row: key block 0, previous block, diagonal
    q, k, v = P.make_qkv(B, H, T, seed=seed)
    k = k.clone()
    k[:, :, :128] *= 6.0  # key block 0: scores up to ~6x the rest
    return q, k, v, rp, ci


def test_running_max_growth_takes_the_rescale_path():
    q, k, v, rp, ci = _growth_inputs(31)
    print("case growth", flush=True)
    o, lse = run_gpu(q, k, v, rp, ci)
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp, ci)
    assert_close(o, oo)
    assert_close(lse, ol, what="LSE")


def test_bf16_running_max_growth():
    """The rescale path with bf16 inputs (default kernel)."""
    q, k, v, rp, ci = _growth_inputs(33)
    q, k, v = (x.to(torch.bfloat16) for x in (q, k, v))
    print("case growth bf16", flush=True)
    o, lse = run_gpu(q, k, v, rp, ci)
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp, ci)
    assert_close(o, oo, rtol=BF16_RTOL)
    assert_close(lse, ol, what="LSE")


def test_sharp_softmax():
    """q and k scaled by 3: scores 9x the unit-variance case (near one-hot rows)."""
    B, H, T = 1, 2, 1024
    rp, ci = P.retrieval_csr(B, H, T, 5, 3)
    q, k, v = P.make_qkv(B, H, T, seed=32)
    q, k = (q.float() * 3.0).half(), (k.float() * 3.0).half()
    print("case sharp", flush=True)
    o, lse = run_gpu(q, k, v, rp, ci)
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp, ci)
    assert_close(o, oo)
    assert_close(lse, ol, what="LSE")


# ------------------------------------------------------------------------------ analytic rows


def run_gpu_window(q, k, v, window, n_global, sl=None):
    from usagi_amd import block_sparse_attn_fwd_window

    dq, dk, dv = (x.to(DEV) for x in (q, k, v))
    dsl = None if sl is None else torch.as_tensor(np.asarray(sl, dtype=np.int32)).to(DEV)
    o, lse = block_sparse_attn_fwd_window(dq, dk, dv, window, n_global, dsl)
    torch.cuda.synchronize()
    return o.float().cpu().numpy(), lse.cpu().numpy()


@pytest.mark.parametrize("B,H,T,w,g", [
    (1, 2, 1024, 4, 0), (1, 2, 1024, 3, 2), (1, 2, 1024, 1, 0), (1, 2, 1024, 1, 3),
    (1, 2, 1024, 100, 0), (1, 2, 1024, 2, 100), (2, 16, 8192, 8, 0), (2, 16, 8192, 4, 4),
])
def test_window_path_equals_csr_path_bitwise(B, H, T, w, g):
    """The analytic rows walk the same blocks in the same order as the CSR of the pattern, so
    O and LSE are bit-identical (the full-size cases are the sliding and global families)."""
    rp, ci = P.global_csr(B, H, T, g, w) if g else P.sliding_csr(B, H, T, w)
    q, k, v = P.make_qkv(B, H, T, seed=41)
    print(f"case window w={w} g={g} B{B} H{H} T{T}", flush=True)
    o_csr, lse_csr = run_csr_walk(q, k, v, rp, ci)
    o_win, lse_win = run_gpu_window(q, k, v, w, g)
    assert np.array_equal(o_win, o_csr)
    assert np.array_equal(lse_win, lse_csr)


@pytest.mark.parametrize("name,pattern", [("sliding", (8, 0)), ("global", (4, 4))])
def test_shim_routes_window_shaped_csr_to_the_analytic_rows(name, pattern):
    """block_sparse_attn_fwd recognises a CSR that is exactly a window (+ global prefix)
    pattern in its first-call check and runs the analytic-row kernel: bit-identical to the CSR
    walk, and the cache entry records the pattern it took."""
    from usagi_amd import submission

    submission.clear_csr_cache()
    w = P.workloads()[name]
    rp, ci = w.csr()
    q, k, v = P.make_qkv(w.B, w.H, w.T, seed=44)
    print(f"case route {name}", flush=True)
    dq, dk, dv = (x.to(DEV) for x in (q, k, v))
    drp, dci = torch.from_numpy(rp).to(DEV), torch.from_numpy(ci).to(DEV)
    o, lse = block_sparse_attn_fwd(dq, dk, dv, drp, dci, None)
    torch.cuda.synchronize()
    (entry,) = submission._csr_cache.values()
    assert entry.window == pattern
    o_csr, lse_csr = run_csr_walk(q, k, v, rp, ci)
    assert np.array_equal(o.float().cpu().numpy(), o_csr)
    assert np.array_equal(lse.cpu().numpy(), lse_csr)


def test_shim_keeps_a_near_window_csr_on_the_csr_walk():
    """A sliding CSR with one entry dropped is no longer the analytic pattern: the shim stays
    on the CSR walk (bit-identical to it) and matches the fp32 walk of the altered rows."""
    from usagi_amd import submission

    submission.clear_csr_cache()
    B, H, T = 2, 16, 8192
    rows = lambda b, h, i: [x for x in P.sliding_row(i, 8) if not (b == 1 and h == 5 and i == 40 and x == 35)]  # noqa: E731,E501
    rp, ci = P.make_csr(B, H, T, rows)
    q, k, v = P.make_qkv(B, H, T, seed=45)
    print("case route near-window", flush=True)
    o, lse = run_gpu(q, k, v, rp, ci)
    (entry,) = submission._csr_cache.values()
    assert entry.window is None
    o_csr, lse_csr = run_csr_walk(q, k, v, rp, ci)
    assert np.array_equal(o, o_csr) and np.array_equal(lse, lse_csr)
    oo, _ = c_oracle(q[1:, 5:6], k[1:, 5:6], v[1:, 5:6], rp[1:, 5:6], ci[1:, 5:6])
    assert_close(o[1:, 5:6], oo)


def test_rows_past_seq_len_may_hold_anything():
    """The walk never reads the rows of query blocks at or past seq_len (v7:63-67), so the shim
    accepts a CSR that leaves them empty when seq_lens is given; O = 0 and LSE = -inf there."""
    from usagi_amd import submission

    submission.clear_csr_cache()
    B, H, T = 2, 2, 1024
    sl = [1024, 300]
    rp, ci = P.sliding_csr(B, H, T, 3)
    rp[1, :, 4:] = rp[1, :, 3:4]  # batch 1: rows 3.. (query blocks from 384 on) left empty
    q, k, v = P.make_qkv(B, H, T, seed=46)
    print("case rows past seq_len", flush=True)
    with pytest.raises(ValueError, match="empty"):
        run_gpu(q, k, v, rp, ci)
    o, lse = run_gpu(q, k, v, rp, ci, sl)
    rp_ok, ci_ok = P.sliding_csr(B, H, T, 3)
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp_ok, ci_ok, np.array(sl))
    assert_close(o, oo)
    assert_close(lse, ol, what="LSE")


@pytest.mark.parametrize("seq_lens", [[1024, 700], [0, 1000], [128, 1]])
def test_window_path_vs_dense_oracle(seq_lens):
    B, H, T, w, g = 2, 2, 1024, 3, 2
    rp, ci = P.global_csr(B, H, T, g, w)
    q, k, v = P.make_qkv(B, H, T, seed=42)
    print(f"case window oracle seq_lens={seq_lens}", flush=True)
    o, lse = run_gpu_window(q, k, v, w, g, seq_lens)
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp, ci, np.array(seq_lens))
    assert_close(o, oo)
    assert_close(lse, ol, what="LSE")


def test_window_path_bf16():
    B, H, T, w, g = 1, 2, 1024, 4, 4
    rp, ci = P.global_csr(B, H, T, g, w)
    q, k, v = P.make_qkv(B, H, T, seed=43, dtype=torch.bfloat16)
    print("case window bf16", flush=True)
    o, lse = run_gpu_window(q, k, v, w, g)
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp, ci)
    assert_close(o, oo, rtol=BF16_RTOL)
    assert_close(lse, ol, what="LSE")
    o_csr, lse_csr = run_gpu(q, k, v, rp, ci)
    assert np.array_equal(o, o_csr) and np.array_equal(lse, lse_csr)


# ------------------------------------------------------------------------------ randomised cases


def _random_case(seed):
    rng = np.random.default_rng(5000 + seed)
    density = float(rng.uniform(0.05, 0.95))
    if seed % 6 == 5:
        B, H, T = 1, 1, 16384  # rows of more than 64 blocks: the column-chunk reload path
        density = max(density, 0.6)
    else:
        B, H = int(rng.choice([1, 2, 3])), int(rng.choice([1, 3, 5, 8]))
        T = 128 * int(rng.integers(1, 25))
    dtype = torch.bfloat16 if seed % 3 == 0 else torch.float16
    seq_lens = None
    if seed % 2 == 1:
        seq_lens = [int(x) for x in rng.integers(0, T + 1, size=B)]
        seq_lens[0] = T  # keep at least one full sequence
    return B, H, T, density, dtype, seq_lens


@pytest.mark.parametrize("seed", range(40))
def test_randomised_shapes_patterns_and_dtypes(seed):
    """Seeded random B, H (B*H not a multiple of 8 takes the row-major work order), T, CSR
    density, seq_lens and dtype against the dense oracle."""
    B, H, T, density, dtype, seq_lens = _random_case(seed)
    rp, ci = P.random_csr(B, H, T, density, seed)
    q, k, v = P.make_qkv(B, H, T, seed=100 + seed, dtype=dtype)
    print(f"case random seed={seed} B{B} H{H} T{T} density={density:.2f} {dtype} "
          f"seq_lens={seq_lens} max_row={int(np.diff(rp, axis=-1).max())}", flush=True)
    o, lse = run_gpu(q, k, v, rp, ci, seq_lens)
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp, ci,
                                     None if seq_lens is None else np.array(seq_lens))
    rtol = BF16_RTOL if dtype == torch.bfloat16 else 2e-3
    assert_close(o, oo, rtol=rtol)
    assert_close(lse, ol, what="LSE")


def test_empty_rows_take_the_implicit_diagonal():
    """max_nnz = 0 (every CSR row empty): like the reference's walk (v7:83-111), each query block
    still attends its implicit diagonal, so O and LSE equal those of a diagonal-only CSR. The
    shim rejects such a CSR (the dense block-mask reading of it attends nothing); the C ABI,
    which does not check rows, runs the walk as the reference does."""
    from usagi_amd import _native

    B, H, T = 1, 3, 512
    nqb = T // 128
    q, k, v = P.make_qkv(B, H, T, seed=51)
    rp0 = np.zeros((B, H, nqb + 1), dtype=np.int32)
    ci0 = np.zeros((B, H, 0), dtype=np.int32)
    rp1, ci1 = P.sliding_csr(B, H, T, 1)
    print("case empty rows", flush=True)
    with pytest.raises(ValueError, match="empty"):
        run_gpu(q, k, v, rp0, ci0)
    dq, dk, dv = (x.to(DEV) for x in (q, k, v))
    drp0 = torch.from_numpy(rp0).to(DEV)
    o0 = torch.empty_like(dq)
    l0 = torch.empty((B, H, T), device=DEV, dtype=torch.float32)
    _native.fwd(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), drp0.data_ptr(), None, None,
                o0.data_ptr(), l0.data_ptr(), B, H, T, 128, 0, _native.FP16, None, 0,
                torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    o0, l0 = o0.float().cpu().numpy(), l0.cpu().numpy()
    o1, l1 = run_gpu(q, k, v, rp1, ci1)
    assert np.array_equal(o0, o1) and np.array_equal(l0, l1)
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp1, ci1)
    assert_close(o0, oo)
    assert_close(l0, ol, what="LSE")


def test_many_heads_single_block():
    """256 (b, h) pairs at T = 128: one query block each, head-major work order."""
    B, H, T = 4, 64, 128
    rp, ci = P.sliding_csr(B, H, T, 1)
    q, k, v = P.make_qkv(B, H, T, seed=52)
    print("case many heads", flush=True)
    o, lse = run_gpu(q, k, v, rp, ci)
    oo, ol = bsa_oracle.dense_masked(q, k, v, rp, ci)
    assert_close(o, oo)
    assert_close(lse, ol, what="LSE")
