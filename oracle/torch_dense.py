"""PyTorch CPU dense-masked attention — TEST INFRASTRUCTURE ONLY (the CPU baseline leg of
bench.py and a cross-check in tests/; never imported by the usagi_amd package).

The reference has no CPU path (kernels/v7_blockptr_warpspec.py:202-203 returns early off CUDA),
so its math is run here the plain way: fp32 scores over the dense token mask
block_mask(CSR) ∧ causal ∧ key < seq_len, softmax, then P·V, in query-row slabs. Keys past the
end of a slab are causally masked for every row of it, so each slab only multiplies against
keys [0, slab end). The result is the same function as oracle.bsa_oracle.dense_masked.
"""

from __future__ import annotations

import math

import torch

BLOCK = 128


def _block_mask(row_ptr_bh, col_idx_bh, nqb: int) -> torch.Tensor:
    m = torch.zeros((nqb, nqb), dtype=torch.bool)
    rp = [int(x) for x in row_ptr_bh]
    for i in range(nqb):
        cols = torch.as_tensor(col_idx_bh[rp[i]:rp[i + 1]], dtype=torch.long)
        m[i, cols] = True
    return m


def dense_masked(q, k, v, row_ptr, col_idx, seq_lens=None, heads=None, slab: int = 1024):
    """q, k, v: CPU tensors [B, H, T, D] (any float dtype, computed in fp32).
    Returns (O fp32 [B, H, T, D], LSE fp32 [B, H, T]); with `heads` (a list of (b, h)) only
    those heads are computed and the rest stay NaN."""
    B, H, T, D = q.shape
    nqb = T // BLOCK
    rp = row_ptr.reshape(B, H, nqb + 1)
    ci = col_idx.reshape(B, H, -1)
    sl = [T] * B if seq_lens is None else [int(x) for x in seq_lens]
    scale = 1.0 / math.sqrt(D)
    out = torch.full((B, H, T, D), float("nan"), dtype=torch.float32)
    lse = torch.full((B, H, T), float("nan"), dtype=torch.float32)
    pairs = heads if heads is not None else [(b, h) for b in range(B) for h in range(H)]
    tok = torch.arange(T)
    for b, h in pairs:
        bm = _block_mask(rp[b, h], ci[b, h], nqb)
        L = sl[b]
        qf, kf, vf = (x[b, h].float() for x in (q, k, v))
        for t0 in range(0, T, slab):
            t1 = min(T, t0 + slab)
            rows = tok[t0:t1]
            keys = tok[:t1]
            mask = bm[rows[:, None] // BLOCK, keys[None, :] // BLOCK]
            mask &= keys[None, :] <= rows[:, None]
            mask &= keys[None, :] < L
            mask &= (rows < L)[:, None]
            s = (qf[t0:t1] @ kf[:t1].T) * scale
            s = s.masked_fill(~mask, float("-inf"))
            lrow = torch.logsumexp(s, dim=1)
            has = torch.isfinite(lrow)
            p = torch.exp(s - torch.where(has, lrow, torch.zeros_like(lrow))[:, None])
            o = p @ vf[:t1]
            out[b, h, t0:t1] = torch.where(has[:, None], o, torch.zeros_like(o))
            lse[b, h, t0:t1] = torch.where(has, lrow, torch.full_like(lrow, float("-inf")))
    return out, lse
