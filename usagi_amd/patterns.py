"""CSR block-pattern generators and the synthetic inputs of the benchmark workloads.

The reference's caller (the challenge harness) is not vendored; its contract is described in
docs/OPTIMIZATION_JOURNAL.md:14-16 (three families: sliding window, sliding window + global
prefix, sliding window + retrieval; scored by the geometric mean of family medians). The CSR
layout follows the reference wrapper: row_ptr [B, H, nqb+1] with offsets local to each (b, h)
row, col_idx [B, H, max_nnz] padded (kernels/v7_blockptr_warpspec.py:77-80, 172-174).
Every generated row is ascending, has all key blocks <= the query block and ends with the
diagonal, which meets the precondition of the implicit-diagonal walk
(kernels/v7_blockptr_warpspec.py:83, 111; see validate_csr).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Sequence

import numpy as np

BLOCK = 128
HEAD_DIM = 128


# ---------------------------------------------------------------------------------------------
# Per-row block sets
# ---------------------------------------------------------------------------------------------

def sliding_row(i: int, w: int) -> list[int]:
    """Query block i attends key blocks max(0, i-w+1) .. i."""
    return list(range(max(0, i - w + 1), i + 1))


def global_row(i: int, g: int, w: int) -> list[int]:
    """Blocks 0..g-1 (global prefix) union max(0, i-w+1)..i, restricted to <= i, sorted."""
    return sorted(set(range(min(g, i + 1))) | set(sliding_row(i, w)))


def retrieval_row(i: int, r: int, seed: int, b: int, h: int) -> list[int]:
    """Diagonal i, block i-1, plus min(r, i-1) distinct blocks drawn uniformly from 0..i-2
    with a generator seeded by (seed, b, h, i)."""
    if i == 0:
        return [0]
    picks: list[int] = []
    n = min(r, i - 1)
    if n > 0:
        rng = np.random.default_rng((seed, b, h, i))
        picks = [int(x) for x in rng.choice(i - 1, size=n, replace=False)]
    return sorted(set(picks) | {i - 1, i})


def rows_to_csr(rows_bh: Sequence[Sequence[Sequence[int]]], pad: int = 0):
    """rows_bh[b][h][qb] -> (row_ptr int32 [B,H,nqb+1], col_idx int32 [B,H,max_nnz])."""
    B = len(rows_bh)
    H = len(rows_bh[0])
    nqb = len(rows_bh[0][0])
    nnz = np.zeros((B, H), dtype=np.int64)
    for b in range(B):
        for h in range(H):
            nnz[b, h] = sum(len(r) for r in rows_bh[b][h])
    max_nnz = int(nnz.max()) if nnz.size else 0
    row_ptr = np.zeros((B, H, nqb + 1), dtype=np.int32)
    col_idx = np.full((B, H, max_nnz), pad, dtype=np.int32)
    for b in range(B):
        for h in range(H):
            off = 0
            for qb, r in enumerate(rows_bh[b][h]):
                col_idx[b, h, off:off + len(r)] = r
                off += len(r)
                row_ptr[b, h, qb + 1] = off
    return row_ptr, col_idx


def make_csr(B: int, H: int, T: int, row_fn: Callable[[int, int, int], list[int]]):
    """row_fn(b, h, qb) -> sorted key blocks of that row."""
    nqb = T // BLOCK
    rows = [[[row_fn(b, h, i) for i in range(nqb)] for h in range(H)] for b in range(B)]
    return rows_to_csr(rows)


def sliding_csr(B, H, T, w):
    return make_csr(B, H, T, lambda b, h, i: sliding_row(i, w))


def global_csr(B, H, T, g, w):
    return make_csr(B, H, T, lambda b, h, i: global_row(i, g, w))


def retrieval_csr(B, H, T, r, seed):
    return make_csr(B, H, T, lambda b, h, i: retrieval_row(i, r, seed, b, h))


def mixed_csr(B, H, T, seed):
    """Heads 0-5 sliding w=16; heads 6-10 global 8 + window 8; heads 11-15 retrieval
    diagonal + previous + 24 seeded earlier blocks (per-head CSR)."""

    def row(b, h, i):
        if h <= 5:
            return sliding_row(i, 16)
        if h <= 10:
            return global_row(i, 8, 8)
        return retrieval_row(i, 24, seed, b, h)

    return make_csr(B, H, T, row)


def random_csr(B, H, T, density: float, seed: int):
    """Random causal rows (each earlier block kept with probability `density`) + diagonal."""
    rng = np.random.default_rng(seed)
    nqb = T // BLOCK

    def row(b, h, i):
        keep = [j for j in range(i) if rng.random() < density]
        return keep + [i]

    return make_csr(B, H, T, row)


def csr_rows(row_ptr: np.ndarray, col_idx: np.ndarray, b: int, h: int) -> list[list[int]]:
    rp = row_ptr[b, h]
    return [list(map(int, col_idx[b, h, rp[i]:rp[i + 1]])) for i in range(len(rp) - 1)]


def active_blocks(row_ptr: np.ndarray) -> int:
    """Number of active (b, h, qb, kb) blocks (the diagonal counts as a full block)."""
    return int(row_ptr[..., -1].astype(np.int64).sum())


def validate_csr(row_ptr: np.ndarray, col_idx: np.ndarray, T: int, seq_lens=None) -> None:
    """Raise ValueError unless every row is non-empty, ends with its diagonal, and lists the
    blocks before it at most once each, all in [0, qb) (any order): the precondition under
    which the implicit-diagonal walk of kernels/v7_blockptr_warpspec.py:83-136 equals
    block-mask ∧ causal attention. With seq_lens ([B]), rows of query blocks starting at or
    past seq_len[b] are skipped: the walk never reads them (v7:63-67). Same rules as
    usagi_bsa_check_csr."""
    B, H, n1 = row_ptr.shape
    nqb = T // BLOCK
    if n1 != nqb + 1:
        raise ValueError(f"row_ptr last dim {n1} != T/128 + 1 = {nqb + 1}")
    max_nnz = col_idx.shape[-1]
    for b in range(B):
        n_rows = nqb
        if seq_lens is not None:
            sl = int(seq_lens[b])
            n_rows = 0 if sl <= 0 else min(nqb, -(-sl // BLOCK))
        for h in range(H):
            rp = row_ptr[b, h]
            if n_rows and rp[0] != 0:
                raise ValueError(f"(b={b},h={h}): row_ptr[0] = {rp[0]}")
            for i in range(n_rows):
                if rp[i + 1] <= rp[i]:
                    raise ValueError(f"(b={b},h={h},qb={i}): empty or decreasing row")
                if rp[i + 1] > max_nnz:
                    raise ValueError(f"(b={b},h={h},qb={i}): row_ptr {rp[i + 1]} > max_nnz {max_nnz}")
                r = col_idx[b, h, rp[i]:rp[i + 1]]
                if r[-1] != i:
                    raise ValueError(f"(b={b},h={h},qb={i}): last entry {r[-1]} is not the diagonal")
                off = r[:-1]
                if len(off) and (off.min() < 0 or off.max() >= i):
                    raise ValueError(f"(b={b},h={h},qb={i}): entries before the diagonal outside [0,{i})")
                if len(np.unique(off)) != len(off):
                    raise ValueError(f"(b={b},h={h},qb={i}): a key block listed twice")


# ---------------------------------------------------------------------------------------------
# Workloads
# ---------------------------------------------------------------------------------------------

@dataclass
class Workload:
    name: str
    B: int
    H: int
    T: int
    csr: Callable[[], tuple]
    family: str = ""
    extra: dict = field(default_factory=dict)

    @property
    def nqb(self) -> int:
        return self.T // BLOCK


PATTERN_SEED = 1234
INPUT_SEED = 0


def workloads(seed: int = PATTERN_SEED) -> dict[str, Workload]:
    """The five workloads: the CPU plumbing case, the three scored families at
    B2 H16 T8192 D128, and the mixed long-context case."""
    return {
        "plumbing": Workload("plumbing", 1, 4, 1024, lambda: sliding_csr(1, 4, 1024, 4), "sliding"),
        "sliding": Workload("sliding", 2, 16, 8192, lambda: sliding_csr(2, 16, 8192, 8), "sliding",
                            {"window": 8, "n_global": 0}),
        "global": Workload("global", 2, 16, 8192, lambda: global_csr(2, 16, 8192, 4, 4), "global",
                           {"window": 4, "n_global": 4}),
        "retrieval": Workload("retrieval", 2, 16, 8192,
                              lambda: retrieval_csr(2, 16, 8192, 14, seed), "retrieval"),
        "mixed": Workload("mixed", 1, 16, 16384, lambda: mixed_csr(1, 16, 16384, seed), "mixed"),
    }


FAMILIES = ("sliding", "global", "retrieval")


def make_qkv(B: int, H: int, T: int, seed: int = INPUT_SEED, dtype=None, D: int = HEAD_DIM):
    """fp16 q, k, v ~ N(0, 1) drawn on the CPU from one torch.Generator, in q, k, v order."""
    import torch

    dtype = dtype or torch.float16
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(3):
        out.append(torch.randn((B, H, T, D), generator=g, dtype=torch.float32).to(dtype))
    return tuple(out)
