"""Write the golden fixtures of this directory (run from the repository root):

    python tests/golden/make_golden.py

The reference (sissississi-013/usagi) ships no tests, golden vectors or fixtures, so these are
computed here by an fp64 brute force that shares no code with oracle/: for every query row it
enumerates the attended key set straight from the CSR semantics of the reference walk
(kernels/v7_blockptr_warpspec.py:83-136: all tokens of the off-diagonal blocks of the row, plus
the diagonal block's tokens at or before the query, nothing for rows at or past seq_len) and
takes softmax(q·k/sqrt(128)) over that set one row at a time.

Fixtures (inputs stored exactly as fp16, outputs as fp32 rounded from fp64):
  golden_families_t512.npz   B=1 H=2 T=512: head 0 sliding window w=2, head 1 retrieval
                             (diagonal + previous + up to 2 seeded earlier blocks)
  golden_seqlens_t256.npz    B=2 H=1 T=256: global prefix 1 + window 2, seq_lens = [256, 150]
  golden_generic_t384.npz    B=2 H=2 T=384, seq_lens = [384, 200], rows for the generic walk of
                             kernels/v1_baseline.py:360-406 (every entry with its multiplicity,
                             an entry equal to the query block causally masked, keys at or past
                             seq_len masked, no implicit diagonal): the diagonal first, in the
                             middle or missing, an empty row, a repeated entry and an entry
                             above the diagonal
"""

from __future__ import annotations

import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
BLOCK = 128
D = 128


def rows_sliding(i, w):
    return list(range(max(0, i - w + 1), i + 1))


def rows_retrieval(i, r, rng):
    if i == 0:
        return [0]
    picks = set()
    if i >= 2:
        picks = set(int(x) for x in rng.choice(i - 1, size=min(r, i - 1), replace=False))
    return sorted(picks | {i - 1, i})


def rows_global(i, g, w):
    return sorted(set(range(min(g, i + 1))) | set(rows_sliding(i, w)))


def to_csr(rows_bh):
    B, H, nqb = len(rows_bh), len(rows_bh[0]), len(rows_bh[0][0])
    max_nnz = max(sum(len(r) for r in rows_bh[b][h]) for b in range(B) for h in range(H))
    rp = np.zeros((B, H, nqb + 1), np.int32)
    ci = np.zeros((B, H, max_nnz), np.int32)
    for b in range(B):
        for h in range(H):
            off = 0
            for i, r in enumerate(rows_bh[b][h]):
                ci[b, h, off:off + len(r)] = r
                off += len(r)
                rp[b, h, i + 1] = off
    return rp, ci


def brute_force(q, k, v, rows_bh, seq_lens):
    """fp64, one query row at a time over an explicitly built key list."""
    B, H, T, _ = q.shape
    out = np.zeros((B, H, T, D), np.float64)
    lse = np.full((B, H, T), -np.inf, np.float64)
    qd, kd, vd = (x.astype(np.float64) for x in (q, k, v))
    for b in range(B):
        L = int(seq_lens[b])
        for h in range(H):
            for t in range(min(T, L)):
                qb = t // BLOCK
                keys = []
                for kb in rows_bh[b][h][qb]:
                    if kb != qb:
                        keys.extend(range(kb * BLOCK, (kb + 1) * BLOCK))
                keys.extend(s for s in range(qb * BLOCK, t + 1) if s < L)
                keys = np.array(keys)
                sc = (kd[b, h, keys] @ qd[b, h, t]) / math.sqrt(D)
                mx = sc.max()
                w = np.exp(sc - mx)
                out[b, h, t] = (w @ vd[b, h, keys]) / w.sum()
                lse[b, h, t] = mx + math.log(w.sum())
    return out, lse


def brute_force_generic(q, k, v, rows_bh, seq_lens):
    """fp64 over the key MULTISET of each query row under the generic walk."""
    B, H, T, _ = q.shape
    out = np.zeros((B, H, T, D), np.float64)
    lse = np.full((B, H, T), -np.inf, np.float64)
    qd, kd, vd = (x.astype(np.float64) for x in (q, k, v))
    for b in range(B):
        L = int(seq_lens[b])
        for h in range(H):
            for t in range(min(T, L)):
                qb = t // BLOCK
                keys = []
                for kb in rows_bh[b][h][qb]:
                    last = t if kb == qb else (kb + 1) * BLOCK - 1
                    keys.extend(s for s in range(kb * BLOCK, last + 1) if s < L)
                if not keys:
                    continue
                keys = np.array(keys)
                sc = (kd[b, h, keys] @ qd[b, h, t]) / math.sqrt(D)
                mx = sc.max()
                w = np.exp(sc - mx)
                out[b, h, t] = (w @ vd[b, h, keys]) / w.sum()
                lse[b, h, t] = mx + math.log(w.sum())
    return out, lse


def make(name, B, H, T, rows_fn, seq_lens, seed, brute=brute_force):
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal((B, H, T, D)).astype(np.float16) for _ in range(3))
    nqb = T // BLOCK
    rows = [[[rows_fn(b, h, i) for i in range(nqb)] for h in range(H)] for b in range(B)]
    rp, ci = to_csr(rows)
    out, lse = brute(q, k, v, rows, seq_lens)
    np.savez_compressed(os.path.join(HERE, name), q=q, k=k, v=v, row_ptr=rp, col_idx=ci,
                        seq_lens=np.asarray(seq_lens, np.int32), out=out.astype(np.float32),
                        lse=lse.astype(np.float32))
    print("wrote", name, "max|O|", float(np.abs(out).max()))


def main():
    rr = np.random.default_rng(77)
    retrieval_rows = [rows_retrieval(i, 2, rr) for i in range(4)]
    make("golden_families_t512.npz", 1, 2, 512,
         lambda b, h, i: rows_sliding(i, 2) if h == 0 else retrieval_rows[i], [512], seed=11)
    make("golden_seqlens_t256.npz", 2, 1, 256, lambda b, h, i: rows_global(i, 1, 2), [256, 150],
         seed=12)
    generic_rows = [
        [[0], [1, 0], [0, 2, 1]],      # diagonal first, diagonal in the middle
        [[], [0, 0, 1, 2], [1, 0]],    # empty row; repeated entry + block above; no diagonal
    ]
    make("golden_generic_t384.npz", 2, 2, 384, lambda b, h, i: generic_rows[h][i], [384, 200],
         seed=13, brute=brute_force_generic)


if __name__ == "__main__":
    main()
