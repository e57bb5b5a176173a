"""CPU oracle of the block-sparse causal attention forward — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this module, and only
to check results (or as the timed CPU baseline); the product path (usagi_amd) never imports it.

Three restatements of the reference's math:

  dense_masked()  fp32 (or fp64) softmax attention over the dense token mask
                  block_mask(CSR) ∧ causal ∧ key < seq_len, rows t >= seq_len -> O = 0,
                  LSE = -inf. This is the parity reference; for a valid CSR (distinct
                  blocks below qb, then the diagonal last) it equals the reference's walk
                  (kernels/v7_blockptr_warpspec.py:83-148).
  blockwise_v7()  the reference's own algorithm, step for step: per (b*h, qb) an online exp2
                  softmax over the off-diagonal CSR entries without a causal mask
                  (kernels/v7_blockptr_warpspec.py:83-108), then the implicit diagonal kb = qb
                  with the causal / seq_len / q-valid mask (v7:111-136), scores scaled after
                  the dot in fp32 (v7:92), P rounded to fp16 before P·V (v7:107), m initialised
                  to -1e30 (v7:73), O = acc / l_safe and LSE = m·ln2 + ln l (v7:138-148).
  blockwise_v1()  the generic walk of kernels/v1_baseline.py:360-406 (every entry, any order,
                  an entry equal to qb causally masked, keys past seq_len masked, no implicit
                  diagonal).

Pins (tests/test_oracle.py): fp64 brute force over explicitly enumerated key sets, the golden
fixtures in tests/golden/ (written by that brute force), torch's scaled_dot_product_attention
for a full lower-triangular CSR and for a diagonal-only CSR, and invariants (V constant,
Q = 0, query row 0, LSE = logsumexp, order invariance of the off-diagonal entries); for
blockwise_v1 also the fixture golden_generic_t384.npz of an fp64 brute force over key
multisets, and duplicating every entry leaving O unchanged while adding ln 2 to LSE.
"""

from __future__ import annotations

import math

import numpy as np

BLOCK = 128
QK_SCALE = (1.0 / math.sqrt(128)) * math.log2(math.e)  # kernels/v7_blockptr_warpspec.py:18-20
LN2 = math.log(2.0)                                       # kernels/v7_blockptr_warpspec.py:21


def _np(x, dtype=np.float32):
    """torch tensor / numpy array -> numpy array of `dtype`."""
    if hasattr(x, "detach"):
        x = x.detach().cpu()
        if str(x.dtype) == "torch.bfloat16":
            x = x.float()
        x = x.numpy()
    return np.asarray(x).astype(dtype, copy=False)


def block_mask(row_ptr_bh: np.ndarray, col_idx_bh: np.ndarray, nqb: int) -> np.ndarray:
    """[nqb, nqb] bool: block (qb, kb) active iff kb is listed in row qb."""
    m = np.zeros((nqb, nqb), dtype=bool)
    for i in range(nqb):
        m[i, col_idx_bh[row_ptr_bh[i]:row_ptr_bh[i + 1]]] = True
    return m


MUTATIONS = ("scale_1_over_d", "mask_transposed", "drop_diagonal", "k_for_v", "lse_log2")


def dense_masked(q, k, v, row_ptr, col_idx, seq_lens=None, dtype=np.float32, slab: int = 1024,
                 heads: list[tuple[int, int]] | None = None, _mutation: str | None = None):
    """fp32 (default) dense-masked attention. Returns (O [B,H,T,D], LSE [B,H,T]) as `dtype`.

    `heads` restricts the work to a list of (b, h) pairs (other rows are left as NaN).
    `_mutation` plants one of MUTATIONS; it exists only so the test suite can show that its
    pins catch such a mistake.
    """
    qn, kn, vn = _np(q, dtype), _np(k, dtype), _np(v, dtype)
    B, H, T, D = qn.shape
    nqb = T // BLOCK
    rp = np.asarray(row_ptr).reshape(B, H, nqb + 1)
    ci = np.asarray(col_idx).reshape(B, H, -1)
    sl = np.full(B, T) if seq_lens is None else np.asarray(seq_lens).reshape(B)
    scale = dtype(1.0 / math.sqrt(D)) if _mutation != "scale_1_over_d" else dtype(1.0 / D)
    out = np.full((B, H, T, D), np.nan, dtype=dtype)
    lse = np.full((B, H, T), np.nan, dtype=dtype)
    pairs = heads if heads is not None else [(b, h) for b in range(B) for h in range(H)]
    tok = np.arange(T)
    for b, h in pairs:
        bm = block_mask(rp[b, h], ci[b, h], nqb)
        L = int(sl[b])
        for t0 in range(0, T, slab):
            t1 = min(T, t0 + slab)
            rows = tok[t0:t1]
            mask = bm[rows[:, None] // BLOCK, tok[None, :] // BLOCK]
            if _mutation == "drop_diagonal":
                mask &= (rows[:, None] // BLOCK) != (tok[None, :] // BLOCK)
            if _mutation == "mask_transposed":
                mask &= (tok[None, :] >= rows[:, None]) | ((tok[None, :] // BLOCK) != (rows[:, None] // BLOCK))
            else:
                mask &= tok[None, :] <= rows[:, None]
            mask &= tok[None, :] < L
            mask &= (rows < L)[:, None]
            s = (qn[b, h, t0:t1] @ kn[b, h].T) * scale
            s = np.where(mask, s, -np.inf)
            mx = s.max(axis=1, keepdims=True)
            has = np.isfinite(mx[:, 0])
            mx = np.where(np.isfinite(mx), mx, 0)
            p = np.exp(s - mx)
            l = p.sum(axis=1, keepdims=True)
            vsrc = kn if _mutation == "k_for_v" else vn
            o = (p @ vsrc[b, h]) / np.where(l > 0, l, 1)
            out[b, h, t0:t1] = np.where(has[:, None], o, 0)
            ln = np.log2 if _mutation == "lse_log2" else np.log
            lse[b, h, t0:t1] = np.where(has, mx[:, 0] + ln(np.where(l[:, 0] > 0, l[:, 0], 1)),
                                        -np.inf)
    return out, lse


def _fp16_round(x: np.ndarray) -> np.ndarray:
    return x.astype(np.float16).astype(np.float32)


def blockwise_v7(q, k, v, row_ptr, col_idx, seq_lens=None, round_p_fp16: bool = True,
                 heads: list[tuple[int, int]] | None = None):
    """The reference's CSR walk restated in numpy (fp32). Returns (O, LSE) float32."""
    qn, kn, vn = _np(q), _np(k), _np(v)
    B, H, T, D = qn.shape
    nqb = T // BLOCK
    rp = np.asarray(row_ptr).reshape(B, H, nqb + 1)
    ci = np.asarray(col_idx).reshape(B, H, -1)
    sl = np.full(B, T) if seq_lens is None else np.asarray(seq_lens).reshape(B)
    out = np.full((B, H, T, D), np.nan, dtype=np.float32)
    lse = np.full((B, H, T), np.nan, dtype=np.float32)
    offs = np.arange(BLOCK)
    qk_scale = np.float32(QK_SCALE)
    pairs = heads if heads is not None else [(b, h) for b in range(B) for h in range(H)]
    v16 = _fp16_round(vn) if round_p_fp16 else vn
    for b, h in pairs:
        seq_len = int(sl[b])                                               # v7:48
        for qb in range(nqb):
            q_start = qb * BLOCK
            q_pos = q_start + offs
            if q_start >= seq_len:                                         # v7:63-67
                out[b, h, q_pos] = 0.0
                lse[b, h, q_pos] = -np.inf
                continue
            q_valid = q_pos < seq_len                                      # v7:69
            qt = qn[b, h, q_pos]                                           # v7:71
            m_i = np.full(BLOCK, -1e30, dtype=np.float32)                  # v7:73
            l_i = np.zeros(BLOCK, dtype=np.float32)                        # v7:74
            acc = np.zeros((BLOCK, D), dtype=np.float32)                   # v7:75
            rs, re = int(rp[b, h, qb]), int(rp[b, h, qb + 1])              # v7:77-79
            kbs = [int(x) for x in ci[b, h, rs:re - 1]] + [qb]             # v7:83, 111
            for j, kb in enumerate(kbs):
                diag = j == len(kbs) - 1
                k_pos = kb * BLOCK + offs
                s = (qt @ kn[b, h, k_pos].T) * qk_scale                    # v7:92 / 117
                if diag:                                                   # v7:119-122
                    mask = (offs[None, :] <= offs[:, None]) & (k_pos[None, :] < seq_len) \
                        & q_valid[:, None]
                else:                                                      # v7:94
                    mask = np.broadcast_to(q_valid[:, None], s.shape)
                s = np.where(mask, s, -np.inf).astype(np.float32)
                m_new = np.maximum(m_i, s.max(axis=1))                    # v7:96-97
                alpha = np.exp2(m_i - m_new)                               # v7:98
                p = np.exp2(s - m_new[:, None])                            # v7:99
                l_i = alpha * l_i + p.sum(axis=1)                          # v7:100
                pv = _fp16_round(p) if round_p_fp16 else p                 # v7:107
                acc = acc * alpha[:, None] + pv @ v16[b, h, k_pos]
                m_i = m_new
            l_safe = np.where(l_i > 0, l_i, 1.0).astype(np.float32)        # v7:138
            o = acc / l_safe[:, None]
            o = np.where(q_valid[:, None], o, 0.0)                         # v7:140
            out[b, h, q_pos] = o
            ls = np.where(l_i > 0, m_i * np.float32(LN2) + np.log(l_safe), -np.inf)
            lse[b, h, q_pos] = np.where(q_valid, ls, -np.inf)              # v7:146-147
    return out, lse


V1_MUTATIONS = ("diag_unmasked", "no_key_mask", "dedupe")


def blockwise_v1(q, k, v, row_ptr, col_idx, seq_lens=None, round_p_fp16: bool = True,
                 heads: list[tuple[int, int]] | None = None, _mutation: str | None = None):
    """The reference's generic CSR walk (kernels/v1_baseline.py:360-406) restated in numpy
    (fp32): every entry of the row in its order (v1:370-376), no implicit diagonal; an entry
    equal to qb is causally masked (v1:382-383); keys at or past seq_len and invalid query rows
    are masked for every entry (v1:385-386); a row with no visible key gives O = 0 and
    LSE = -inf (v1:398-406, output pre-filled with zeros / -inf at v1:421-422). Entries outside
    [0, nqb) are clamped into it, as the build does (the reference would read outside K/V).
    `_mutation` plants one of V1_MUTATIONS for the test suite's pins."""
    qn, kn, vn = _np(q), _np(k), _np(v)
    B, H, T, D = qn.shape
    nqb = T // BLOCK
    rp = np.asarray(row_ptr).reshape(B, H, nqb + 1)
    ci = np.asarray(col_idx).reshape(B, H, -1)
    sl = np.full(B, T) if seq_lens is None else np.asarray(seq_lens).reshape(B)
    out = np.full((B, H, T, D), np.nan, dtype=np.float32)
    lse = np.full((B, H, T), np.nan, dtype=np.float32)
    offs = np.arange(BLOCK)
    qk_scale = np.float32(QK_SCALE)
    pairs = heads if heads is not None else [(b, h) for b in range(B) for h in range(H)]
    v16 = _fp16_round(vn) if round_p_fp16 else vn
    for b, h in pairs:
        seq_len = int(sl[b])
        for qb in range(nqb):
            q_start = qb * BLOCK
            q_pos = q_start + offs
            if q_start >= seq_len:                                         # v1:360
                out[b, h, q_pos] = 0.0
                lse[b, h, q_pos] = -np.inf
                continue
            q_valid = q_pos < seq_len                                      # v1:362
            qt = qn[b, h, q_pos]
            m_i = np.full(BLOCK, -1e30, dtype=np.float32)                  # v1:366
            l_i = np.zeros(BLOCK, dtype=np.float32)
            acc = np.zeros((BLOCK, D), dtype=np.float32)
            rs, re = int(rp[b, h, qb]), int(rp[b, h, qb + 1])              # v1:370-373
            kbs = [min(max(int(x), 0), nqb - 1) for x in ci[b, h, rs:re]]
            if _mutation == "dedupe":
                kbs = sorted(set(kbs))
            for kb in kbs:                                                 # v1:375-376
                k_pos = kb * BLOCK + offs
                s = (qt @ kn[b, h, k_pos].T) * qk_scale                    # v1:380
                mask = np.broadcast_to(q_valid[:, None], s.shape).copy()   # v1:386
                if kb == qb and _mutation != "diag_unmasked":              # v1:382-383
                    mask &= offs[None, :] <= offs[:, None]
                if _mutation != "no_key_mask":                             # v1:385
                    mask &= k_pos[None, :] < seq_len
                s = np.where(mask, s, -np.inf).astype(np.float32)
                m_new = np.maximum(m_i, s.max(axis=1))                    # v1:388-389
                alpha = np.exp2(m_i - m_new)                               # v1:390
                p = np.exp2(s - m_new[:, None])                            # v1:391
                l_i = alpha * l_i + p.sum(axis=1)                          # v1:392
                pv = _fp16_round(p) if round_p_fp16 else p                 # v1:395
                acc = acc * alpha[:, None] + pv @ v16[b, h, k_pos]
                m_i = m_new
            l_safe = np.where(l_i > 0, l_i, 1.0).astype(np.float32)        # v1:398
            o = np.where(q_valid[:, None], acc / l_safe[:, None], 0.0)     # v1:399-404
            out[b, h, q_pos] = o
            ls = np.where(l_i > 0, m_i * np.float32(LN2) + np.log(l_safe), -np.inf)
            lse[b, h, q_pos] = np.where(q_valid, ls, -np.inf)              # v1:405-406
    return out, lse


def block_flops(active_blocks: int) -> int:
    """Algorithmic work: each active 128x128 block is Q·K^T + P·V = 4·128^3 FLOP."""
    return int(active_blocks) * 4 * BLOCK * BLOCK * 128
