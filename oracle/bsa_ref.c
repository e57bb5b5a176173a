/*
 * bsa_ref.c — plain-C restatement of the reference's CSR block-sparse causal attention walk.
 * TEST INFRASTRUCTURE ONLY: built by oracle/build.py into oracle/_build/ and loaded by tests/
 * and by bench.py's cpu_baseline leg to check results / as the timed CPU port. The product library
 * (usagi_amd/lib/libusagi_bsa.so) never links or calls it.
 *
 * Follows the Triton program _fwd_csr of kernels/v7_blockptr_warpspec.py:45-148 step for step,
 * on host fp32 copies of q/k/v:
 *   seq_len per batch (v7:48, host side repeat_interleave at v7:175);
 *   query block past seq_len -> O = 0, LSE = -inf (v7:63-67);
 *   m = -1e30, l = 0, acc = 0 (v7:73-75); row range from per-(b,h) local row_ptr (v7:77-80);
 *   off-diagonal loop over col_idx[rs .. re-2], unmasked except invalid query rows (v7:83-108);
 *   implicit diagonal kb = qb with c <= r, key < seq_len, q valid (v7:111-136);
 *   scores = dot * QK_SCALE in fp32 after the dot (v7:92); exp2 online softmax (v7:96-100);
 *   P (and V) rounded to fp16 before P·V when round_p_fp16 != 0 (v7:107);
 *   O = acc / l_safe, invalid rows 0, LSE = m·ln2 + ln(l_safe) or -inf (v7:138-148).
 * With walk = 1 it follows the generic walk of kernels/v1_baseline.py:360-406 instead: every
 * entry of the row in its order (v1:375-376), with no implicit diagonal; an entry equal to qb takes
 * the causal mask c <= r (v1:382-383), every entry masks keys at or past seq_len and invalid
 * query rows (v1:385-386). Entries outside [0, nqb) are clamped into it (the reference would
 * read outside K/V there; the build clamps the same way).
 * The argument list mirrors usagi_bsa_fwd (include/usagi_bsa.h) with host float arrays.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define BLK 128

/* IEEE binary16 round-to-nearest-even of a float, returned as float (overflow -> inf). */
static float round_fp16(float x) {
  if (!isfinite(x) || x == 0.0f) return x;
  const float ax = fabsf(x);
  if (ax >= 65520.0f) return copysignf(INFINITY, x);
  if (ax < 6.103515625e-05f) { /* subnormal range: multiples of 2^-24 */
    return nearbyintf(x * 16777216.0f) / 16777216.0f;
  }
  int e;
  const float m = frexpf(x, &e); /* x = m * 2^e, 0.5 <= |m| < 1 */
  return ldexpf(nearbyintf(ldexpf(m, 11)), e - 11);
}

int oracle_bsa_fwd(const float* q, const float* k, const float* v, const int32_t* row_ptr,
                   const int32_t* col_idx, const int32_t* seq_lens, float* out, float* lse,
                   int32_t batch, int32_t heads, int32_t seq_len_max, int32_t head_dim,
                   int32_t max_nnz, int32_t round_p_fp16, int32_t walk) {
  if (!q || !k || !v || !row_ptr || !out || batch <= 0 || heads <= 0 || seq_len_max <= 0 ||
      seq_len_max % BLK || head_dim <= 0 || max_nnz < 0 || (max_nnz > 0 && !col_idx))
    return -1;
  const int T = seq_len_max, D = head_dim, nqb = T / BLK;
  const int64_t nbh = (int64_t)batch * heads;
  const float qk_scale = (float)((1.0 / sqrt((double)D)) * 1.4426950408889634); /* v7:18-20 */
  const float ln2 = (float)0.6931471805599453;                                /* v7:21 */

#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t item = 0; item < nbh * nqb; ++item) {
    const int64_t bh = item / nqb;
    const int qb = (int)(item % nqb);
    const int seq_len = seq_lens ? seq_lens[bh / heads] : T;
    const size_t base = (size_t)bh * T * D;
    const int q_start = qb * BLK;
    float* o_blk = out + base + (size_t)q_start * D;
    float* l_blk = lse ? lse + (size_t)bh * T + q_start : NULL;
    if (q_start >= seq_len) {
      memset(o_blk, 0, sizeof(float) * BLK * D);
      if (l_blk)
        for (int r = 0; r < BLK; ++r) l_blk[r] = -INFINITY;
      continue;
    }
    float* s = (float*)malloc(sizeof(float) * BLK * BLK);
    float* acc = (float*)calloc((size_t)BLK * D, sizeof(float));
    float* vb = (float*)malloc(sizeof(float) * BLK * D);
    float m_i[BLK], l_i[BLK];
    for (int r = 0; r < BLK; ++r) {
      m_i[r] = -1e30f;
      l_i[r] = 0.0f;
    }
    const int32_t* rp = row_ptr + bh * (nqb + 1);
    const int rs = rp[qb], re = rp[qb + 1];
    const int n_off = re - rs - 1 > 0 ? re - rs - 1 : 0;
    const int32_t* cols = col_idx ? col_idx + bh * max_nnz + rs : NULL;
    /* v7: off-diagonal entries then the implicit diagonal (n_off + 1 blocks); v1: every entry. */
    const int n_blk = walk ? (cols && re - rs > 0 ? re - rs : 0) : n_off + 1;
    for (int j = 0; j < n_blk; ++j) {
      int kb, diag;
      if (walk) {
        kb = cols[j] < 0 ? 0 : (cols[j] >= nqb ? nqb - 1 : cols[j]);
        diag = kb == qb;
      } else {
        diag = (j == n_off);
        kb = diag ? qb : cols[j];
      }
      const int k_start = kb * BLK;
      const float* kp = k + base + (size_t)k_start * D;
      const float* vp = v + base + (size_t)k_start * D;
      for (int r = 0; r < BLK; ++r) {
        const float* qr = q + base + (size_t)(q_start + r) * D;
        const int q_valid = q_start + r < seq_len;
        for (int c = 0; c < BLK; ++c) {
          const float* kr = kp + (size_t)c * D;
          float dot = 0.0f;
          for (int d = 0; d < D; ++d) dot += qr[d] * kr[d];
          float sc = dot * qk_scale;
          int keep = q_valid;
          if (diag) keep = keep && (c <= r) && (k_start + c < seq_len);
          if (walk) keep = keep && (k_start + c < seq_len);
          s[r * BLK + c] = keep ? sc : -INFINITY;
        }
      }
      for (int c = 0; c < BLK * D; ++c) vb[c] = round_p_fp16 ? round_fp16(vp[c]) : vp[c];
      for (int r = 0; r < BLK; ++r) {
        float* sr = s + r * BLK;
        float mj = -INFINITY;
        for (int c = 0; c < BLK; ++c) mj = sr[c] > mj ? sr[c] : mj;
        const float m_new = m_i[r] > mj ? m_i[r] : mj;
        const float alpha = exp2f(m_i[r] - m_new);
        float rsum = 0.0f;
        for (int c = 0; c < BLK; ++c) {
          const float p = exp2f(sr[c] - m_new);
          rsum += p;
          sr[c] = round_p_fp16 ? round_fp16(p) : p;
        }
        l_i[r] = alpha * l_i[r] + rsum;
        float* ar = acc + (size_t)r * D;
        for (int d = 0; d < D; ++d) ar[d] *= alpha;
        for (int c = 0; c < BLK; ++c) {
          const float p = sr[c];
          if (p == 0.0f) continue;
          const float* vr = vb + (size_t)c * D;
          for (int d = 0; d < D; ++d) ar[d] += p * vr[d];
        }
        m_i[r] = m_new;
      }
    }
    for (int r = 0; r < BLK; ++r) {
      const int q_valid = q_start + r < seq_len;
      const float l_safe = l_i[r] > 0.0f ? l_i[r] : 1.0f;
      for (int d = 0; d < D; ++d) o_blk[(size_t)r * D + d] = q_valid ? acc[(size_t)r * D + d] / l_safe : 0.0f;
      if (l_blk) {
        const float ls = l_i[r] > 0.0f ? m_i[r] * ln2 + logf(l_safe) : -INFINITY;
        l_blk[r] = q_valid ? ls : -INFINITY;
      }
    }
    free(s);
    free(acc);
    free(vb);
  }
  return 0;
}
