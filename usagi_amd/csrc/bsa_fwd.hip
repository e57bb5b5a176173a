// Block-sparse causal attention forward for MI355X (gfx950 / CDNA4).
//
// Semantics follow the reference Triton kernel _fwd_csr (kernels/v7_blockptr_warpspec.py:30-148,
// same math as kernels/v4_leaderboard_0740ms.py:31-136): for each (b*h, query block qb) the
// CSR row col_idx[row_ptr[qb] : row_ptr[qb+1]] lists key blocks, ascending, with the diagonal
// last. Entries before the diagonal are attended unmasked (v7:83-108); the diagonal is taken
// implicitly as kb = qb and causally masked (v7:111-136). Softmax is an online exp2 softmax
// over fp32 scores scaled AFTER the dot product (v7:92, v7:96-100); P is rounded to fp16 before
// P·V (v7:107). O = acc / l and LSE = m·ln2 + ln l (v7:138-148).
//
// Three kernels share that structure:
//   bsa_fwd_dma_kernel<bf16, window>  the default for fp16 and bf16: K/V tiles DMA'd HBM -> LDS,
//                           V read transposed out of LDS, two workgroups per CU, diagonal block
//                           first, speculative softmax (see the comment at the kernel). With
//                           window = true the rows are a window (+ global prefix) computed in
//                           the kernel instead of read from the CSR (usagi_bsa_fwd_window).
//   bsa_fwd_kernel<bf16>    register-staged K/V (global -> VGPR -> LDS, V transposed and
//                           converted to fp16 on the way in); USAGI_BSA_FP16_KERNEL=staged.
//   bsa_fwd_split_kernel    fp16, one workgroup per CU, each wave 64 rows x 64 keys, K/V
//                           double-buffered; USAGI_BSA_FP16_KERNEL=split.
//
// Common MI355X design points (not a translation of the Triton program):
//   * One 256-thread workgroup (4 wave64s) per (b*h, qb); each wave owns 32 query rows (the
//     split kernel: 64 rows and half the keys).
//   * Everything is computed transposed so that one lane owns one query row:
//       S^T[key][q] = K · Q^T      (MFMA A = K rows from LDS, B = Q fragment in VGPRs)
//       O^T[d][q]  += V^T · P^T    (MFMA A = V^T rows from LDS, B = P taken straight from the
//                                   S^T accumulator registers, no LDS round trip)
//     With v_mfma_f32_32x32x16_{f16,bf16}, lane l holds query (l % 32); the other 64 keys of
//     that query sit in lane l ^ 32, so the row max is one v_permlane32_swap and the running
//     row sum needs no cross-lane work until the epilogue.
//   * Work order (item_coords): longest row first; when B*H is a multiple of 8, head-major per
//     XCD, so the K/V tiles of the head an XCD is walking stay in its L2.
//   * The O rescale is skipped for almost every block: the DMA kernel computes P with the
//     running max as it stands and checks the row sum of P (a sum <= 2^12 proves every P finite
//     in fp16); the other two move the running max only when it grows by more than 2^8.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <type_traits>

#include "usagi_bsa.h"

namespace {

constexpr int kBlk = USAGI_BSA_BLOCK;    // rows per query / key block
constexpr int kHd = USAGI_BSA_HEAD_DIM;  // head dimension
constexpr int kThreads = 256;            // 4 wave64s
constexpr int kRow = kHd + 8;            // halfs per padded LDS row (272 B)
constexpr float kTau = 8.0f;             // lazy-rescale threshold, log2 units
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kSpecSum = 4096.0f;      // acceptance bound of a speculative P row sum

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct Args {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;
  const int32_t* row_ptr;
  const int32_t* col_idx;
  const int32_t* seq_lens;
  int heads;
  int T;
  int nqb;
  int bh_count;
  int max_nnz;
  float qk_scale;  // log2(e) / sqrt(128)
  int head_major;  // work-item order, see item_coords
  int window;      // analytic rows (bsa_fwd_dma_kernel<*, true>): window length in blocks
  int n_global;    // analytic rows: global prefix blocks
};

// Work item (workgroup index) -> (query block, b*h).
// head_major == 0: longest rows first over the whole grid (query blocks in descending order,
//   b*h fastest).
// head_major == 1 (B*H a multiple of 8): workgroups are dealt to the 8 XCDs round-robin by
//   index, so item i runs on XCD i % 8; each XCD walks its heads x, x+8, ... one at a time, and
//   within a head takes the query blocks longest row first. The key/value tiles of the head being
//   walked (4 MiB at T = 8192) then stay in that XCD's L2 while all its query blocks read them.
__device__ __forceinline__ void item_coords(const Args& a, int item, int& qb, int& bh) {
  if (a.head_major) {
    const int x = item & 7;
    const int j = item >> 3;
    const int hl = j / a.nqb;
    qb = a.nqb - 1 - (j - hl * a.nqb);
    bh = x + 8 * hl;
  } else {
    const int qslot = item / a.bh_count;
    qb = a.nqb - 1 - qslot;
    bh = item - qslot * a.bh_count;
  }
}

__device__ __forceinline__ float wave_pair_max(float x) {
  // {x[l], x[l ^ 32]} in some order; max is symmetric.
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float wave_pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Two bf16 (one dword) -> two fp16 (one dword), round to nearest even.
__device__ __forceinline__ uint32_t bf16x2_to_f16x2(uint32_t w) {
  const float lo = __uint_as_float(w << 16);
  const float hi = __uint_as_float(w & 0xffff0000u);
  const _Float16 a = (_Float16)lo;
  const _Float16 b = (_Float16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

__device__ __forceinline__ uint16_t to_out_bits(float x, bool bf16) {
  if (bf16) return __builtin_bit_cast(uint16_t, (__bf16)x);
  return __builtin_bit_cast(uint16_t, (_Float16)x);
}

template <bool kBf16>
__device__ __forceinline__ floatx16 mfma_qk(u32x4 a, u32x4 b, floatx16 c) {
  if constexpr (kBf16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a),
                                                  __builtin_bit_cast(half8, b), c, 0, 0, 0);
  }
}

__device__ __forceinline__ floatx16 mfma_pv(u32x4 a, half8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), b, c, 0, 0, 0);
}

template <bool kBf16>
__global__ __launch_bounds__(kThreads) void bsa_fwd_kernel(Args a) {
  __shared__ __attribute__((aligned(16))) uint16_t k_lds[kBlk * kRow];   // K[key][d]
  __shared__ __attribute__((aligned(16))) uint16_t vt_lds[kHd * kRow];   // V^T[d][key'] (fp16)

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 31;
  const int lh = lane >> 5;

  // Longest-row-first issue order: descending query block, b*h fastest.
  int qb, bh;
  item_coords(a, blockIdx.x, qb, bh);
  const int seq_len = a.seq_lens ? a.seq_lens[bh / a.heads] : a.T;
  const int q0 = qb * kBlk;
  const size_t base = (size_t)bh * a.T * kHd;
  uint16_t* out_blk = a.o + base + (size_t)q0 * kHd;

  if (q0 >= seq_len) {
    // Whole query block past the sequence: O = 0, LSE = -inf (v7:63-67).
#pragma unroll
    for (int i = 0; i < (kBlk * kHd) / (8 * kThreads); ++i) {
      *(u32x4*)(out_blk + (size_t)(i * kThreads + tid) * 8) = u32x4{0, 0, 0, 0};
    }
    if (a.lse && tid < kBlk) a.lse[(size_t)bh * a.T + q0 + tid] = -INFINITY;
    return;
  }

  const int q_local = wave * 32 + li;
  const int qrow = q0 + q_local;
  const bool qvalid = qrow < seq_len;
  const bool full_q = q0 + kBlk <= seq_len;  // uniform: no query row of the block is masked

  // Q^T fragment (MFMA B operand): lane holds Q[qrow][16s + 8lh .. +8] for s = 0..7.
  u32x4 qf[8];
  {
    const uint16_t* qp = a.q + base + (size_t)qrow * kHd + 8 * lh;
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = *(const u32x4*)(qp + 16 * s);
  }

  // CSR row (offsets local to this b*h, v7:77-80). Clamped so a malformed row cannot index
  // outside col_idx or outside K/V; the host validator reports such rows as errors.
  const int32_t* rp = a.row_ptr + (size_t)bh * (a.nqb + 1) + qb;
  int rs = rp[0];
  int re = rp[1];
  rs = min(max(rs, 0), a.max_nnz);
  re = min(max(re, rs), a.max_nnz);
  const int n_off = max(re - rs - 1, 0);  // off-diagonal entries; the last entry is the diagonal
  const int32_t* cols = a.col_idx + (size_t)bh * a.max_nnz + rs;
  const int nqb_m1 = a.nqb - 1;
  auto key_block = [&](int j) -> int {
    if (j >= n_off) return qb;
    const int kb = cols[j];
    return min(max(kb, 0), nqb_m1);
  };

  // Tile staging. K: chunk c = i*256 + tid -> row c/16, 8 halfs at (c%16)*8.
  // V: thread owns 8 keys x 8 d: d chunk dc, key group kg holding keys
  //    16*(kg/2) + 4*(kg%2) + {0,1,2,3} and +8 + {0,1,2,3}, written transposed so that
  //    V^T row d, positions 8kg .. 8kg+7 hold exactly those keys in that order.
  const int v_dc = (tid >> 2) & 15;
  const int v_kg = (tid & 3) + 4 * wave;
  const int v_key0 = 16 * (v_kg >> 1) + 4 * (v_kg & 1);
  u32x4 kst[8];
  u32x4 vst[8];

  auto load_tile = [&](int kb) {
    const uint16_t* kp = a.k + base + (size_t)kb * kBlk * kHd;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = i * kThreads + tid;
      kst[i] = *(const u32x4*)(kp + (c >> 4) * kHd + (c & 15) * 8);
    }
    const uint16_t* vp = a.v + base + (size_t)kb * kBlk * kHd + v_dc * 8;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int key = v_key0 + (e & 3) + 8 * (e >> 2);
      vst[e] = *(const u32x4*)(vp + key * kHd);
    }
  };

  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = i * kThreads + tid;
      *(u32x4*)(k_lds + (c >> 4) * kRow + (c & 15) * 8) = kst[i];
    }
    if constexpr (kBf16) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
#pragma unroll
        for (int w = 0; w < 4; ++w) vst[e][w] = bf16x2_to_f16x2(vst[e][w]);
      }
    }
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const uint32_t sel = (d & 1) ? 0x07060302u : 0x05040100u;
      u32x4 w;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        w[j] = __builtin_amdgcn_perm(vst[2 * j + 1][d >> 1], vst[2 * j][d >> 1], sel);
      }
      *(u32x4*)(vt_lds + (v_dc * 8 + d) * kRow + v_kg * 8) = w;
    }
  };

  floatx16 o_acc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[u][r] = 0.0f;
  }
  float m_used = -1e30f;  // running max in log2 units (v7:73)
  float l_part = 0.0f;    // this lane's half of the running row sum
  const float scale = a.qk_scale;

  const int nblk = n_off + 1;
  load_tile(key_block(0));

  for (int j = 0; j < nblk; ++j) {
    if (j) __syncthreads();  // every wave is done reading the previous tile
    store_tile();
    __syncthreads();
    const bool diag = (j == n_off);
    if (j + 1 < nblk) load_tile(key_block(j + 1));

    // S^T = K · Q^T: st[t][r] = S[q_local][key], key = 32t + 8(r/4) + 4lh + r%4.
    floatx16 st[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) st[t][r] = 0.0f;
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const u32x4 ka = *(const u32x4*)(k_lds + (32 * t + li) * kRow + 16 * s + 8 * lh);
        st[t] = mfma_qk<kBf16>(ka, qf[s], st[t]);
      }
    }

    // Masks: causal on the diagonal (v7:119-122), invalid query rows everywhere (v7:94).
    if (diag) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = 32 * t + 8 * (r >> 2) + 4 * lh + (r & 3);
          if (key > q_local || !qvalid) st[t][r] = -INFINITY;
        }
      }
    } else if (!full_q && !qvalid) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) st[t][r] = -INFINITY;
      }
    }

    // Online softmax in log2 units.
    float mx = st[0][0];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, st[t][r]);
    }
    mx = wave_pair_max(mx);
    const float m_cand = fmaxf(m_used, mx * scale);
    const bool grow = m_cand > m_used + kTau;
    if (__any(grow)) {
      const float alpha = grow ? __builtin_amdgcn_exp2f(m_used - m_cand) : 1.0f;
      m_used = grow ? m_cand : m_used;
      l_part *= alpha;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int r = 0; r < 16; ++r) o_acc[u][r] *= alpha;
      }
    }
    const float neg_m = -m_used;
    float psum = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(fmaf(st[t][r], scale, neg_m));
        st[t][r] = p;
        psum += p;
      }
    }
    l_part += psum;

    // P^T fragments (MFMA B operand of P·V): k-step s covers keys 16s + 8(e/4) + 4lh + e%4.
    half8 pb[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[s][e] = (_Float16)st[s >> 1][8 * (s & 1) + e];
    }

    // O^T += V^T · P^T: o_acc[u][r] = O[q_local][d], d = 32u + 8(r/4) + 4lh + r%4.
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const u32x4 va = *(const u32x4*)(vt_lds + (32 * u + li) * kRow + 16 * s + 8 * lh);
        o_acc[u] = mfma_pv(va, pb[s], o_acc[u]);
      }
    }
  }

  // Epilogue (v7:138-148).
  const float l_tot = wave_pair_sum(l_part);
  float inv = l_tot > 0.0f ? 1.0f / l_tot : 1.0f;
  if (!qvalid) inv = 0.0f;
  uint16_t* orow = a.o + base + (size_t)qrow * kHd + 4 * lh;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      u32x2 w;
      w[0] = (uint32_t)to_out_bits(o_acc[u][4 * g + 0] * inv, kBf16) |
             ((uint32_t)to_out_bits(o_acc[u][4 * g + 1] * inv, kBf16) << 16);
      w[1] = (uint32_t)to_out_bits(o_acc[u][4 * g + 2] * inv, kBf16) |
             ((uint32_t)to_out_bits(o_acc[u][4 * g + 3] * inv, kBf16) << 16);
      *(u32x2*)(orow + 32 * u + 8 * g) = w;
    }
  }
  if (a.lse && lh == 0) {
    const float lse = (qvalid && l_tot > 0.0f) ? (m_used + log2f(l_tot)) * kLn2 : -INFINITY;
    a.lse[(size_t)bh * a.T + qrow] = lse;
  }
}


// ---------------------------------------------------------------------------------------------
// DMA kernel (fp16; bf16 with the V tile turned into fp16 in LDS): K and V tiles go HBM -> LDS by
// direct DMA (global_load_lds_dwordx4), so no VGPRs stage them; V is read transposed out of LDS
// with ds_read_b64_tr_b16. That keeps the wave at <= 256 registers, so two workgroups share each
// CU (2 waves per SIMD): while one workgroup waits at a barrier or runs softmax VALU, the other
// keeps the matrix core busy.
//
// LDS tiles are 128 rows x 256 B, unpadded, with 16-byte chunks XOR-swizzled inside each row
// (K: chunk ^ (row % 16), V: chunk ^ 4 * (row % 4)) so that both the DMA writes (1 KiB
// lane-contiguous per wave instruction) and the MFMA operand reads spread over all banks.
//
// Per key block j (two barriers, tiles single-buffered per workgroup, 64 KiB of LDS):
//   wait K(j) | barrier | S^T = K·Q^T, DMA of V(j) spread between the MFMAs | P = exp2 in fp16
//   and its row sum (diagonal: exact row max first; otherwise the running max, checked by the sum)
//   wait V(j) | barrier | O^T += V^T·P^T, DMA of K(j+1) spread between the MFMAs
// The diagonal block goes first, so its K tile is requested at entry without reading col_idx.
// O leaves through LDS as whole rows.
// A 16-byte-per-lane LDS DMA holds the issuing wave for tens of cycles, so the eight 1 KiB
// pieces of a wave's share are interleaved with MFMAs instead of being issued back to back.
// ---------------------------------------------------------------------------------------------

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) const void global_cvoid;

// One 16-byte-per-lane DMA: global (uniform base + per-lane byte offset) -> LDS at the uniform
// byte address lds_addr + 16 * lane. Issued as inline asm so that the compiler's wait-count pass
// does not treat it as aliasing every later LDS read; the kernel waits for it explicitly
// (s_waitcnt vmcnt + s_barrier) before any wave reads the tile.
template <int kImm>
__device__ __forceinline__ void dma_16b(const void* gbase, uint32_t voff, uint32_t lds_addr) {
  // M0 holds the LDS destination. Nothing else in these kernels uses M0 (gfx950 LDS
  // instructions do not read it), so it is not saved.
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2 offset:%3"
      :
      : "s"(lds_addr), "v"(voff), "s"(gbase), "i"(kImm)
      : "memory");
}

// 8 DMAs of one wave's 8 KiB share of a tile: instruction i moves row group i (1 KiB). The
// instruction's immediate offset moves both the global and the LDS address, so 1024 (i % 4) goes
// there and i >= 4 use global and LDS bases 4096 bytes further on.
__device__ __forceinline__ void dma_tile8(const char* src, const uint32_t off[4], uint32_t lds) {
  const char* src_hi = src + 4096;
  const uint32_t lds_hi = lds + 4096;
  dma_16b<0>(src, off[0], lds);
  dma_16b<1024>(src, off[1], lds);
  dma_16b<2048>(src, off[2], lds);
  dma_16b<3072>(src, off[3], lds);
  dma_16b<0>(src_hi, off[0], lds_hi);
  dma_16b<1024>(src_hi, off[1], lds_hi);
  dma_16b<2048>(src_hi, off[2], lds_hi);
  dma_16b<3072>(src_hi, off[3], lds_hi);
}

__device__ __forceinline__ uint32_t lds_addr_of(const void* p) {
  return (uint32_t)(uintptr_t)(lds_void*)p;
}

#define USAGI_BARRIER() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")
#define USAGI_WAIT_VM(n) asm volatile("s_waitcnt vmcnt(" #n ")" ::: "memory")
#define USAGI_FENCE() __builtin_amdgcn_sched_barrier(0)

// kWindow: analytic rows instead of the CSR (no row_ptr / col_idx reads): query block qb attends
// the global prefix 0 .. n_global-1 and the window max(0, qb-window+1) .. qb, deduplicated and
// ascending, the rows of kernels/v1_baseline.py:141-322 (_fwd_window, _fwd_window_global).
template <bool kBf16, bool kWindow>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void bsa_fwd_dma_kernel(Args a) {
  __shared__ __attribute__((aligned(1024))) uint16_t k_lds[kBlk * kHd];  // K[key][d], swizzled
  __shared__ __attribute__((aligned(1024))) uint16_t v_lds[kBlk * kHd];  // V[key][d], swizzled

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 31;
  const int lh = lane >> 5;

  int qb, bh;
  item_coords(a, blockIdx.x, qb, bh);
  const size_t base = (size_t)bh * a.T * kHd;
  constexpr size_t kTileBytes = (size_t)kBlk * kHd * 2;
  auto tile_k = [&](int kb) { return (const char*)(a.k + base) + (size_t)kb * kTileBytes; };
  auto tile_v = [&](int kb) { return (const char*)(a.v + base) + (size_t)kb * kTileBytes; };

  // DMA: wave w, instruction i writes row group 8w + i (rows 32w + 4i + L/16, 1 KiB per wave
  // instruction). Lane L covers physical chunk L%16 = logical chunk (L%16) ^ swz(row). The
  // per-lane byte offsets repeat for every tile, so only the uniform tile base changes.
  const int dma_r = lane >> 4;
  const int dma_pc = lane & 15;
  // Row 32w + 4i + L/16 has (row % 16) = 4(i % 4) + L/16 and (row % 4) = L/16.
  uint32_t k_off[4];
  uint32_t v_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    k_off[i] = (uint32_t)((32 * wave + dma_r) * 256 + 16 * (dma_pc ^ (4 * i + dma_r)));
    v_off[i] = (uint32_t)((32 * wave + dma_r) * 256 + 16 * (dma_pc ^ (4 * dma_r)));
  }
  const uint32_t k_dst = __builtin_amdgcn_readfirstlane(lds_addr_of(k_lds) + wave * 8192);
  const uint32_t v_dst = __builtin_amdgcn_readfirstlane(lds_addr_of(v_lds) + wave * 8192);

  // The diagonal block is processed first: its key block is qb itself, so its K tile goes out
  // before anything else is read, while Q, seq_len and the row's column indices are in flight.
  // (The reference walks it last; online softmax does not depend on the order, up to the fp16
  // rounding of P.)
  dma_tile8(tile_k(qb), k_off, k_dst);

  const int seq_len = a.seq_lens ? a.seq_lens[bh / a.heads] : a.T;
  const int q0 = qb * kBlk;
  if (q0 >= seq_len) {
    // The whole query block is past seq_len: O = 0, LSE = -inf (v7:63-67).
    uint16_t* out_blk = a.o + base + (size_t)q0 * kHd;
#pragma unroll
    for (int i = 0; i < (kBlk * kHd) / (8 * kThreads); ++i) {
      *(u32x4*)(out_blk + (size_t)(i * kThreads + tid) * 8) = u32x4{0, 0, 0, 0};
    }
    if (a.lse && tid < kBlk) a.lse[(size_t)bh * a.T + q0 + tid] = -INFINITY;
    USAGI_WAIT_VM(0);  // the K tile DMA lands before the workgroup's LDS is released
    return;
  }

  const int q_local = wave * 32 + li;
  const int qrow = q0 + q_local;
  const bool qvalid = qrow < seq_len;

  u32x4 qf[8];
  {
    const uint16_t* qp = a.q + base + (size_t)qrow * kHd + 8 * lh;
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = *(const u32x4*)(qp + 16 * s);
  }

  const int nqb_m1 = a.nqb - 1;
  int n_off = 0;
  // CSR rows: column indices are held 64 at a time in one VGPR (lane i: entry 64c + i) and
  // picked with v_readlane, so no vector load sits inside the loop behind the in-flight tile
  // DMAs. Rows longer than 64 blocks reload the next chunk when they reach it.
  const int32_t* cols = nullptr;
  int col_chunk = 0;
  int colv = 0;
  // Analytic rows: entries 0 .. win_ng-1 are the global blocks below the window, then the
  // window from win_lo up to qb - 1.
  int win_lo = 0;
  int win_ng = 0;
  if constexpr (kWindow) {
    win_lo = max(qb - a.window + 1, 0);
    win_ng = min(a.n_global, win_lo);
    n_off = win_ng + (qb - win_lo);
  } else {
    const int32_t* rp = a.row_ptr + (size_t)bh * (a.nqb + 1) + qb;
    int rs = rp[0];
    int re = rp[1];
    rs = min(max(rs, 0), a.max_nnz);
    re = min(max(re, rs), a.max_nnz);
    n_off = max(re - rs - 1, 0);
    cols = a.col_idx + (size_t)bh * a.max_nnz + rs;
    colv = lane < n_off ? cols[lane] : 0;
  }
  auto key_block = [&](int j) -> int {
    if constexpr (kWindow) {
      return j < win_ng ? j : win_lo + (j - win_ng);
    } else {
      const int c = j >> 6;
      if (c != col_chunk) {
        col_chunk = c;
        const int e = c * 64 + lane;
        colv = e < n_off ? cols[e] : 0;
      }
      const int kb = __builtin_amdgcn_readlane(colv, j & 63);
      return min(max(kb, 0), nqb_m1);
    }
  };

  // Piece i (0..7) of this wave's 8 KiB share of a tile: one 1 KiB DMA. The pieces are spread
  // between MFMAs: a 16-byte-per-lane DMA holds the issuing wave for tens of cycles, which then
  // overlaps the previous MFMA instead of stalling a whole phase.
  auto dma_piece = [&](const char* tile, const uint32_t off[4], uint32_t dst, int i) {
    const char* src = tile + (i >= 4 ? 4096 : 0);
    const uint32_t lds = dst + (i >= 4 ? 4096 : 0);
    switch (i & 3) {
      case 0: dma_16b<0>(src, off[0], lds); break;
      case 1: dma_16b<1024>(src, off[1], lds); break;
      case 2: dma_16b<2048>(src, off[2], lds); break;
      default: dma_16b<3072>(src, off[3], lds); break;
    }
  };

  // K operand (MFMA A, 32 keys x 16 d): lane reads row 32t + li, logical chunk 2s + lh.
  const char* k_rd = (const char*)k_lds + li * 256;
  const int k_x = lh ^ (li & 15);
  // V^T operand via transpose reads: source lane l supplies row key0 + (l%16)/4 and the
  // 8 bytes at d = 32u + 16((l/16)%2) + 4(l%4); key0 = 16s + 8r + 4lh.
  const int tq = (lane & 15) >> 2;
  const int t_x = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
  const char* v_rd = (const char*)v_lds + (4 * lh + tq) * 256 + 8 * (lane & 1);

  floatx16 o_acc[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[u][r] = 0.0f;
  }
  float m_used = -1e30f;
  float l_part = 0.0f;
  const float scale = a.qk_scale;

  // vmcnt(0): Q, the column chunk (CSR rows) and the diagonal K tile have landed. Issued as a
  // real s_waitcnt so the compiler knows no load of its own is outstanding inside the loop.
  __builtin_amdgcn_s_waitcnt(0x0F70);

  // One key block: the diagonal (kDiag, j = -1, causal mask) or off-diagonal entry j.
  // kMaskQ: some query rows of this block are past seq_len. kNext: DMA the K tile of entry
  // j + 1 during this block's P·V.
  auto block = [&](auto diag_tag, auto maskq_tag, auto next_tag, int j) {
    constexpr bool kDiag = decltype(diag_tag)::value;
    constexpr bool kMaskQ = decltype(maskq_tag)::value;
    constexpr bool kNext = decltype(next_tag)::value;
    USAGI_WAIT_VM(0);  // this wave's K(j) DMA has landed
    USAGI_BARRIER();   // K(j) complete; every wave is done reading V of the previous block
    const char* vt_src = tile_v(kDiag ? qb : key_block(j));

    // Matrix-core sections run at raised wave priority, so when both waves of a SIMD (one per
    // workgroup) can issue, the MFMA stream goes first and the other wave's exponentials fill
    // the gaps.
    __builtin_amdgcn_s_setprio(1);
    // ---- S^T = K · Q^T: 32 MFMAs, K operands read one step ahead.
    floatx16 st[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) st[t][r] = 0.0f;
    }
    // V(j) DMA pieces go out between the QK MFMAs (the V buffer is free after the barrier).
    u32x4 kop[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (!kDiag || t <= wave) kop[t] = *(const u32x4*)(k_rd + t * 8192 + 16 * (0 ^ k_x));
    }
    // On the diagonal, key tile t (keys 32t .. 32t+31) lies above every row of wave w when t > w:
    // those tiles are skipped here, in the softmax and in P·V.
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (!kDiag || t <= wave) {
          const u32x4 ka = kop[t];
          if (s < 7) kop[t] = *(const u32x4*)(k_rd + t * 8192 + 16 * ((2 * (s + 1)) ^ k_x));
          st[t] = mfma_qk<kBf16>(ka, qf[s], st[t]);
        }
      }
      dma_piece(vt_src, v_off, v_dst, s);
    }
    // Schedule: each step's 4 K operands are read one step ahead of its 4 MFMAs (deeper
    // read-ahead only adds registers: the reads complete within one step).
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
#pragma unroll
    for (int i = 0; i < 7; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 1);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 1);

    // ---- masks (v7:94, v7:119-122), row max, lazy rescale
    if constexpr (kDiag) {
      // Key tiles below the wave's own (t < wave) are visible to all its rows, its own tile
      // (t == wave) takes the causal mask, and the tiles above (t > wave) were skipped by the
      // MFMAs: their softmax is skipped too (P·V never reads them).
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (t == wave) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = 32 * t + 8 * (r >> 2) + 4 * lh + (r & 3);
            if (key > q_local || !qvalid) st[t][r] = -INFINITY;
          }
        } else if (t < wave && !qvalid) {
#pragma unroll
          for (int r = 0; r < 16; ++r) st[t][r] = -INFINITY;
        }
      }
    } else if constexpr (kMaskQ) {
      if (!qvalid) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
          for (int r = 0; r < 16; ++r) st[t][r] = -INFINITY;
        }
      }
    }
    __builtin_amdgcn_s_setprio(0);
    // ---- P = exp2(S·scale - m) in fp16 and its row sum (this lane's 64 keys).
    // The diagonal block (always the first block of a row) takes the exact row max. Later blocks
    // compute P with the running max as it stands: each P is <= the lane's fp32 sum of its P,
    // so a sum <= 2^12 proves every P finite in fp16 and the result exact in the normalised
    // output; otherwise (rare) the row max moves to the block's exact max, O and l are rescaled
    // and P recomputed.
    half8 pb[8];
    float pblk = 0.0f;
    auto make_p = [&]() {
      const float neg_m = -m_used;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        if (kDiag && (s >> 1) > wave) continue;  // a key tile above the wave's rows
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          pb[s][e] = (_Float16)__builtin_amdgcn_exp2f(fmaf(st[s >> 1][8 * (s & 1) + e], scale, neg_m));
        }
      }
      float acc = 0.0f;
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        if (kDiag && (s >> 1) > wave) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const half2 pp = {pb[s][2 * e], pb[s][2 * e + 1]};
          acc = __builtin_amdgcn_fdot2(pp, half2{1.0f16, 1.0f16}, acc, false);
        }
      }
      pblk = acc;
    };
    auto row_max = [&]() {
      float mx = st[0][0];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (kDiag && t > wave) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, st[t][r]);
      }
      return wave_pair_max(mx);
    };
    auto rescale = [&](float m_new) {
      const float alpha = __builtin_amdgcn_exp2f(m_used - m_new);
      m_used = m_new;
      l_part *= alpha;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int r = 0; r < 16; ++r) o_acc[u][r] *= alpha;
      }
    };
    if constexpr (kDiag) {
      // The diagonal block is the item's first: O and l are still zero, so the row max is taken
      // without a rescale.
      m_used = fmaxf(m_used, row_max() * scale);
      make_p();
    } else {
      make_p();
      asm volatile("" ::"v"(pb[0]), "v"(pb[1]), "v"(pb[2]), "v"(pb[3]), "v"(pb[4]), "v"(pb[5]),
                   "v"(pb[6]), "v"(pb[7]));
      if (__builtin_expect(__any(!(pblk <= kSpecSum)), 0)) {
        rescale(fmaxf(m_used, row_max() * scale));
        make_p();
      }
    }
    l_part += pblk;

    USAGI_WAIT_VM(0);  // V(j) has landed
    if constexpr (kBf16) {
      // bf16 inputs: this wave turns its own 8 KiB of the V tile (the rows its DMA wrote) into
      // fp16 in place before the barrier publishes the tile, so P·V runs on fp16 P and fp16 V as
      // the reference's does (v7:107). Element positions do not matter: every 16-bit value is
      // converted where it lies.
      char* slice = (char*)v_lds + wave * 8192 + lane * 16;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        u32x4 x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = *(const u32x4*)(slice + (4 * h + i) * 1024);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int w = 0; w < 4; ++w) x[i][w] = bf16x2_to_f16x2(x[i][w]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) *(u32x4*)(slice + (4 * h + i) * 1024) = x[i];
      }
    }
    USAGI_BARRIER();   // every wave is done reading K(j); V(j) is complete
    const char* kt_src = kNext ? tile_k(key_block(j + 1)) : nullptr;

    __builtin_amdgcn_s_setprio(1);
    // ---- O^T += V^T · P^T (32 MFMAs, V operands 2 ahead)
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        // Diagonal: k-step s holds keys 16s .. 16s+15, all above wave w's rows when s > 2w + 1.
        if (kDiag && s > 2 * wave + 1) continue;
        const char* vb = v_rd + 16 * (4 * (u ^ tq) + t_x) + s * 4096;
        const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)vb);
        const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vb + 2048));
        const half8 va = __builtin_shufflevector(__builtin_bit_cast(half4, lo),
                                                 __builtin_bit_cast(half4, hi), 0, 1, 2, 3, 4, 5, 6, 7);
        o_acc[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb[s], o_acc[u], 0, 0, 0);
      }
      // K(j+1) DMA pieces between the P·V MFMAs (the K buffer is free after the barrier).
      if constexpr (kNext) dma_piece(kt_src, k_off, k_dst, s);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_s_setprio(0);
    // No closing barrier: the next block's first barrier orders every wave's reads of this V
    // tile before the DMA of the next one, which is issued after it.
  };

  using T_ = std::true_type;
  using F_ = std::false_type;
  // Off-diagonal blocks use the kMaskQ form even when every query row is valid (the masking
  // branch is then skipped for the whole wave): separate full-block copies of the block body
  // push the register allocation of the whole kernel into spills.
  if (n_off > 0) {
    block(T_{}, T_{}, T_{}, -1);
    for (int j = 0; j < n_off - 1; ++j) block(F_{}, T_{}, T_{}, j);
    block(F_{}, T_{}, F_{}, n_off - 1);
  } else {
    block(T_{}, T_{}, F_{}, -1);
  }

  const float l_tot = wave_pair_sum(l_part);
  float inv = l_tot > 0.0f ? 1.0f / l_tot : 1.0f;
  if (!qvalid) inv = 0.0f;
  // O: normalise, stage this wave's 32 rows in its 8 KiB slice of the K tile and store whole
  // 256-byte rows (1 KiB contiguous per instruction); written straight from the accumulator
  // layout, each store instruction would touch 32 rows with 8 bytes each. The last block DMA'd
  // no K tile and every wave finished reading its K at that block's second barrier, so the
  // K tile is free.
  {
    char* stage = (char*)k_lds + wave * 8192;  // 32 rows x 256 B, chunk c at c ^ (row % 16)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        u32x2 wv;
        // Rows past seq_len were computed on whatever their Q holds: select, never multiply.
        float ov[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[e] = qvalid ? o_acc[u][4 * g + e] * inv : 0.0f;
        wv[0] = (uint32_t)to_out_bits(ov[0], kBf16) | ((uint32_t)to_out_bits(ov[1], kBf16) << 16);
        wv[1] = (uint32_t)to_out_bits(ov[2], kBf16) | ((uint32_t)to_out_bits(ov[3], kBf16) << 16);
        // d = 32u + 8g + 4lh .. +3: 16-byte chunk 4u + g, half lh.
        *(u32x2*)(stage + li * 256 + 16 * ((4 * u + g) ^ (li & 15)) + 8 * lh) = wv;
      }
    }
    // Only this wave's rows: LDS operations of one wave complete in order, no barrier.
    uint16_t* oblk = a.o + base + (size_t)(q0 + 32 * wave) * kHd;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = 4 * i + (lane >> 4);
      const int c = lane & 15;
      const u32x4 x = *(const u32x4*)(stage + row * 256 + 16 * (c ^ (row & 15)));
      *(u32x4*)(oblk + (size_t)row * kHd + 8 * c) = x;
    }
  }
  if (a.lse && lh == 0) {
    const float lse = (qvalid && l_tot > 0.0f) ? (m_used + log2f(l_tot)) * kLn2 : -INFINITY;
    a.lse[(size_t)bh * a.T + qrow] = lse;
  }
}

// ---------------------------------------------------------------------------------------------
// fp16 split kernel: one workgroup per CU (4 waves, one per SIMD), K/V double-buffered in LDS.
//
// Wave w = (rw, cw) = (w / 2, w % 2) owns query rows 64 rw .. 64 rw + 63 and keys
// 64 cw .. 64 cw + 63 of every key block. Every K or V^T operand a wave reads from LDS feeds two
// MFMAs (one per 32-row query fragment f), so LDS reads per FLOP are half of the 32-row layout.
// The two waves of a row pair keep separate online-softmax states over their key halves; the
// states are merged once, in the epilogue (m = max, O and l rescaled by 2^(m_i - m)).
//
// Tiles: stage s holds K and V of one key block (2 x 32 KiB); the DMA of block p+1 goes to the
// other stage during block p, so each tile is requested a whole block ahead. One barrier per
// block. Inside a block each wave works in 32-key sub-tiles t:
//   QK(t0) [16 MFMAs, next block's 16 DMA pieces between them]
//   QK(t1) [16 MFMAs] alongside exp2 of sub-tile 0 computed with the running max
//   row max over the 64 keys; if it grew by more than 2^8 anywhere (rare after the first block):
//   rescale O, l and recompute sub-tile 0's P
//   PV(t0) [16 MFMAs] alongside exp2 of sub-tile 1
//   PV(t1) [16 MFMAs]
// The diagonal block goes first (non-speculative, causally masked; waves with cw > rw have no
// key at or before any of their query rows there and skip it).
// Query rows at or past seq_len are computed like the others and written as O = 0, LSE = -inf
// at the end: off-diagonal keys and causally visible diagonal keys of a valid row are all before
// seq_len, so no other mask is needed.
// ---------------------------------------------------------------------------------------------

// Multiplies an MFMA accumulator that lives in AGPRs by alpha, in place. Written with AGPR
// operands so the compiler never copies the accumulators into VGPRs for it: a plain multiply on
// a rarely taken path makes it read all of them out of the AGPRs on every loop iteration.
__device__ __forceinline__ void scale_acc_agpr(floatx16& acc, float alpha) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    float x = acc[r];
    float t;
    asm volatile(
        "v_accvgpr_read_b32 %1, %0\n\t"
        "v_mul_f32 %1, %1, %2\n\t"
        "v_accvgpr_write_b32 %0, %1"
        : "+a"(x), "=&v"(t)
        : "v"(alpha));
    acc[r] = x;
  }
}

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void bsa_fwd_split_kernel(Args a) {
  __shared__ __attribute__((aligned(1024))) uint16_t lds[4 * kBlk * kHd];  // [stage][K | V]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rw = wave >> 1;
  const int cw = wave & 1;
  const int li = lane & 31;
  const int lh = lane >> 5;

  int qb, bh;
  item_coords(a, blockIdx.x, qb, bh);
  const size_t base = (size_t)bh * a.T * kHd;
  constexpr size_t kTileBytes = (size_t)kBlk * kHd * 2;
  auto tile_k = [&](int kb) { return (const char*)(a.k + base) + (size_t)kb * kTileBytes; };
  auto tile_v = [&](int kb) { return (const char*)(a.v + base) + (size_t)kb * kTileBytes; };

  // DMA: wave w moves tile rows 32w .. 32w+31 (8 x 1 KiB), swizzled as in bsa_fwd_dma_kernel.
  const int dma_r = lane >> 4;
  const int dma_pc = lane & 15;
  uint32_t k_off[4];
  uint32_t v_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    k_off[i] = (uint32_t)((32 * wave + dma_r) * 256 + 16 * (dma_pc ^ (4 * i + dma_r)));
    v_off[i] = (uint32_t)((32 * wave + dma_r) * 256 + 16 * (dma_pc ^ (4 * dma_r)));
  }
  const uint32_t lds0 = lds_addr_of(lds);
  auto k_dst = [&](int stage) {
    return __builtin_amdgcn_readfirstlane(lds0 + 65536u * stage + wave * 8192);
  };
  auto v_dst = [&](int stage) {
    return __builtin_amdgcn_readfirstlane(lds0 + 65536u * stage + 32768u + wave * 8192);
  };

  dma_tile8(tile_k(qb), k_off, k_dst(0));
  dma_tile8(tile_v(qb), v_off, v_dst(0));

  const int seq_len = a.seq_lens ? a.seq_lens[bh / a.heads] : a.T;
  const int q0 = qb * kBlk;
  if (q0 >= seq_len) {
    uint16_t* out_blk = a.o + base + (size_t)q0 * kHd;
#pragma unroll
    for (int i = 0; i < (kBlk * kHd) / (8 * kThreads); ++i) {
      *(u32x4*)(out_blk + (size_t)(i * kThreads + tid) * 8) = u32x4{0, 0, 0, 0};
    }
    if (a.lse && tid < kBlk) a.lse[(size_t)bh * a.T + q0 + tid] = -INFINITY;
    USAGI_WAIT_VM(0);
    return;
  }

  // Q^T fragments (MFMA B operand): qf[f][s] = Q[q0 + 64 rw + 32 f + li][16 s + 8 lh .. +8].
  u32x4 qf[2][8];
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    const uint16_t* qp = a.q + base + (size_t)(q0 + 64 * rw + 32 * f + li) * kHd + 8 * lh;
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[f][s] = *(const u32x4*)(qp + 16 * s);
  }

  const int32_t* rp = a.row_ptr + (size_t)bh * (a.nqb + 1) + qb;
  int rs = rp[0];
  int re = rp[1];
  rs = min(max(rs, 0), a.max_nnz);
  re = min(max(re, rs), a.max_nnz);
  const int n_off = max(re - rs - 1, 0);
  const int32_t* cols = a.col_idx + (size_t)bh * a.max_nnz + rs;
  const int nqb_m1 = a.nqb - 1;
  int col_chunk = 0;
  int colv = lane < n_off ? cols[lane] : 0;
  auto key_block = [&](int j) -> int {
    const int c = j >> 6;
    if (c != col_chunk) {
      col_chunk = c;
      const int e = c * 64 + lane;
      colv = e < n_off ? cols[e] : 0;
    }
    const int kb = __builtin_amdgcn_readlane(colv, j & 63);
    return min(max(kb, 0), nqb_m1);
  };

  auto dma_piece = [&](const char* tile, const uint32_t off[4], uint32_t dst, int i) {
    const char* src = tile + (i >= 4 ? 4096 : 0);
    const uint32_t l = dst + (i >= 4 ? 4096 : 0);
    switch (i & 3) {
      case 0: dma_16b<0>(src, off[0], l); break;
      case 1: dma_16b<1024>(src, off[1], l); break;
      case 2: dma_16b<2048>(src, off[2], l); break;
      default: dma_16b<3072>(src, off[3], l); break;
    }
  };

  // LDS read addresses (bytes, relative to a stage): K operand rows 64 cw + 32 t + li, logical
  // chunk 2 s + lh at physical chunk (2 s + lh) ^ (li % 16).
  const int k_rd = (64 * cw + li) * 256;
  const int k_x = lh ^ (li & 15);
  // V^T operand via transpose reads (as in bsa_fwd_dma_kernel), global k-step S = 4 cw + 2 t + s2.
  const int tq = (lane & 15) >> 2;
  const int t_x = 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
  const int v_rd = 32768 + (4 * lh + tq) * 256 + 8 * (lane & 1) + cw * 4 * 4096;
  const char* lds_c = (const char*)lds;

  floatx16 o_acc[4][2];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
#pragma unroll
    for (int f = 0; f < 2; ++f) {
#pragma unroll
      for (int r = 0; r < 16; ++r) o_acc[u][f][r] = 0.0f;
    }
  }
  float m_used[2] = {-1e30f, -1e30f};
  float l_part[2] = {0.0f, 0.0f};
  const float scale = a.qk_scale;

  auto k_op = [&](int stage, int t, int s) -> u32x4 {
    return *(const u32x4*)(lds_c + stage * 65536 + k_rd + t * 8192 + 16 * ((2 * s) ^ k_x));
  };
  auto v_op = [&](int stage, int t, int s2, int u) -> half8 {
    const char* vb = lds_c + stage * 65536 + v_rd + 16 * (4 * (u ^ tq) + t_x) + (2 * t + s2) * 4096;
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)vb);
    const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vb + 2048));
    return __builtin_shufflevector(__builtin_bit_cast(half4, lo), __builtin_bit_cast(half4, hi),
                                   0, 1, 2, 3, 4, 5, 6, 7);
  };
  // P of sub-tile t as two k-steps x two query fragments (MFMA B operands).
  auto exp_tile = [&](const floatx16 (&s)[2], half8 (&p)[2][2]) {
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const float neg_m = -m_used[f];
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          p[s2][f][e] = (_Float16)__builtin_amdgcn_exp2f(fmaf(s[f][8 * s2 + e], scale, neg_m));
        }
      }
    }
  };
  auto psum = [&](const half8 (&p)[2][2]) {
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      float acc = l_part[f];
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const half2 pp = {p[s2][f][2 * e], p[s2][f][2 * e + 1]};
          acc = __builtin_amdgcn_fdot2(pp, half2{1.0f16, 1.0f16}, acc, false);
        }
      }
      l_part[f] = acc;
    }
  };
  auto qk_tile = [&](int stage, int t, floatx16 (&s)[2]) {
#pragma unroll
    for (int f = 0; f < 2; ++f) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[f][r] = 0.0f;
    }
#pragma unroll
    for (int ss = 0; ss < 8; ++ss) {
      const u32x4 ka = k_op(stage, t, ss);
      s[0] = mfma_qk<false>(ka, qf[0][ss], s[0]);
      s[1] = mfma_qk<false>(ka, qf[1][ss], s[1]);
    }
  };
  auto pv_tile = [&](int stage, int t, const half8 (&p)[2][2]) {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const half8 va = v_op(stage, t, s2, u);
        o_acc[u][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, p[s2][0], o_acc[u][0], 0, 0, 0);
        o_acc[u][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, p[s2][1], o_acc[u][1], 0, 0, 0);
      }
    }
  };
  auto tile_max = [&](const floatx16& s) {
    float mx = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
    return mx;
  };

  // vmcnt(0): Q, the column chunk and the diagonal tiles have landed.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  USAGI_BARRIER();

  // ---- the diagonal block (stage 0); the first off-diagonal block's tiles go to stage 1.
  if (n_off > 0) {
    const int kb = key_block(0);
    dma_tile8(tile_k(kb), k_off, k_dst(1));
    dma_tile8(tile_v(kb), v_off, v_dst(1));
  }
  if (cw <= rw) {
    floatx16 s0[2], s1[2];
    qk_tile(0, 0, s0);
    qk_tile(0, 1, s1);
    if (cw == rw) {
#pragma unroll
      for (int f = 0; f < 2; ++f) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = 8 * (r >> 2) + 4 * lh + (r & 3);
          if (key > 32 * f + li) s0[f][r] = -INFINITY;
          if (32 + key > 32 * f + li) s1[f][r] = -INFINITY;
        }
      }
    }
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const float mx = wave_pair_max(fmaxf(tile_max(s0[f]), tile_max(s1[f])));
      m_used[f] = fmaxf(m_used[f], mx * scale);
    }
    half8 p0[2][2], p1[2][2];
    exp_tile(s0, p0);
    exp_tile(s1, p1);
    pv_tile(0, 0, p0);
    pv_tile(0, 1, p1);
    psum(p0);
    psum(p1);
  }

  // ---- off-diagonal blocks: processing index p = 1 .. n_off is CSR entry p - 1, stage p % 2.
  //
  // The body is written as explicit steps separated by scheduling fences
  // (__builtin_amdgcn_sched_barrier(0)): each step issues the LDS operand read two steps ahead,
  // its MFMAs, and a chunk of VALU work that does not depend on them, so the matrix core runs
  // while the wave computes exponentials. Without the fences the compiler groups all DMAs, all
  // reads and all MFMAs and sinks the speculative exponentials past the rescale test.
  int koff[8];
#pragma unroll
  for (int ss = 0; ss < 8; ++ss) koff[ss] = k_rd + 16 * ((2 * ss) ^ k_x);
  int voff[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) voff[u] = v_rd + 16 * (4 * (u ^ tq) + t_x);

  // Four elements of sub-tile sv (chunk c = 0..7: query fragment c / 4, elements 4 (c % 4) ..)
  // -> fp16 P with the running max as it stands, and their row sum into sum[f].
  auto exp_chunk = [&](const floatx16 (&sv)[2], half8 (&p)[2][2], float (&sum)[2], int c) {
    const int f = c >> 2;
    const int j0 = 4 * (c & 3);
    const int s2 = j0 >> 3;
    const int e0 = j0 & 7;
    const float neg_m = -m_used[f];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      p[s2][f][e0 + e] = (_Float16)__builtin_amdgcn_exp2f(fmaf(sv[f][j0 + e], scale, neg_m));
    }
    float acc = sum[f];
    acc = __builtin_amdgcn_fdot2(half2{p[s2][f][e0], p[s2][f][e0 + 1]}, half2{1.0f16, 1.0f16}, acc, false);
    acc = __builtin_amdgcn_fdot2(half2{p[s2][f][e0 + 2], p[s2][f][e0 + 3]}, half2{1.0f16, 1.0f16}, acc, false);
    sum[f] = acc;
  };
  // A sub-tile's P was computed with the running max as it stands. Every P is <= the lane's
  // fp32 sum of its 16 P values, so a sum <= 2^12 proves all of them finite in fp16 and the
  // speculation good (and it is, for almost every block after the first). Otherwise (rare) take
  // the exact row max of the sub-tile, move the running max to it, rescale O and l, and
  // recompute the sub-tile's P and sum. Then the sum joins l.
  auto check = [&](const floatx16 (&sv)[2], half8 (&p)[2][2], float (&sum)[2]) {
    // The speculative P is consumed here, so the compiler cannot sink its computation past the
    // branch (into the common path after the MFMAs it was meant to overlap).
    asm volatile("" ::"v"(p[0][0]), "v"(p[0][1]), "v"(p[1][0]), "v"(p[1][1]));
    const bool big = !(sum[0] <= kSpecSum) || !(sum[1] <= kSpecSum);
    if (__builtin_expect(__any(big), 0)) {
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const float mx = wave_pair_max(tile_max(sv[f]));
        const float m_new = fmaxf(m_used[f], mx * scale);
        const float alpha = __builtin_amdgcn_exp2f(m_used[f] - m_new);
        m_used[f] = m_new;
        l_part[f] *= alpha;
#pragma unroll
        for (int u = 0; u < 4; ++u) scale_acc_agpr(o_acc[u][f], alpha);
      }
      exp_tile(sv, p);
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        float acc = 0.0f;
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
#pragma unroll
          for (int e = 0; e < 8; e += 2) {
            acc = __builtin_amdgcn_fdot2(half2{p[s2][f][e], p[s2][f][e + 1]}, half2{1.0f16, 1.0f16}, acc, false);
          }
        }
        sum[f] = acc;
      }
    }
    l_part[0] += sum[0];
    l_part[1] += sum[1];
  };

  auto block = [&](auto next_tag, int p) {
    constexpr bool kNext = decltype(next_tag)::value;
    const int stage = p & 1;
    USAGI_WAIT_VM(0);  // this wave's share of block p's tiles has landed
    USAGI_BARRIER();   // every share has landed; every wave is done with block p - 1
    const char* nk = nullptr;
    const char* nv = nullptr;
    uint32_t nkd = 0, nvd = 0;
    if constexpr (kNext) {
      const int kb = key_block(p);
      nk = tile_k(kb);
      nv = tile_v(kb);
      nkd = k_dst(stage ^ 1);
      nvd = v_dst(stage ^ 1);
    }
    const char* st_base = lds_c + stage * 65536;
    auto kread = [&](int t, int ss) -> u32x4 {
      return *(const u32x4*)(st_base + koff[ss] + t * 8192);
    };
    auto vread = [&](int t, int s2, int u) -> half8 {
      const char* vb = st_base + voff[u] + (2 * t + s2) * 4096;
      const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)vb);
      const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(vb + 2048));
      return __builtin_shufflevector(__builtin_bit_cast(half4, lo), __builtin_bit_cast(half4, hi),
                                     0, 1, 2, 3, 4, 5, 6, 7);
    };
    floatx16 s0[2], s1[2];
#pragma unroll
    for (int f = 0; f < 2; ++f) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s0[f][r] = 0.0f;
        s1[f][r] = 0.0f;
      }
    }

    // A: QK(t0) with the next block's K tile DMA (one 1 KiB piece per two MFMAs).
    u32x4 kA = kread(0, 0);
    u32x4 kB = kread(0, 1);
    USAGI_FENCE();
#pragma unroll
    for (int ss = 0; ss < 8; ++ss) {
      const u32x4 kN = ss < 6 ? kread(0, ss + 2) : kread(1, ss - 6);
      s0[0] = mfma_qk<false>(kA, qf[0][ss], s0[0]);
      if constexpr (kNext) dma_piece(nk, k_off, nkd, ss);
      s0[1] = mfma_qk<false>(kA, qf[1][ss], s0[1]);
      kA = kB;
      kB = kN;
      USAGI_FENCE();
    }

    // B: QK(t1) with sub-tile 0's P (speculative: the running max as it stands) and row sums.
    half8 p0[2][2];
    float sum0[2] = {0.0f, 0.0f};
#pragma unroll
    for (int ss = 0; ss < 8; ++ss) {
      u32x4 kN = kB;
      if (ss < 6) kN = kread(1, ss + 2);
      s1[0] = mfma_qk<false>(kA, qf[0][ss], s1[0]);
      exp_chunk(s0, p0, sum0, ss);
      s1[1] = mfma_qk<false>(kA, qf[1][ss], s1[1]);
      kA = kB;
      kB = kN;
      USAGI_FENCE();
    }
    check(s0, p0, sum0);

    // D: PV(t0) with sub-tile 1's P and row sums.
    half8 p1[2][2];
    float sum1[2] = {0.0f, 0.0f};
    half8 vA = vread(0, 0, 0);
    half8 vB = vread(0, 0, 1);
    USAGI_FENCE();
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int s2 = i >> 2;
      const int u = i & 3;
      const half8 vN = i < 6 ? vread(0, (i + 2) >> 2, (i + 2) & 3) : vread(1, 0, i - 6);
      o_acc[u][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vA, p0[s2][0], o_acc[u][0], 0, 0, 0);
      exp_chunk(s1, p1, sum1, i);
      o_acc[u][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vA, p0[s2][1], o_acc[u][1], 0, 0, 0);
      vA = vB;
      vB = vN;
      USAGI_FENCE();
    }
    check(s1, p1, sum1);

    // E: PV(t1) with the next block's V tile DMA (one piece per two MFMAs).
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int s2 = i >> 2;
      const int u = i & 3;
      half8 vN = vB;
      if (i < 6) vN = vread(1, (i + 2) >> 2, (i + 2) & 3);
      o_acc[u][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vA, p1[s2][0], o_acc[u][0], 0, 0, 0);
      if constexpr (kNext) dma_piece(nv, v_off, nvd, i);
      o_acc[u][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vA, p1[s2][1], o_acc[u][1], 0, 0, 0);
      vA = vB;
      vB = vN;
      USAGI_FENCE();
    }
  };

  using T_ = std::true_type;
  using F_ = std::false_type;
  for (int p = 1; p < n_off; ++p) block(T_{}, p);
  if (n_off > 0) block(F_{}, n_off);

  // ---- epilogue: merge the two key halves of each row pair, normalise, store.
  USAGI_BARRIER();  // every wave is done with the tiles; the LDS is reused below
  float l_tot[2];
#pragma unroll
  for (int f = 0; f < 2; ++f) l_tot[f] = wave_pair_sum(l_part[f]);
  // Wave (rw, cw) keeps d-tiles u = 2 cw, 2 cw + 1 and hands the other two to its partner:
  // region (rw, cw) = 16 KiB at 32 KiB rw + 16 KiB cw, float index (i * 64 + lane) with
  // i = ((u % 2) * 2 + f) * 16 + r; m and l at 64 KiB + 1 KiB (2 rw + cw).
  {
    // (register arrays are only ever indexed with compile-time indices: a run-time index would
    // move o_acc to scratch memory)
    float* xo = (float*)(lds_c + rw * 32768 + cw * 16384);
#pragma unroll
    for (int uu = 0; uu < 2; ++uu) {
#pragma unroll
      for (int f = 0; f < 2; ++f) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          xo[((uu * 2 + f) * 16 + r) * 64 + lane] = cw ? o_acc[uu][f][r] : o_acc[2 + uu][f][r];
        }
      }
    }
    float* xm = (float*)(lds_c + 65536 + 1024 * (2 * rw + cw));
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      xm[f * 64 + lane] = m_used[f];
      xm[128 + f * 64 + lane] = l_tot[f];
    }
  }
  USAGI_BARRIER();
  const float* po = (const float*)(lds_c + rw * 32768 + (1 - cw) * 16384);
  const float* pm = (const float*)(lds_c + 65536 + 1024 * (2 * rw + (1 - cw)));
  float inv[2], a0[2], a1[2], m_fin[2], l_fin[2];
  bool qv[2];
#pragma unroll
  for (int f = 0; f < 2; ++f) {
    const float mp = pm[f * 64 + lane];
    const float lp = pm[128 + f * 64 + lane];
    const float mn = fmaxf(m_used[f], mp);
    a0[f] = __builtin_amdgcn_exp2f(m_used[f] - mn);
    a1[f] = __builtin_amdgcn_exp2f(mp - mn);
    const float l = l_tot[f] * a0[f] + lp * a1[f];
    m_fin[f] = mn;
    l_fin[f] = l;
    qv[f] = q0 + 64 * rw + 32 * f + li < seq_len;
    inv[f] = l > 0.0f ? 1.0f / l : 1.0f;
  }
  // Stage this wave's 64 rows x 64 d (128 B per row) at 72 KiB + 8 KiB wave, 16-byte chunk c of
  // row r at c ^ (r % 8); then store whole 128-byte row halves.
  char* stage_o = (char*)lds_c + 73728 + wave * 8192;
#pragma unroll
  for (int uu = 0; uu < 2; ++uu) {
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const int row = 32 * f + li;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g + e;
          // Rows past seq_len were computed on whatever their Q holds: select, never multiply.
          const float own = cw ? o_acc[2 + uu][f][r] : o_acc[uu][f][r];
          const float x = (own * a0[f] + po[((uu * 2 + f) * 16 + r) * 64 + lane] * a1[f]) * inv[f];
          v[e] = qv[f] ? x : 0.0f;
        }
        u32x2 wv;
        wv[0] = (uint32_t)to_out_bits(v[0], false) | ((uint32_t)to_out_bits(v[1], false) << 16);
        wv[1] = (uint32_t)to_out_bits(v[2], false) | ((uint32_t)to_out_bits(v[3], false) << 16);
        const int chunk = 4 * uu + g;  // d_local = 32 uu + 8 g + 4 lh
        *(u32x2*)(stage_o + row * 128 + 16 * (chunk ^ (row & 7)) + 8 * lh) = wv;
      }
    }
  }
  // Only this wave's rows: LDS operations of one wave complete in order, no barrier.
  uint16_t* oblk = a.o + base + (size_t)(q0 + 64 * rw) * kHd + 64 * cw;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = 8 * i + (lane >> 3);
    const int c = lane & 7;
    const u32x4 x = *(const u32x4*)(stage_o + row * 128 + 16 * (c ^ (row & 7)));
    *(u32x4*)(oblk + (size_t)row * kHd + 8 * c) = x;
  }
  if (a.lse && cw == 0 && lh == 0) {
#pragma unroll
    for (int f = 0; f < 2; ++f) {
      const int qrow = q0 + 64 * rw + 32 * f + li;
      const float lse = (qv[f] && l_fin[f] > 0.0f) ? (m_fin[f] + log2f(l_fin[f])) * kLn2 : -INFINITY;
      a.lse[(size_t)bh * a.T + qrow] = lse;
    }
  }
}


thread_local char g_err[512] = "";

// USAGI_BSA_FP16_KERNEL selects the kernel for A/B runs, read on every call: "dma" (default,
// fp16 and bf16), "split" (fp16 only; bf16 inputs stay on "dma") or "staged" (the
// register-staged kernel, fp16 and bf16).
int fp16_kernel() {
  const char* e = getenv("USAGI_BSA_FP16_KERNEL");
  if (e && strcmp(e, "staged") == 0) return 2;
  if (e && strcmp(e, "split") == 0) return 0;
  return 1;
}

// USAGI_BSA_ORDER=rows forces the longest-row-first grid order (A/B runs); default: head-major
// per XCD whenever B*H is a multiple of 8.
int item_order() {
  const char* e = getenv("USAGI_BSA_ORDER");
  return (e && strcmp(e, "rows") == 0) ? 0 : 1;
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

}  // namespace

extern "C" const char* usagi_bsa_version(void) { return "usagi_bsa 0.1.0 gfx950"; }

extern "C" const char* usagi_bsa_last_error(void) { return g_err; }

namespace {

// Checks shared by both forward entry points; fills the fields of `a` they have in common.
int prepare(Args& a, const void* q, const void* k, const void* v, const int32_t* seq_lens,
            void* out, float* lse, int32_t batch, int32_t heads, int32_t seq_len,
            int32_t head_dim, int32_t dtype) {
  if (!q || !k || !v || !out) return fail(USAGI_BSA_EINVAL, "null tensor pointer");
  if (dtype != USAGI_BSA_FP16 && dtype != USAGI_BSA_BF16)
    return fail(USAGI_BSA_EDTYPE, "unknown dtype code %d", (int)dtype);
  if (head_dim != kHd) return fail(USAGI_BSA_EHEADDIM, "head_dim must be %d, got %d", kHd, (int)head_dim);
  if (seq_len <= 0 || seq_len % kBlk != 0)
    return fail(USAGI_BSA_ESEQ, "T must be a positive multiple of %d, got %d", kBlk, (int)seq_len);
  if (batch <= 0 || heads <= 0) return fail(USAGI_BSA_EINVAL, "batch and heads must be positive");
  const long long bh = (long long)batch * heads;
  const long long nqb = seq_len / kBlk;
  if (bh * nqb > 0x7fffffffLL || bh > 0x7fffffffLL / ((long long)seq_len * kHd) ||
      bh * (nqb + 1) > 0x7fffffffLL)
    return fail(USAGI_BSA_EINVAL, "problem too large");
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.o = static_cast<uint16_t*>(out);
  a.lse = lse;
  a.row_ptr = nullptr;
  a.col_idx = nullptr;
  a.seq_lens = seq_lens;
  a.heads = heads;
  a.T = seq_len;
  a.nqb = (int)nqb;
  a.bh_count = (int)bh;
  a.max_nnz = 0;
  a.qk_scale = (float)(1.4426950408889634 / sqrt((double)kHd));
  a.head_major = (bh % 8 == 0 && item_order() != 0) ? 1 : 0;
  a.window = 0;
  a.n_global = 0;
  return USAGI_BSA_OK;
}

int launched() {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail((int)err, "kernel launch failed: %s", hipGetErrorString(err));
  return USAGI_BSA_OK;
}

}  // namespace

extern "C" int usagi_bsa_fwd(const void* q, const void* k, const void* v,
                             const int32_t* row_ptr, const int32_t* col_idx,
                             const int32_t* seq_lens, void* out, float* lse, int32_t batch,
                             int32_t heads, int32_t seq_len, int32_t head_dim, int32_t max_nnz,
                             int32_t dtype, void* stream) {
  g_err[0] = '\0';
  Args a;
  const int rc = prepare(a, q, k, v, seq_lens, out, lse, batch, heads, seq_len, head_dim, dtype);
  if (rc != USAGI_BSA_OK) return rc;
  if (!row_ptr) return fail(USAGI_BSA_EINVAL, "null tensor pointer");
  if (max_nnz < 0 || (max_nnz > 0 && !col_idx))
    return fail(USAGI_BSA_EINVAL, "max_nnz must be >= 0 and col_idx non-null when max_nnz > 0");
  if ((long long)a.bh_count * (long long)max_nnz > 0x7fffffffLL * 4LL)
    return fail(USAGI_BSA_EINVAL, "problem too large");
  a.row_ptr = row_ptr;
  a.col_idx = col_idx;
  a.max_nnz = max_nnz;

  const dim3 grid((unsigned)((long long)a.bh_count * a.nqb));
  const dim3 block(kThreads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == USAGI_BSA_BF16) {
    if (fp16_kernel() == 2) {
      hipLaunchKernelGGL(bsa_fwd_kernel<true>, grid, block, 0, s, a);
    } else {
      hipLaunchKernelGGL((bsa_fwd_dma_kernel<true, false>), grid, block, 0, s, a);
    }
  } else if (fp16_kernel() == 2) {
    hipLaunchKernelGGL(bsa_fwd_kernel<false>, grid, block, 0, s, a);
  } else if (fp16_kernel() == 1) {
    hipLaunchKernelGGL((bsa_fwd_dma_kernel<false, false>), grid, block, 0, s, a);
  } else {
    hipLaunchKernelGGL(bsa_fwd_split_kernel, grid, block, 0, s, a);
  }
  return launched();
}

extern "C" int usagi_bsa_fwd_window(const void* q, const void* k, const void* v,
                                    int32_t window, int32_t n_global, const int32_t* seq_lens,
                                    void* out, float* lse, int32_t batch, int32_t heads,
                                    int32_t seq_len, int32_t head_dim, int32_t dtype,
                                    void* stream) {
  g_err[0] = '\0';
  Args a;
  const int rc = prepare(a, q, k, v, seq_lens, out, lse, batch, heads, seq_len, head_dim, dtype);
  if (rc != USAGI_BSA_OK) return rc;
  if (window < 1) return fail(USAGI_BSA_EINVAL, "window must be >= 1, got %d", (int)window);
  if (n_global < 0) return fail(USAGI_BSA_EINVAL, "n_global must be >= 0, got %d", (int)n_global);
  a.window = window;
  a.n_global = n_global;

  const dim3 grid((unsigned)((long long)a.bh_count * a.nqb));
  const dim3 block(kThreads);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == USAGI_BSA_BF16) {
    hipLaunchKernelGGL((bsa_fwd_dma_kernel<true, true>), grid, block, 0, s, a);
  } else {
    hipLaunchKernelGGL((bsa_fwd_dma_kernel<false, true>), grid, block, 0, s, a);
  }
  return launched();
}

extern "C" int usagi_bsa_check_csr(const int32_t* row_ptr, const int32_t* col_idx, int32_t batch,
                                   int32_t heads, int32_t num_q_blocks, int32_t max_nnz) {
  g_err[0] = '\0';
  if (!row_ptr || batch <= 0 || heads <= 0 || num_q_blocks <= 0 || max_nnz < 0 ||
      (max_nnz > 0 && !col_idx))
    return fail(USAGI_BSA_EINVAL, "bad arguments");
  const int64_t bh_count = (int64_t)batch * heads;
  for (int64_t bh = 0; bh < bh_count; ++bh) {
    const int32_t* rp = row_ptr + bh * (num_q_blocks + 1);
    const int32_t* ci = col_idx ? col_idx + bh * (int64_t)max_nnz : nullptr;
    const int b = (int)(bh / heads), h = (int)(bh % heads);
    if (rp[0] != 0) return fail(USAGI_BSA_ECSR, "(b=%d,h=%d): row_ptr[0]=%d, expected 0", b, h, rp[0]);
    if (rp[num_q_blocks] > max_nnz)
      return fail(USAGI_BSA_ECSR, "(b=%d,h=%d): row_ptr[%d]=%d exceeds max_nnz=%d", b, h,
                  num_q_blocks, rp[num_q_blocks], max_nnz);
    for (int qb = 0; qb < num_q_blocks; ++qb) {
      const int rs = rp[qb], re = rp[qb + 1];
      if (re <= rs)
        return fail(USAGI_BSA_ECSR, "(b=%d,h=%d,qb=%d): empty or decreasing row (%d..%d)", b, h,
                    qb, rs, re);
      for (int j = rs; j < re; ++j) {
        const int kb = ci[j];
        if (kb < 0 || kb > qb)
          return fail(USAGI_BSA_ECSR, "(b=%d,h=%d,qb=%d): key block %d outside [0, %d]", b, h,
                      qb, kb, qb);
        if (j > rs && kb <= ci[j - 1])
          return fail(USAGI_BSA_ECSR, "(b=%d,h=%d,qb=%d): col_idx not strictly ascending", b, h, qb);
      }
      if (ci[re - 1] != qb)
        return fail(USAGI_BSA_ECSR, "(b=%d,h=%d,qb=%d): last entry %d is not the diagonal", b, h,
                    qb, ci[re - 1]);
    }
  }
  return USAGI_BSA_OK;
}
