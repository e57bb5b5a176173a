/*
 * usagi_bsa.h — C ABI of the MI355X (gfx950) block-sparse causal attention forward.
 *
 * The reference exposes this path only as a Python submission module whose timed call is
 *   block_sparse_attn_fwd(q, k, v, row_ptr, col_idx, seq_lens) -> (O, LSE)
 * (kernels/v7_blockptr_warpspec.py:251-252), which flattens to [B*H, T, D] and launches one
 * Triton program per (query block, b*h) (kernels/v7_blockptr_warpspec.py:155-191). The entry
 * points below replace that launch (and the ctypes cuLaunchKernel hop of
 * kernels/v1_baseline.py:93-128) with plain pointers and sizes: no torch types cross the
 * boundary, and the library allocates no device memory.
 *
 * Conventions
 *   - All tensor pointers are borrowed device pointers. Inputs are never written.
 *   - q, k, v, out: contiguous [B, H, T, 128] of `dtype` (fp16, or bf16 with fp16 P·V).
 *   - row_ptr: int32 [B, H, T/128 + 1]; values are offsets local to each (b, h) row of col_idx
 *     (kernels/v7_blockptr_warpspec.py:77-80).
 *   - col_idx: int32 [B, H, max_nnz]; row qb lists key blocks in
 *     col_idx[b, h, row_ptr[qb] : row_ptr[qb+1]] with the diagonal (kb == qb) as the LAST entry
 *     (the reference's rows are ascending; distinct blocks below qb in any order before the
 *     diagonal give the same result). The diagonal is processed implicitly and causally masked;
 *     entries before it are processed unmasked (kernels/v7_blockptr_warpspec.py:83-136).
 *   - seq_lens: int32 [B] or NULL (NULL: every sequence has length T). Query rows at or past
 *     seq_len get O = 0 and LSE = -inf (kernels/v7_blockptr_warpspec.py:63-67, 138-148).
 *   - lse: float32 [B, H, T], natural-log log-sum-exp of the scaled scores, or NULL to skip.
 *   - sched / n_slots: an optional work plan from usagi_bsa_plan (device copy of its int32 array
 *     and its return value), or NULL / 0 for the kernel's built-in order. Any plan of the same
 *     CSR gives bit-identical results: it only decides which GPU slot runs which query block.
 *   - stream: a hipStream_t (NULL = the default stream). The launch is asynchronous.
 *   - Kernel: calls without seq_lens whose rows hold at most 4 key blocks on average
 *     (max_nnz <= 4 * T/128, or the analytic pattern's own count) run a software-pipelined
 *     kernel; other calls, and every call when USAGI_BSA_PIPE=0 is set in the environment, run
 *     the two-phase kernel (USAGI_BSA_PIPE=1 makes every call without seq_lens on CSR or
 *     analytic rows use the pipelined one; read at each launch). Both meet the same parity
 *     bound; between them results can differ in the last bits.
 *   - Return: 0 on success; a negative USAGI_BSA_E* code for a rejected argument; a positive
 *     hipError_t value when the HIP runtime reports an error. usagi_bsa_last_error() gives a
 *     message for the calling thread's last failure.
 */
#ifndef USAGI_BSA_H
#define USAGI_BSA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define USAGI_BSA_BLOCK 128
#define USAGI_BSA_HEAD_DIM 128
/* Capacity of the sched array usagi_bsa_plan needs for B*H*(T/128) items. */
#define USAGI_BSA_PLAN_CAP(n_items) (2 * (int64_t)(n_items) + 8)

enum usagi_bsa_dtype {
  USAGI_BSA_FP16 = 0, /* fp16 q/k/v/out (the build's contract) */
  USAGI_BSA_BF16 = 1  /* bf16 q/k/v/out, fp16 P·V (kernels/v7_blockptr_warpspec.py:107) */
};

enum usagi_bsa_status {
  USAGI_BSA_OK = 0,
  USAGI_BSA_EINVAL = -1,   /* a null pointer or an out-of-range size */
  USAGI_BSA_EDTYPE = -2,   /* unknown dtype code */
  USAGI_BSA_EHEADDIM = -3, /* head_dim != 128 */
  USAGI_BSA_ESEQ = -4,     /* T is not a positive multiple of 128 */
  USAGI_BSA_ECSR = -5      /* malformed CSR (usagi_bsa_check_csr only) */
};

/* Forward pass. Replaces _run_csr + the _fwd_csr launch,
 * kernels/v7_blockptr_warpspec.py:155-191 (same in kernels/v4_leaderboard_0740ms.py:143-179). */
int usagi_bsa_fwd(const void* q, const void* k, const void* v,
                  const int32_t* row_ptr, const int32_t* col_idx, const int32_t* seq_lens,
                  void* out, float* lse,
                  int32_t batch, int32_t heads, int32_t seq_len, int32_t head_dim,
                  int32_t max_nnz, int32_t dtype, const int32_t* sched, int32_t n_slots,
                  void* stream);

/* Forward pass with the generic CSR walk of kernels/v1_baseline.py:331-406 (launched by its
 * _run_csr, v1:411-441): every entry of a row is attended, in any order, with no implicit
 * diagonal; an entry equal to the query block takes the causal mask, keys at or past seq_len
 * are masked, and an empty row (or a row of fully masked entries) gives O = 0 and LSE = -inf.
 * Entries are clamped to [0, T/128) for memory safety. Same arguments and conventions as
 * usagi_bsa_fwd (a plan for it comes from usagi_bsa_plan with generic = 1). */
int usagi_bsa_fwd_generic(const void* q, const void* k, const void* v,
                          const int32_t* row_ptr, const int32_t* col_idx,
                          const int32_t* seq_lens, void* out, float* lse,
                          int32_t batch, int32_t heads, int32_t seq_len, int32_t head_dim,
                          int32_t max_nnz, int32_t dtype, const int32_t* sched,
                          int32_t n_slots, void* stream);

/* Forward pass over an analytic pattern instead of a CSR: query block qb attends the global
 * prefix 0 .. n_global-1 and the window max(0, qb-window+1) .. qb (deduplicated; the diagonal is
 * causally masked), with no row_ptr / col_idx reads. Same tensors, dtype, seq_lens, lse, stream
 * and return conventions as usagi_bsa_fwd; the result equals usagi_bsa_fwd on the CSR of that
 * pattern. Replaces the analytic kernels _fwd_window (window only) and _fwd_window_global of
 * kernels/v1_baseline.py:141-322. window >= 1, n_global >= 0. */
int usagi_bsa_fwd_window(const void* q, const void* k, const void* v,
                         int32_t window, int32_t n_global, const int32_t* seq_lens,
                         void* out, float* lse,
                         int32_t batch, int32_t heads, int32_t seq_len, int32_t head_dim,
                         int32_t dtype, void* stream);

/* Host-side CSR validator over HOST copies of row_ptr / col_idx (and of seq_lens, int32 [B], or
 * NULL for all T); no counterpart in the reference, which does not validate its input
 * (kernels/v7_blockptr_warpspec.py:155-191). It checks the preconditions under which the
 * implicit-diagonal walk of kernels/v7_blockptr_warpspec.py:83-136 equals block-mask ∧ causal
 * attention: row_ptr[0] == 0, every row non-empty and within max_nnz, its last entry == qb, and
 * the entries before it distinct and in [0, qb) (in any order: the walk's result does not depend
 * on it). Rows of query blocks starting at or past seq_len[b] are not checked: the walk never
 * reads them (kernels/v7_blockptr_warpspec.py:63-67). Returns 0, or USAGI_BSA_ECSR with the
 * first offending (b, h, qb) in usagi_bsa_last_error(). */
int usagi_bsa_check_csr(const int32_t* row_ptr, const int32_t* col_idx, const int32_t* seq_lens,
                        int32_t batch, int32_t heads, int32_t num_q_blocks, int32_t max_nnz);

/* Work plan over a HOST copy of row_ptr; no counterpart in the reference, whose grid is
 * (nqb, B*H) in index order (kernels/v7_blockptr_warpspec.py:178-179). When rows of different
 * heads differ in length, it spreads the work evenly over the GPU's 8 XCDs (each XCD on a few
 * heads at a time, its longest rows first) and writes the slot -> item table (item
 * b*H*nqb + h*nqb + qb, or -1 for an idle slot) to sched[0 .. n_slots). generic: 1 plans for
 * usagi_bsa_fwd_generic, 0 for usagi_bsa_fwd. sched_cap >= USAGI_BSA_PLAN_CAP(B*H*nqb).
 * Returns n_slots (> 0), 0 when the built-in order is already balanced (launch with sched
 * NULL), or a negative USAGI_BSA_E* code. */
int usagi_bsa_plan(const int32_t* row_ptr, int32_t batch, int32_t heads, int32_t num_q_blocks,
                   int32_t generic, int32_t* sched, int32_t sched_cap);

/* Timing hook for benchmarks; no counterpart in the reference. The calling thread's next
 * forward launch (any usagi_bsa_fwd* entry point) records start_event when its kernel starts
 * and stop_event when it completes (hipExtLaunchKernel's events, attached to the dispatch
 * itself), so their elapsed time is the kernel's own duration, without the launch gap and event
 * packets that events recorded around the call include. hipEvent_t handles created with timing,
 * either may be NULL. The setting is used up by the thread's next forward call, whether that call
 * launches or rejects its arguments, so it never attaches to a later launch. Returns 0. */
int usagi_bsa_time_next_launch(void* start_event, void* stop_event);

/* Version string of this library, e.g. "usagi_bsa 0.2.0 gfx950". No counterpart in the
 * reference (its module has no version). */
const char* usagi_bsa_version(void);

/* Message for the calling thread's most recent nonzero return ("" if none). Stands in for the
 * reference's exceptions: the RuntimeError carrying the driver's code at
 * kernels/v1_baseline.py:126-128 (the Triton versions raise from the JIT launch). */
const char* usagi_bsa_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* USAGI_BSA_H */
