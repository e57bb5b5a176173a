// Host-side half of libusagi_bsa.so: the error state, the CSR validator and the work planner.
//
// The planner decides which workgroup slot runs which (b*h, query block) item. The GPU deals
// workgroup slots to its 8 XCDs round-robin (slot s runs on XCD s % 8), and each XCD hands its
// slots to its own 32 CUs in slot order as they free up. The kernel's built-in order
// (item_coords in bsa_fwd.hip) gives every XCD the same number of items, which balances the
// chip only when every head costs the same; with rows whose lengths vary by head (e.g. a mix of
// window and retrieval heads) whole XCDs finish early. The plan gives every XCD the same total
// work instead, keeps each XCD on a few heads at a time (their K/V tiles stay in its L2), and
// orders each XCD's items longest row first, so its CUs finish together.

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <algorithm>
#include <numeric>
#include <vector>

#include "bsa_internal.h"
#include "usagi_bsa.h"

namespace {

thread_local char g_err[512] = "";

constexpr int kXcds = 8;
// Fixed cost of one item in units of one key block: its prologue (Q, CSR row, first K tile)
// and epilogue (O and LSE stores) take about as long as one and a half off-diagonal blocks.
constexpr double kItemOverhead = 1.5;
// The built-in order is kept when its most loaded XCD carries at most this much more than the
// mean.
constexpr double kKeepImbalance = 1.02;

// Key blocks one item walks: its row's entries, with the implicit diagonal of the CSR walk
// (kernels/v7_blockptr_warpspec.py:83-136) counted once whatever the row holds.
int item_blocks(const int32_t* rp, int qb, bool generic) {
  const int n = std::max(rp[qb + 1] - rp[qb], 0);
  return generic ? n : std::max(n - 1, 0) + 1;
}

// The kernel's built-in order (item_coords in bsa_fwd.hip): slot -> item b*h*nqb + qb.
int builtin_item(int slot, int bh_count, int nqb) {
  if (bh_count % kXcds == 0) {
    const int x = slot % kXcds;
    const int j = slot / kXcds;
    const int hl = j / nqb;
    const int qb = nqb - 1 - (j - hl * nqb);
    return (x + kXcds * hl) * nqb + qb;
  }
  const int qslot = slot / bh_count;
  const int qb = nqb - 1 - qslot;
  const int bh = slot - qslot * bh_count;
  return bh * nqb + qb;
}

}  // namespace

int usagi_bsa_fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void usagi_bsa_clear_error(void) { g_err[0] = '\0'; }

extern "C" const char* usagi_bsa_last_error(void) { return g_err; }

extern "C" int usagi_bsa_check_csr(const int32_t* row_ptr, const int32_t* col_idx,
                                   const int32_t* seq_lens, int32_t batch, int32_t heads,
                                   int32_t num_q_blocks, int32_t max_nnz) {
  usagi_bsa_clear_error();
  if (!row_ptr || batch <= 0 || heads <= 0 || num_q_blocks <= 0 || max_nnz < 0 ||
      (max_nnz > 0 && !col_idx))
    return usagi_bsa_fail(USAGI_BSA_EINVAL, "bad arguments");
  const int64_t bh_count = (int64_t)batch * heads;
  // seen[kb] == stamp: key block kb already listed in the row being checked.
  std::vector<int64_t> seen(num_q_blocks, -1);
  int64_t stamp = 0;
  for (int64_t bh = 0; bh < bh_count; ++bh) {
    const int32_t* rp = row_ptr + bh * (num_q_blocks + 1);
    const int32_t* ci = col_idx ? col_idx + bh * (int64_t)max_nnz : nullptr;
    const int b = (int)(bh / heads), h = (int)(bh % heads);
    // Rows of query blocks that start at or past seq_len are never read by the walk (their
    // output is O = 0, LSE = -inf: kernels/v7_blockptr_warpspec.py:63-67), so they may hold
    // anything; only the rows before them are checked.
    int n_rows = num_q_blocks;
    if (seq_lens) {
      const int64_t sl = seq_lens[b];
      n_rows = sl <= 0 ? 0
                     : (int)std::min<int64_t>(num_q_blocks,
                                              (sl + USAGI_BSA_BLOCK - 1) / USAGI_BSA_BLOCK);
    }
    if (n_rows > 0 && rp[0] != 0)
      return usagi_bsa_fail(USAGI_BSA_ECSR, "(b=%d,h=%d): row_ptr[0]=%d, expected 0", b, h, rp[0]);
    for (int qb = 0; qb < n_rows; ++qb, ++stamp) {
      const int rs = rp[qb], re = rp[qb + 1];
      if (re <= rs)
        return usagi_bsa_fail(USAGI_BSA_ECSR, "(b=%d,h=%d,qb=%d): empty or decreasing row (%d..%d)",
                              b, h, qb, rs, re);
      if (re > max_nnz)
        return usagi_bsa_fail(USAGI_BSA_ECSR, "(b=%d,h=%d,qb=%d): row_ptr %d exceeds max_nnz=%d",
                              b, h, qb, re, max_nnz);
      if (ci[re - 1] != qb)
        return usagi_bsa_fail(USAGI_BSA_ECSR, "(b=%d,h=%d,qb=%d): last entry %d is not the diagonal",
                              b, h, qb, ci[re - 1]);
      for (int j = rs; j < re - 1; ++j) {
        const int kb = ci[j];
        if (kb < 0 || kb >= qb)
          return usagi_bsa_fail(USAGI_BSA_ECSR,
                                "(b=%d,h=%d,qb=%d): entry %d before the diagonal outside [0, %d)", b,
                                h, qb, kb, qb);
        if (seen[kb] == stamp)
          return usagi_bsa_fail(USAGI_BSA_ECSR, "(b=%d,h=%d,qb=%d): key block %d listed twice", b,
                                h, qb, kb);
        seen[kb] = stamp;
      }
    }
  }
  return USAGI_BSA_OK;
}

extern "C" int usagi_bsa_plan(const int32_t* row_ptr, int32_t batch, int32_t heads,
                              int32_t num_q_blocks, int32_t generic, int32_t* sched,
                              int32_t sched_cap) {
  usagi_bsa_clear_error();
  if (!row_ptr || !sched || batch <= 0 || heads <= 0 || num_q_blocks <= 0)
    return usagi_bsa_fail(USAGI_BSA_EINVAL, "bad arguments");
  const int64_t bh_count = (int64_t)batch * heads;
  const int64_t n_items = bh_count * num_q_blocks;
  if (n_items > 0x3fffffffLL) return usagi_bsa_fail(USAGI_BSA_EINVAL, "problem too large");
  if (sched_cap < USAGI_BSA_PLAN_CAP(n_items))
    return usagi_bsa_fail(USAGI_BSA_EINVAL, "sched_cap %d below USAGI_BSA_PLAN_CAP(%lld) = %lld",
                          (int)sched_cap, (long long)n_items,
                          (long long)USAGI_BSA_PLAN_CAP(n_items));
  const int G = (int)n_items;
  const int nqb = num_q_blocks;
  std::vector<double> cost(G);
  double total = 0.0;
  for (int64_t bh = 0; bh < bh_count; ++bh) {
    const int32_t* rp = row_ptr + bh * (nqb + 1);
    for (int qb = 0; qb < nqb; ++qb) {
      const double c = item_blocks(rp, qb, generic != 0) + kItemOverhead;
      cost[bh * nqb + qb] = c;
      total += c;
    }
  }
  const double mean = total / kXcds;

  // Load of each XCD under the built-in order.
  double load[kXcds] = {0};
  for (int s = 0; s < G; ++s) load[s % kXcds] += cost[builtin_item(s, (int)bh_count, nqb)];
  if (*std::max_element(load, load + kXcds) <= kKeepImbalance * mean) return 0;

  // Items head by head, each head's longest rows first (ties: later query block first).
  std::vector<int> seq(G);
  std::iota(seq.begin(), seq.end(), 0);
  std::stable_sort(seq.begin(), seq.end(), [&](int x, int y) {
    const int hx = x / nqb, hy = y / nqb;
    if (hx != hy) return hx < hy;
    if (cost[x] != cost[y]) return cost[x] > cost[y];
    return x > y;
  });
  // Cut that sequence into 8 runs of equal cost, each run one XCD's queue.
  std::vector<int> cut(kXcds + 1, 0);
  cut[kXcds] = G;
  {
    double prefix = 0.0;
    int p = 0;
    for (int x = 1; x < kXcds; ++x) {
      const double target = mean * x;
      while (p < G && prefix + cost[seq[p]] <= target) prefix += cost[seq[p++]];
      // Take the item that straddles the target too if that lands nearer to it.
      if (p < G && prefix + cost[seq[p]] - target < target - prefix) prefix += cost[seq[p++]];
      cut[x] = std::max(p, cut[x - 1]);
    }
  }
  int longest = 0;
  for (int x = 0; x < kXcds; ++x) longest = std::max(longest, cut[x + 1] - cut[x]);
  std::vector<std::vector<int>> queue(kXcds);
  if ((int64_t)kXcds * longest <= USAGI_BSA_PLAN_CAP(n_items)) {
    for (int x = 0; x < kXcds; ++x) {
      queue[x].assign(seq.begin() + cut[x], seq.begin() + cut[x + 1]);
      // Longest rows first within the XCD; equal rows stay head by head.
      std::stable_sort(queue[x].begin(), queue[x].end(),
                       [&](int a, int b) { return cost[a] > cost[b]; });
    }
  } else {
    // Heads too unequal for equal-cost runs within the slot budget: deal the items, longest
    // first, to the XCDs in a snake order (equal counts, near-equal cost, no head locality).
    std::vector<int> order(seq);
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return cost[a] > cost[b]; });
    for (int i = 0; i < G; ++i) {
      const int r = i / kXcds, c = i % kXcds;
      queue[(r & 1) ? kXcds - 1 - c : c].push_back(order[i]);
    }
    longest = 0;
    for (int x = 0; x < kXcds; ++x) longest = std::max(longest, (int)queue[x].size());
  }
  const int n_slots = kXcds * longest;
  for (int s = 0; s < n_slots; ++s) {
    const int x = s % kXcds, r = s / kXcds;
    sched[s] = r < (int)queue[x].size() ? queue[x][r] : -1;
  }
  return n_slots;
}
