// Work split of the chunked-prefill kernel's stream-K schedule, kept free of HIP types so
// that host code (a CPU test) runs the same arithmetic as the kernel.
//
// The work list is every task's key-step pairs, tasks in order: task t holds positions
// [P_t, P_t+1) (P = exclusive prefix sums of the tasks' pair counts, each count >= 1), and
// `total` = P_ntasks. The launch has `groups` workgroups; `shares` = min(groups, total) of
// them each take the contiguous positions [floor(l total / shares), floor((l + 1) total /
// shares)) (share l), so every share holds at least one position and the shares holding
// a task's positions are consecutive. A share's part of a task that does not cover the
// whole task is stored as a partial at slot 2 l + (0 if it is the share's first task, 1
// if its last), and the task's last contributor to take the ticket folds them.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define MSATTN_SK_HD __host__ __device__
#else
#define MSATTN_SK_HD
#endif

namespace msattn {

MSATTN_SK_HD inline int pf_sk_shares(int groups, int total) {
  return groups < total ? groups : total;
}

// Share l's positions [begin, end); empty for l >= shares.
MSATTN_SK_HD inline void pf_sk_range(int l, int total, int shares, int* begin, int* end) {
  if (l >= shares || shares <= 0) {
    *begin = *end = 0;
    return;
  }
  *begin = static_cast<int>(static_cast<int64_t>(l) * total / shares);
  *end = static_cast<int>(static_cast<int64_t>(l + 1) * total / shares);
}

// The share holding position x (0 <= x < total): the largest l with l total / shares <= x.
MSATTN_SK_HD inline int pf_sk_owner(int x, int total, int shares) {
  return static_cast<int>((static_cast<int64_t>(x + 1) * shares - 1) / total);
}

// The slot of share l's partial of the task whose entry in the list (its head included)
// starts at position p0: its first task's slot unless the share began in an earlier task.
MSATTN_SK_HD inline int pf_sk_partial_slot(int l, int p0, int total, int shares) {
  const bool began_before = static_cast<int64_t>(l) * total / shares < p0;
  return 2 * l + (began_before ? 1 : 0);
}

}  // namespace msattn
