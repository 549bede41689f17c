// CPU simulation of the chunked-prefill kernel's stream-K schedule
// (miniserve_amd/csrc/pf_streamk.h and the task loop of prefill_mfma.h): for random task
// sizes and workgroup counts, every workgroup's segment loop is run as the kernel runs it,
// and the result is checked (each task's entry in the list is a head of `head` positions
// that hold no work, then its pairs):
//   - every pair position is taken by exactly one share, no head position by any;
//   - a task covered by one share is written whole (no partial), and the fold launch
//     skips it (its first and last contributors are one share);
//   - a split task's partial slots are exactly the slots the fold launch reads, each slot
//     is written once in the launch, and the number of its partials is the contributor
//     count the fold reads (l_hi - l_lo + 1, more than one).
// Built with g++ and run by tests/test_pf_streamk.py:
//   pf_streamk_sim <trials> <mode>   mode 1 plants a mistake: shares = groups unclamped.
// Prints "violations trials_with_splits" and exits 0.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <set>
#include <vector>

#include "pf_streamk.h"

int main(int argc, char** argv) {
  const long trials = argc > 1 ? std::atol(argv[1]) : 20000;
  const int mode = argc > 2 ? std::atoi(argv[2]) : 0;
  std::mt19937_64 rng(31337);
  auto pick = [&](long lo, long hi) { return lo + static_cast<long>(rng() % (hi - lo + 1)); };
  long violations = 0, with_splits = 0;
  for (long tr = 0; tr < trials; ++tr) {
    const int ntasks = static_cast<int>(pick(1, 300));
    std::vector<int> P(ntasks + 1, 0);
    const int kind = static_cast<int>(pick(0, 2));
    const int head = static_cast<int>(pick(0, 4));
    for (int t = 0; t < ntasks; ++t) {
      const int c = kind == 0 ? 1 : static_cast<int>(kind == 1 ? pick(1, 4) : pick(1, 200));
      P[t + 1] = P[t] + head + c;
    }
    const int total = P[ntasks];
    const int groups = static_cast<int>(pick(1, 320));
    const int shares = mode == 1 ? groups : msattn::pf_sk_shares(groups, total);
    std::vector<int> taken(total, 0), full(ntasks, 0), parts(ntasks, 0);
    std::vector<std::vector<int>> written(ntasks);
    std::vector<int> slot_writes(2 * groups, 0);
    bool split = false;
    for (int l = 0; l < groups; ++l) {
      int rb = 0, re = 0;
      if (mode == 1) {
        if (l < shares) {
          rb = static_cast<int>(static_cast<int64_t>(l) * total / shares);
          re = static_cast<int>(static_cast<int64_t>(l + 1) * total / shares);
        }
      } else {
        msattn::pf_sk_range(l, total, shares, &rb, &re);
      }
      int lo = 0, hi = ntasks;
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (P[mid] <= rb) lo = mid;
        else hi = mid;
      }
      for (int t = lo, seg = 0;; ++t, ++seg) {
        if (t >= ntasks || rb >= re) break;
        const int p0 = P[t] + head, p1 = P[t + 1];
        if (p0 >= re) break;
        const int it_lo = rb > p0 ? rb - p0 : 0;
        const int it_hi = std::min(re, p1) - p0;
        for (int x = p0 + it_lo; x < p0 + it_hi; ++x) taken[x]++;
        if (it_lo == 0 && it_hi == p1 - p0) {
          full[t]++;
        } else {
          const int slot = 2 * l + (seg == 0 ? 0 : 1);
          written[t].push_back(slot);
          slot_writes[slot]++;
          parts[t]++;
          split = true;
        }
      }
    }
    with_splits += split;
    for (int t = 0; t < ntasks; ++t)
      for (int x = P[t]; x < P[t + 1]; ++x) violations += taken[x] != (x >= P[t] + head ? 1 : 0);
    for (int s : slot_writes) violations += s > 1;
    for (int t = 0; t < ntasks; ++t) {
      if (full[t]) {
        violations += full[t] != 1 || !written[t].empty();
        // the fold launch's test: one contributor, nothing to fold
        violations += msattn::pf_sk_owner(P[t] + head, total, shares) !=
                      msattn::pf_sk_owner(P[t + 1] - 1, total, shares);
        continue;
      }
      if (written[t].empty()) {  // nobody wrote this task's output
        ++violations;
        continue;
      }
      const int l_lo = msattn::pf_sk_owner(P[t] + head, total, shares);
      const int l_hi = msattn::pf_sk_owner(P[t + 1] - 1, total, shares);
      if (parts[t] != l_hi - l_lo + 1 || l_lo == l_hi) ++violations;  // a part unread, or none folded
      std::set<int> reads;
      for (int l = l_lo; l <= l_hi; ++l) reads.insert(msattn::pf_sk_partial_slot(l, P[t], total, shares));
      const std::set<int> wrote(written[t].begin(), written[t].end());
      if (reads != wrote) ++violations;
      for (int s : reads) violations += s < 0 || s >= 2 * groups;
    }
  }
  std::printf("%ld %ld\n", violations, with_splits);
  return 0;
}
