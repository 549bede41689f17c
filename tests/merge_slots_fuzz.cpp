// CPU fuzz of merge_slot_range (miniserve_amd/csrc/merge_slots.h), the slot arithmetic of
// the merge kernel: whatever the workspace header and a row's prefix entries hold, every
// slot it names lies in [0, slots). Built with g++ and run by tests/test_merge_slots.py.
//
//   merge_slots_fuzz <iterations> <mode>
// mode 0 checks merge_slot_range; mode 1 checks a copy without the final clamp (a planted
// mistake the fuzz must catch). Prints "violations nonempty" and exits 0.
#include <climits>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <random>

#include "merge_slots.h"

namespace {

std::mt19937_64 rng(20260);

int64_t pick(int64_t lo, int64_t hi) {  // uniform in [lo, hi]
  return lo + static_cast<int64_t>(rng() % static_cast<uint64_t>(hi - lo + 1));
}

// A header word: small values (the range real layouts use), boundary values and noise.
int word() {
  switch (pick(0, 5)) {
    case 0: return static_cast<int>(pick(-4, 64));
    case 1: return static_cast<int>(pick(0, 1 << 20));
    case 2: return INT_MAX - static_cast<int>(pick(0, 3));
    case 3: return INT_MIN + static_cast<int>(pick(0, 3));
    case 4: return static_cast<int>(pick(-(1 << 20), 1 << 20));
    default: return static_cast<int>(static_cast<uint32_t>(rng()));
  }
}

// merge_slot_range without its last clamp_slots call (kind 1), for the planted check.
msattn::SlotRange unclamped(const int* hv, int pb, int pe, int64_t row, int batch, int H,
                            int KVH, int G, int max_parts, int64_t slots, int kind_hint) {
  msattn::SlotRange s = msattn::merge_slot_range(hv, pb, pe, row, batch, H, KVH, G, max_parts,
                                                 slots, kind_hint);
  if (kind_hint == 0 || hv[0] != 1 || s.n == 0) return s;
  const int sumT = hv[1], c = hv[2], UG = hv[4], RT = hv[7];
  const int64_t b = row / H;
  const int h = static_cast<int>(row - b * H);
  const int kvh = h / G, gi = h - kvh * G;
  const int64_t unit = static_cast<int64_t>(gi / RT) * KVH + kvh;
  const int64_t seg_start = unit / UG * sumT + pb;
  s.n = (seg_start + (pe - pb) - 1) / c - seg_start / c + 1;
  return s;
}

}  // namespace

int main(int argc, char** argv) {
  const long iters = argc > 1 ? std::atol(argv[1]) : 1000000;
  const int mode = argc > 2 ? std::atoi(argv[2]) : 0;
  long violations = 0, nonempty = 0;
  for (long it = 0; it < iters; ++it) {
    const int batch = static_cast<int>(pick(1, 300));
    const int KVH = static_cast<int>(pick(1, 16));
    const int G = static_cast<int>(pick(1, 16));
    const int H = KVH * G;
    const int max_parts = static_cast<int>(pick(1, 600));
    const int64_t rows = static_cast<int64_t>(batch) * H;
    int64_t slots;
    switch (pick(0, 3)) {
      case 0: slots = rows * max_parts; break;
      case 1: slots = pick(0, 64); break;
      case 2: slots = pick(0, rows * max_parts); break;
      default: slots = pick(0, int64_t(1) << 40); break;
    }
    int hv[8];
    for (int& w : hv) w = word();
    switch (pick(0, 3)) {  // kind: mostly the two layouts the merge reads
      case 0: hv[0] = 0; break;
      case 1:
      case 2: hv[0] = 1; break;
      default: break;
    }
    if (pick(0, 1)) hv[6] = batch;  // a header of this batch, so the stream-K branch runs
    if (pick(0, 1)) {               // plausible unit groups and row tiles
      hv[4] = static_cast<int>(pick(1, 8));
      hv[7] = static_cast<int>(pick(1, 16));
    }
    int pb = word(), pe = word();
    if (pick(0, 1)) {  // an ordered pair of entries below sumT
      const int sumT = hv[1] > 0 ? hv[1] : 1;
      pb = static_cast<int>(pick(0, sumT - 1));
      pe = static_cast<int>(pick(pb, sumT));
    }
    const int64_t row = pick(0, rows + 8);
    const int kind_hint = pick(0, 4) == 0 ? 0 : -1;
    const msattn::SlotRange s =
        mode == 0 ? msattn::merge_slot_range(hv, pb, pe, row, batch, H, KVH, G, max_parts, slots,
                                             kind_hint)
                  : unclamped(hv, pb, pe, row, batch, H, KVH, G, max_parts, slots, kind_hint);
    if (s.n <= 0) continue;
    ++nonempty;
    const __int128 last = static_cast<__int128>(s.base) +
                          static_cast<__int128>(s.n - 1) * static_cast<__int128>(s.stride);
    if (s.base < 0 || s.stride <= 0 || last >= slots) ++violations;
  }
  std::printf("%ld %ld\n", violations, nonempty);
  return 0;
}
