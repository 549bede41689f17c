// Where a merged row's split-K partials sit in a workspace: the index arithmetic of the
// merge kernel (merge.hip), kept free of HIP types so that host code can run it too.
//
// The partials kernels record their layout in the workspace header (split_kernel.h):
//   kind 0 (partition kernels): row r owns slots r * max_parts .. + max_parts - 1, closed
//     by an end marker;
//   kind 1 (stream-K decode): words [1] sumT, [2] chunk c, [4] UG, [6] B, [7] RT, and the
//     per-sequence tile prefix sums pb = P_b, pe = P_{b+1}; decode row (b, h) lies in unit
//     u = ((h % G) / RT) * KVH + h / G, unit group ug = u / UG, lane ul = u % UG, and its
//     segment spans work-list positions [ug * sumT + pb, ug * sumT + pe), cut into chunks
//     of c; the chunk r holding a piece of it stored that piece at slot
//     ((r + ug * B + b) * UG + ul) * RT + (h % G) % RT.
// A header that does not describe a layout of this workspace (another geometry wrote it,
// or it was never written) must not send the merge outside the workspace: every header
// word is checked, and the count of slots is clamped so that the last slot read,
// base + (n - 1) * stride, stays below `slots`, the workspace's slot count. Words that
// describe no layout give n = 0 (the row has no partials and merges to zeros).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define MSATTN_HD __host__ __device__
#else
#define MSATTN_HD
#endif

namespace msattn {

// Largest unit group and row tile a stream-K layout uses (waves per workgroup, query rows
// per MFMA tile); a header claiming more describes no layout of this library.
constexpr int kSlotsMaxUG = 64;
constexpr int kSlotsMaxRT = 16;

struct SlotRange {
  int64_t base;    // slot of the row's first partial
  int64_t stride;  // slots between consecutive partials
  int64_t n;       // partials to read (0: none)
  bool markers;    // the partials end at the first end marker (kind 0)
};

// Slots [base, base + (n - 1) * stride] clamped into [0, slots).
MSATTN_HD inline SlotRange clamp_slots(SlotRange s, int64_t slots) {
  if (s.n <= 0 || s.base < 0 || s.stride <= 0 || s.base >= slots) {
    s.n = 0;
    return s;
  }
  const int64_t fit = (slots - 1 - s.base) / s.stride + 1;  // partials with a slot below `slots`
  if (s.n > fit) s.n = fit;
  return s;
}

// The partials of output row `row` (decode row b * H + h) under the layout of header
// words hv[0..7] and the row's prefix entries pb, pe (stream-K only), for a workspace of
// `slots` slots whose partition layout has max_parts slots per row. kind_hint 0: the
// caller knows the partition layout was used (the header is not read).
MSATTN_HD inline SlotRange merge_slot_range(const int* hv, int pb, int pe, int64_t row,
                                            int batch, int H, int KVH, int G, int max_parts,
                                            int64_t slots, int kind_hint) {
  SlotRange s{0, 1, 0, false};
  if (batch <= 0 || H <= 0 || KVH <= 0 || G <= 0 || row < 0) return s;
  const int kind = kind_hint == 0 ? 0 : hv[0];
  if (kind == 0) {
    s.markers = true;
    s.base = row * max_parts;
    s.n = max_parts;
    return clamp_slots(s, slots);
  }
  if (kind != 1) return s;  // no layout this merge reads (kind 2 merged in-kernel)
  const int sumT = hv[1], c = hv[2], UG = hv[4], B = hv[6], RT = hv[7];
  if (c <= 0 || UG <= 0 || UG > kSlotsMaxUG || RT <= 0 || RT > kSlotsMaxRT || B != batch ||
      sumT < 0 || pb < 0 || pe <= pb || pe > sumT)
    return s;
  const int64_t b = row / H;
  if (b >= batch) return s;
  const int h = static_cast<int>(row - b * H);
  const int kvh = h / G;
  const int gi = h - kvh * G;
  const int64_t unit = static_cast<int64_t>(gi / RT) * KVH + kvh;
  const int64_t ug = unit / UG;
  const int64_t ul = unit - ug * UG;
  const int64_t seg_start = ug * sumT + pb;  // < 2^62: ug < 2^31, sumT and pb < 2^31
  const int64_t r0 = seg_start / c;
  // Every slot of the row is at least its first piece id, so a piece id past the slots
  // means none is in the workspace (and keeps the products below in range).
  const int64_t piece = r0 + ug * B + b;
  if (piece >= slots) return s;
  s.n = (seg_start + (pe - pb) - 1) / c - r0 + 1;
  s.base = (piece * UG + ul) * RT + gi % RT;
  s.stride = static_cast<int64_t>(UG) * RT;
  return clamp_slots(s, slots);
}

}  // namespace msattn
