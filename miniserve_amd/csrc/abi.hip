// C ABI of libmsattn.so (declared in include/msattn.h): argument checks,
// partition policy and kernel dispatch. No exception crosses this boundary.
#include <cmath>
#include <cstdint>

#include <algorithm>
#include <atomic>
#include <mutex>

#include "decode_mfma.h"
#include "decode_streamk.h"
#include "prefill_mfma.h"
#include "kernels.h"
#include "msattn.h"

namespace {

using namespace msattn;

// Partition sizes, largest first: a launch takes the largest that reaches kTargetSlots
// workgroups, else the smallest. The smallest serves the small, latency-bound decodes
// (C1: 4 sequences of at most 512 tokens), where more, shorter workgroups shorten the
// launch; every choice holds a whole number of 16-token tiles per MFMA wave.
constexpr int kPartitionChoices[] = {kPartMax, kPartMax / 2, kPartMax / 4, kPartMax / 8};
static_assert(kPartMax / 8 >= 16 * kMfmaWaves && (kPartMax / 8) % (16 * kMfmaWaves) == 0,
              "every partition choice splits into whole tiles per wave");
#ifndef MSATTN_TARGET_SLOTS
#define MSATTN_TARGET_SLOTS 512
#endif
constexpr int64_t kTargetSlots = MSATTN_TARGET_SLOTS;  // workgroup slots wanted in a launch
#ifndef MSATTN_STREAMK_MIN_TILES
#define MSATTN_STREAMK_MIN_TILES 65536
#endif
#ifndef MSATTN_STREAMK_MIN_TILES_D64
#define MSATTN_STREAMK_MIN_TILES_D64 131072
#endif
// Decode launches whose (batch x KV heads x table tiles) reach this use stream-K, below it
// the partition kernel. Measured on 40 shapes (graph steps, both kernels on each): at
// head_dim 128, stream-K was 12-25 % faster from 65,536 tiles up (bf16, fp8, fp32 caches;
// H32/KVH8 and H28/KVH4), level or 10 % slower only where the contexts fill little of
// the table (16 log-uniform 1-8k contexts: 41.3 against 37.3 us); at head_dim 64
// (H14/KVH2) the partition kernel stays 9-14 % faster up to 98,304 tiles and stream-K
// wins from 131,072 (5-14 %). At 49,152 tiles the two are level.
constexpr int64_t kStreamKMinTiles = MSATTN_STREAMK_MIN_TILES;
constexpr int64_t kStreamKMinTilesD64 = MSATTN_STREAMK_MIN_TILES_D64;
// The same for a 16-bit query over an fp8 cache at 8 rows per tile (G = 5..8), where
// stream-K's two waves per SIMD win from 65,536 tiles (37.0 against 44.3 us for 64 x
// H14/KVH2 at 2-8k tokens); below it the partition kernel does (11.8 against 20.4 us).
#ifndef MSATTN_STREAMK_MIN_TILES_FP8_RT8
#define MSATTN_STREAMK_MIN_TILES_FP8_RT8 65536
#endif
constexpr int64_t kStreamKMinTilesFp8Rt8 = MSATTN_STREAMK_MIN_TILES_FP8_RT8;
#ifndef MSATTN_FUSED_MERGE
#define MSATTN_FUSED_MERGE 1
#endif
// 1: msattn_paged_attention's partition-kernel decodes merge in-kernel (no merge launch).
constexpr bool kFusedMerge = MSATTN_FUSED_MERGE != 0;
#ifndef MSATTN_FUSED_APPEND
#define MSATTN_FUSED_APPEND 1
#endif
// 1: msattn_paged_attention_append writes the new K/V rows inside the partition decode
// launch; 0: always a write_kv launch, then the decode.
constexpr bool kFusedAppend = MSATTN_FUSED_APPEND != 0;

int write_kv_impl(void* k_cache, void* v_cache, int64_t cache_block_stride,
                  int64_t cache_slot_stride, int64_t cache_head_stride, const void* k,
                  const void* v, const int32_t* block_table, const int32_t* starts,
                  int start_offset, int batch, int tokens, int num_kv_heads, int head_dim,
                  int block_size, int num_blocks, int table_width, int src_dtype, int kv_dtype,
                  void* stream);
#ifndef MSATTN_WIDE_ROUTE
#define MSATTN_WIDE_ROUTE 1
#endif
#ifndef MSATTN_WIDE_SLOTS_PCT
#define MSATTN_WIDE_SLOTS_PCT 100
#endif
// 1: long-context decodes with few (sequence, KV head) pairs take the wide partition
// shape; its partitions are sized for kWideSlotsPct percent of a workgroup per CU.
constexpr bool kWideRoute = MSATTN_WIDE_ROUTE != 0;
constexpr int kWideSlotsPct = MSATTN_WIDE_SLOTS_PCT;
#ifndef MSATTN_WIDE_MAX_PCT
#define MSATTN_WIDE_MAX_PCT 150
#endif
// The wide shape only when its launch holds at most this percentage of the aimed-for
// workgroups (two 8-wave workgroups on one CU run one after the other).
constexpr int kWideMaxPct = MSATTN_WIDE_MAX_PCT;
#ifndef MSATTN_WIDE_FP8_UNCAPPED
#define MSATTN_WIDE_FP8_UNCAPPED 1
#endif
constexpr bool kWideFp8Uncapped = MSATTN_WIDE_FP8_UNCAPPED != 0;
#ifndef MSATTN_DEEP_MIN_PER_CU
#define MSATTN_DEEP_MIN_PER_CU 4
#endif
// Workgroups per CU from which a head_dim-64 partition launch takes the deeper residency.
constexpr int kDeepMinPerCu = MSATTN_DEEP_MIN_PER_CU;

// Stream-K scheduling of the prefill kernel's tasks: 1 where the cost model below prefers
// it, 2 always (where it fits), 0 never (one task per workgroup).
#ifndef MSATTN_PF_STREAMK
#define MSATTN_PF_STREAMK 1
#endif
constexpr int kPfStreamK = MSATTN_PF_STREAMK;
// The cost model, in units of one task's key-step pair (about 2 us on MI355X), fitted on
// ten chunked-prefill shapes of 16-224 tasks timed both ways: one task per workgroup costs
// P x rounds + kPfOneFixed (P: key-step pairs of a task, rounds: of one task per CU; the
// fixed part: a task's start and end); stream-K costs P x tasks / G + kPfSkFixed (a share's
// starts and ends, its partials and the fold launch), in tenths of a pair. Stream-K is
// taken when it costs under 90 % of the other.
#ifndef MSATTN_PF_SK_FIXED_TENTHS
#define MSATTN_PF_SK_FIXED_TENTHS 90
#endif
#ifndef MSATTN_PF_ONE_FIXED_TENTHS
#define MSATTN_PF_ONE_FIXED_TENTHS 40
#endif
constexpr int64_t kPfSkFixedTenths = MSATTN_PF_SK_FIXED_TENTHS;
constexpr int64_t kPfOneFixedTenths = MSATTN_PF_ONE_FIXED_TENTHS;
#ifndef MSATTN_PF_SK_MIN_PAIRS
#define MSATTN_PF_SK_MIN_PAIRS 4
#endif
constexpr int64_t kPfSkMinPairs = MSATTN_PF_SK_MIN_PAIRS;  // key-step pairs a share holds at least
constexpr int64_t kPfSkMaxGroups = 256;  // workgroups of a stream-K prefill launch, at most

// Workgroups of a stream-K prefill launch on a device of `cus` CUs for this geometry (a
// multiple of 8 when it has at least 8, so that shares are dealt to the XCDs evenly; no
// more than kPfSkMaxGroups; each share at least kPfSkMinPairs of the work list's key-step
// pairs at the table capacity), or 0 where the geometry cannot take stream-K: not a
// prefill the MFMA kernel's head sizes allow, or more tasks than its work-list table holds.
int64_t prefill_sk_groups(int batch, int q_len, int num_heads, int num_kv_heads, int head_dim,
                          int max_context, int64_t cus) {
  if (kPfStreamK == 0 || q_len <= 1 || (head_dim != 64 && head_dim != 128)) return 0;
  const int64_t rows = static_cast<int64_t>(q_len) * (num_heads / num_kv_heads);
  const int64_t tasks = (rows + kPfRows - 1) / kPfRows * num_kv_heads * batch;
  if (tasks > kPfSkMaxTasks) return 0;
  const int64_t pairs_max = std::max<int64_t>(1, ceil_div(ceil_div(max_context, kPfStep), 2));
  int64_t G = std::min<int64_t>(cus, kPfSkMaxGroups);
  if (G >= kXcds) G = G / kXcds * kXcds;
  return std::min<int64_t>(G, std::max<int64_t>(1, tasks * pairs_max / kPfSkMinPairs));
}

bool dtype_ok(int d) { return d >= MSATTN_F32 && d <= MSATTN_FP8_E4M3; }
int dtype_bytes(int d) { return d == MSATTN_F32 ? 4 : (d == MSATTN_FP8_E4M3 ? 1 : 2); }
bool aligned(const void* ptr, uintptr_t a) { return (reinterpret_cast<uintptr_t>(ptr) % a) == 0; }

// Head sizes: every even size up to kMaxHeadDim (miniserve/attention.py:87-88 accepts any
// positive even head_dim; the generic kernel spreads a row over at most one wave, and the
// merge kernel holds rows of up to 256 dims).
constexpr int kMaxHeadDim = 256;

bool geometry_ok(int batch, int q_len, int num_heads, int num_kv_heads, int head_dim,
                 int max_context) {
  if (batch <= 0 || q_len <= 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0) return false;
  if (num_heads % num_kv_heads) return false;
  if (max_context < 0) return false;
  if (head_dim % 2 || head_dim > kMaxHeadDim) return false;
  const int64_t rows = static_cast<int64_t>(batch) * q_len * num_heads;
  return rows < (int64_t(1) << 31);
}

int rows_per_tile(int rows_per_kvh) { return rows_per_kvh >= 8 ? 8 : next_pow2(rows_per_kvh); }

int choose_partition(int batch, int q_len, int num_heads, int num_kv_heads, int max_context) {
  const int G = num_heads / num_kv_heads;
  const int rows = q_len * G;
  const int RT = rows_per_tile(rows);
  const int64_t base = static_cast<int64_t>(batch) * num_kv_heads * ceil_div(rows, RT);
  for (int part : kPartitionChoices) {
    const int64_t parts = max_context > 0 ? (max_context + part - 1) / part : 1;
    if (base * parts >= kTargetSlots) return part;
  }
  return kPartitionChoices[sizeof(kPartitionChoices) / sizeof(int) - 1];
}

int largest_pow2_divisor_upto(int x, int cap) {
  int u = 1;
  while (u * 2 <= cap && x % (u * 2) == 0) u *= 2;
  return u;
}

// Stream-K grid: one workgroup per CU (MI355X has 256 CUs; 4 waves for a 2-byte cache,
// 8 for fp8); devices with fewer CUs launch proportionally fewer.
#ifndef MSATTN_SK_GRID
#define MSATTN_SK_GRID 256
#endif
constexpr int kSkGrid = MSATTN_SK_GRID;
#ifndef MSATTN_SK_MIN_CHUNK
#define MSATTN_SK_MIN_CHUNK 4
#endif
constexpr int kSkMinChunk = MSATTN_SK_MIN_CHUNK;  // stream-K: smallest chunk (tiles)

int mfma_rows_per_tile(int rows_per_kvh) { return rows_per_kvh >= 16 ? 16 : next_pow2(rows_per_kvh); }

// Workspace: [header][ml: slots x 2 floats][acc: slots x head_dim floats], each
// region 256-byte aligned. Slots cover both partial layouts: rows x max_parts for
// the partition kernels, and pieces x UG x RT for stream-K decode, where pieces
// <= chunks + NUG * batch and chunks <= min(grid * 8 / UG, tiles / min chunk).
struct Layout {
  int part;
  int max_parts;
  int64_t rows;
  int64_t slots;
  size_t hdr_bytes;
  size_t ml_bytes;
  size_t acc_bytes;
  size_t total() const { return hdr_bytes + ml_bytes + acc_bytes; }
};

size_t round256(size_t x) { return (x + 255) / 256 * 256; }

Layout workspace_layout(int batch, int q_len, int num_heads, int num_kv_heads, int head_dim,
                        int max_context) {
  Layout L;
  L.part = choose_partition(batch, q_len, num_heads, num_kv_heads, max_context);
  // Partition kernels: one slot per partition plus the end marker.
  L.max_parts = (max_context > 0 ? ceil_div(max_context, L.part) : 1) + 1;
  L.rows = static_cast<int64_t>(batch) * q_len * num_heads;
  L.slots = L.rows * L.max_parts;
  if (q_len == 1 && batch <= kSkMaxBatch) {
    // Either stream-K shape (2- or 4-byte or fp8 cache: the size does not depend on the
    // dtype).
    const int RT = mfma_rows_per_tile(num_heads / num_kv_heads);
    const int units = num_kv_heads * ceil_div(num_heads / num_kv_heads, RT);
    for (const int waves : {sk_waves(2), sk_waves(1)}) {
      const int UG = largest_pow2_divisor_upto(units, waves);
      const int64_t segments = static_cast<int64_t>(units / UG) * batch;
      const int64_t tiles = segments * ceil_div(max_context, 16);
      const int64_t by_grid = static_cast<int64_t>(kSkGrid) * (waves / UG);
      const int64_t by_size = (tiles + kSkMinChunk - 1) / kSkMinChunk;
      const int64_t chunks = by_grid < by_size ? by_grid : by_size;
      const int64_t sk = streamk_pieces(chunks, segments) * UG * RT;
      if (sk > L.slots) L.slots = sk;
    }
  }
  // A chunked prefill on the prefill kernel's stream-K schedule keeps two partials of
  // kPfRows rows per workgroup in the same regions: sized for the largest launch any
  // device takes, so that a call with this workspace and the no-allocation entry point
  // (whose scratch holds it) take the same schedule.
  const int64_t pf_groups = prefill_sk_groups(batch, q_len, num_heads, num_kv_heads, head_dim,
                                              max_context, kPfSkMaxGroups);
  if (2 * pf_groups * kPfRows > L.slots) L.slots = 2 * pf_groups * kPfRows;
  // The header's prefix area: a stream-K decode's tiles per sequence (batch + 1 words), or a
  // stream-K prefill's task offsets and head size for its fold launch (tasks + 2).
  size_t prefix_words = static_cast<size_t>(batch) + 1;
  if (pf_groups > 0) {
    const int64_t rows = static_cast<int64_t>(q_len) * (num_heads / num_kv_heads);
    const size_t tasks = static_cast<size_t>((rows + kPfRows - 1) / kPfRows * num_kv_heads * batch);
    if (tasks + 2 > prefix_words) prefix_words = tasks + 2;
  }
  L.hdr_bytes = round256(sizeof(int) * (kHdrPrefix + prefix_words));
  L.ml_bytes = round256(static_cast<size_t>(L.slots) * 2 * sizeof(float));
  L.acc_bytes = static_cast<size_t>(L.slots) * head_dim * sizeof(float);
  return L;
}

// The prefill launch's schedule: stream-K over `groups` workgroups (partials at the given
// workspace offsets), or groups = 0 for one task per workgroup. Stream-K is taken where
// prefill_sk_groups allows it, the cost model prefers it (MSATTN_PF_STREAMK 1; 2 takes it
// wherever it fits) and the workspace holds its partials.
int device_cus();

struct PfSkPlan {
  int64_t groups = 0;
  size_t ml_offset = 0;
  size_t acc_offset = 0;
};

PfSkPlan prefill_sk_plan(int batch, int q_len, int num_heads, int num_kv_heads, int head_dim,
                         int max_context, size_t workspace_bytes) {
  PfSkPlan plan;
  const int64_t cus = device_cus();
  const int64_t G = prefill_sk_groups(batch, q_len, num_heads, num_kv_heads, head_dim,
                                      max_context, cus);
  if (G < 2) return plan;
  const int64_t rows = static_cast<int64_t>(q_len) * (num_heads / num_kv_heads);
  const int64_t tasks = (rows + kPfRows - 1) / kPfRows * num_kv_heads * batch;
  const int64_t rounds = (tasks + cus - 1) / cus;
  const int64_t P = std::max<int64_t>(1, ceil_div(ceil_div(max_context, kPfStep), 2));
  // costs in tenths of a pair, times `tasks` (which divides the stream-K work term)
  const int64_t one_cost = (10 * P * rounds + kPfOneFixedTenths) * tasks;
  const int64_t sk_cost = 10 * P * tasks * tasks / G + kPfSkFixedTenths * tasks;
  if (kPfStreamK != 2 && 10 * sk_cost >= 9 * one_cost) return plan;
  const Layout L = workspace_layout(batch, q_len, num_heads, num_kv_heads, head_dim, max_context);
  const size_t ml_bytes = round256(static_cast<size_t>(2 * G * kPfRows) * 2 * sizeof(float));
  const size_t acc_bytes = static_cast<size_t>(2 * G * kPfRows) * head_dim * sizeof(float);
  if (workspace_bytes < L.hdr_bytes + ml_bytes + acc_bytes) return plan;
  plan.groups = G;
  plan.ml_offset = L.hdr_bytes;
  plan.acc_offset = L.hdr_bytes + ml_bytes;
  return plan;
}

// Cascade decode: the shared-prefix pass splits the prefix into npart key partitions
// so that (row blocks x KV heads x npart) workgroups about reach kPxGrid, each at least
// kPxMinPart tokens; its partials follow the regular workspace layout.
#ifndef MSATTN_PX_GRID
#define MSATTN_PX_GRID 256
#endif
#ifndef MSATTN_PX_MIN_PART
#define MSATTN_PX_MIN_PART 128
#endif
constexpr int kPxGrid = MSATTN_PX_GRID;          // workgroups the prefix pass aims for
constexpr int kPxMinPart = MSATTN_PX_MIN_PART;   // shortest key partition (tokens)
static_assert(kPxMinPart % kPfStep == 0, "partitions of whole steps");
struct PrefixLayout {
  Layout base;
  int prefix;     // shared tokens
  int key_part;   // tokens per partition (a multiple of kPfStep)
  int npart;
  size_t pml_off, pacc_off;
  size_t total;
};

PrefixLayout prefix_layout(int batch, int num_heads, int num_kv_heads, int head_dim,
                           int block_size, int max_context, int prefix_pages) {
  PrefixLayout X;
  X.base = workspace_layout(batch, 1, num_heads, num_kv_heads, head_dim, max_context);
  const int64_t pt = static_cast<int64_t>(prefix_pages) * block_size;
  X.prefix = static_cast<int>(pt < max_context ? pt : max_context);
  const int rblocks = ceil_div(batch * (num_heads / num_kv_heads), kPfRows);
  const int64_t per_part = static_cast<int64_t>(rblocks) * num_kv_heads;
  int want = static_cast<int>((kPxGrid + per_part - 1) / per_part);
  const int most = X.prefix > 0 ? ceil_div(X.prefix, kPxMinPart) : 1;
  want = want < 1 ? 1 : (want > most ? most : want);
  X.key_part = X.prefix > 0 ? ceil_div(ceil_div(X.prefix, want), kPfStep) * kPfStep : kPfStep;
  X.npart = X.prefix > 0 ? ceil_div(X.prefix, X.key_part) : 1;
  const int64_t slots = static_cast<int64_t>(batch) * num_heads * X.npart;
  X.pml_off = round256(X.base.total());
  X.pacc_off = X.pml_off + round256(static_cast<size_t>(slots) * 2 * sizeof(float));
  X.total = X.pacc_off + static_cast<size_t>(slots) * head_dim * sizeof(float);
  return X;
}

// The MFMA kernels (decode partition, stream-K, prefill) read a 16-token tile through a
// buffer descriptor with 32-bit byte offsets from the tile's first row: the tile's span
// (15 slot strides plus one row) must stay below 2^31 bytes. Caches laid out with a
// larger slot stride (a permuted view of a large pool) take the generic kernel, which
// addresses with 64-bit offsets.
bool tile_span_ok(int64_t slot_stride, int head_dim, int kv_dtype) {
  if (slot_stride >= (int64_t(1) << 31)) return false;
  return (15 * slot_stride + head_dim) * dtype_bytes(kv_dtype) < (int64_t(1) << 31);
}

int hip_status(hipError_t e) { return e == hipSuccess ? MSATTN_OK : MSATTN_ERR_HIP; }

// Compute units of the current device (cached per device).
int device_cus() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64) {
    const int c = cache[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  if (dev < 64) cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

// Generic kernel for every (query, cache) type pair: the cache is read as stored and
// cast to the query type (miniserve/attention.py:240-241).
template <typename QT>
hipError_t dispatch_split_q(const SplitParams& p, int kv_dtype, int D, int RT, bool rows16,
                            hipStream_t s, bool* sup) {
  switch (kv_dtype) {
    case MSATTN_F32: return launch_split<QT, float>(p, D, RT, rows16, s, sup);
    case MSATTN_F16: return launch_split<QT, _Float16>(p, D, RT, rows16, s, sup);
    case MSATTN_BF16: return launch_split<QT, bf16_t>(p, D, RT, rows16, s, sup);
    case MSATTN_FP8_E4M3: return launch_split<QT, fp8_t>(p, D, RT, rows16, s, sup);
    default: break;
  }
  *sup = false;
  return hipSuccess;
}

// rows16: the cache rows start on 16-byte boundaries and span whole 16-byte chunks, so
// the generic kernel may read them with 16-byte loads (else element by element).
hipError_t dispatch_split(const SplitParams& p, int q_dtype, int kv_dtype, int D, int RT,
                          bool rows16, hipStream_t s, bool* sup) {
  *sup = false;
  switch (q_dtype) {
    case MSATTN_F32: return dispatch_split_q<float>(p, kv_dtype, D, RT, rows16, s, sup);
    case MSATTN_F16: return dispatch_split_q<_Float16>(p, kv_dtype, D, RT, rows16, s, sup);
    case MSATTN_BF16: return dispatch_split_q<bf16_t>(p, kv_dtype, D, RT, rows16, s, sup);
    default: break;
  }
  return hipSuccess;
}

// The MFMA kernels (partition and stream-K decode, chunked prefill, the cascade's prefix
// pass) take a bf16/fp16 query over a cache of its own type, of fp8 e4m3 (widened
// exactly) or of fp32 (rounded to the query type as loaded), head_dim 64 or 128, pages
// of whole 16-token tiles, a tile span their 32-bit offsets reach, and a query they can
// read with 16-byte loads.
bool mfma_route_ok(const void* query, int q_dtype, int kv_dtype, int head_dim, int block_size,
                   int64_t slot_stride, bool rows16) {
  return (q_dtype == MSATTN_BF16 || q_dtype == MSATTN_F16) &&
         (kv_dtype == q_dtype || kv_dtype == MSATTN_FP8_E4M3 || kv_dtype == MSATTN_F32) &&
         (head_dim == 64 || head_dim == 128) && block_size % 16 == 0 && rows16 &&
         tile_span_ok(slot_stride, head_dim, kv_dtype) && aligned(query, 16);
}

// Launch an MFMA kernel family for (query type T, the cache's type): F is a generic
// callable taking (T{}, KT{}) tags.
template <typename T, typename F>
hipError_t with_kv_type(int kv_dtype, F&& f) {
  if (kv_dtype == MSATTN_FP8_E4M3) return f(T{}, fp8_t{});
  if (kv_dtype == MSATTN_F32) return f(T{}, float{});
  return f(T{}, T{});
}
template <typename F>
hipError_t with_mfma_types(int q_dtype, int kv_dtype, F&& f) {
  if (q_dtype == MSATTN_BF16) return with_kv_type<bf16_t>(kv_dtype, f);
  return with_kv_type<_Float16>(kv_dtype, f);
}

// The decode kernels (partition and stream-K) also take an fp32 query over any cache:
// an fp32 cache is the reference runner's default (miniserve/model_runner.py:122-123), and
// its fp8 kv_dtype (miniserve/attention.py:151-152) under the runner's fp32 model gives an
// fp32 query over fp8. Scores on fp32 MFMAs over the cache widened exactly to fp32; P.V on
// fp32 FMAs, or fp32 MFMAs at 16 rows per tile over an fp32 cache. The cascade's prefix
// pass keeps the generic kernel for an fp32 query.
bool mfma_decode_route_ok(const void* query, int q_dtype, int kv_dtype, int head_dim,
                          int block_size, int64_t slot_stride, bool rows16) {
  if (q_dtype == MSATTN_F32)
    return (head_dim == 64 || head_dim == 128) && block_size % 16 == 0 && rows16 &&
           tile_span_ok(slot_stride, head_dim, kv_dtype) && aligned(query, 16);
  return mfma_route_ok(query, q_dtype, kv_dtype, head_dim, block_size, slot_stride, rows16);
}
template <typename F>
hipError_t with_mfma_decode_types(int q_dtype, int kv_dtype, F&& f) {
  if (q_dtype != MSATTN_F32) return with_mfma_types(q_dtype, kv_dtype, f);
  switch (kv_dtype) {
    case MSATTN_F32: return f(float{}, float{});
    case MSATTN_BF16: return f(float{}, bf16_t{});
    case MSATTN_F16: return f(float{}, _Float16{});
    case MSATTN_FP8_E4M3: return f(float{}, fp8_t{});
    default: return hipErrorNotSupported;
  }
}

// Caches must be element-aligned with non-negative strides. Rows that start on 16-byte
// boundaries (pointers and every stride) and span whole 16-byte chunks are read with
// 16-byte loads (cache_rows16); other layouts (odd head sizes such as 6 or 40 over a
// 2-byte cache, padded strides) take the generic kernel's element loads.
int check_cache_args(const void* k_cache, const void* v_cache, int64_t blk, int64_t slot,
                     int64_t head, int kv_dtype, int block_size, int num_blocks, int table_width) {
  if (!k_cache || !v_cache) return MSATTN_ERR_INVALID_ARG;
  if (block_size <= 0 || num_blocks <= 0 || table_width <= 0) return MSATTN_ERR_INVALID_ARG;
  if (blk < 0 || slot < 0 || head < 0) return MSATTN_ERR_INVALID_ARG;
  const int eb = dtype_bytes(kv_dtype);
  if (!aligned(k_cache, eb) || !aligned(v_cache, eb)) return MSATTN_ERR_INVALID_ARG;
  return MSATTN_OK;
}

bool cache_rows16(const void* k_cache, const void* v_cache, int64_t blk, int64_t slot,
                  int64_t head, int head_dim, int kv_dtype) {
  const int eb = dtype_bytes(kv_dtype);
  return aligned(k_cache, 16) && aligned(v_cache, 16) && (blk * eb) % 16 == 0 &&
         (slot * eb) % 16 == 0 && (head * eb) % 16 == 0 && (head_dim * eb) % 16 == 0;
}

}  // namespace

extern "C" {

int msattn_abi_version(void) { return MSATTN_ABI_VERSION; }

const char* msattn_status_string(int status) {
  switch (status) {
    case MSATTN_OK: return "ok";
    case MSATTN_ERR_INVALID_ARG: return "invalid argument";
    case MSATTN_ERR_UNSUPPORTED: return "unsupported geometry or dtype";
    case MSATTN_ERR_WORKSPACE: return "workspace too small";
    case MSATTN_ERR_HIP: return "HIP error";
    default: return "unknown status";
  }
}

int msattn_partition_tokens(int batch, int q_len, int num_heads, int num_kv_heads, int head_dim,
                            int max_context) {
  if (!geometry_ok(batch, q_len, num_heads, num_kv_heads, head_dim, max_context)) return -1;
  return choose_partition(batch, q_len, num_heads, num_kv_heads, max_context);
}

size_t msattn_workspace_bytes(int batch, int q_len, int num_heads, int num_kv_heads, int head_dim,
                              int max_context) {
  if (!geometry_ok(batch, q_len, num_heads, num_kv_heads, head_dim, max_context)) return 0;
  const Layout L = workspace_layout(batch, q_len, num_heads, num_kv_heads, head_dim, max_context);
  return L.total();
}

}  // extern "C"

namespace {

// Optional query RoPE of the decode entry point (null cos: none).
struct RopeArgs {
  const float* cos;
  const float* sin;
  const int32_t* pos;
  int max_pos;
};

// Which partials kernel a call takes (kind as the workspace header records it: 1 stream-K,
// 2 the partition kernel merging in-kernel, 0 the partition or generic kernel with a merge
// launch after it), from sizes, types and alignment only, so the choice is capture-safe.
struct PartialsPlan {
  bool use_mfma;  // the MFMA decode kernels (else the generic kernel)
  int RT;         // query rows per tile
  int kind;
};

PartialsPlan plan_partials(const void* query, int q_dtype, int kv_dtype, int head_dim,
                           int block_size, int64_t slot_stride, bool rows16, int batch,
                           int q_len, int num_heads, int num_kv_heads, int max_context,
                           bool has_out, int key_lo) {
  PartialsPlan pl;
  const int rows = q_len * (num_heads / num_kv_heads);
  pl.use_mfma = mfma_decode_route_ok(query, q_dtype, kv_dtype, head_dim, block_size, slot_stride,
                                     rows16);
  pl.RT = pl.use_mfma ? mfma_rows_per_tile(rows) : rows_per_tile(rows);
  // Decode with enough work to fill the chip: stream-K over every (sequence, KV head)
  // tile run, one workgroup per CU. Small decodes keep the partition kernel, whose short
  // runs start faster.
  const int64_t tile_capacity =
      static_cast<int64_t>(batch) * num_kv_heads * ceil_div(max_context, 16);
  const bool kv_fp8 = kv_dtype == MSATTN_FP8_E4M3;
  const int64_t sk_min_tiles =
      kv_fp8 && q_dtype != MSATTN_F32 && pl.RT == 8 ? kStreamKMinTilesFp8Rt8
      : head_dim == 64                               ? kStreamKMinTilesD64
                                                     : kStreamKMinTiles;
  const int64_t triples = static_cast<int64_t>(batch) * num_kv_heads * ceil_div(rows, pl.RT);
  if (pl.use_mfma && q_len == 1 && batch <= kSkMaxBatch && tile_capacity >= sk_min_tiles)
    pl.kind = 1;
  // With an output to write, the MFMA partition kernel merges in-kernel (the last
  // partition of each (sequence, KV head, row tile) to finish folds the others in), so
  // no merge launch follows; it needs one header ticket per such triple.
  else if (pl.use_mfma && has_out && key_lo == 0 && kFusedMerge && triples <= kMaxTickets)
    pl.kind = 2;
  else
    pl.kind = 0;
  return pl;
}

int partials_impl(const void* query, const void* k_cache, const void* v_cache,
                  int64_t cache_block_stride, int64_t cache_slot_stride,
                  int64_t cache_head_stride, const int32_t* block_table,
                  const int32_t* context_lens, void* workspace, size_t workspace_bytes, int batch,
                  int q_len, int num_heads, int num_kv_heads, int head_dim, int block_size,
                  int num_blocks, int table_width, int max_context, int causal, int window,
                  float scale, int q_dtype, int kv_dtype, const RopeArgs& rope, int key_lo,
                  int* kind, void* stream, void* fused_out = nullptr,
                  const void* k_new = nullptr, const void* v_new = nullptr) {
  *kind = -1;
  if (!query || !block_table || !context_lens || !workspace) return MSATTN_ERR_INVALID_ARG;
  if (!geometry_ok(batch, q_len, num_heads, num_kv_heads, head_dim, max_context))
    return MSATTN_ERR_INVALID_ARG;
  if (!dtype_ok(q_dtype) || q_dtype == MSATTN_FP8_E4M3 || !dtype_ok(kv_dtype))
    return MSATTN_ERR_INVALID_ARG;
  if (!std::isfinite(scale)) return MSATTN_ERR_INVALID_ARG;
  const int rc = check_cache_args(k_cache, v_cache, cache_block_stride, cache_slot_stride,
                                  cache_head_stride, kv_dtype, block_size, num_blocks, table_width);
  if (rc != MSATTN_OK) return rc;
  if (!aligned(query, dtype_bytes(q_dtype)) || !aligned(workspace, 16)) return MSATTN_ERR_INVALID_ARG;
  const Layout L = workspace_layout(batch, q_len, num_heads, num_kv_heads, head_dim, max_context);
  if (workspace_bytes < L.total()) return MSATTN_ERR_WORKSPACE;

  const int G = num_heads / num_kv_heads;
  const int rows = q_len * G;
  // MFMA path where mfma_decode_route_ok allows it; everything else takes the generic kernel.
  const bool kv_fp8 = kv_dtype == MSATTN_FP8_E4M3;
  const bool rows16 = cache_rows16(k_cache, v_cache, cache_block_stride, cache_slot_stride,
                                   cache_head_stride, head_dim, kv_dtype);
  const PartialsPlan plan =
      plan_partials(query, q_dtype, kv_dtype, head_dim, block_size, cache_slot_stride, rows16,
                    batch, q_len, num_heads, num_kv_heads, max_context, fused_out != nullptr,
                    key_lo);
  const bool use_mfma = plan.use_mfma;
  const int RT = plan.RT;
  char* ws = static_cast<char*>(workspace);
  SplitParams p;
  p.hdr = reinterpret_cast<int*>(ws);
  p.q = query;
  p.k = k_cache;
  p.v = v_cache;
  p.table = block_table;
  p.lens = context_lens;
  p.ml = reinterpret_cast<float*>(ws + L.hdr_bytes);
  p.acc = reinterpret_cast<float*>(ws + L.hdr_bytes + L.ml_bytes);
  p.blk_stride = cache_block_stride;
  p.slot_stride = cache_slot_stride;
  p.head_stride = cache_head_stride;
  p.batch = batch;
  p.q_len = q_len;
  p.H = num_heads;
  p.KVH = num_kv_heads;
  p.G = G;
  p.bs = block_size;
  p.num_blocks = num_blocks;
  p.W = table_width;
  p.max_ctx = max_context;
  p.max_parts = L.max_parts;
  p.part = L.part;
  p.causal = causal ? 1 : 0;
  p.window = window > 0 ? window : 0;
  p.scale_log2 = scale * kLog2e;
  p.rows_per_kvh = rows;
  p.rtiles = ceil_div(rows, RT);
  p.sk_group = 1;
  p.sk_unit_groups = 0;
  p.sk_min_chunk = kSkMinChunk;
  p.mfma_waves = kMfmaWaves;
  p.mfma_deep = 0;
  p.key_lo = key_lo;
  p.rope_cos = rope.cos;
  p.rope_sin = rope.sin;
  p.rope_pos = rope.pos;
  p.rope_max_pos = rope.max_pos;
  p.out = nullptr;
  p.tickets = nullptr;
  p.k_new = nullptr;
  p.v_new = nullptr;
  p.part_major = 0;  // the partition kernel's launcher chooses its grid order
  p.head_dim = head_dim;
  p.rows16 = rows16 ? 1 : 0;
  const int64_t gx = static_cast<int64_t>(p.max_parts) * num_kv_heads * p.rtiles;
  if (gx >= (int64_t(1) << 31) || batch > 65535) return MSATTN_ERR_UNSUPPORTED;

  bool sup = false;
  hipError_t e = hipSuccess;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (plan.kind == 1) {  // stream-K
    *kind = 1;
    if (k_new != nullptr) {  // fused append: the caller checked the route and types
      p.k_new = k_new;
      p.v_new = v_new;
    }
    const int units = num_kv_heads * p.rtiles;
    p.sk_group = largest_pow2_divisor_upto(
        units, sk_waves(kv_fp8 ? 1 : 2, q_dtype == MSATTN_F32 ? 4 : 2));
    p.sk_unit_groups = units / p.sk_group;
    const int grid = device_cus() < 256 ? kSkGrid * device_cus() / 256 : kSkGrid;
    e = with_mfma_decode_types(q_dtype, kv_dtype, [&](auto t, auto kt) {
      return launch_decode_streamk<decltype(t), decltype(kt)>(p, head_dim, RT, grid, st, &sup);
    });
    if (!sup) return MSATTN_ERR_UNSUPPORTED;
    return hip_status(e);
  }
  *kind = 0;  // the partition kernels below
  if (plan.kind == 2) {  // the partition kernel merging in-kernel
    *kind = 2;
    p.out = fused_out;
    p.tickets = p.hdr + kHdrTickets;
    if (k_new != nullptr) {  // fused append: the caller checked append_fusable
      p.k_new = k_new;
      p.v_new = v_new;
    }
    // The fp32 16-row route (P.V on the matrix core; its kernel unrolls kPartLongF32
    // tokens per workgroup) takes partitions of up to kPartLongF32 tokens when the grid
    // still reaches kTargetSlots: chunked prefill. Only the in-kernel merge reads these
    // slots, so their count may shrink to the partitions launched.
    if (MSATTN_PV_MFMA32 && q_dtype == MSATTN_F32 && kv_dtype == MSATTN_F32 && RT == 16) {
      const int np = ceil_div(max_context, kPartLongF32);
      const int step = 16 * kMfmaWaves;
      const int part_l = ceil_div(ceil_div(max_context, np), step) * step;
      if (part_l > p.part &&
          static_cast<int64_t>(np) * num_kv_heads * p.rtiles * batch >= kTargetSlots) {
        p.part = part_l;
        p.max_parts = np;
      }
    }
    // Few (sequence, KV head, row tile) triples over long contexts: when partitions that
    // give about one workgroup per CU would hold kPartWide tokens or more, and the launch
    // stays within 1.5 workgroups per CU, the partition kernel's wide shape (8 waves, two
    // per SIMD) over kPartWide-token partitions. Its
    // two waves per SIMD fill each other's waits (C5-decode: 24.1 -> 22.6 us); shorter
    // wide partitions, and wide workgroups two to a CU, measured slower than the regular
    // shape.
    if (kWideRoute && q_len == 1 && (RT == 4 || RT == 8) && q_dtype != MSATTN_F32 &&
        kv_dtype != MSATTN_F32) {
      const int64_t triples = static_cast<int64_t>(batch) * num_kv_heads * p.rtiles;
      const int64_t want = static_cast<int64_t>(device_cus()) * kWideSlotsPct / 100;
      const int64_t np = std::max<int64_t>(1, want / triples);
      const int64_t launched = triples * ceil_div(max_context, kPartWide);
      // An fp8 cache at 4 rows per tile and head_dim 128 takes the wide shape however many
      // workgroups the launch holds: its widening work per byte fills two waves per SIMD
      // (5-10 % faster on H32/KVH8 decodes of 6-20 workgroups per CU); at 8 rows per tile,
      // at head_dim 64 and over a 16-bit cache the cap stands (7-18 % slower without it).
      const bool uncapped = kWideFp8Uncapped && kv_fp8 && RT == 4 && head_dim == 128;
      if (static_cast<int64_t>(max_context) >= np * kPartWide &&
          (uncapped || 100 * launched <= static_cast<int64_t>(kWideMaxPct) * want)) {
        p.part = kPartWide;
        p.max_parts = ceil_div(max_context, kPartWide);
        p.mfma_waves = kWideWaves;
      }
    }
  }
  // A regular-shape launch at head_dim 64 of kDeepMinPerCu or more workgroups per CU
  // holds three a CU instead of two (kMfmaWgPerCuDeep).
  if (use_mfma && p.mfma_waves == kMfmaWaves && head_dim == 64 && (RT == 4 || RT == 8) &&
      q_dtype != MSATTN_F32) {
    const int64_t launched = static_cast<int64_t>(p.max_parts) * num_kv_heads * p.rtiles * batch;
    if (launched >= static_cast<int64_t>(kDeepMinPerCu) * device_cus()) p.mfma_deep = 1;
  }
  if (use_mfma) {
    e = with_mfma_decode_types(q_dtype, kv_dtype, [&](auto t, auto kt) {
      return launch_decode_mfma<decltype(t), decltype(kt)>(p, head_dim, RT, st, &sup);
    });
  } else {
    e = dispatch_split(p, q_dtype, kv_dtype, head_dim, RT, rows16, st, &sup);
  }
  if (!sup) return MSATTN_ERR_UNSUPPORTED;
  return hip_status(e);
}

}  // namespace

extern "C" {

int msattn_paged_attention_partials(const void* query, const void* k_cache, const void* v_cache,
                                    int64_t cache_block_stride, int64_t cache_slot_stride,
                                    int64_t cache_head_stride, const int32_t* block_table,
                                    const int32_t* context_lens, void* workspace,
                                    size_t workspace_bytes, int batch, int q_len, int num_heads,
                                    int num_kv_heads, int head_dim, int block_size,
                                    int num_blocks, int table_width, int max_context, int causal,
                                    int window, float scale, int q_dtype, int kv_dtype,
                                    void* stream) {
  int kind = -1;
  return partials_impl(query, k_cache, v_cache, cache_block_stride, cache_slot_stride,
                       cache_head_stride, block_table, context_lens, workspace, workspace_bytes,
                       batch, q_len, num_heads, num_kv_heads, head_dim, block_size, num_blocks,
                       table_width, max_context, causal, window, scale, q_dtype, kv_dtype,
                       RopeArgs{nullptr, nullptr, nullptr, 0}, 0, &kind, stream);
}

}  // extern "C"

namespace {

int merge_impl(const void* workspace, size_t workspace_bytes, const int32_t* context_lens,
               void* out, int batch, int q_len, int num_heads, int num_kv_heads, int head_dim,
               int max_context, int q_dtype, const float* pml, const float* pacc, int npp,
               int kind_hint, void* stream) {
  if (!workspace || !context_lens || !out) return MSATTN_ERR_INVALID_ARG;
  if (!geometry_ok(batch, q_len, num_heads, num_kv_heads, head_dim, max_context))
    return MSATTN_ERR_INVALID_ARG;
  if (!dtype_ok(q_dtype) || q_dtype == MSATTN_FP8_E4M3) return MSATTN_ERR_INVALID_ARG;
  if (head_dim > 1024) return MSATTN_ERR_UNSUPPORTED;
  if (!aligned(out, dtype_bytes(q_dtype)) || !aligned(workspace, 16)) return MSATTN_ERR_INVALID_ARG;
  const Layout L = workspace_layout(batch, q_len, num_heads, num_kv_heads, head_dim, max_context);
  if (workspace_bytes < L.total()) return MSATTN_ERR_WORKSPACE;
  const char* ws = static_cast<const char*>(workspace);
  MergeParams p;
  p.hdr = reinterpret_cast<const int*>(ws);
  p.ml = reinterpret_cast<const float*>(ws + L.hdr_bytes);
  p.acc = reinterpret_cast<const float*>(ws + L.hdr_bytes + L.ml_bytes);
  p.out = out;
  p.rows = L.rows;
  p.batch = batch;
  p.H = num_heads;
  p.KVH = num_kv_heads;
  p.G = num_heads / num_kv_heads;
  p.D = head_dim;
  p.max_parts = L.max_parts;
  p.slots = L.slots;
  p.pml = pml;
  p.pacc = pacc;
  p.npp = npp;
  p.pslots = npp > 0 ? L.rows * npp : 0;
  p.kind_hint = kind_hint;
  bool sup = false;
  const hipError_t e = launch_merge(p, q_dtype, static_cast<hipStream_t>(stream), &sup);
  if (!sup) return MSATTN_ERR_UNSUPPORTED;
  return hip_status(e);
}

}  // namespace

extern "C" {

int msattn_merge_partials(const void* workspace, size_t workspace_bytes,
                          const int32_t* context_lens, void* out, int batch, int q_len,
                          int num_heads, int num_kv_heads, int head_dim, int max_context,
                          int q_dtype, void* stream) {
  return merge_impl(workspace, workspace_bytes, context_lens, out, batch, q_len, num_heads,
                    num_kv_heads, head_dim, max_context, q_dtype, nullptr, nullptr, 0, -1, stream);
}

}  // extern "C"

namespace {

// Chunked prefill (more than one 16-row tile of query rows per KV head) on the MFMA
// prefill kernel, which writes the normalised output directly, four elements (8 bytes)
// a store, and uses no workspace.
// Query rows per KV head (q_len x G) above which a multi-token query may take the chunked
// prefill kernel; at or below it, the partition decode kernel's 16-row tiles.
#ifndef MSATTN_PREFILL_MIN_ROWS
#define MSATTN_PREFILL_MIN_ROWS 16
#endif
constexpr int64_t kPrefillMinRows = MSATTN_PREFILL_MIN_ROWS;
// Past that, the prefill kernel runs one workgroup per (sequence, KV head, 128-row block)
// over the whole context, so a launch of few such tasks leaves CUs idle, while the
// partition kernel splits the keys over many workgroups but reads the K/V rows once per
// 16-row tile. The partition kernel is taken when (16-row tiles x sequences x KV heads)
// is at most kPrefillSplitPct percent of (CUs x the prefill launch's rounds of one task
// per CU): measured speculative-decoding shapes (q_len 3-16, G 4-7, contexts 1-8k) ran
// 1.1-3x faster there (8 x q_len 4 at G 7: 150.6 -> 49.7 us) and slower past it (64 x
// q_len 6 at G 4: 157.5 against 241.8 us on the partition kernel).
#ifndef MSATTN_PREFILL_SPLIT_PCT
#define MSATTN_PREFILL_SPLIT_PCT 100
#endif
constexpr int64_t kPrefillSplitPct = MSATTN_PREFILL_SPLIT_PCT;
// The rule above holds over the measured shapes, at most 64 query rows per KV head (4
// tiles); longer chunks stay on the prefill kernel, since every 16-row tile of the
// partition kernel streams the whole context again.
#ifndef MSATTN_PREFILL_SPLIT_MAX_ROWS
#define MSATTN_PREFILL_SPLIT_MAX_ROWS 64
#endif
constexpr int64_t kPrefillSplitMaxRows = MSATTN_PREFILL_SPLIT_MAX_ROWS;


// Whether the chunked-prefill kernel can run this call: a multi-token bf16/fp16 query
// with more than kPrefillMinRows rows per KV head on the MFMA route's types and layouts.
bool prefill_kernel_ok(const void* query, const void* out, int64_t cache_slot_stride,
                       bool rows16, int batch, int q_len, int num_heads, int num_kv_heads,
                       int head_dim, int block_size, int q_dtype, int kv_dtype) {
  if (!(q_len > 1 &&
        mfma_route_ok(query, q_dtype, kv_dtype, head_dim, block_size, cache_slot_stride,
                      rows16) &&
        aligned(out, 8) && batch <= 65535 && num_heads > 0 && num_kv_heads > 0 &&
        num_heads % num_kv_heads == 0))
    return false;
  const int64_t rows = static_cast<int64_t>(q_len) * (num_heads / num_kv_heads);
  return rows > kPrefillMinRows;
}

// Whether the cost model prefers the prefill kernel to the partition kernel (for a call
// both can run).
bool prefill_preferred(int batch, int q_len, int num_heads, int num_kv_heads) {
  const int64_t rows = static_cast<int64_t>(q_len) * (num_heads / num_kv_heads);
  if (rows > kPrefillSplitMaxRows) return true;
  const int64_t pairs = static_cast<int64_t>(batch) * num_kv_heads;
  const int64_t tasks = pairs * ((rows + kPfRows - 1) / kPfRows);
  const int64_t cus = device_cus();
  const int64_t rounds = (tasks + cus - 1) / cus;
  return 100 * ((rows + 15) / 16) * pairs > kPrefillSplitPct * cus * rounds;
}

// The route of msattn_paged_attention (and of the no-allocation entry point, whose
// workspace is its scratch): the prefill kernel when it can run and the cost model
// prefers it, or when the partition layout does not fit the workspace (the prefill
// kernel uses none); else the partials kernel plan_partials names.
int choose_route(const void* query, const void* out, const void* k_cache, const void* v_cache,
                 int64_t cache_block_stride, int64_t cache_slot_stride, int64_t cache_head_stride,
                 int batch, int q_len, int num_heads, int num_kv_heads, int head_dim,
                 int block_size, int max_context, int q_dtype, int kv_dtype,
                 size_t workspace_bytes) {
  const bool rows16 = cache_rows16(k_cache, v_cache, cache_block_stride, cache_slot_stride,
                                   cache_head_stride, head_dim, kv_dtype);
  const Layout L = workspace_layout(batch, q_len, num_heads, num_kv_heads, head_dim, max_context);
  const bool fits = workspace_bytes >= L.total();
  if (prefill_kernel_ok(query, out, cache_slot_stride, rows16, batch, q_len, num_heads,
                        num_kv_heads, head_dim, block_size, q_dtype, kv_dtype) &&
      (!fits || prefill_preferred(batch, q_len, num_heads, num_kv_heads)))
    return MSATTN_ROUTE_PREFILL;
  const PartialsPlan pl =
      plan_partials(query, q_dtype, kv_dtype, head_dim, block_size, cache_slot_stride, rows16,
                    batch, q_len, num_heads, num_kv_heads, max_context, true, 0);
  if (pl.kind == 1) return MSATTN_ROUTE_STREAMK;
  if (pl.kind == 2) return MSATTN_ROUTE_PARTITION_FUSED;
  return pl.use_mfma ? MSATTN_ROUTE_PARTITION : MSATTN_ROUTE_GENERIC;
}

// msattn_paged_attention's body. `prefill_needs_ws`: whether the direct prefill route
// checks the workspace size too (the workspace entry point's contract), although that
// route does not touch it.
int attention_impl(const void* query, const void* k_cache, const void* v_cache,
                   int64_t cache_block_stride, int64_t cache_slot_stride,
                   int64_t cache_head_stride, const int32_t* block_table,
                   const int32_t* context_lens, void* out, void* workspace,
                   size_t workspace_bytes, int batch, int q_len, int num_heads,
                   int num_kv_heads, int head_dim, int block_size, int num_blocks,
                   int table_width, int max_context, int causal, int window, float scale,
                   int q_dtype, int kv_dtype, bool prefill_needs_ws, void* stream,
                   const void* k_new = nullptr, const void* v_new = nullptr) {
  if (!out) return MSATTN_ERR_INVALID_ARG;
  if (!dtype_ok(q_dtype) || !aligned(out, dtype_bytes(q_dtype))) return MSATTN_ERR_INVALID_ARG;
  if (!geometry_ok(batch, q_len, num_heads, num_kv_heads, head_dim, max_context))
    return MSATTN_ERR_INVALID_ARG;
  if (choose_route(query, out, k_cache, v_cache, cache_block_stride, cache_slot_stride,
                   cache_head_stride, batch, q_len, num_heads, num_kv_heads, head_dim, block_size,
                   max_context, q_dtype, kv_dtype, workspace_bytes) == MSATTN_ROUTE_PREFILL) {
    if (!query || !block_table || !context_lens || !workspace) return MSATTN_ERR_INVALID_ARG;
    if (!std::isfinite(scale)) return MSATTN_ERR_INVALID_ARG;
    const int rc = check_cache_args(k_cache, v_cache, cache_block_stride, cache_slot_stride,
                                    cache_head_stride, kv_dtype, block_size, num_blocks,
                                    table_width);
    if (rc != MSATTN_OK) return rc;
    const Layout L = workspace_layout(batch, q_len, num_heads, num_kv_heads, head_dim, max_context);
    if (prefill_needs_ws && workspace_bytes < L.total()) return MSATTN_ERR_WORKSPACE;
    PrefillParams pp{};
    pp.q = query;
    pp.k = k_cache;
    pp.v = v_cache;
    pp.table = block_table;
    pp.lens = context_lens;
    pp.out = out;
    pp.blk_stride = cache_block_stride;
    pp.slot_stride = cache_slot_stride;
    pp.head_stride = cache_head_stride;
    pp.batch = batch;
    pp.q_len = q_len;
    pp.H = num_heads;
    pp.KVH = num_kv_heads;
    pp.G = num_heads / num_kv_heads;
    pp.bs = block_size;
    pp.num_blocks = num_blocks;
    pp.W = table_width;
    pp.max_ctx = max_context;
    pp.causal = causal ? 1 : 0;
    pp.window = window > 0 ? window : 0;
    pp.scale_log2 = scale * kLog2e;
    pp.rows_per_kvh = q_len * pp.G;
    pp.rblocks = ceil_div(pp.rows_per_kvh, kPfRows);
    pp.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz(static_cast<unsigned>(block_size)) : -1;
    const int64_t tasks = static_cast<int64_t>(pp.rblocks) * num_kv_heads * batch;
    if (tasks >= (int64_t(1) << 31) - kXcds) return MSATTN_ERR_UNSUPPORTED;
    pp.xcd_per = static_cast<int>((tasks + kXcds - 1) / kXcds);
    // Stream-K scheduling where the cost model prefers it (prefill_sk_plan): one workgroup
    // per CU, each taking an equal share of all tasks' key-step pairs; a task split
    // between shares is merged by the fold launch that follows (the work list's task
    // offsets in the workspace header, two partial slots per workgroup after it).
    pp.sk_groups = 0;
    const PfSkPlan sk = prefill_sk_plan(batch, q_len, num_heads, num_kv_heads, head_dim,
                                        max_context, workspace_bytes);
    if (sk.groups > 0) {
      char* ws = static_cast<char*>(workspace);
      pp.sk_groups = static_cast<int>(sk.groups);
      pp.ntasks = static_cast<int>(tasks);
      pp.sk_ml = reinterpret_cast<float*>(ws + sk.ml_offset);
      pp.sk_acc = reinterpret_cast<float*>(ws + sk.acc_offset);
      pp.sk_pre = reinterpret_cast<int*>(ws) + kHdrPrefix;
    }
    bool sup = false;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const hipError_t e = with_mfma_types(q_dtype, kv_dtype, [&](auto t, auto kt) {
      return launch_prefill_mfma<decltype(t), decltype(kt)>(pp, head_dim, st, &sup);
    });
    if (!sup) return MSATTN_ERR_UNSUPPORTED;
    return hip_status(e);
  }
  int kind = -1;
  const int rc = partials_impl(
      query, k_cache, v_cache, cache_block_stride, cache_slot_stride, cache_head_stride,
      block_table, context_lens, workspace, workspace_bytes, batch, q_len, num_heads,
      num_kv_heads, head_dim, block_size, num_blocks, table_width, max_context, causal, window,
      scale, q_dtype, kv_dtype, RopeArgs{nullptr, nullptr, nullptr, 0}, 0, &kind, stream, out,
      k_new, v_new);
  if (rc != MSATTN_OK) return rc;
  if (kind == 2) return MSATTN_OK;  // merged in-kernel
  return merge_impl(workspace, workspace_bytes, context_lens, out, batch, q_len, num_heads,
                    num_kv_heads, head_dim, max_context, q_dtype, nullptr, nullptr, 0, kind, stream);
}

// ---------------------------------------------------------------------------
// Scratch of msattn_paged_attention_noalloc: one fixed array per device, allocated with
// the code object (no hipMalloc at call time) and held until the process ends. Host code
// must not use the array's name as a device address: its address on each device comes
// from hipGetSymbolAddress, looked up once per device on that device's first call.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = MSATTN_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of `scratch` (its address found on the first call).
int current_scratch(void** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return MSATTN_ERR_HIP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr)
      return MSATTN_ERR_HIP;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return MSATTN_OK;
}

}  // namespace

extern "C" {

int msattn_paged_attention(const void* query, const void* k_cache, const void* v_cache,
                           int64_t cache_block_stride, int64_t cache_slot_stride,
                           int64_t cache_head_stride, const int32_t* block_table,
                           const int32_t* context_lens, void* out, void* workspace,
                           size_t workspace_bytes, int batch, int q_len, int num_heads,
                           int num_kv_heads, int head_dim, int block_size, int num_blocks,
                           int table_width, int max_context, int causal, int window,
                           float scale, int q_dtype, int kv_dtype, void* stream) {
  return attention_impl(query, k_cache, v_cache, cache_block_stride, cache_slot_stride,
                        cache_head_stride, block_table, context_lens, out, workspace,
                        workspace_bytes, batch, q_len, num_heads, num_kv_heads, head_dim,
                        block_size, num_blocks, table_width, max_context, causal, window, scale,
                        q_dtype, kv_dtype, true, stream);
}

int msattn_paged_attention_noalloc(const void* query, const void* k_cache, const void* v_cache,
                                   int64_t cache_block_stride, int64_t cache_slot_stride,
                                   int64_t cache_head_stride, const int32_t* block_table,
                                   const int32_t* context_lens, void* out, int batch, int q_len,
                                   int num_heads, int num_kv_heads, int head_dim, int block_size,
                                   int num_blocks, int table_width, int max_context, int causal,
                                   int window, float scale, int q_dtype, int kv_dtype,
                                   void* stream) {
  // Every size check comes before the first HIP call.
  if (!out || !dtype_ok(q_dtype) || q_dtype == MSATTN_FP8_E4M3) return MSATTN_ERR_INVALID_ARG;
  if (!geometry_ok(batch, q_len, num_heads, num_kv_heads, head_dim, max_context))
    return MSATTN_ERR_INVALID_ARG;
  // A partition layout that does not fit the scratch sends a chunked prefill the prefill
  // kernel can run there (it uses no scratch); any other call past the scratch is refused.
  if (choose_route(query, out, k_cache, v_cache, cache_block_stride, cache_slot_stride,
                   cache_head_stride, batch, q_len, num_heads, num_kv_heads, head_dim, block_size,
                   max_context, q_dtype, kv_dtype, kScratchBytes) != MSATTN_ROUTE_PREFILL) {
    const Layout L = workspace_layout(batch, q_len, num_heads, num_kv_heads, head_dim, max_context);
    if (L.total() > kScratchBytes) return MSATTN_ERR_WORKSPACE;
  }
  void* ws = nullptr;
  const int rc = current_scratch(&ws);
  if (rc != MSATTN_OK) return rc;
  return attention_impl(query, k_cache, v_cache, cache_block_stride, cache_slot_stride,
                        cache_head_stride, block_table, context_lens, out, ws, kScratchBytes,
                        batch, q_len, num_heads, num_kv_heads, head_dim, block_size, num_blocks,
                        table_width, max_context, causal, window, scale, q_dtype, kv_dtype,
                        false, stream);
}

int msattn_paged_attention_route(const void* query, const void* out, const void* k_cache,
                                 const void* v_cache, int64_t cache_block_stride,
                                 int64_t cache_slot_stride, int64_t cache_head_stride, int batch,
                                 int q_len, int num_heads, int num_kv_heads, int head_dim,
                                 int block_size, int max_context, int q_dtype, int kv_dtype,
                                 size_t workspace_bytes, int* route) {
  if (!route) return MSATTN_ERR_INVALID_ARG;
  *route = 0;
  if (!geometry_ok(batch, q_len, num_heads, num_kv_heads, head_dim, max_context))
    return MSATTN_ERR_INVALID_ARG;
  if (!dtype_ok(q_dtype) || q_dtype == MSATTN_FP8_E4M3 || !dtype_ok(kv_dtype))
    return MSATTN_ERR_INVALID_ARG;
  if (block_size <= 0 || cache_block_stride < 0 || cache_slot_stride < 0 || cache_head_stride < 0)
    return MSATTN_ERR_INVALID_ARG;
  const int r = choose_route(query, out, k_cache, v_cache, cache_block_stride, cache_slot_stride,
                             cache_head_stride, batch, q_len, num_heads, num_kv_heads, head_dim,
                             block_size, max_context, q_dtype, kv_dtype, workspace_bytes);
  if (r != MSATTN_ROUTE_PREFILL &&
      workspace_bytes < workspace_layout(batch, q_len, num_heads, num_kv_heads, head_dim,
                                         max_context).total())
    return MSATTN_ERR_WORKSPACE;
  *route = r == MSATTN_ROUTE_PREFILL &&
                   prefill_sk_plan(batch, q_len, num_heads, num_kv_heads, head_dim, max_context,
                                   workspace_bytes).groups > 0
               ? MSATTN_ROUTE_PREFILL_STREAMK
               : r;
  return MSATTN_OK;
}

int msattn_paged_attention_rope(const void* query, const void* k_cache, const void* v_cache,
                                int64_t cache_block_stride, int64_t cache_slot_stride,
                                int64_t cache_head_stride, const int32_t* block_table,
                                const int32_t* context_lens, void* out, void* workspace,
                                size_t workspace_bytes, int batch, int q_len, int num_heads,
                                int num_kv_heads, int head_dim, int block_size, int num_blocks,
                                int table_width, int max_context, int causal, int window,
                                float scale, int q_dtype, int kv_dtype, const float* rope_cos,
                                const float* rope_sin, const int32_t* position,
                                int max_position, void* stream) {
  if (!out || !rope_cos || !rope_sin || !position || max_position <= 0)
    return MSATTN_ERR_INVALID_ARG;
  if (!aligned(rope_cos, 16) || !aligned(rope_sin, 16) || !aligned(position, 4))
    return MSATTN_ERR_INVALID_ARG;
  if (!dtype_ok(q_dtype) || !aligned(out, dtype_bytes(q_dtype))) return MSATTN_ERR_INVALID_ARG;
  if (q_len != 1 || head_dim % 2) return MSATTN_ERR_UNSUPPORTED;  // decode-only, as the reference
  int kind = -1;
  const int rc = partials_impl(
      query, k_cache, v_cache, cache_block_stride, cache_slot_stride, cache_head_stride,
      block_table, context_lens, workspace, workspace_bytes, batch, q_len, num_heads,
      num_kv_heads, head_dim, block_size, num_blocks, table_width, max_context, causal, window,
      scale, q_dtype, kv_dtype, RopeArgs{rope_cos, rope_sin, position, max_position}, 0, &kind,
      stream, out);
  if (rc != MSATTN_OK) return rc;
  if (kind == 2) return MSATTN_OK;  // merged in-kernel
  return merge_impl(workspace, workspace_bytes, context_lens, out, batch, q_len, num_heads,
                    num_kv_heads, head_dim, max_context, q_dtype, nullptr, nullptr, 0, kind, stream);
}

size_t msattn_prefix_workspace_bytes(int batch, int num_heads, int num_kv_heads, int head_dim,
                                     int block_size, int max_context, int prefix_pages) {
  if (!geometry_ok(batch, 1, num_heads, num_kv_heads, head_dim, max_context) ||
      block_size <= 0 || prefix_pages < 0)
    return 0;
  return prefix_layout(batch, num_heads, num_kv_heads, head_dim, block_size, max_context,
                       prefix_pages).total;
}

int msattn_paged_attention_prefix(const void* query, const void* k_cache, const void* v_cache,
                                  int64_t cache_block_stride, int64_t cache_slot_stride,
                                  int64_t cache_head_stride, const int32_t* block_table,
                                  const int32_t* context_lens, void* out, void* workspace,
                                  size_t workspace_bytes, int batch, int num_heads,
                                  int num_kv_heads, int head_dim, int block_size, int num_blocks,
                                  int table_width, int max_context, int prefix_pages, float scale,
                                  int q_dtype, int kv_dtype, void* stream) {
  if (!query || !block_table || !context_lens || !out || !workspace) return MSATTN_ERR_INVALID_ARG;
  if (!geometry_ok(batch, 1, num_heads, num_kv_heads, head_dim, max_context))
    return MSATTN_ERR_INVALID_ARG;
  if (!dtype_ok(q_dtype) || q_dtype == MSATTN_FP8_E4M3 || !dtype_ok(kv_dtype))
    return MSATTN_ERR_INVALID_ARG;
  if (!std::isfinite(scale) || prefix_pages < 0 || prefix_pages > table_width)
    return MSATTN_ERR_INVALID_ARG;
  const int rc = check_cache_args(k_cache, v_cache, cache_block_stride, cache_slot_stride,
                                  cache_head_stride, kv_dtype, block_size, num_blocks, table_width);
  if (rc != MSATTN_OK) return rc;
  if (!aligned(query, dtype_bytes(q_dtype)) || !aligned(out, dtype_bytes(q_dtype)) ||
      !aligned(workspace, 16))
    return MSATTN_ERR_INVALID_ARG;
  const PrefixLayout X = prefix_layout(batch, num_heads, num_kv_heads, head_dim, block_size,
                                       max_context, prefix_pages);
  if (workspace_bytes < X.total) return MSATTN_ERR_WORKSPACE;
  // The shared-prefix pass runs the MFMA prefill kernel; other types and head sizes,
  // and calls without a shared prefix, attend in one pass over the whole context.
  const bool rows16 = cache_rows16(k_cache, v_cache, cache_block_stride, cache_slot_stride,
                                   cache_head_stride, head_dim, kv_dtype);
  const bool cascade = X.prefix > 0 && mfma_route_ok(query, q_dtype, kv_dtype, head_dim,
                                                     block_size, cache_slot_stride, rows16);
  if (!cascade)
    return msattn_paged_attention(query, k_cache, v_cache, cache_block_stride, cache_slot_stride,
                                  cache_head_stride, block_table, context_lens, out, workspace,
                                  workspace_bytes, batch, 1, num_heads, num_kv_heads, head_dim,
                                  block_size, num_blocks, table_width, max_context, 1, 0, scale,
                                  q_dtype, kv_dtype, stream);
  char* ws = static_cast<char*>(workspace);
  float* pml = reinterpret_cast<float*>(ws + X.pml_off);
  float* pacc = reinterpret_cast<float*>(ws + X.pacc_off);
  const hipStream_t st = static_cast<hipStream_t>(stream);

  // Pass 1: every sequence's query against the shared pages (table row 0), once per
  // KV head, as one virtual sequence of `batch` query positions.
  PrefillParams pp{};
  pp.q = query;
  pp.k = k_cache;
  pp.v = v_cache;
  pp.table = block_table;
  pp.lens = context_lens;
  pp.out = nullptr;
  pp.blk_stride = cache_block_stride;
  pp.slot_stride = cache_slot_stride;
  pp.head_stride = cache_head_stride;
  pp.batch = 1;
  pp.q_len = batch;
  pp.H = num_heads;
  pp.KVH = num_kv_heads;
  pp.G = num_heads / num_kv_heads;
  pp.bs = block_size;
  pp.num_blocks = num_blocks;
  pp.W = table_width;
  pp.max_ctx = X.prefix;
  pp.causal = 0;
  pp.window = 0;
  pp.scale_log2 = scale * kLog2e;
  pp.rows_per_kvh = batch * pp.G;
  pp.rblocks = ceil_div(pp.rows_per_kvh, kPfRows);
  pp.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz(static_cast<unsigned>(block_size)) : -1;
  pp.row_lens = context_lens;
  pp.pml = pml;
  pp.pacc = pacc;
  pp.key_part = X.key_part;
  pp.npart = X.npart;
  if (static_cast<int64_t>(pp.rblocks) * num_kv_heads >= (int64_t(1) << 31) || X.npart > 65535)
    return MSATTN_ERR_UNSUPPORTED;
  bool sup = false;
  const hipError_t e = with_mfma_types(q_dtype, kv_dtype, [&](auto t, auto kt) {
    return launch_prefix_partials<decltype(t), decltype(kt)>(pp, head_dim, st, &sup);
  });
  if (!sup) return MSATTN_ERR_UNSUPPORTED;
  if (e != hipSuccess) return MSATTN_ERR_HIP;

  // Pass 2: each sequence's own pages, keys from the end of the prefix on.
  int kind = -1;
  const int rc2 = partials_impl(
      query, k_cache, v_cache, cache_block_stride, cache_slot_stride, cache_head_stride,
      block_table, context_lens, workspace, workspace_bytes, batch, 1, num_heads, num_kv_heads,
      head_dim, block_size, num_blocks, table_width, max_context, 1, 0, scale, q_dtype, kv_dtype,
      RopeArgs{nullptr, nullptr, nullptr, 0}, X.prefix, &kind, stream);
  if (rc2 != MSATTN_OK) return rc2;
  // Merge: both passes' partials of every row.
  return merge_impl(workspace, workspace_bytes, context_lens, out, batch, 1, num_heads,
                    num_kv_heads, head_dim, max_context, q_dtype, pml, pacc, X.npart, kind,
                    stream);
}

int msattn_write_kv(void* k_cache, void* v_cache, int64_t cache_block_stride,
                    int64_t cache_slot_stride, int64_t cache_head_stride, const void* k,
                    const void* v, const int32_t* block_table, const int32_t* starts, int batch,
                    int tokens, int num_kv_heads, int head_dim, int block_size, int num_blocks,
                    int table_width, int src_dtype, int kv_dtype, void* stream) {
  return write_kv_impl(k_cache, v_cache, cache_block_stride, cache_slot_stride,
                       cache_head_stride, k, v, block_table, starts, 0, batch, tokens,
                       num_kv_heads, head_dim, block_size, num_blocks, table_width, src_dtype,
                       kv_dtype, stream);
}

int msattn_paged_attention_append(const void* query, const void* k_new, const void* v_new,
                                  void* k_cache, void* v_cache, int64_t cache_block_stride,
                                  int64_t cache_slot_stride, int64_t cache_head_stride,
                                  const int32_t* block_table, const int32_t* context_lens,
                                  void* out, void* workspace, size_t workspace_bytes, int batch,
                                  int num_heads, int num_kv_heads, int head_dim, int block_size,
                                  int num_blocks, int table_width, int max_context, int window,
                                  float scale, int q_dtype, int kv_dtype, void* stream) {
  if (!k_new || !v_new || !k_cache || !v_cache || !context_lens || !out)
    return MSATTN_ERR_INVALID_ARG;
  if (!dtype_ok(q_dtype) || q_dtype == MSATTN_FP8_E4M3 || !dtype_ok(kv_dtype))
    return MSATTN_ERR_INVALID_ARG;
  if (!geometry_ok(batch, 1, num_heads, num_kv_heads, head_dim, max_context))
    return MSATTN_ERR_INVALID_ARG;
  const int route = choose_route(query, out, k_cache, v_cache, cache_block_stride,
                                 cache_slot_stride, cache_head_stride, batch, 1, num_heads,
                                 num_kv_heads, head_dim, block_size, max_context, q_dtype,
                                 kv_dtype, workspace_bytes);
  // The partition and stream-K kernels built with the append: a bf16/fp16 query at up to
  // 8 query rows per KV head (stream-K: not over an fp8 cache).
  const bool append_kernel = (q_dtype == MSATTN_BF16 || q_dtype == MSATTN_F16) &&
                             mfma_rows_per_tile(num_heads / num_kv_heads) <= 8;
  if (kFusedAppend && append_kernel && aligned(k_new, 16) && aligned(v_new, 16) &&
      (route == MSATTN_ROUTE_PARTITION_FUSED ||
       (route == MSATTN_ROUTE_STREAMK && kv_dtype != MSATTN_FP8_E4M3))) {
    return attention_impl(query, k_cache, v_cache, cache_block_stride, cache_slot_stride,
                          cache_head_stride, block_table, context_lens, out, workspace,
                          workspace_bytes, batch, 1, num_heads, num_kv_heads, head_dim,
                          block_size, num_blocks, table_width, max_context, 1, window, scale,
                          q_dtype, kv_dtype, true, stream, k_new, v_new);
  }
  // Other routes: the write, then the decode (two launches, the same result).
  const int rc = write_kv_impl(k_cache, v_cache, cache_block_stride, cache_slot_stride,
                               cache_head_stride, k_new, v_new, block_table, context_lens, -1,
                               batch, 1, num_kv_heads, head_dim, block_size, num_blocks,
                               table_width, q_dtype, kv_dtype, stream);
  if (rc != MSATTN_OK) return rc;
  return msattn_paged_attention(query, k_cache, v_cache, cache_block_stride, cache_slot_stride,
                                cache_head_stride, block_table, context_lens, out, workspace,
                                workspace_bytes, batch, 1, num_heads, num_kv_heads, head_dim,
                                block_size, num_blocks, table_width, max_context, 1, window,
                                scale, q_dtype, kv_dtype, stream);
}

}  // extern "C"

namespace {

int write_kv_impl(void* k_cache, void* v_cache, int64_t cache_block_stride,
                  int64_t cache_slot_stride, int64_t cache_head_stride, const void* k,
                  const void* v, const int32_t* block_table, const int32_t* starts,
                  int start_offset, int batch, int tokens, int num_kv_heads, int head_dim,
                  int block_size, int num_blocks, int table_width, int src_dtype, int kv_dtype,
                  void* stream) {
  if (!k_cache || !v_cache || !k || !v || !block_table || !starts) return MSATTN_ERR_INVALID_ARG;
  if (batch <= 0 || tokens < 0 || num_kv_heads <= 0 || head_dim <= 0) return MSATTN_ERR_INVALID_ARG;
  if (block_size <= 0 || num_blocks <= 0 || table_width <= 0) return MSATTN_ERR_INVALID_ARG;
  if (cache_block_stride < 0 || cache_slot_stride < 0 || cache_head_stride < 0)
    return MSATTN_ERR_INVALID_ARG;
  if (!dtype_ok(src_dtype) || !dtype_ok(kv_dtype)) return MSATTN_ERR_INVALID_ARG;
  if (src_dtype == MSATTN_FP8_E4M3 && kv_dtype != MSATTN_FP8_E4M3) return MSATTN_ERR_UNSUPPORTED;
  if (!aligned(k_cache, dtype_bytes(kv_dtype)) || !aligned(v_cache, dtype_bytes(kv_dtype)) ||
      !aligned(k, dtype_bytes(src_dtype)) || !aligned(v, dtype_bytes(src_dtype)))
    return MSATTN_ERR_INVALID_ARG;
  if (tokens == 0) return MSATTN_OK;
  WriteKVParams p;
  p.k_cache = k_cache;
  p.v_cache = v_cache;
  p.k = k;
  p.v = v;
  p.table = block_table;
  p.starts = starts;
  p.blk_stride = cache_block_stride;
  p.slot_stride = cache_slot_stride;
  p.head_stride = cache_head_stride;
  p.batch = batch;
  p.tokens = tokens;
  p.KVH = num_kv_heads;
  p.D = head_dim;
  p.bs = block_size;
  p.num_blocks = num_blocks;
  p.W = table_width;
  p.start_offset = start_offset;
  bool sup = false;
  const hipError_t e = launch_write_kv(p, src_dtype, kv_dtype, static_cast<hipStream_t>(stream), &sup);
  if (!sup) return MSATTN_ERR_UNSUPPORTED;
  return hip_status(e);
}

}  // namespace

extern "C" {

int msattn_gather_kv(const void* cache, int64_t cache_block_stride, int64_t cache_slot_stride,
                     int64_t cache_head_stride, const int32_t* block_table,
                     const int32_t* context_lens, void* out, int batch, int max_context,
                     int num_kv_heads, int head_dim, int block_size, int num_blocks,
                     int table_width, int kv_dtype, void* stream) {
  if (!cache || !block_table || !context_lens || !out) return MSATTN_ERR_INVALID_ARG;
  if (batch <= 0 || max_context < 0 || num_kv_heads <= 0 || head_dim <= 0) return MSATTN_ERR_INVALID_ARG;
  if (block_size <= 0 || num_blocks <= 0 || table_width <= 0) return MSATTN_ERR_INVALID_ARG;
  if (cache_block_stride < 0 || cache_slot_stride < 0 || cache_head_stride < 0)
    return MSATTN_ERR_INVALID_ARG;
  if (!dtype_ok(kv_dtype)) return MSATTN_ERR_INVALID_ARG;
  const int eb = dtype_bytes(kv_dtype);
  if (!aligned(cache, eb) || !aligned(out, eb)) return MSATTN_ERR_INVALID_ARG;
  if (max_context == 0) return MSATTN_OK;
  GatherParams p;
  p.cache = cache;
  p.table = block_table;
  p.lens = context_lens;
  p.out = out;
  p.blk_stride = cache_block_stride;
  p.slot_stride = cache_slot_stride;
  p.head_stride = cache_head_stride;
  p.batch = batch;
  p.max_ctx = max_context;
  p.KVH = num_kv_heads;
  p.D = head_dim;
  p.bs = block_size;
  p.num_blocks = num_blocks;
  p.W = table_width;
  return hip_status(launch_gather(p, eb, static_cast<hipStream_t>(stream)));
}

}  // extern "C"
