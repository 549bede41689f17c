// Stream-K paged decode (q_len == 1) for gfx950: a bf16/fp16 query over a cache of its
// type, of fp8 e4m3 or of fp32, head_dim 64 or 128.
//
// Work decomposition. A "unit" is (row tile, KV head): the up-to-16 GQA query
// rows that read one KV head. Units are grouped UG at a time (UG KV heads side
// by side); the work of a unit group over sequence b is its T_b 16-token tiles
// (the tiles of b's key range). Listing every unit group's sequences in order
// gives `total` slabs. The grid is fixed by the device (one workgroup of kSkWaves
// waves per CU: 4 for a 2-byte cache, 8 for fp8); the slab list is cut into equal
// contiguous chunks of c slabs, one per wave sub-group (kSkWaves / UG sub-groups per
// workgroup), and each of the UG waves of a sub-group walks that chunk for its own KV
// head.
// So every wave streams the same amount of KV (no ragged tails), pays its
// set-up once per run of tiles, and the UG heads of a page are read together.
//
// A chunk that crosses sequence boundaries is split into pieces. With
// segment index seg = ug * B + b, the piece of chunk r inside segment seg has the
// id r + seg: ids are unique and below n_chunks + NUG * B, whatever the lengths.
// Each piece stores, for each of its UG units' rows, the partial (m, l, acc) at
// [id][unit in group][row]. Workgroup 0 writes the layout (chunk size, prefix sums
// of T_b) into the workspace header; merge.hip finds a row's pieces from it.
//
// The per-tile arithmetic is decode_mfma.h's: MFMA scores, online softmax, P.V on
// v_dot2 with DPP row broadcasts, a ring of per-tile buffer descriptors keeping the
// next tiles' loads in flight. A wave walks its chunk in runs of up to kSkTableRun
// tiles and requests the next run's page ids (and, at a sequence boundary, the next
// piece's query rows) before it streams the current one; the tile ring runs on across
// runs and pieces. The algorithm is the split decomposition of
// kernels/paged_attn_triton.py:102-171 with the masking of
// miniserve/attention.py:135-153 (for q_len == 1: keys in [ctx - window, ctx)).
#pragma once

#include "decode_mfma.h"

namespace msattn {

// Waves per workgroup: one per SIMD. With two waves on a SIMD the older one's loads
// win every issue slot of a saturated memory pipe, so the younger one streams only after
// the older has finished its chunk; the page's other heads are then read late, and the
// kernel's end is set by the starved half.
// An fp8 cache spends about twice the VALU work per byte (widening), so there a second
// wave per SIMD pays: its conversions fill the first wave's waits (C3 4 %, C4 2 % faster
// than one wave per SIMD; the same on a 2-byte cache is 2 % slower).
#ifndef MSATTN_SK_WAVES
#define MSATTN_SK_WAVES 4
#endif
#ifndef MSATTN_SK_WAVES_FP8
#define MSATTN_SK_WAVES_FP8 8
#endif
// Waves per workgroup for a cache of kv_bytes-byte elements under a query of q_bytes-byte
// elements. An fp32 query keeps one wave per SIMD: its query chunks take twice the
// registers, and two waves on a SIMD would spill.
__host__ __device__ constexpr int sk_waves(int kv_bytes, int q_bytes = 2) {
  return kv_bytes == 1 && q_bytes < 4 ? MSATTN_SK_WAVES_FP8 : MSATTN_SK_WAVES;
}
constexpr int kSkMaxBatch = 4096;   // sequences per launch on this path
constexpr int kSkTableRun = 64;     // tile page ids fetched per table load
// Tiles whose loads are in flight per wave (ring depth) for 2-byte and for fp8
// caches, and ring turns per loop iteration.
#ifndef MSATTN_SK_DEPTH
#define MSATTN_SK_DEPTH 2
#endif
#ifndef MSATTN_SK_DEPTH_FP8
#define MSATTN_SK_DEPTH_FP8 2
#endif
#ifndef MSATTN_SK_ROUNDS
#define MSATTN_SK_ROUNDS 1
#endif
// 1: a run's page ids are decoded in the previous run's last ring turn, a run after
// their request, so the wave does not wait for the table at each run's start.
#ifndef MSATTN_SK_LATE_IDS
#define MSATTN_SK_LATE_IDS 1
#endif
// Two waves on a SIMD (workgroups of more than 4 waves): the hardware issues the older
// wave's loads first whenever both are ready, so the younger one streams its chunk
// behind it and ends well after it (C3 fp8: waves 0-3 at 55 us, waves 4-7 at 67 us),
// with the SIMD half-used meanwhile. With MSATTN_SK_BALANCE, each wave posts the tiles
// it has consumed in LDS and runs at raised priority while it is not ahead of its SIMD
// partner (wave w ^ waves/2), so the two keep pace and end together.
#ifndef MSATTN_SK_BALANCE
#define MSATTN_SK_BALANCE 1
#endif

// Pieces a launch can produce: one per chunk plus one per segment boundary.
__host__ __device__ constexpr int64_t streamk_pieces(int64_t n_chunks, int64_t n_segments) {
  return n_chunks + n_segments;
}

template <typename T, typename KT, int D, int RT, bool APPEND = false>
__global__ __launch_bounds__(sk_waves(sizeof(KT), sizeof(T)) * kWave) void decode_streamk_kernel(
    const SplitParams p) {
  constexpr int kSkWaves = sk_waves(sizeof(KT), sizeof(T));
  constexpr int kSkThreads = kSkWaves * kWave;
  typedef Kv8<T, KT> KV;
  typedef typename KV::raw_t raw_t;
  constexpr int DEPTH = sizeof(KT) == 1 ? MSATTN_SK_DEPTH_FP8 : MSATTN_SK_DEPTH;
  constexpr int STEP = DEPTH * MSATTN_SK_ROUNDS;  // tiles per loop iteration
  static_assert(D == 64 || D == 128, "stream-K decode handles head_dim 64 and 128");
  constexpr int JD = D / 32;
  constexpr int LPR = D / 8;
  constexpr int TPI = 64 / LPR;
  constexpr int NJ = 16 / TPI;
  constexpr int APR = 16 / LPR;
  constexpr int EB = static_cast<int>(sizeof(KT));

  __shared__ int s_pre[kSkMaxBatch + 1];  // exclusive prefix of T_b
  __shared__ int s_ctx[kSkMaxBatch];      // context length of b, clamped to max_ctx
  __shared__ int s_wsum[2][kSkWaves];
  constexpr bool kBalance = MSATTN_SK_BALANCE && kSkWaves > 4;
  __shared__ int s_prog[kSkWaves];        // tiles consumed per wave (kBalance)

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  if (kBalance && tid < kSkWaves) s_prog[tid] = 0;  // ordered by the scan's barriers
  const int g = lane >> 4;
  const int n = lane & 15;
  const int va = lane / LPR;
  const int vc = lane % LPR;
  const int B = p.batch;

  // ---- tiles per sequence and their exclusive prefix sum (block scan) ----
  // Sequence b = k * kSkThreads + tid: one coalesced load per slice of the batch, every
  // slice's loads issued together; each slice is scanned in registers and across the
  // waves through LDS (two buffers, so one barrier a slice), carrying the running total.
  constexpr int kSlices = (kSkMaxBatch + kSkThreads - 1) / kSkThreads;
  const int nslices = (B + kSkThreads - 1) / kSkThreads;
  // Every live slice's length load goes out before any is used (lanes past the batch
  // read sequence 0's and drop it): one memory round trip for the whole batch.
  int lraw[kSlices];
#pragma unroll
  for (int k = 0; k < kSlices; ++k)
    if (k < nslices) {
      const int b = k * kSkThreads + tid;
      lraw[k] = p.lens[b < B ? b : 0];
    }
  int tb[kSlices];
#pragma unroll
  for (int k = 0; k < kSlices; ++k) {
    const int b = k * kSkThreads + tid;
    int t = 0;
    if (k < nslices && b < B) {
      int ctx = lraw[k];
      ctx = ctx < 0 ? 0 : (ctx > p.max_ctx ? p.max_ctx : ctx);
      s_ctx[b] = ctx;
      const int lo = max(p.key_lo, p.window > 0 ? max(0, ctx - p.window) : 0);
      t = ctx > lo ? ceil_div(ctx, 16) - lo / 16 : 0;
    }
    tb[k] = t;
  }
  int sumT = 0;
#pragma unroll
  for (int k = 0; k < kSlices; ++k) {
    if (k < nslices) {
      const int incl = wave_inclusive_sum(tb[k]);
      if (lane == kWave - 1) s_wsum[k & 1][w] = incl;
      __syncthreads();
      int off = sumT;
      int tot = 0;
#pragma unroll
      for (int i = 0; i < kSkWaves; ++i) {
        const int v = s_wsum[k & 1][i];
        if (i < w) off += v;
        tot += v;
      }
      const int b = k * kSkThreads + tid;
      if (b < B) s_pre[b] = off + incl - tb[k];
      sumT += tot;
    }
  }
  if (tid == 0) s_pre[B] = sumT;
  __syncthreads();

  // ---- chunking ----
  const int UG = p.sk_group;                 // KV heads per unit group (divides kSkWaves)
  const int SG = kSkWaves / UG;              // sub-groups per workgroup
  const int64_t total = static_cast<int64_t>(p.sk_unit_groups) * sumT;
  const int64_t nsub = static_cast<int64_t>(gridDim.x) * SG;
  const int64_t c = max(static_cast<int64_t>(p.sk_min_chunk), (total + nsub - 1) / nsub);

  // Workgroup 0 publishes the layout for the merge.
  if (blockIdx.x == 0) {
    if (tid == 0) {
      p.hdr[kHdrKind] = 1;
      p.hdr[kHdrSumT] = sumT;
      p.hdr[kHdrChunk] = static_cast<int>(c);
      p.hdr[kHdrNsub] = static_cast<int>(nsub);
      p.hdr[kHdrUG] = UG;
      p.hdr[kHdrNUG] = p.sk_unit_groups;
      p.hdr[kHdrB] = B;
      p.hdr[kHdrRT] = RT;
    }
    for (int b = tid; b <= B; b += kSkThreads) p.hdr[kHdrPrefix + b] = s_pre[b];
  }
  if (sumT == 0) return;
  const int sg = w / UG;
  const int ul = w - sg * UG;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * SG + sg;
  int64_t s = r * c;
  const int64_t s_end = min(s + c, total);

  const KT* kbase = static_cast<const KT*>(p.k);
  const KT* vbase = static_cast<const KT*>(p.v);
  const uint32_t k_lane_tok = static_cast<uint32_t>(tile_token<D>(n));
  const int tile_bytes = static_cast<int>((15 * p.slot_stride + D) * EB);

  // A piece: the part of this chunk's tiles inside one segment (unit group ug, sequence b).
  struct Piece {
    int b, kvh, row0, nrows, t_first, ntiles, a0, a1;
    int64_t pid, pe;
  };
  auto locate = [&](int64_t s0) __attribute__((always_inline)) {
    Piece pc;
    const int ug = static_cast<int>(s0 / sumT);
    const int o = static_cast<int>(s0 - static_cast<int64_t>(ug) * sumT);
    int lo_b = 0, hi_b = B;  // largest b with s_pre[b] <= o: s_pre[lo_b] <= o < s_pre[hi_b]
    while (hi_b - lo_b > 1) {
      const int mid = (lo_b + hi_b) >> 1;
      if (s_pre[mid] <= o) lo_b = mid; else hi_b = mid;
    }
    pc.b = lo_b;
    const int64_t seg_start = static_cast<int64_t>(ug) * sumT + s_pre[pc.b];
    const int64_t seg_end = static_cast<int64_t>(ug) * sumT + s_pre[pc.b + 1];
    pc.pe = min(s_end, seg_end);
    pc.pid = r + static_cast<int64_t>(ug) * B + pc.b;  // piece id
    const int unit = ug * UG + ul;  // unit = rtile * KVH + kvh
    pc.kvh = unit % p.KVH;
    pc.row0 = (unit / p.KVH) * RT;  // query row n of the tile is head kvh * G + row0 + n
    pc.nrows = min(RT, p.G - pc.row0);
    const int ctx = s_ctx[pc.b];  // stored before the scan's barriers
    const int lo_key = max(p.key_lo, p.window > 0 ? max(0, ctx - p.window) : 0);
    pc.t_first = lo_key / 16 + static_cast<int>(s0 - seg_start);
    pc.ntiles = static_cast<int>(pc.pe - s0);
    pc.a0 = max(lo_key, pc.t_first * 16);
    pc.a1 = min(ctx, (pc.t_first + pc.ntiles) * 16);
    return pc;
  };
  // Lane k: element offset of tile t_first + run0 + k of the piece, or -1 for a hole or
  // a lane past the run.
  auto table_run = [&](const Piece& pc, int run0) -> int64_t __attribute__((always_inline)) {
    const int nt = min(kSkTableRun, pc.ntiles - run0);
    int64_t mb = -1;
    if (lane < nt) {
      const int t = pc.t_first + run0 + lane;
      const int pg = (t * 16) / p.bs;
      const int slot0 = t * 16 - pg * p.bs;
      if (pg < p.W) {
        const int phys = p.table[static_cast<int64_t>(pc.b) * p.W + pg];
        if (phys >= 0 && phys < p.num_blocks)
          mb = static_cast<int64_t>(phys) * p.blk_stride +
               static_cast<int64_t>(slot0) * p.slot_stride +
               static_cast<int64_t>(pc.kvh) * p.head_stride;
      }
    }
    return mb;
  };
  // The same in two halves, so that the page id's load and its use are a run apart:
  // table_issue requests lane k's page id (-1 past the run or the table) and the
  // id-independent part of the offset; table_decode turns them into table_run's value.
  struct RunIds {
    int phys;
    int64_t rest;
  };
  auto table_issue = [&](const Piece& pc, int run0) -> RunIds __attribute__((always_inline)) {
    const int nt = min(kSkTableRun, pc.ntiles - run0);
    RunIds r{-1, 0};
    if (lane < nt) {
      const int t = pc.t_first + run0 + lane;
      const int pg = (t * 16) / p.bs;
      const int slot0 = t * 16 - pg * p.bs;
      r.rest = static_cast<int64_t>(slot0) * p.slot_stride +
               static_cast<int64_t>(pc.kvh) * p.head_stride;
      if (pg < p.W) r.phys = p.table[static_cast<int64_t>(pc.b) * p.W + pg];
    }
    return r;
  };
  auto table_decode = [&](const RunIds& r) -> int64_t __attribute__((always_inline)) {
    return r.phys >= 0 && r.phys < p.num_blocks
               ? static_cast<int64_t>(r.phys) * p.blk_stride + r.rest
               : int64_t(-1);
  };
  // The piece's query rows as the MFMA B operand (lane (g, n): row n, chunk j at dim
  // KV::qk_dim0(j, g), the split the K loads use).
  typedef typename QChunk<T>::type qchunk_t;
  auto load_q = [&](const Piece& pc, qchunk_t (&q)[JD]) __attribute__((always_inline)) {
    const T* qp = static_cast<const T*>(p.q);
    const int64_t orow_n = static_cast<int64_t>(pc.b) * p.H + pc.kvh * p.G + pc.row0 + n;
#pragma unroll
    for (int j = 0; j < JD; ++j) {
      q[j] = QChunk<T>::zero();
      if (n < pc.nrows) q[j] = QChunk<T>::load(qp + orow_n * D + KV::qk_dim0(j, g, JD));
    }
    if (p.rope_cos != nullptr && n < pc.nrows) {
      const int64_t po = static_cast<int64_t>(rope_position(p, pc.b)) * D;
      rope_chunks<T, KT, D>(q, p.rope_cos + po, p.rope_sin + po, g);
    }
  };

  // The first piece's query rows and first run's page ids, requested together and with
  // no branch around either load, so that the wave waits once for both (a load under a
  // lane condition whose result must merge with a default value makes the compiler wait
  // for it on the spot: four query chunks and the page id were five round trips).
  auto load_q_first = [&](const Piece& pc, qchunk_t (&q)[JD]) __attribute__((always_inline)) {
    const T* qp = static_cast<const T*>(p.q);
    // Lanes past the piece's rows load row 0 again: their MFMA columns' scores are
    // replaced by -inf before use (the masking in the tile loop tests n < nrows), and no
    // output or partial row is stored for them.
    const bool live = n < pc.nrows;
    const int64_t orow_n =
        static_cast<int64_t>(pc.b) * p.H + pc.kvh * p.G + pc.row0 + (live ? n : 0);
#pragma unroll
    for (int j = 0; j < JD; ++j) q[j] = QChunk<T>::load(qp + orow_n * D + KV::qk_dim0(j, g, JD));
    if (p.rope_cos != nullptr && live) {
      const int64_t po = static_cast<int64_t>(rope_position(p, pc.b)) * D;
      rope_chunks<T, KT, D>(q, p.rope_cos + po, p.rope_sin + po, g);
    }
  };
  auto table_first = [&](const Piece& pc) -> int64_t __attribute__((always_inline)) {
    const int nt = min(kSkTableRun, pc.ntiles);
    const int t = pc.t_first + lane;
    const int pg = (t * 16) / p.bs;
    const int slot0 = t * 16 - pg * p.bs;
    const bool ok = lane < nt && pg < p.W;  // other lanes read entry 0 and drop it
    const int phys = p.table[static_cast<int64_t>(pc.b) * p.W + (ok ? pg : 0)];
    const int64_t rest = static_cast<int64_t>(slot0) * p.slot_stride +
                         static_cast<int64_t>(pc.kvh) * p.head_stride;
    return ok && phys >= 0 && phys < p.num_blocks
               ? static_cast<int64_t>(phys) * p.blk_stride + rest
               : int64_t(-1);
  };

  if (s >= s_end) return;
  Piece cur = locate(s);
  int run0 = 0;
  qchunk_t qb[JD];
  load_q_first(cur, qb);
  int64_t my_base = table_first(cur);

  float m_run = -INFINITY;
  float l_run = 0.0f;
  float acc[RT][8];
#pragma unroll
  for (int rr = 0; rr < RT; ++rr)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[rr][e] = 0.0f;

  // Runs of up to kSkTableRun tiles, piece after piece. The next run's page ids (and a
  // new piece's query rows) are requested before this run streams, so they have landed
  // when it starts: a piece boundary costs no page-table round trip. The tile ring runs
  // on across runs: a run is rounded up to whole ring turns (the extra tiles read
  // nothing), and its last turn already issues the next run's first tiles, whose loads
  // are in flight while the piece's partial is written.
  // Fused append (APPEND instantiation, p.k_new set): the new token's K/V rows go to
  // cache position ctx - 1 of each sequence, in the last tile of its segment. The wave
  // whose piece holds that tile (one per KV head) requests the rows when the piece
  // starts, writes them to the cache (cast as msattn_write_kv casts them) and puts the
  // same values into the tile's registers in place of the row it loaded. No other piece
  // reads that position, so nothing waits for the store.
  // (Not over an fp8 cache: its 8-wave workgroups keep two waves a SIMD, where the held
  // chunks would spill.)
  constexpr bool kAppendOk = APPEND && sizeof(T) == 2 && sizeof(KT) != 1 && RT <= 8;
  int app_t = -1;  // absolute tile index of the current piece to patch, or -1
  int app_r = 0;   // the new token's row in that tile
  SrcChunk<T> kn[JD], vn;
  auto app_setup = [&](const Piece& pc) __attribute__((always_inline)) {
    const int ctx = s_ctx[pc.b];
    const int t_new = (ctx - 1) / 16;
    app_t = ctx > 0 && t_new >= pc.t_first && t_new < pc.t_first + pc.ntiles ? t_new : -1;
    if (app_t < 0) return;
    app_r = (ctx - 1) & 15;
    const int64_t row = (static_cast<int64_t>(pc.b) * p.KVH + pc.kvh) * D;
    if (tile_token<D>(n) == app_r) {
#pragma unroll
      for (int j = 0; j < JD; ++j)
        kn[j] = *reinterpret_cast<const SrcChunk<T>*>(static_cast<const T*>(p.k_new) + row +
                                                      KV::qk_dim0(j, g, JD));
    }
    if (va <= app_r && (app_r - va) % TPI == 0)
      vn = *reinterpret_cast<const SrcChunk<T>*>(static_cast<const T*>(p.v_new) + row + vc * 8);
  };
  auto app_patch = [&](raw_t (&kb)[JD], raw_t (&vb)[NJ], int64_t base) __attribute__((always_inline)) {
    if (base < 0) return;  // a hole: write_kv writes nothing there either
    const int64_t rowoff = base + static_cast<int64_t>(app_r) * p.slot_stride;
    if (tile_token<D>(n) == app_r) {
#pragma unroll
      for (int j = 0; j < JD; ++j) {
        const raw_t x = append_raw<KT, T, raw_t>(kn[j]);
        kb[j] = x;
        *reinterpret_cast<raw_t*>(const_cast<KT*>(kbase) + rowoff + KV::qk_dim0(j, g, JD)) = x;
      }
    }
    if (va <= app_r && (app_r - va) % TPI == 0) {
      const raw_t x = append_raw<KT, T, raw_t>(vn);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (TPI * j + va == app_r) vb[j] = x;
      *reinterpret_cast<raw_t*>(const_cast<KT*>(vbase) + rowoff + vc * 8) = x;
    }
  };
  if constexpr (kAppendOk) app_setup(cur);

  raw_t kq[DEPTH][JD], vq[DEPTH][NJ];
  int64_t bq[DEPTH];
  bool primed = false;  // the ring holds the run's first DEPTH - 1 tiles
  int prog = 0;         // ring positions consumed (kBalance)
  while (true) {
    const bool more_here = run0 + kSkTableRun < cur.ntiles;
    const bool next_piece = !more_here && cur.pe < s_end;
    Piece nxt = cur;
    int run_n = run0 + kSkTableRun;
    qchunk_t qn[JD];
    if (next_piece) {
      nxt = locate(cur.pe);
      run_n = 0;
      load_q(nxt, qn);
    }
    const bool has_next = more_here || next_piece;
    // The next run's page ids are requested now and decoded in this run's last ring turn,
    // where its first tiles are issued: the wait for them then falls a run after the
    // request (MSATTN_SK_LATE_IDS; decoding at once makes the wave wait here for the
    // table's round trip and for the tile in flight).
    RunIds ids_n{-1, 0};
    int64_t base_n = -1;
    if constexpr (MSATTN_SK_LATE_IDS) {
      if (has_next) ids_n = table_issue(nxt, run_n);
    } else {
      base_n = has_next ? table_run(nxt, run_n) : -1;
    }

    const int nt = min(kSkTableRun, cur.ntiles - run0);
    const int nt_ring = (nt + STEP - 1) / STEP * STEP;  // positions the ring walks
    const int nt_next = has_next ? min(kSkTableRun, nxt.ntiles - run_n) : 0;
    // Ring position k: tile k of this run, nothing (k < nt_ring), or tile k - nt_ring
    // of the next run.
    auto tile_base = [&](int k) -> int64_t __attribute__((always_inline)) {
      int64_t src = my_base;
      if (k >= nt) {
        k -= nt_ring;
        if (k < 0 || k >= nt_next) return -1;
        src = base_n;
      }
      const uint32_t lo = static_cast<uint32_t>(
          __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(src)), k));
      const int hi = __builtin_amdgcn_readlane(static_cast<int>(src >> 32), k);
      return static_cast<int64_t>(lo) | (static_cast<int64_t>(hi) << 32);
    };
    auto issue = [&](int64_t base, raw_t (&kb)[JD], raw_t (&vb)[NJ]) __attribute__((always_inline)) {
      const bool ok = base >= 0;
      const int64_t b0 = ok ? base : 0;
      const __amdgpu_buffer_rsrc_t rk = tile_rsrc(kbase + b0, ok ? tile_bytes : 0);
      const __amdgpu_buffer_rsrc_t rv = tile_rsrc(vbase + b0, ok ? tile_bytes : 0);
      KV::template load_k<MSATTN_LOAD_AUX, JD>(
          rk, k_lane_tok * static_cast<uint32_t>(p.slot_stride) * EB, g, kb);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        vb[j] = KV::template load<MSATTN_LOAD_AUX>(
            rv, ((static_cast<uint32_t>(TPI * j + va) * static_cast<uint32_t>(p.slot_stride)) +
                 vc * 8) * EB);
    };
    auto consume = [&](int k, const raw_t (&kb)[JD], const raw_t (&vb)[NJ], int64_t base) __attribute__((always_inline)) {
      mf_f32x4 sv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < JD; ++j) sv = Mfma16<T>::mac(KV::operand(kb[j]), qb[j], sv);
      const int t0 = (cur.t_first + run0 + k) * 16;
      const bool hole = base < 0;
      float sc[4];
      float mt = -INFINITY;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int tok = t0 + tile_token<D>(4 * g + q);
        const bool ok = !hole && n < cur.nrows && tok >= cur.a0 && tok < cur.a1;
        sc[q] = ok ? sv[q] * p.scale_log2 : -INFINITY;
        mt = fmaxf(mt, sc[q]);
      }
      mt = rows4_max(mt);
      const float m_new = fmaxf(m_run, mt);
      const bool live = m_new != -INFINITY;
      const float alpha = live ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
      float pr[4];
      float psum = 0.0f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        pr[q] = live ? __builtin_amdgcn_exp2f(sc[q] - m_new) : 0.0f;
        psum += pr[q];
      }
      l_run = fmaf(l_run, alpha, psum);
      m_run = m_new;
      if (!MSATTN_LAZY_RESCALE || __any(alpha != 1.0f)) {
        static_for<RT>([&](auto nc) {
          constexpr int rn = decltype(nc)::value;
          const float al = row_bcast<rn>(alpha);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[rn][e] *= al;
        });
      }
      const bool partial = hole || t0 < cur.a0 || t0 + 16 > cur.a1;
      raw_t vm[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        vm[j] = vb[j];
        if (partial) {
          const int vtok = t0 + TPI * j + va;
          vm[j] = KV::keep_if(vm[j], !hole && vtok >= cur.a0 && vtok < cur.a1);
        }
      }
      pv_tile<T, KT, D, RT>(acc, pr, vm, va);
    };

    // A ring of DEPTH tile buffers: DEPTH - 1 tiles' loads stay in flight while a
    // tile is consumed, the next tile's loads going into the slot just freed.
    // A position in [nt, nt_ring) reads nothing and adds nothing (its descriptor has
    // no records, all its keys are masked).
    {
      if (!primed) {
        static_for<DEPTH - 1>([&](auto dc) {
          constexpr int d = decltype(dc)::value;
          bq[d] = tile_base(d);
          issue(bq[d], kq[d], vq[d]);
        });
      }
      // The next run's ids are decoded after the issues of the turn before the last (the
      // last turn issues the next run's first tiles): those issues are younger than the
      // id's load on every path, so the wait for it holds back no tile in flight. (An
      // empty asm that rewrites the id keeps the decode, and that wait, here rather than
      // hoisted to the request.) A run of one turn decodes before it.
      auto decode_next = [&]() __attribute__((always_inline)) {
        asm volatile("" : "+v"(ids_n.phys));
        base_n = table_decode(ids_n);
      };
      if constexpr (MSATTN_SK_LATE_IDS) {
        if (nt <= STEP) decode_next();
      }
      for (int k = 0; k < nt; k += STEP) {
        static_for<STEP>([&](auto dc) {
          constexpr int d = decltype(dc)::value;
          constexpr int cu = d % DEPTH;
          constexpr int nx = (d + DEPTH - 1) % DEPTH;
          bq[nx] = tile_base(k + d + DEPTH - 1);
          issue(bq[nx], kq[nx], vq[nx]);
          if constexpr (kAppendOk) {
            if (k + d < nt && cur.t_first + run0 + k + d == app_t)
              app_patch(kq[cu], vq[cu], bq[cu]);
          }
          consume(k + d, kq[cu], vq[cu], bq[cu]);
        });
        if constexpr (MSATTN_SK_LATE_IDS) {
          if (k + STEP < nt && k + 2 * STEP >= nt) decode_next();
        }
        if constexpr (kBalance) {
          // Post this wave's progress; take priority while not ahead of the partner.
          // Both walk the same chunk, ring positions included, so counts compare.
          prog += STEP;
          if (lane == 0)
            __hip_atomic_store(&s_prog[w], prog, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
          const int other = __hip_atomic_load(&s_prog[w ^ (kSkWaves / 2)], __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_WORKGROUP);
          if (prog <= __builtin_amdgcn_readfirstlane(other))
            __builtin_amdgcn_s_setprio(1);
          else
            __builtin_amdgcn_s_setprio(0);
        }
      }
      primed = has_next;
    }

    if (!more_here) {
      // ---- wave totals and the piece's partial ----
      l_run = rows4_sum(l_run);
      // acc over the V token groups (lanes of equal lane % LPR), reduce-scattered: a
      // lane keeps dims vc * 8 + 2 * share + {0, 1} of each row.
      float red[RT * 2];
      reduce_scatter<LPR>(acc, red);
      const int64_t slot0 = (cur.pid * UG + ul) * RT;  // this unit's rows in the piece
      if (rs_owner<LPR>(lane)) {
        const int d0 = vc * 8 + 2 * rs_share<LPR>(lane);
#pragma unroll
        for (int rr = 0; rr < RT; ++rr) {
          if (rr < cur.nrows)
            *reinterpret_cast<float2*>(p.acc + (slot0 + rr) * D + d0) =
                make_float2(red[2 * rr], red[2 * rr + 1]);
        }
      }
      if (lane < cur.nrows) {
        float* ml = p.ml + (slot0 + lane) * 2;
        ml[0] = m_run;
        ml[1] = l_run;
      }
      if (!next_piece) break;
      m_run = -INFINITY;
      l_run = 0.0f;
#pragma unroll
      for (int rr = 0; rr < RT; ++rr)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[rr][e] = 0.0f;
#pragma unroll
      for (int j = 0; j < JD; ++j) qb[j] = qn[j];
    }
    cur = nxt;
    run0 = run_n;
    my_base = base_n;
    if constexpr (kAppendOk) {
      if (run0 == 0) app_setup(cur);  // a new piece
    }
  }
}

template <typename T, typename KT, int D, int RT>
hipError_t launch_decode_streamk_one(const SplitParams& p, int grid, hipStream_t stream) {
  // the fused append's instantiation (the host sets k_new only where it is built)
  if constexpr (sizeof(T) == 2 && sizeof(KT) != 1 && RT <= 8) {
    if (p.k_new != nullptr) {
      hipLaunchKernelGGL((decode_streamk_kernel<T, KT, D, RT, true>),
                         dim3(static_cast<unsigned>(grid)),
                         dim3(sk_waves(sizeof(KT), sizeof(T)) * kWave), 0, stream, p);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((decode_streamk_kernel<T, KT, D, RT>), dim3(static_cast<unsigned>(grid)),
                     dim3(sk_waves(sizeof(KT), sizeof(T)) * kWave), 0, stream, p);
  return hipGetLastError();
}

// Launch for T in {bf16_t, _Float16} and a KV cache of T or of fp8_t;
// *supported = false when (D, RT) is not compiled.
template <typename T, typename KT>
hipError_t launch_decode_streamk(const SplitParams& p, int D, int RT, int grid, hipStream_t stream,
                                 bool* supported);

#define MSATTN_DECLARE_SK_LAUNCHER(T, KT)                                                    \
  template <>                                                                                \
  hipError_t launch_decode_streamk<T, KT>(const SplitParams& p, int D, int RT, int grid,     \
                                          hipStream_t stream, bool* supported);
MSATTN_DECLARE_SK_LAUNCHER(bf16_t, bf16_t)
MSATTN_DECLARE_SK_LAUNCHER(_Float16, _Float16)
MSATTN_DECLARE_SK_LAUNCHER(bf16_t, fp8_t)
MSATTN_DECLARE_SK_LAUNCHER(_Float16, fp8_t)
MSATTN_DECLARE_SK_LAUNCHER(bf16_t, float)
MSATTN_DECLARE_SK_LAUNCHER(_Float16, float)
MSATTN_DECLARE_SK_LAUNCHER(float, float)
MSATTN_DECLARE_SK_LAUNCHER(float, bf16_t)
MSATTN_DECLARE_SK_LAUNCHER(float, _Float16)
MSATTN_DECLARE_SK_LAUNCHER(float, fp8_t)
#undef MSATTN_DECLARE_SK_LAUNCHER

#define MSATTN_SK_RT(T, KT, D)                                                      \
  switch (RT) {                                                                     \
    case 1: return launch_decode_streamk_one<T, KT, D, 1>(p, grid, stream);         \
    case 2: return launch_decode_streamk_one<T, KT, D, 2>(p, grid, stream);         \
    case 4: return launch_decode_streamk_one<T, KT, D, 4>(p, grid, stream);         \
    case 8: return launch_decode_streamk_one<T, KT, D, 8>(p, grid, stream);         \
    case 16: return launch_decode_streamk_one<T, KT, D, 16>(p, grid, stream);       \
    default: break;                                                                 \
  }

#define MSATTN_SK_LAUNCHER(T, KT)                                                            \
  template <>                                                                                \
  hipError_t launch_decode_streamk<T, KT>(const SplitParams& p, int D, int RT, int grid,     \
                                          hipStream_t stream, bool* supported) {             \
    *supported = true;                                                                       \
    if (D == 64) { MSATTN_SK_RT(T, KT, 64) }                                                 \
    if (D == 128) { MSATTN_SK_RT(T, KT, 128) }                                               \
    *supported = false;                                                                      \
    return hipSuccess;                                                                       \
  }

}  // namespace msattn
