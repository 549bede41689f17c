// Split-K paged attention partials for gfx950 (templates; instantiated per dtype
// pair in split_*.hip).
//
// One workgroup (4 waves) owns one (sequence b, KV head, row tile, context
// partition). A row tile packs up to RT query rows that read the same KV head:
// the `group` GQA heads of that KV head, times the q_len query tokens. The
// workgroup walks the partition's tokens through the block table and writes a
// partial (m, l, acc) per row into workspace slot `part`:
//   m   = max_k  s_k              with s_k = scale * log2(e) * q . K[k]
//   l   = sum_k  2^(s_k - m)
//   acc = sum_k  2^(s_k - m) V[k]
// over the row's unmasked keys in the partition. The slot after a row's last
// partition gets the end marker (m = -inf, l = -1) unless it is past the
// workspace. merge.hip combines a row's slots up to that marker.
//
// Phases (barriers between them):
//   0  page-table walk: one byte offset per token of the partition into LDS
//      (holes and positions outside every row's key range get -1);
//   1  scores: each wave streams K rows with 16-byte loads, LPR lanes per row,
//      so one wave load instruction covers TPI = 64 / LPR tokens; per-lane dot
//      products are summed across the LPR lanes;
//   2  softmax statistics per row over the partition (wave reductions);
//   3  P.V: the same token walk over V, fp32 accumulators per lane, reduced
//      across lanes and waves through LDS.
//
// K/V elements are widened to fp32 and, when the cache type is wider than or differs
// from the query type, rounded to the query type first (KvCast, common.h): the cast of
// the gathered K/V to query.dtype in miniserve/attention.py:240-241.
//
// The algorithm is the split decomposition of kernels/paged_attn_triton.py
// (_split_kernel :176-248, reference restatement :102-171); the masking rules
// are PagedAttention.build_mask (miniserve/attention.py:135-153).
#pragma once

#include <climits>

#include "common.h"

namespace msattn {

constexpr int kSplitThreads = 256;
constexpr int kSplitWaves = kSplitThreads / kWave;
// Largest context partition (tokens) one workgroup covers.
#ifndef MSATTN_PART_MAX
#define MSATTN_PART_MAX 512
#endif
constexpr int kPartMax = MSATTN_PART_MAX;

// Workspace header (first bytes of every workspace): which partial layout the
// partials kernel used, so the merge can read it back.
//   hdr[0] kind: 0 = per-row slots closed by end markers (partition kernels);
//                1 = stream-K pieces (decode_streamk.h);
//                2 = partition kernel that merged in-kernel and wrote the output
//   kind 1 also: hdr[1] sumT, [2] chunk c, [3] sub-ranges, [4] UG, [5] NUG, [6] B,
//   [7] RT, and hdr[kHdrPrefix + b] = tiles of sequences before b (b = 0..B).
//   A chunked prefill on the prefill kernel's stream-K schedule writes hdr[kHdrPrefix + t]
//   = work-list offset of task t (t = 0..tasks) and hdr[kHdrPrefix + tasks + 1] = the
//   list's head size, for its fold launch.
//   kinds 0 and 2 (partition kernels) also: hdr[8] partition tokens, [9] waves per
//   workgroup, [14] workgroups a CU may hold (the launch's shape, for tests and
//   measurements; the merge does not read them).
//   hdr[kHdrTickets + t], t < kMaxTickets: arrival counters of the in-kernel merge, one
//   per (sequence, KV head, row tile). They sit at the same offset for every geometry,
//   must be zero when a workspace is first used, and every call leaves them zero.
constexpr int kHdrTickets = 64;
constexpr int kMaxTickets = 4096;
constexpr int kHdrPrefix = kHdrTickets + kMaxTickets;
constexpr int kHdrKind = 0, kHdrSumT = 1, kHdrChunk = 2, kHdrNsub = 3, kHdrUG = 4,
              kHdrNUG = 5, kHdrB = 6, kHdrRT = 7, kHdrPart = 8, kHdrWaves = 9,
              kHdrResidency = 14;

struct SplitParams {
  int* hdr;
  const void* q;
  const void* k;
  const void* v;
  const int32_t* table;
  const int32_t* lens;
  float* ml;   // [rows][max_parts][2]
  float* acc;  // [rows][max_parts][D]
  int64_t blk_stride, slot_stride, head_stride;  // elements
  int batch, q_len, H, KVH, G;
  int bs, num_blocks, W;
  int max_ctx, max_parts, part;
  int causal, window;
  float scale_log2;
  int rows_per_kvh;  // q_len * G
  int rtiles;        // ceil(rows_per_kvh / RT)
  // The MFMA partition kernel's grid order (set by its launcher): 1 = one flat x index
  // kvh + KVH (rtile + rtiles (b + batch part)), partition-major, so that every sequence's
  // first partitions are dispatched before any sequence's later (often empty) ones;
  // 0 = x = kvh + KVH (part + max_parts rtile), z = b.
  int part_major;
  int sk_group;        // stream-K: KV-head units per unit group
  int sk_unit_groups;  // stream-K: number of unit groups
  int sk_min_chunk;    // stream-K: smallest chunk (tiles)
  // Optional rotate-half RoPE of the query at position rope_pos[b] (decode):
  // q' = q * cos[pos] + rotate_half(q) * sin[pos], fp32 tables [rope_max_pos, D].
  int key_lo;             // keys below this position are excluded (a shared prefix
                          // handled by another pass); 0 for none
  const float* rope_cos;  // nullptr: no RoPE
  const float* rope_sin;
  const int32_t* rope_pos;
  int rope_max_pos;
  // In-kernel merge (partition MFMA kernel only): non-null `out` [rows][D] of the query
  // type makes the last partition of each (sequence, KV head, row tile) to arrive merge
  // its partials and write the output; `tickets` are the header's arrival counters.
  void* out;
  int* tickets;
  int mfma_waves;  // partition MFMA kernel: waves per workgroup (4, or 8 for long partitions)
  int mfma_deep;   // partition MFMA kernel, regular shape at head_dim 64: the deeper residency
  int head_dim;    // the row's head size (the generic kernel's element mode compiles a larger
                   // capacity and masks the dims past it)
  int rows16;      // cache rows start on 16-byte boundaries and hold whole 16-byte chunks
  // Fused append (partition MFMA kernel, q_len 1): non-null k_new / v_new, contiguous
  // [batch, KVH, D] rows of the query type, 16-byte aligned: row (b, kvh) goes to cache
  // position lens[b] - 1 (cast to the cache type) before the decode reads it.
  const void* k_new;
  const void* v_new;
};

// One 16-byte chunk of a K/V row as the generic kernel's lanes read it. Whole chunks of
// rows on 16-byte boundaries load as one 16-byte load; otherwise the `valid` leading
// elements (the row's last, partial chunk, or rows on 2- or 4-byte boundaries) load one
// by one and the rest of the chunk reads as zeros.
template <typename KT>
__device__ __forceinline__ uint4 load_kv_chunk(const KT* src, int valid, bool vec16) {
  constexpr int EB = Elt<KT>::kBytes;
  constexpr int N = 16 / EB;
  if (vec16 && valid >= N) return *reinterpret_cast<const uint4*>(src);
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int e = 0; e < N; ++e) {
    if (e < valid) {
      uint32_t bits;
      if constexpr (EB == 4) bits = reinterpret_cast<const uint32_t*>(src)[e];
      else if constexpr (EB == 2) bits = reinterpret_cast<const uint16_t*>(src)[e];
      else bits = reinterpret_cast<const uint8_t*>(src)[e];
      w[(e * EB) / 4] |= bits << (8 * ((e * EB) % 4));
    }
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Position of row b's query for RoPE, clamped into the tables.
__device__ __forceinline__ int rope_position(const SplitParams& p, int b) {
  int pos = p.rope_pos[b];
  pos = pos < 0 ? 0 : (pos >= p.rope_max_pos ? p.rope_max_pos - 1 : pos);
  return pos;
}

// q * c + r * s in fp32 with every product and sum rounded on its own (contraction
// into a fused multiply-add is switched off here), the evaluation of (q * cos + rotate_half(q) * sin) as separate
// elementwise tensor ops.
__device__ __forceinline__ float rope_mix(float q, float r, float c, float s) {
#pragma clang fp contract(off)
  const float a = q * c;
  const float b = r * s;
  return a + b;
}

// ELEM = false: head_dim == D, rows read with 16-byte loads. ELEM = true: D is a capacity
// (16, 32, 64, 128 or 256) and the row's head_dim (p.head_dim <= D) any even size; rows
// load chunk by chunk through load_kv_chunk, dims past head_dim read as zeros and are
// not written.
template <typename QT, typename KT, int D, int RT, bool ELEM>
__global__ __launch_bounds__(kSplitThreads) void split_kernel(const SplitParams p) {
  using CK = Chunk<KT>;
  constexpr int EPL = CK::kElems;                      // KV elements per 16 B
  static_assert((D * Elt<KT>::kBytes) % 16 == 0, "row must be whole 16-byte chunks");
  constexpr int CHUNKS = D * Elt<KT>::kBytes / 16;     // 16-byte chunks per row (capacity)
  const int HD = ELEM ? p.head_dim : D;                // the row's head size
  constexpr int LPR = next_pow2(CHUNKS);               // lanes per K/V row
  static_assert(LPR <= kWave, "row wider than a wave");
  constexpr int TPI = kWave / LPR;                     // tokens per wave instruction
  constexpr int U = TPI >= 8 ? 2 : 4;                  // load instructions in flight
  constexpr int SC_SCORES = kPartMax * RT;
  constexpr int SC_REDUCE = kSplitWaves * RT * D;
  constexpr int SC = SC_SCORES > SC_REDUCE ? SC_SCORES : SC_REDUCE;

  __shared__ int64_t s_off[kPartMax];
  __shared__ float s_sc[SC];
  __shared__ float s_m[RT];
  __shared__ float s_l[RT];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int w = tid / kWave;
  if (tid == 0 && blockIdx.x == 0 && blockIdx.z == 0) {
    p.hdr[kHdrKind] = 0;
    p.hdr[kHdrPart] = p.part;
    p.hdr[kHdrWaves] = kSplitWaves;
    p.hdr[kHdrResidency] = 0;
  }

  // blockIdx.x = part + max_parts * (kvh + KVH * rtile); blockIdx.z = b.
  const int part = static_cast<int>(blockIdx.x % static_cast<unsigned>(p.max_parts));
  const int rest = static_cast<int>(blockIdx.x / static_cast<unsigned>(p.max_parts));
  const int kvh = rest % p.KVH;
  const int rtile = rest / p.KVH;
  const int b = blockIdx.z;

  int ctx = p.lens[b];
  ctx = ctx < 0 ? 0 : (ctx > p.max_ctx ? p.max_ctx : ctx);
  const int nparts = ctx > 0 ? ceil_div(ctx, p.part) : 1;
  if (part >= nparts) return;

  const int row0 = rtile * RT;
  const int nrows = min(RT, p.rows_per_kvh - row0);

  // Per-row key ranges [lo, hi) (attention.py:143-153 with q_pos = ctx - q_len + i).
  int lo_r[RT], hi_r[RT];
  int lo_all = INT_MAX, hi_all = INT_MIN;
  int64_t orow[RT];
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    lo_r[r] = 0;
    hi_r[r] = 0;
    orow[r] = 0;
    if (r < nrows) {
      const int gr = row0 + r;
      const int i = gr / p.G;
      const int g = gr - i * p.G;
      const int qpos = ctx - p.q_len + i;
      int hi = p.causal ? min(ctx, qpos + 1) : ctx;
      int lo = max(p.key_lo, p.window > 0 ? max(0, qpos - p.window + 1) : 0);
      if (hi < lo) hi = lo;
      lo_r[r] = lo;
      hi_r[r] = hi;
      if (hi > lo) {
        lo_all = min(lo_all, lo);
        hi_all = max(hi_all, hi);
      }
      orow[r] = (static_cast<int64_t>(b) * p.q_len + i) * p.H + (kvh * p.G + g);
    }
  }

  const int tok0 = part * p.part;
  const int tok1 = min(tok0 + p.part, ctx);
  const int a0 = max(tok0, lo_all);
  const int a1 = min(tok1, hi_all);
  if (a1 <= a0) {  // nothing to attend to in this partition: m = -inf, l = 0
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      if (r < nrows && tid == r) {
        float* ml = p.ml + (orow[r] * p.max_parts + part) * 2;
        ml[0] = -INFINITY;
        ml[1] = 0.0f;
        if (part + 1 == nparts && nparts < p.max_parts) {  // end marker
          ml[2] = -INFINITY;
          ml[3] = -1.0f;
        }
      }
    }
    return;
  }
  const int n_tok = tok1 - tok0;

  // Phase 0: page-table walk (attention.py:163-171; paged_attn_triton.py:228-231).
  for (int t = tid; t < n_tok; t += kSplitThreads) {
    const int tok = tok0 + t;
    int64_t off = -1;
    if (tok >= a0 && tok < a1) {
      const int pg = tok / p.bs;
      const int slot = tok - pg * p.bs;
      if (pg < p.W) {
        const int phys = p.table[static_cast<int64_t>(b) * p.W + pg];
        if (phys >= 0 && phys < p.num_blocks)
          off = static_cast<int64_t>(phys) * p.blk_stride +
                static_cast<int64_t>(slot) * p.slot_stride +
                static_cast<int64_t>(kvh) * p.head_stride;
      }
    }
    s_off[t] = off;
  }

  // Query rows for this lane's chunk of dims, pre-scaled by scale*log2(e).
  const int c = lane % LPR;
  const int tg = lane / LPR;
  // Lanes past the row's last (possibly partial) chunk hold no dims.
  const bool c_ok = ELEM ? c * EPL < HD : c < CHUNKS;
  const int c_valid = HD - c * EPL;  // elements of this lane's chunk inside the row
  const bool vec16 = !ELEM || p.rows16 != 0;
  float qreg[RT][EPL];
  {
    const QT* qp = static_cast<const QT*>(p.q);
#pragma unroll
    for (int r = 0; r < RT; ++r) {
#pragma unroll
      for (int e = 0; e < EPL; ++e) qreg[r][e] = 0.0f;
      if (r < nrows && c_ok) {
        const QT* src = qp + orow[r] * HD + c * EPL;
        float qv[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) qv[e] = (!ELEM || e < c_valid) ? Elt<QT>::load(src + e) : 0.0f;
        if (p.rope_cos != nullptr) {  // rotate-half RoPE, rounded back to QT
          const int64_t po = static_cast<int64_t>(rope_position(p, b)) * HD;
#pragma unroll
          for (int e = 0; e < EPL; ++e) {
            const int d = c * EPL + e;
            if (ELEM && d >= HD) continue;
            const bool lo_half = d < HD / 2;
            const float partner =
                Elt<QT>::load(qp + orow[r] * HD + (lo_half ? d + HD / 2 : d - HD / 2));
            qv[e] = round_to<QT>(rope_mix(qv[e], lo_half ? -partner : partner, p.rope_cos[po + d],
                                          p.rope_sin[po + d]));
          }
        }
#pragma unroll
        for (int e = 0; e < EPL; ++e) qreg[r][e] = qv[e] * p.scale_log2;
      }
    }
  }
  __syncthreads();

  const int nslots = ceil_div(n_tok, TPI);
  const KT* kbase = static_cast<const KT*>(p.k);
  const KT* vbase = static_cast<const KT*>(p.v);

  // Phase 1: scores into s_sc[t * RT + r].
  for (int s0 = w; s0 < nslots; s0 += kSplitWaves * U) {
    uint4 raw[U];
    int64_t offs[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = s0 + u * kSplitWaves;
      const int t = s * TPI + tg;
      const int64_t off = (s < nslots && t < n_tok) ? s_off[t] : -1;
      offs[u] = off;
      raw[u] = make_uint4(0u, 0u, 0u, 0u);
      if (off >= 0 && c_ok) raw[u] = load_kv_chunk(kbase + off + c * EPL, c_valid, vec16);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float kf[EPL];
      CK::unpack(raw[u], kf);
      KvCast<QT, KT>::apply(kf);
      float dot[RT];
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        float a = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) a = fmaf(qreg[r][e], kf[e], a);
        dot[r] = group_sum<LPR>(a);
      }
      const int s = s0 + u * kSplitWaves;
      const int t = s * TPI + tg;
      if (c == 0 && s < nslots && t < n_tok) {
        const int tok = tok0 + t;
#pragma unroll
        for (int r = 0; r < RT; ++r) {
          const bool ok = offs[u] >= 0 && tok >= lo_r[r] && tok < hi_r[r];
          s_sc[t * RT + r] = ok ? dot[r] : -INFINITY;
        }
      }
    }
  }
  __syncthreads();

  // Phase 2: per-row max and sum over the partition; scores become weights.
  for (int r = w; r < RT; r += kSplitWaves) {
    float mx = -INFINITY;
    for (int t = lane; t < n_tok; t += kWave) mx = fmaxf(mx, s_sc[t * RT + r]);
    mx = group_max<kWave>(mx);
    float sum = 0.0f;
    for (int t = lane; t < n_tok; t += kWave) {
      const float pr = mx == -INFINITY ? 0.0f : exp2f(s_sc[t * RT + r] - mx);
      s_sc[t * RT + r] = pr;
      sum += pr;
    }
    sum = group_sum<kWave>(sum);
    if (lane == 0) {
      s_m[r] = mx;
      s_l[r] = sum;
    }
  }
  __syncthreads();

  // Phase 3: acc[r][:] = sum_t w[t][r] V[t][:].
  float acc[RT][EPL];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[r][e] = 0.0f;

  for (int s0 = w; s0 < nslots; s0 += kSplitWaves * U) {
    uint4 raw[U];
    int tt[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = s0 + u * kSplitWaves;
      const int t = s * TPI + tg;
      const int64_t off = (s < nslots && t < n_tok) ? s_off[t] : -1;
      tt[u] = off >= 0 ? t : -1;
      raw[u] = make_uint4(0u, 0u, 0u, 0u);
      if (off >= 0 && c_ok) raw[u] = load_kv_chunk(vbase + off + c * EPL, c_valid, vec16);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (tt[u] >= 0) {
        float vf[EPL];
        CK::unpack(raw[u], vf);
        KvCast<QT, KT>::apply(vf);
#pragma unroll
        for (int r = 0; r < RT; ++r) {
          const float pr = s_sc[tt[u] * RT + r];
#pragma unroll
          for (int e = 0; e < EPL; ++e) acc[r][e] = fmaf(pr, vf[e], acc[r][e]);
        }
      }
    }
  }

  // Reduce over the TPI token groups of the wave (lanes c, c + LPR, ...), reduce-scattered:
  // a lane keeps elements share * PER .. + PER - 1 of its chunk in every row.
  constexpr int RSP = rs_parts(LPR);
  constexpr int PER = EPL / RSP;
  float red[RT * PER];
  reduce_scatter<LPR>(acc, red);
  __syncthreads();  // every wave is done reading weights from s_sc
  if (rs_owner<LPR>(lane) && c_ok) {
    const int e0 = c * EPL + rs_share<LPR>(lane) * PER;
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int e = 0; e < PER; ++e) s_sc[(w * RT + r) * D + e0 + e] = red[r * PER + e];
  }
  __syncthreads();

  for (int idx = tid; idx < nrows * HD; idx += kSplitThreads) {
    const int r = idx / HD;
    const int d = idx - r * HD;
    float a = 0.0f;
#pragma unroll
    for (int ww = 0; ww < kSplitWaves; ++ww) a += s_sc[(ww * RT + r) * D + d];
    int64_t orr = 0;
#pragma unroll
    for (int rr = 0; rr < RT; ++rr)
      if (rr == r) orr = orow[rr];
    p.acc[(orr * p.max_parts + part) * HD + d] = a;
  }
#pragma unroll
  for (int r = 0; r < RT; ++r) {
    if (r < nrows && tid == r) {
      float* ml = p.ml + (orow[r] * p.max_parts + part) * 2;
      ml[0] = s_m[r];
      ml[1] = s_l[r];
      if (part + 1 == nparts && nparts < p.max_parts) {  // end marker
        ml[2] = -INFINITY;
        ml[3] = -1.0f;
      }
    }
  }
}

// Host-side launch for one dtype pair; defined in split_<pair>.hip.
template <typename QT, typename KT>
hipError_t launch_split(const SplitParams& p, int D, int RT, bool rows16, hipStream_t stream,
                        bool* supported);

template <typename QT, typename KT, int D, int RT, bool ELEM>
hipError_t launch_split_one(const SplitParams& p, hipStream_t stream) {
  const unsigned gx = static_cast<unsigned>(p.max_parts) * static_cast<unsigned>(p.KVH) *
                      static_cast<unsigned>(p.rtiles);
  dim3 grid(gx, 1, static_cast<unsigned>(p.batch));
  hipLaunchKernelGGL((split_kernel<QT, KT, D, RT, ELEM>), grid, dim3(kSplitThreads), 0, stream, p);
  return hipGetLastError();
}

// One head size (or, ELEM, capacity): row tiles of 1, 2, 4 or 8 query rows; head sizes
// whose K/V row is not whole 16-byte chunks of the cache type are not compiled.
template <typename QT, typename KT, int D, bool ELEM>
hipError_t launch_split_d(const SplitParams& p, int RT, hipStream_t stream, bool* supported) {
  if constexpr ((D * Elt<KT>::kBytes) % 16 == 0) {
    switch (RT) {
      case 1: return launch_split_one<QT, KT, D, 1, ELEM>(p, stream);
      case 2: return launch_split_one<QT, KT, D, 2, ELEM>(p, stream);
      case 4: return launch_split_one<QT, KT, D, 4, ELEM>(p, stream);
      case 8: return launch_split_one<QT, KT, D, 8, ELEM>(p, stream);
      default: break;
    }
  }
  *supported = false;
  return hipSuccess;
}

// Explicit specializations, one per compiled dtype pair (split_<pair>.hip): head dims
// 16, 24, 32, 64, 96, 128 and 256 with 16-byte rows (24 only where a row is whole 16-byte
// chunks); any other even head_dim up to 256, or rows off 16-byte boundaries, on the
// element mode at the next capacity of 16, 32, 64, 128 or 256.
#define MSATTN_SPLIT_LAUNCHER(QT, KT)                                                      \
  template <>                                                                              \
  hipError_t launch_split<QT, KT>(const SplitParams& p, int D, int RT, bool rows16,        \
                                  hipStream_t stream, bool* supported) {                   \
    *supported = true;                                                                     \
    if (rows16 && (D * Elt<KT>::kBytes) % 16 == 0) {                                       \
      switch (D) {                                                                         \
        case 16: return launch_split_d<QT, KT, 16, false>(p, RT, stream, supported);       \
        case 24: return launch_split_d<QT, KT, 24, false>(p, RT, stream, supported);       \
        case 32: return launch_split_d<QT, KT, 32, false>(p, RT, stream, supported);       \
        case 64: return launch_split_d<QT, KT, 64, false>(p, RT, stream, supported);       \
        case 96: return launch_split_d<QT, KT, 96, false>(p, RT, stream, supported);       \
        case 128: return launch_split_d<QT, KT, 128, false>(p, RT, stream, supported);     \
        case 256: return launch_split_d<QT, KT, 256, false>(p, RT, stream, supported);     \
        default: break;                                                                    \
      }                                                                                    \
    }                                                                                      \
    if (D <= 16) return launch_split_d<QT, KT, 16, true>(p, RT, stream, supported);        \
    if (D <= 32) return launch_split_d<QT, KT, 32, true>(p, RT, stream, supported);        \
    if (D <= 64) return launch_split_d<QT, KT, 64, true>(p, RT, stream, supported);        \
    if (D <= 128) return launch_split_d<QT, KT, 128, true>(p, RT, stream, supported);      \
    if (D <= 256) return launch_split_d<QT, KT, 256, true>(p, RT, stream, supported);      \
    *supported = false;                                                                    \
    return hipSuccess;                                                                     \
  }

#define MSATTN_DECLARE_SPLIT(QT, KT)                                                   \
  template <>                                                                          \
  hipError_t launch_split<QT, KT>(const SplitParams& p, int D, int RT, bool rows16,    \
                                  hipStream_t stream, bool* supported);
MSATTN_DECLARE_SPLIT(float, float)
MSATTN_DECLARE_SPLIT(float, _Float16)
MSATTN_DECLARE_SPLIT(float, bf16_t)
MSATTN_DECLARE_SPLIT(float, fp8_t)
MSATTN_DECLARE_SPLIT(_Float16, float)
MSATTN_DECLARE_SPLIT(_Float16, _Float16)
MSATTN_DECLARE_SPLIT(_Float16, bf16_t)
MSATTN_DECLARE_SPLIT(_Float16, fp8_t)
MSATTN_DECLARE_SPLIT(bf16_t, float)
MSATTN_DECLARE_SPLIT(bf16_t, _Float16)
MSATTN_DECLARE_SPLIT(bf16_t, bf16_t)
MSATTN_DECLARE_SPLIT(bf16_t, fp8_t)
#undef MSATTN_DECLARE_SPLIT

}  // namespace msattn
