// Chunked-prefill paged attention on MFMA (gfx950): q_len > 1, bf16/fp16 query (over a
// cache of its type or of fp8 e4m3), head_dim 64 or 128.
//
// One workgroup owns 128 query rows of one (sequence b, KV head): rows are the (query
// token i, GQA head g) pairs r = i * group + g. It has two groups of 4 waves, one wave of
// each group per SIMD: both groups hold the same rows (32 per wave, one 32-row MFMA
// block, so every K/V operand it reads from LDS feeds a 32-row product) and split the
// keys, group 0 taking the even 64-token steps and group 1 the odd ones; the two running
// (m, l, O) are merged through LDS at the end. With two waves per SIMD, one wave's softmax
// and LDS traffic overlap the other's MFMAs. Per group and step:
//   * K and V of the step are staged through the group's LDS buffers, double-buffered
//     (copied there by the load unit for a cache of the query's type, through registers
//     for the converted caches); one barrier per step pair;
//   * S^T = K Q^T on v_mfma_f32_32x32x16, one 32-key tile at a time: A = K rows read from
//     LDS, B = the wave's query rows kept in registers, so lane (cc = l % 32, hh = l / 32)
//     holds the scores of query row cc for keys (v & 3) + 8 (v >> 2) + 4 hh of the tile
//     in register v. The longer MFMA (32 cycles, half as many per step as 16x16x32) leaves
//     more issue slots between MFMAs for the softmax's VALU work (a standalone probe with
//     two waves per SIMD: 810 -> 688 cycles for the same MFMA and VALU work);
//   * online softmax per row (fp32, base 2), causal / window masks only on the steps that
//     cross a row's key range; a row's keys are split over the two lane halves;
//   * O^T += V^T P^T on the same MFMA, in 16-key chunks: B = P^T comes straight from the
//     score registers (registers 8 c .. 8 c + 7 are chunk c's keys 4 hh .. + 3 and
//     8 + 4 hh .. + 3), A = V^T is read transposed from the row-major V rows with
//     ds_read_b64_tr_b16 (each lane names 4 dims of one token; lane i of a 16-lane group
//     receives dim i of four tokens), so lane (cc, hh) accumulates O[row cc][dims
//     32 t + (v & 3) + 8 (v >> 2) + 4 hh] and the softmax rescale stays in the lane.
// LDS rows of copied K/V are unpadded with a 16-byte chunk swizzle; the register-staged
// rows are padded (K rows D + 8 elements apart, V rows D + 16).
// A task's rows are normalised and written directly, or, on the stream-K schedule, left as
// partials for the fold launch when the task is split between workgroups.
//
// Semantics: PagedAttention.forward with q_len > 1 (miniserve/attention.py:205-250,
// mask :135-153; the trailing query positions q_pos = len - q_len + i, :146).
#pragma once

#include "decode_mfma.h"
#include "pf_streamk.h"

#ifndef MSATTN_PF_RB
#define MSATTN_PF_RB 2
#endif
// K/V of a cache of the query's type copied into LDS by the load unit (1), or staged
// through registers like the converted caches (0).
#ifndef MSATTN_PF_DMA
#define MSATTN_PF_DMA 1
#endif
// Interleaving of MFMA and VALU work requested from the scheduler on the copy path:
// MSATTN_PF_NV VALU instructions after each MFMA of a half-step block.
#ifndef MSATTN_PF_SCHED
#define MSATTN_PF_SCHED 1
#endif
#ifndef MSATTN_PF_NV
#define MSATTN_PF_NV 3
#endif
// Wave priority of key group 1 over its loop (copy path).
#ifndef MSATTN_PF_G1PRIO
#define MSATTN_PF_G1PRIO 1
#endif
// Wave priority of the copy path's MFMA-only blocks (the first half-step's scores and the
// second half-step's P.V), above both groups' loop priorities, so that a SIMD's matrix core
// is fed first when both waves are ready; 0 leaves them at the group's priority.
#ifndef MSATTN_PF_MPRIO
#define MSATTN_PF_MPRIO 2
#endif

namespace msattn {

typedef float mf_f32x16 __attribute__((ext_vector_type(16)));
// One 32x32x16 MFMA: C[32 x 32] += A[32 x 16] B[16 x 32]. Lane l holds A's row l % 32 and
// B's column l % 32, elements k = 8 (l / 32) .. + 7 of each; and C's column l % 32, rows
// (v & 3) + 8 (v >> 2) + 4 (l / 32) in its registers v = 0 .. 15.
template <typename T> struct Mfma32;
template <> struct Mfma32<bf16_t> {
  __device__ static mf_f32x16 mac(const uint4& a, const uint4& b, mf_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(mf_bf16x8, a),
                                                   __builtin_bit_cast(mf_bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma32<_Float16> {
  __device__ static mf_f32x16 mac(const uint4& a, const uint4& b, mf_f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(mf_f16x8, a),
                                                  __builtin_bit_cast(mf_f16x8, b), c, 0, 0, 0);
  }
};
__device__ __forceinline__ mf_f32x16 zero16() {
  mf_f32x16 z;
#pragma unroll
  for (int e = 0; e < 16; ++e) z[e] = 0.0f;
  return z;
}
// Max / sum over the two 32-lane halves of the wave (lanes i and i + 32), every lane
// receiving it (v_permlane32_swap; with MSATTN_ROW_SWAPS=0 a lane shuffle).
__device__ __forceinline__ float halves_max(float v) {
#if MSATTN_ROW_SWAPS
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
#else
  return fmaxf(v, __shfl_xor(v, 32, kWave));
#endif
}
__device__ __forceinline__ float halves_sum(float v) {
#if MSATTN_ROW_SWAPS
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
#else
  return v + __shfl_xor(v, 32, kWave);
#endif
}

constexpr int kPfWaves = 4;                     // waves per key group (one per SIMD)
constexpr int kPfGroups = 2;                    // key groups: even / odd steps
constexpr int kPfGroupThreads = kPfWaves * kWave;
constexpr int kPfThreads = kPfGroups * kPfGroupThreads;
constexpr int kPfRB = MSATTN_PF_RB;             // query rows per wave / 16 (2: one 32-row block)
constexpr int kPfRows = 16 * kPfRB * kPfWaves;  // query rows per workgroup
constexpr int kPfStep = 64;                     // key tokens per step
constexpr int kPfPageChunk = 512;               // page ids cached in LDS at a time
// Workgroups are dispatched to the 8 XCDs round-robin (workgroup i runs on XCD i % 8),
// and each XCD has its own L2. The (sequence, KV head, row block) tasks are dealt so
// that XCD x takes a contiguous run of them: the row blocks of one (sequence, KV
// head) then share one L2, where their common K/V stream stays.
#ifndef MSATTN_PF_XCD
#define MSATTN_PF_XCD 1
#endif
constexpr int kXcds = 8;
// Wave priority (s_setprio) raised for the two MFMA blocks of a step: when both waves of
// a SIMD are ready, the one feeding the matrix core issues first.
#ifndef MSATTN_PF_PRIO
#define MSATTN_PF_PRIO 1
#endif
constexpr float kPfRescaleSlack = 8.0f;  // base-2 headroom before the max moves
constexpr float kPfSumBound = 256.0f;      // 2^kPfRescaleSlack
// l's increment as the sum of the rounded weights (v_dot2), which is also the fast path's
// test for a weight over the bound (no per-score max); 0: fp32 sum and a per-lane max.
#ifndef MSATTN_PF_SUM_CHECK
#define MSATTN_PF_SUM_CHECK 1
#endif
constexpr bool kPfSumCheck = MSATTN_PF_SUM_CHECK != 0;
// s_waitcnt immediate (gfx9 encoding) waiting for every vector memory operation only.
constexpr int kWaitVm0 = 0x0F70;

typedef short pf_s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) pf_s4 lds_s4;  // an LDS pointer target
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) uint4 lds_u4;

// Chunk swizzle of the copied K/V rows (16-byte chunk c of token row r stored at chunk
// position c ^ pf_swz(r); depends on r % 16 only). head_dim 128 (16 chunks per row): the
// 16 rows of a K operand read get 16 distinct positions, and the 8 rows of a transposed V
// read (tokens 8k .. 8k + 7, one 32-byte chunk pair each) 8 distinct pairs. head_dim 64
// (8 chunks, two rows per 64 banks): the same within each row parity.
// A use of v's registers at this point of the program (no instruction): values computed
// before it stay before it.
__device__ __forceinline__ void keep_here(const uint4& v) {
#if defined(__HIP_DEVICE_COMPILE__)  // the constraint names a GPU register class
  asm volatile("" ::"v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w));
#endif
}

// Instruction order asked of the scheduler for a half-step block of the copy path: NM
// MFMAs, each followed by NV VALU instructions (the other half-step's softmax), and the
// block's NC copy instructions spread among them; the LDS reads of the MFMA operands are
// free to move. Group masks: 0x008 MFMA, 0x002 VALU, 0x020 vector memory read.
template <int NM, int NV, int NC>
__device__ __forceinline__ void pf_sched_half() {
#pragma unroll
  for (int m = 0; m < NM; ++m) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, NV, 0);
    if (m % (NM / NC) == NM / NC - 1) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
  }
}

// One copy instruction: lane l's 16 bytes at buffer offset voff land at LDS dst + 16 l
// bytes (buffer_load_dwordx4 ... lds; the LDS address is wave-uniform).
__device__ __forceinline__ void lds_copy16(__amdgpu_buffer_rsrc_t r, uint16_t* dst, uint32_t voff) {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass of this file drops kernels that use it
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)dst, 16, voff, 0, 0, 0);
#endif
}

template <int D>
__device__ __forceinline__ int pf_swz(int r) {
  if constexpr (D == 128) return ((r & 7) << 1) | ((r >> 3) & 1);
  const int x = (r >> 1) & 7;
  return ((x & 3) << 1) | (x >> 2);
}

struct PrefillParams {
  const void* q;
  const void* k;
  const void* v;
  const int32_t* table;
  const int32_t* lens;
  void* out;
  int64_t blk_stride, slot_stride, head_stride;
  int batch, q_len, H, KVH, G;
  int bs, num_blocks, W, max_ctx;
  int causal, window;
  float scale_log2;
  int rows_per_kvh;  // q_len * G
  int rblocks;       // ceil(rows_per_kvh / kPfRows)
  int bs_shift;      // log2(bs) when bs is a power of two, else -1
  int xcd_per;       // tasks per XCD (the grid is kXcds * xcd_per workgroups)
  // Shared-prefix partials mode (the PX kernels): the rows are the decode queries of
  // every sequence (query index i = sequence), the keys are the first max_ctx positions
  // of table row 0 (the pages every sequence shares), split into partitions of key_part
  // tokens (blockIdx.y); row i sees keys below min(max_ctx, row_lens[i]); each
  // (row, partition) writes an unnormalised partial (m, l, acc) at slot row * npart + part.
  const int32_t* row_lens;
  float* pml;
  float* pacc;
  int key_part, npart;
  // Stream-K mode (sk_groups > 0, prefill only): the grid is sk_groups workgroups, which
  // take equal contiguous shares of the work list (every task's key-step pairs, tasks in
  // order). A task split between workgroups has each share store an unnormalised partial
  // (m, l, acc) per row at slot 2 * share + (0: the share's first task, 1: its last);
  // the fold launch that follows (prefill_sk_fold_kernel) merges them into the output.
  int sk_groups;
  int ntasks;         // rblocks * KVH * batch
  float* sk_ml;       // [2 * sk_groups][kPfRows][2]
  float* sk_acc;      // [2 * sk_groups][kPfRows][D]
  int* sk_pre;        // [ntasks + 2]: the work list's task offsets and its head size,
                      // written by workgroup 0
};

// Largest task count of a stream-K prefill launch (its work-list prefix sums sit in LDS).
constexpr int kPfSkMaxTasks = 2048;
// Positions of the stream-K work list ahead of each task's key-step pairs that hold no work
// (a head): a share whose range takes a task's start past its own pays a second task start
// and end (context length, table window, first copies; the key groups' merge and stores),
// and the head gives it that much less of the pairs, so that the shares end together.
// Where every task boundary already falls on a share boundary (equal shares of whole tasks,
// or tasks of whole shares), no share holds a second start and the list has no heads.
#ifndef MSATTN_PF_SK_HEAD
#define MSATTN_PF_SK_HEAD 3
#endif
constexpr int kPfSkHead = MSATTN_PF_SK_HEAD;

// Geometry of one prefill task (sequence b, KV head, 128-row block; not the cascade's
// PX tasks): its rows, context and the key range [lo_all, hi_all) its rows see, and the
// 64-key steps covering that range.
struct PfTask {
  int b, kvh, rblock, ctx, row0, rows_here, i_first, i_last, lo_all, hi_all;
  int step_first, step_end;
  __device__ int iterations() const {  // key-step pairs, at least one (rows without keys)
    const int n = (step_end - step_first + 1) / 2;
    return n > 0 ? n : 1;
  }
};

template <int BROWS>
__device__ __forceinline__ PfTask pf_task(const PrefillParams& p, unsigned task) {
  PfTask t;
  const unsigned per_b = static_cast<unsigned>(p.rblocks) * static_cast<unsigned>(p.KVH);
  t.b = static_cast<int>(task / per_b);
  const unsigned bx = task - static_cast<unsigned>(t.b) * per_b;
  // larger (later) row blocks first: they see the most keys under a causal mask
  t.rblock = p.rblocks - 1 - static_cast<int>(bx % static_cast<unsigned>(p.rblocks));
  t.kvh = static_cast<int>(bx / static_cast<unsigned>(p.rblocks));
  int ctx = p.lens[t.b];
  t.ctx = ctx < 0 ? 0 : (ctx > p.max_ctx ? p.max_ctx : ctx);
  t.row0 = t.rblock * BROWS;
  t.rows_here = min(BROWS, p.rows_per_kvh - t.row0);
  t.i_first = t.row0 / p.G;
  t.i_last = (t.row0 + t.rows_here - 1) / p.G;
  t.lo_all = p.window > 0 ? max(0, t.ctx - p.q_len + t.i_first - p.window + 1) : 0;
  t.hi_all = p.causal ? min(t.ctx, t.ctx - p.q_len + t.i_last + 1) : t.ctx;
  t.step_first = t.hi_all > t.lo_all ? t.lo_all / kPfStep : 0;
  t.step_end = t.hi_all > t.lo_all ? ceil_div(t.hi_all, kPfStep) : 0;
  return t;
}

template <typename T, typename KT, int D, int RB, bool PX>
__global__ __launch_bounds__(kPfThreads) void prefill_mfma_kernel(const PrefillParams p) {
  typedef Kv8<T, KT> KV;  // a cache of T, or of fp8 e4m3 / fp32 converted to T in registers
  typedef typename KV::raw_t raw_t;
  constexpr int EB = static_cast<int>(sizeof(KT));
  static_assert(D == 64 || D == 128, "prefill MFMA kernel handles head_dim 64 and 128");
  // A cache of the query's type is copied into LDS by the load unit; other caches pass
  // through registers, where they are converted.
  constexpr bool DMA = MSATTN_PF_DMA && std::is_same<T, KT>::value;
  constexpr int JD = D / 16;              // k-steps of S^T (16 dims each)
  constexpr int ND = D / 32;              // 32-dim tiles of O^T
  static_assert(16 * RB == 32, "one 32-row MFMA block per wave");
  // LDS row strides (elements): unpadded, swizzled rows for the copies; padded rows for
  // register staging (K: 68 / 36 dwords, V: 72 / 40 dwords).
  constexpr int RSK = DMA ? D : D + 8;
  constexpr int RSV = DMA ? D : D + 16;
  constexpr int WROWS = 16 * RB;          // query rows per wave
  constexpr int BROWS = WROWS * kPfWaves; // query rows per workgroup

  // One array per buffer slot, [key group][token row * stride]: the compiler then sees
  // that a copy into one slot does not write the slots being read.
  __shared__ __attribute__((aligned(256))) uint16_t s_k0[kPfGroups][kPfStep * RSK];
  __shared__ __attribute__((aligned(256))) uint16_t s_k1[kPfGroups][kPfStep * RSK];
  __shared__ __attribute__((aligned(256))) uint16_t s_v0[kPfGroups][kPfStep * RSV];
  __shared__ __attribute__((aligned(256))) uint16_t s_v1[kPfGroups][kPfStep * RSV];
  // Page window: kPfPageChunk page ids (register staging) or 16-token tile offsets (copies).
  __shared__ __attribute__((aligned(8))) int s_pg[2 * kPfPageChunk];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wg = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int grp = wg / kPfWaves;  // key group: steps step_first + grp, + 2, ...
  const int w = wg - grp * kPfWaves;  // wave within the group: its query rows
  const int g = lane >> 4;
  const int n = lane & 15;
  // Stream-K mode: the work list is every task's key-step pairs (PfTask::iterations),
  // tasks in order; s_skpre[t] = pairs of tasks 0 .. t - 1 (an exclusive scan over the
  // tasks' counts, computed here from the context lengths, so the launch is capture-safe),
  // and this workgroup's share is [r_begin, r_end) of the list.
  __shared__ int s_skpre[PX ? 1 : kPfSkMaxTasks + 1];
  const bool sk = !PX && p.sk_groups > 0;
  int r_begin = 0, r_end = 0, sk_task = 0, sk_share = 0, sk_head = 0;
  if constexpr (!PX) {
    if (sk) {
      constexpr int kPer = (kPfSkMaxTasks + kPfThreads - 1) / kPfThreads;
      int cnt[kPer];
      int sum = 0;
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        const int t = tid * kPer + k;
        cnt[k] = t < p.ntasks ? pf_task<BROWS>(p, static_cast<unsigned>(t)).iterations() : 0;
        sum += cnt[k];
      }
      const int incl = wave_inclusive_sum(sum);
      if (lane == kWave - 1) s_pg[wg] = incl;  // the page window is free before the tasks
      __syncthreads();
      int excl = incl - sum;
      for (int k = 0; k < wg; ++k) excl += s_pg[k];
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        const int t = tid * kPer + k;
        if (t < p.ntasks) s_skpre[t] = excl;
        excl += cnt[k];
      }
      if (tid == kPfThreads - 1) s_skpre[p.ntasks] = excl;  // the list's length
      if (tid == 0) s_pg[kPfThreads / kWave] = 1;  // every boundary on a share boundary, so far
      __syncthreads();
      {
        // Heads unless every task boundary sits on a share boundary of the list without them.
        const int total0 = s_skpre[p.ntasks];
        const int shares0 = pf_sk_shares(p.sk_groups, total0);
        const int q = shares0 > 0 && total0 % shares0 == 0 ? total0 / shares0 : 0;
        bool off = q == 0;
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
          const int t = tid * kPer + k;
          if (t < p.ntasks && q > 0) off = off || s_skpre[t] % q != 0;
        }
        if (off) s_pg[kPfThreads / kWave] = 0;  // (any writer stores the same value)
        __syncthreads();
        sk_head = s_pg[kPfThreads / kWave] ? 0 : kPfSkHead;
        if (sk_head > 0) {
#pragma unroll
          for (int k = 0; k < kPer; ++k) {
            const int t = tid * kPer + k;
            if (t < p.ntasks) s_skpre[t] += sk_head * t;
          }
          if (tid == kPfThreads - 1) s_skpre[p.ntasks] += sk_head * p.ntasks;
        }
        __syncthreads();
      }
      if (blockIdx.x == 0) {  // for the fold launch: the list, then the head size
        for (int t = tid; t <= p.ntasks; t += kPfThreads) p.sk_pre[t] = s_skpre[t];
        if (tid == 0) p.sk_pre[p.ntasks + 1] = sk_head;
      }
      const unsigned i = blockIdx.x;
      // shares dealt to the XCDs in contiguous runs, as tasks are without stream-K
      sk_share = (MSATTN_PF_XCD && p.sk_groups % kXcds == 0)
                     ? static_cast<int>((i % kXcds) * static_cast<unsigned>(p.sk_groups / kXcds) +
                                        i / kXcds)
                     : static_cast<int>(i);
      // (values read from LDS are the same in every lane: readfirstlane keeps them, and
      // all the task arithmetic that follows, in scalar registers)
      const int total = __builtin_amdgcn_readfirstlane(s_skpre[p.ntasks]);
      // Shares: no more than the list's length, so that every share holds work (a task's
      // contributors are then consecutive shares, each storing a partial); workgroups
      // past them have none.
      pf_sk_range(sk_share, total, pf_sk_shares(p.sk_groups, total), &r_begin, &r_end);
      int lo = 0, hi = p.ntasks;  // the task holding r_begin: s_skpre[lo] <= r_begin < s_skpre[hi]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (__builtin_amdgcn_readfirstlane(s_skpre[mid]) <= r_begin) lo = mid;
        else hi = mid;
      }
      sk_task = lo;
    }
  }

  // One task at a time: without stream-K the workgroup's one task; with it, the tasks its
  // share touches, each over the part [it_lo, it_hi) of its key-step pairs in the share.
  for (int seg = 0;; ++seg) {
  // The lane's constants are derived again in each task from an opaque copy of the thread
  // index, so the compiler does not hoist the task's lane arithmetic out of this loop and
  // hold it across the key loop.
  int tid_opaque = static_cast<int>(threadIdx.x);
  asm volatile("" : "+v"(tid_opaque));
  const int tid = tid_opaque;
  const int lane = tid & (kWave - 1);
  const int wg = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int grp = wg / kPfWaves;
  const int w = wg - grp * kPfWaves;
  const int hh = lane >> 5;  // lane half: keys / dims 4 hh .. of each group of 8
  const int cc = lane & 31;  // the lane's query row in the wave's 32-row block
  int it_lo = 0, it_hi = 1 << 28;
  bool full = true;  // the whole task: normalised output; else a partial
  unsigned task = 0;
  // Task = (sequence, KV head) pair-major, then row block; larger (later) row blocks
  // first: they see the most keys under a causal mask.
  unsigned bx = blockIdx.x;
  int b = 0;
  if constexpr (!PX) {
    const unsigned per_b = static_cast<unsigned>(p.rblocks) * static_cast<unsigned>(p.KVH);
    if (sk) {
      if (sk_task >= p.ntasks || r_begin >= r_end) break;
      // the task's pairs: positions p0 .. p1 - 1, after its head
      const int p0 = __builtin_amdgcn_readfirstlane(s_skpre[sk_task]) + sk_head;
      const int p1 = __builtin_amdgcn_readfirstlane(s_skpre[sk_task + 1]);
      if (p0 >= r_end) break;  // the share ends before (or in the head of) this task
      it_lo = r_begin > p0 ? r_begin - p0 : 0;
      it_hi = (r_end < p1 ? r_end : p1) - p0;
      full = it_lo == 0 && it_hi == p1 - p0;
      task = static_cast<unsigned>(sk_task++);
    } else {
      if (seg > 0) break;
      const unsigned i = blockIdx.x;
      task = MSATTN_PF_XCD ? (i % kXcds) * static_cast<unsigned>(p.xcd_per) + i / kXcds : i;
      if (task >= per_b * static_cast<unsigned>(p.batch)) break;  // the grid's tail
    }
    b = static_cast<int>(task / per_b);
    bx = task - static_cast<unsigned>(b) * per_b;
  } else {
    if (seg > 0) break;
  }
  const int rblock = p.rblocks - 1 - static_cast<int>(bx % static_cast<unsigned>(p.rblocks));
  const int kvh = static_cast<int>(bx / static_cast<unsigned>(p.rblocks));

  // Copy path: the task's first window of tile offsets starts at tile pre_t whenever no
  // sliding window moves its first key (the task's steps then start at step 0, or at the
  // prefix partition's first step, and a share's part at its first pair): that window's
  // table entries are requested here, before the context length is known, so that their
  // round trip overlaps the length's and the query's instead of following them.
  int pre_t = -1, pre_phys = -1;
  if constexpr (DMA) {
    static_assert(kPfPageChunk == kPfThreads, "one window entry per thread");
    int s0 = -1;
    if constexpr (PX) {
      const int lo = static_cast<int>(blockIdx.y) * p.key_part;
      s0 = lo < p.max_ctx ? lo / kPfStep : 0;
    } else if (p.window <= 0) {
      s0 = 2 * it_lo;
    }
    if (s0 >= 0) {
      pre_t = s0 * (kPfStep / 16);
      const int tok = (pre_t + tid) * 16;
      const int pg = p.bs_shift >= 0 ? tok >> p.bs_shift : tok / p.bs;
      if (pg < p.W) pre_phys = p.table[static_cast<int64_t>(b) * p.W + pg];
    }
  }
  int ctx = PX ? p.max_ctx : p.lens[b];
  ctx = ctx < 0 ? 0 : (ctx > p.max_ctx ? p.max_ctx : ctx);
  const int row0 = rblock * BROWS;
  const int rows_here = min(BROWS, p.rows_per_kvh - row0);

  // Key range of the block (query index grows with the row).
  const int i_first = row0 / p.G;
  const int i_last = (row0 + rows_here - 1) / p.G;
  int lo_all, hi_all;
  if constexpr (PX) {  // the block's key partition of the shared prefix
    const int part = blockIdx.y;
    lo_all = part * p.key_part;
    hi_all = min(ctx, lo_all + p.key_part);
  } else {
    lo_all = p.window > 0 ? max(0, ctx - p.q_len + i_first - p.window + 1) : 0;
    hi_all = p.causal ? min(ctx, ctx - p.q_len + i_last + 1) : ctx;
  }

  // This lane's query row: MFMA column cc of the wave's 32-row block (both lane halves hold
  // it, each for half of every 8 keys or dims).
  const bool row_ok = row0 + w * WROWS + cc < p.rows_per_kvh;
  int lo_n = 0, hi_n = 0;
  // Index of the lane's query row in the [tokens, heads] query / output arrays
  // (recomputed where needed rather than held through the key loop).
  auto out_row = [&]() {
    const int row = row0 + w * WROWS + cc;
    const int i = row / p.G;
    return (static_cast<int64_t>(b) * p.q_len + i) * p.H + kvh * p.G + (row - i * p.G);
  };
  if (row_ok) {
    const int i = (row0 + w * WROWS + cc) / p.G;
    const int qpos = ctx - p.q_len + i;
    if constexpr (PX) {
      lo_n = lo_all;
      hi_n = min(hi_all, max(0, p.row_lens[i]));
    } else {
      hi_n = p.causal ? min(ctx, qpos + 1) : ctx;
      lo_n = p.window > 0 ? max(0, qpos - p.window + 1) : 0;
    }
    if (hi_n < lo_n) hi_n = lo_n;
  }
  // Keys every row of this wave sees: [wave_lo, wave_hi) (rows grow with the query).
  int wave_lo = 0, wave_hi = 0;
  {
    const int wr0 = row0 + w * WROWS;
    const int wr1 = min(wr0 + WROWS, p.rows_per_kvh) - 1;
    if (wr1 >= wr0) {
      const int qa = ctx - p.q_len + wr0 / p.G;  // first row's query position
      const int qb_ = ctx - p.q_len + wr1 / p.G; // last row's
      wave_hi = p.causal ? min(ctx, qa + 1) : ctx;
      wave_lo = p.window > 0 ? max(0, qb_ - p.window + 1) : 0;
    }
    if constexpr (PX) {  // the smallest per-row limit of the wave's valid rows
      int h = row_ok ? hi_n : INT_MAX;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) h = min(h, __shfl_xor(h, o, kWave));
      wave_lo = lo_all;
      wave_hi = h == INT_MAX ? 0 : h;
    }
  }
  // The B operand Q^T of k-step j: the row's dims 16 j + 8 hh .. + 7.
  uint4 qb[JD];
  {
    const T* qp = static_cast<const T*>(p.q);
#pragma unroll
    for (int j = 0; j < JD; ++j) {
      qb[j] = make_uint4(0u, 0u, 0u, 0u);
      if (row_ok) qb[j] = *reinterpret_cast<const uint4*>(qp + out_row() * D + 16 * j + 8 * hh);
    }
  }

  // O^T in 32-dim tiles: acc[t] register v = dim 32 t + (v & 3) + 8 (v >> 2) + 4 hh.
  mf_f32x16 acc[ND];
  float m_run = -INFINITY, l_run = 0.0f;
#pragma unroll
  for (int t = 0; t < ND; ++t) acc[t] = zero16();

  const KT* kbase = static_cast<const KT*>(p.k);
  const KT* vbase = static_cast<const KT*>(p.v);
  // The task's steps (pf_task's rule), then this share's part of them: pairs it_lo ..
  // it_hi - 1 (group 0 takes the pair's first step, group 1 its second, as without
  // stream-K).
  const int step_first0 = hi_all > lo_all ? lo_all / kPfStep : 0;
  const int step_end0 = hi_all > lo_all ? ceil_div(hi_all, kPfStep) : 0;
  const int step_first = step_first0 + 2 * it_lo;
  const int step_end = min(step_end0, step_first0 + 2 * it_hi);

  int pg_base = -(1 << 30);  // s_pg[i] = physical page of logical page pg_base + i
  auto page_of = [&](int tok) { return p.bs_shift >= 0 ? tok >> p.bs_shift : tok / p.bs; };
  // Make s_pg cover the pages of steps [s_lo, s_hi]: called by every thread (it may
  // hold barriers); reloads the window from the first page of s_lo when needed.
  auto ensure_pages = [&](int s_lo, int s_hi) {
    const int p_lo = page_of(s_lo * kPfStep);
    const int p_hi = page_of(s_hi * kPfStep + kPfStep - 1);
    if (p_lo < pg_base || p_hi >= pg_base + kPfPageChunk) {
      __syncthreads();
      for (int j = tid; j < kPfPageChunk; j += kPfThreads) {
        const int pg = p_lo + j;
        int phys = -1;
        if (pg < p.W) {
          phys = p.table[static_cast<int64_t>(b) * p.W + pg];
          if (phys < 0 || phys >= p.num_blocks) phys = -1;
        }
        s_pg[j] = phys;
      }
      pg_base = p_lo;
      __syncthreads();
    }
  };
  const int64_t row_bytes = p.slot_stride * EB;

  // ---- one step's arithmetic, shared by both staging schemes ----
  // Keys of a step all visible to every row of the wave: no per-key mask.
  auto step_full = [&](int step) {
    const int t_base = step * kPfStep;
    return t_base >= wave_lo && t_base + kPfStep <= wave_hi;
  };
  // S^T of a step's 32-key tile TL for the wave's 32 rows; ka_of(TL, j) reads the K
  // operand of k-step j (key row 32 TL + cc, dims 16 j + 8 hh ..). Lane (cc, hh) then holds
  // row cc's scores of keys 32 TL + (v & 3) + 8 (v >> 2) + 4 hh in register v.
  auto scores = [&](auto&& ka_of, mf_f32x16 (&sv)[2], auto tile_c) {
    constexpr int TL = decltype(tile_c)::value;
    mf_f32x16 st = zero16();
#pragma unroll
    for (int j = 0; j < JD; ++j) st = Mfma32<T>::mac(ka_of(TL, j), qb[j], st);
    sv[TL] = st;
  };
  // Keys outside the row's range score -inf (steps that cross some row's range).
  auto mask_scores = [&](int step, mf_f32x16 (&sv)[2], auto tile_c) {
    constexpr int TL = decltype(tile_c)::value;
    const int t_base = step * kPfStep + 32 * TL + 4 * hh;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int tok = t_base + (v & 3) + 8 * (v >> 2);
      sv[TL][v] = (tok >= lo_n && tok < hi_n) ? sv[TL][v] : -INFINITY;
    }
  };
  // Online softmax of the lane's row over one half-step (the 32-key tile ks: 16 keys per
  // lane half).
  // The weights are exp2(s * scale_log2 - m) for the row's running max m (base 2; the row
  // max is taken on raw scores, scale_log2 > 0 keeps the order). m moves only when some
  // weight would exceed 2^kPfRescaleSlack: the weights stay within what fp32 sums and the
  // bf16/fp16 P operand hold, and the normalisation by l is exact whatever reference max
  // the sums share.
  // Fast path (almost every half-step): the weights are taken with the current m, with no
  // cross-lane reduction, and l's increment is the sum of the rounded weights the P.V
  // MFMAs take (v_dot2 of each packed pair with (1, 1)). Every weight is at most that
  // sum, so a lane whose sum is within 2^kPfRescaleSlack holds no weight over it: the
  // sum is the test, and the scores' max is taken only on the slow path. A row whose m
  // is still -inf (no key seen yet) takes the slow path too. softmax_redo moves m to the
  // row max (over both lane halves) when it is above m, rescales l and acc, and takes
  // the weights again. (MSATTN_PF_SUM_CHECK=0: each lane tests its scores' max against
  // m + kPfRescaleSlack instead, l's increment summed in fp32 before rounding.)
  // The B operand P^T of the 16-key chunk c2 of tile ks: registers v = 8 c2 .. 8 c2 + 7,
  // i.e. keys 16 c2 + 4 hh .. + 3 and 16 c2 + 8 + 4 hh .. + 3, the two 4-token reads of V.
  uint4 pb[2][2];
  float psum;
  float lmax;
  auto softmax_exp = [&](const mf_f32x16 (&sv)[2], auto ks_c) __attribute__((always_inline)) {
    constexpr int KS = decltype(ks_c)::value;
    const float m_use = m_run != -INFINITY ? m_run : 0.0f;
    float pr[16];
#pragma unroll
    for (int v = 0; v < 16; ++v)
      pr[v] = __builtin_amdgcn_exp2f(fmaf(sv[KS][v], p.scale_log2, -m_use));
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2)
      pb[KS][c2] = make_uint4(Pack2<T>::pack(pr[8 * c2], pr[8 * c2 + 1]),
                              Pack2<T>::pack(pr[8 * c2 + 2], pr[8 * c2 + 3]),
                              Pack2<T>::pack(pr[8 * c2 + 4], pr[8 * c2 + 5]),
                              Pack2<T>::pack(pr[8 * c2 + 6], pr[8 * c2 + 7]));
    if constexpr (kPfSumCheck) {
      const uint32_t one2 = Pack2<T>::pack(1.0f, 1.0f);
      float s2[2];
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        const uint4 wv = pb[KS][c2];
        s2[c2] = Dot2<T>::dot(wv.w, one2, Dot2<T>::dot(wv.z, one2, Dot2<T>::dot(wv.y, one2,
                 Dot2<T>::dot(wv.x, one2, 0.0f))));
      }
      psum = s2[0] + s2[1];
    } else {
      float sum = 0.0f;
#pragma unroll
      for (int v = 0; v < 16; ++v) sum += pr[v];
      psum = sum;
    }
  };
  // The lane's scores' max over the half-step.
  auto lane_max = [&](const mf_f32x16 (&sv)[2], auto ks_c) __attribute__((always_inline)) {
    constexpr int KS = decltype(ks_c)::value;
    float lm = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) lm = fmaxf(lm, sv[KS][v]);
    return lm;
  };
  // The weights with the current m (and, without the sum test, the lane's max).
  auto softmax_fast = [&](const mf_f32x16 (&sv)[2], auto ks_c) __attribute__((always_inline)) {
    if constexpr (!kPfSumCheck) lmax = lane_max(sv, ks_c);
    softmax_exp(sv, ks_c);
  };
  auto over_bound = [&]() __attribute__((always_inline)) {
    bool over;
    if constexpr (kPfSumCheck)
      over = psum > kPfSumBound || m_run == -INFINITY;
    else
      over = lmax * p.scale_log2 > m_run + kPfRescaleSlack;
    return __any(over);
  };
  // Slow path for the wave: move m, rescale l and acc, take the weights again.
  auto softmax_redo = [&](const mf_f32x16 (&sv)[2], auto ks_c) __attribute__((always_inline)) {
    if constexpr (kPfSumCheck) lmax = lane_max(sv, ks_c);
    const float mt = halves_max(lmax) * p.scale_log2;  // the row max, base-2 units
    const float m_new = mt > m_run + (kPfSumCheck ? 0.0f : kPfRescaleSlack) ? mt : m_run;
    const float alpha = m_new != -INFINITY ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
    l_run *= alpha;
    m_run = m_new;
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int t = 0; t < ND; ++t) acc[t] *= alpha;
    }
    softmax_exp(sv, ks_c);
  };
  // After a half-step's weights (fast, and the redo when needed): l += their sum.
  auto softmax_end = [&](const mf_f32x16 (&sv)[2], auto ks_c) __attribute__((always_inline)) {
    if (__builtin_expect(over_bound(), 0)) softmax_redo(sv, ks_c);
    l_run += psum;
  };
  // O^T += V^T P^T over half-step ks (the 32-key tile ks, in 16-key chunks c2); va_of(ks,
  // c2, t) reads the A operand V^T (dims 32 t + cc, the chunk's keys as pb's).
  auto pv = [&](auto&& va_of, auto ks_c) {
    constexpr int KS = decltype(ks_c)::value;
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2) {
      uint4 va[ND];
#pragma unroll
      for (int t = 0; t < ND; ++t) va[t] = va_of(KS, c2, t);
#pragma unroll
      for (int t = 0; t < ND; ++t) acc[t] = Mfma32<T>::mac(va[t], pb[KS][c2], acc[t]);
    }
  };
  // Transposed reads: lane s of a 16-lane group names 4 dims of one token (tokens
  // base + (s >> 2), dims 4 * (s & 3) ..); lane i then receives dim i of those four
  // tokens. Group q = lane / 16 reads dims 16 (q & 1) .. of its tile for tokens 4 hh ..
  // (lo) and 8 + 4 hh .. (hi) of the 16-key chunk: lane (cc, hh) receives dim cc.
  const int tr_tok = lane >> 2 & 3;        // the token a lane names, within its 4
  const int tr_dim = 16 * (lane >> 4 & 1) + 4 * (lane & 3);  // the dims it names
  auto tr_pair = [&](uint16_t* lo, uint16_t* hi) {
    const uint2 a = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)lo));
    const uint2 c = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)hi));
    return make_uint4(a.x, a.y, c.x, c.y);
  };

  if constexpr (DMA) {
    // ---- K and V copied into LDS by the load unit (buffer_load ... lds) ----
    // Wave w of a group copies token rows 16 w .. 16 w + 15 of a step, K and V, each
    // instruction 1 KiB: lane l writes LDS bytes 16 l .. of the instruction's block. Rows
    // are unpadded; the 16-byte chunk c of token row r sits at position c ^ pf_swz(r), so a
    // lane reads global chunk (l % chunks per row) ^ pf_swz(row). K operand reads (16 rows,
    // one chunk each) and the transposed V reads (8 rows, 32 bytes each) then fall on
    // distinct banks. Tokens past hi_all, below a window's first key, or on a page the table
    // does not map lie outside the tile's descriptor: their copies write zeros.
    constexpr int CPRD = D / 8;        // 16-byte chunks per row
    constexpr int RPI = kWave / CPRD;  // rows per copy instruction (4 or 8)
    constexpr int NI = 16 / RPI;       // copy instructions per 16-row tile
    // Lane byte offsets of the reads, as one base XORed with a constant per k-step / dim
    // tile, so no register per j or t is held (slots are 256-byte aligned, rows 2 D
    // bytes): the K chunk (2 j + hh) of key row cc sits at (2 j + hh) ^ s, s = pf_swz(cc),
    // byte 16 (hh ^ s) ^ 32 j; the V chunk (4 t + c) (c < 4) of token row r at
    // 16 ((c ^ s) ^ 4 t), and token row r + 8 (r < 8) has s ^ 1, one chunk over.
    const uint32_t kx = static_cast<uint32_t>(cc * 2 * D + 16 * (hh ^ pf_swz<D>(cc)));
    const int vrow = 4 * hh + tr_tok;
    const uint32_t vx = static_cast<uint32_t>(vrow * 2 * D + 16 * ((tr_dim >> 3) ^ pf_swz<D>(vrow)) +
                                              8 * (lane & 1));
    uint32_t dvo[NI];
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int lr = RPI * j + lane / CPRD;
      dvo[j] = static_cast<uint32_t>(lr * row_bytes + 16 * ((lane % CPRD) ^ pf_swz<D>(lr)));
    }
    // This wave's 16-row tile of a step (token rows 16 w ..): one descriptor for its K
    // rows and one for its V rows, and the offset that pushes rows below a window's first
    // key out of range. ok = false gives empty descriptors (the copies then write zeros).
    struct TileCopy {
      __amdgpu_buffer_rsrc_t rk, rv;
      uint32_t skip;
    };
    // Window of tile offsets: s_tile[i] = element offset of 16-token tile tb_base + i of
    // this (sequence, KV head) in the caches, or -1 for a tile on an unmapped page.
    // Reloaded (between barriers, by every thread) when a step leaves it.
    int64_t* const s_tile = reinterpret_cast<int64_t*>(s_pg);
    int tb_base = -(1 << 30);
    // first: the prologue's call, which may take the entries requested at the task's start
    auto ensure_tiles = [&](int s_lo, int s_hi, auto first_c) {
      constexpr bool first = decltype(first_c)::value;
      const int t_lo = s_lo * (kPfStep / 16);
      const int t_hi = s_hi * (kPfStep / 16) + kPfStep / 16 - 1;
      if (t_lo < tb_base || t_hi >= tb_base + kPfPageChunk) {
        __syncthreads();
        for (int j = tid; j < kPfPageChunk; j += kPfThreads) {
          const int tok = (t_lo + j) * 16;
          const int pg = page_of(tok);
          int64_t off = -1;
          if (pg < p.W) {
            const int phys = first && t_lo == pre_t ? pre_phys
                                                    : p.table[static_cast<int64_t>(b) * p.W + pg];
            if (phys >= 0 && phys < p.num_blocks)
              off = static_cast<int64_t>(phys) * p.blk_stride +
                    static_cast<int64_t>(tok - pg * p.bs) * p.slot_stride +
                    static_cast<int64_t>(kvh) * p.head_stride;
          }
          s_tile[j] = off;
        }
        tb_base = t_lo;
        __syncthreads();
      }
    };
    auto plan_tile = [&](int step, bool ok) {
      const int t0 = step * kPfStep + 16 * w;
      const int64_t o = s_tile[ok ? t0 / 16 - tb_base : 0];
      const uint32_t lo32 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(o));
      const uint32_t hi32 = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(o) >> 32));
      const int64_t off = ok ? static_cast<int64_t>((static_cast<uint64_t>(hi32) << 32) | lo32) : -1;
      const int rows_valid = min(16, hi_all - t0);
      const bool tile_in = off >= 0 && rows_valid > 0 && t0 + 16 > lo_all;
      const int skip = tile_in && t0 < lo_all ? lo_all - t0 : 0;  // rows below the window
      const int64_t tbase = tile_in ? off + static_cast<int64_t>(skip) * p.slot_stride : 0;
      const int nbytes = tile_in ? static_cast<int>((rows_valid - 1 - skip) * row_bytes + D * EB) : 0;
      TileCopy c;
      c.rk = tile_rsrc(kbase + tbase, nbytes);
      c.rv = tile_rsrc(vbase + tbase, nbytes);
      c.skip = static_cast<uint32_t>(skip * row_bytes);  // rows below wrap out of range
      return c;
    };
    // Copy instruction j of the tile (RPI token rows) into the LDS slot dst.
    auto copy_rows = [&](__amdgpu_buffer_rsrc_t r, uint32_t skip, uint16_t* dst, int j) {
      lds_copy16(r, dst + (16 * w + RPI * j) * D, dvo[j] - skip);
    };
    uint16_t* const k0 = &s_k0[grp][0];
    uint16_t* const k1 = &s_k1[grp][0];
    uint16_t* const v0 = &s_v0[grp][0];
    uint16_t* const v1 = &s_v1[grp][0];
    // Reads address the slot arrays themselves (so the compiler can tell a read of one
    // slot from a copy into another); each slot is 256-byte aligned.
    static_assert(sizeof(s_k0[0]) % 256 == 0 && sizeof(s_v0[0]) % 256 == 0, "slot alignment");
    auto k_from = [&](uint16_t* buf) {
      return [&, buf](int tl, int j) {
        const uint32_t a = (kx ^ static_cast<uint32_t>(32 * j)) + static_cast<uint32_t>(64 * tl * D);
        return *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(buf) + a);
      };
    };
    auto v_from = [&](uint16_t* buf) {
      return [&, buf](int ks, int c2, int t) {
        const uint32_t x = vx ^ static_cast<uint32_t>(64 * t);
        const uint32_t row = static_cast<uint32_t>((32 * ks + 16 * c2) * 2 * D);
        char* const base = reinterpret_cast<char*>(buf);
        return tr_pair(reinterpret_cast<uint16_t*>(base + x + row),
                       reinterpret_cast<uint16_t*>(base + (x ^ 16u) + row + 16 * D));
      };
    };

    // Group grp takes steps s_first + 2 i from slots k(i & 1), v(i & 1); iteration i
    // copies the group's next step into the other slots while it computes step i in
    // half-steps of 32 keys, pairing independent MFMA and VALU work of the wave:
    //   scores of keys 0-31 | scores of keys 32-63 with the softmax of keys 0-31 |
    //   P.V of keys 0-31 with the softmax of keys 32-63 | P.V of keys 32-63.
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    // A step in four blocks (half-steps of 32 keys), each pairing independent MFMA and
    // VALU work where it can:
    //   r0: scores of keys 0-31;
    //   r1: scores of keys 32-63 | softmax of keys 0-31;
    //   r2: P.V of keys 0-31 | softmax of keys 32-63;
    //   r3: P.V of keys 32-63.
    // The scores sv and weights pb of a step live across blocks (and, for group 1, across
    // an iteration's barrier). `copies` issues copy instructions among the block's MFMAs.
    mf_f32x16 sv[2];
    // The MFMA-only blocks run at MSATTN_PF_MPRIO and return to the group's priority.
    auto prio_up = [] {
      if constexpr (MSATTN_PF_MPRIO > 0) __builtin_amdgcn_s_setprio(MSATTN_PF_MPRIO);
    };
    auto prio_down = [&] {
      if constexpr (MSATTN_PF_MPRIO > 0) {
        if (grp) __builtin_amdgcn_s_setprio(MSATTN_PF_G1PRIO);
        else __builtin_amdgcn_s_setprio(0);
      }
    };
    auto r0 = [&](uint16_t* kc, int step, bool full, auto&& side) {
      prio_up();
      scores(k_from(kc), sv, I0{});
      side();
      prio_down();
      if (!full) mask_scores(step, sv, I0{});
    };
    auto r1 = [&](uint16_t* kc, int step, bool full, auto&& copies) {
      scores(k_from(kc), sv, I1{});
      copies();
      softmax_fast(sv, I0{});
      if constexpr (MSATTN_PF_SCHED) pf_sched_half<JD, MSATTN_PF_NV, NI>();
      // The weights stay in this block (the compiler would otherwise move them past the
      // branches below, next to their use and away from the MFMAs they overlap).
      keep_here(pb[0][0]);
      keep_here(pb[0][1]);
      softmax_end(sv, I0{});
      if (!full) mask_scores(step, sv, I1{});
    };
    auto r2 = [&](uint16_t* vc, auto&& copies) {
      pv(v_from(vc), I0{});
      copies();
      softmax_fast(sv, I1{});
      if constexpr (MSATTN_PF_SCHED) pf_sched_half<2 * ND, MSATTN_PF_NV, NI>();
      keep_here(pb[1][0]);
      keep_here(pb[1][1]);
      softmax_end(sv, I1{});
    };
    auto r3 = [&](uint16_t* vc) {
      prio_up();
      pv(v_from(vc), I1{});
      prio_down();
    };
    auto no_copies = [] {};

    // Group grp takes steps s_first + 2 i; the K and V of its i-th step go to slots
    // k(i & 1) and v(i & 1). Both groups meet at one barrier per iteration, but run half a
    // step apart so that a SIMD's two waves are in complementary blocks: iteration i of
    // group 0 is r0 r1 r2 r3 of its step i; of group 1, r2 r3 of its step i - 1, then r0
    // r1 of its step i. While one wave's block is MFMA-only, the other's is MFMA + VALU.
    // The copy plans (scalar work) of an iteration are made during the one before, in its
    // MFMA-only blocks.
    const int s_first = step_first + grp;
    const int n_it = ceil_div(step_end - step_first, 2);
    TileCopy ck = plan_tile(0, false), cv = ck;  // this iteration's copies: K, V
    if (n_it > 0) {
      ensure_tiles(step_first, min(step_first + 5, step_end - 1), std::true_type{});
      const TileCopy c = plan_tile(s_first, s_first < step_end);
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        copy_rows(c.rk, c.skip, k0, j);
        if (grp == 0) copy_rows(c.rv, c.skip, v0, j);  // group 1 copies V a step later
      }
      // group 0 copies step i + 1 in iteration i; group 1, K of step i + 1 and V of step i
      ck = plan_tile(s_first + 2, s_first + 2 < step_end);
      cv = grp == 0 ? ck : c;
    }
    // The copies and the query loads have landed: the compiler does not order reads of
    // the copies' LDS after their completion itself (and without a wait here on every
    // path into the loop, it puts one for the query into each iteration).
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    // Each group runs its own copy of the loop (the two meet at the same barriers: one
    // per iteration and the window reloads, all at the same iterations).
    auto iteration0 = [&](int i, auto cur_c) {
      constexpr int cur = decltype(cur_c)::value;
      uint16_t* const k_cur = cur ? k1 : k0;  // K of the group's step i
      uint16_t* const k_nxt = cur ? k0 : k1;  // K of step i + 1 goes here
      uint16_t* const v_cur = cur ? v1 : v0;  // V of step i
      uint16_t* const v_nxt = cur ? v0 : v1;  // V of step i + 1 goes here
      const int step = s_first + 2 * i;
      const int pn = step_first + 2 * i + 2;
      if (pn < step_end) ensure_tiles(pn, min(pn + 3, step_end - 1), std::false_type{});
      if (step < step_end) {
        const bool full = step_full(step);
        TileCopy cn;  // the next iteration's copies (step + 4)
        r0(k_cur, step, full, [&] { cn = plan_tile(step + 4, step + 4 < step_end); });
        r1(k_cur, step, full, [&] {
#pragma unroll
          for (int j = 0; j < NI; ++j) copy_rows(ck.rk, ck.skip, k_nxt, j);
        });
        r2(v_cur, [&] {
#pragma unroll
          for (int j = 0; j < NI; ++j) copy_rows(ck.rv, ck.skip, v_nxt, j);
        });
        r3(v_cur);
        ck = cn;
      }
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
      __syncthreads();  // this iteration's copies landed; the reads of their slots are done
    };
    auto iteration1 = [&](int i, auto cur_c) {
      constexpr int cur = decltype(cur_c)::value;
      uint16_t* const k_cur = cur ? k1 : k0;  // K of the group's step i
      uint16_t* const k_nxt = cur ? k0 : k1;  // K of step i + 1 goes here
      uint16_t* const v_cur = cur ? v1 : v0;  // V of step i goes here
      uint16_t* const v_prv = cur ? v0 : v1;  // V of step i - 1
      const int step = s_first + 2 * i;
      const int pn = step_first + 2 * i + 2;
      if (pn < step_end) ensure_tiles(pn, min(pn + 3, step_end - 1), std::false_type{});
      if (i > 0 && step - 2 < step_end) {  // the second half of step i - 1
        r2(v_prv, [&] {
#pragma unroll
          for (int j = 0; j < NI; ++j) copy_rows(ck.rk, ck.skip, k_nxt, j);
        });
        r3(v_prv);
      } else {
#pragma unroll
        for (int j = 0; j < NI; ++j) copy_rows(ck.rk, ck.skip, k_nxt, j);
      }
      if (step < step_end) {
        const bool full = step_full(step);
        TileCopy ckn, cvn;  // the next iteration's copies: K of step + 4, V of step + 2
        r0(k_cur, step, full, [&] {
          ckn = plan_tile(step + 4, step + 4 < step_end);
          cvn = plan_tile(step + 2, step + 2 < step_end);
        });
        r1(k_cur, step, full, [&] {
#pragma unroll
          for (int j = 0; j < NI; ++j) copy_rows(cv.rv, cv.skip, v_cur, j);
        });
        ck = ckn;
        cv = cvn;
      }
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
      __syncthreads();  // this iteration's copies landed; the reads of their slots are done
    };
    if (grp == 0) {
      int i = 0;
      for (; i + 1 < n_it; i += 2) {
        iteration0(i, I0{});
        iteration0(i + 1, I1{});
      }
      if (i < n_it) iteration0(i, I0{});
    } else {
      // Group 1 carries the iteration's critical path (its blocks include the plans of two
      // copies): its waves issue first when both waves of a SIMD are ready.
      if constexpr (MSATTN_PF_G1PRIO > 0) __builtin_amdgcn_s_setprio(MSATTN_PF_G1PRIO);
      int i = 0;
      for (; i + 1 < n_it; i += 2) {
        iteration1(i, I0{});
        iteration1(i + 1, I1{});
      }
      if (i < n_it) iteration1(i, I0{});
      if constexpr (MSATTN_PF_G1PRIO > 0) __builtin_amdgcn_s_setprio(0);
    }
    // Group 1: the second half of its last step (its V landed at the last barrier).
    if (grp == 1 && n_it > 0 && s_first + 2 * (n_it - 1) < step_end) {
      uint16_t* const v_last = ((n_it - 1) & 1) ? v1 : v0;
      r2(v_last, no_copies);
      r3(v_last);
    }
  } else {
    // ---- register staging (caches converted on the way: fp8 e4m3, fp32) ----
    // A group's thread gtid loads chunk st_c of token rows st_r + ROWS_PER_PASS * j of the
    // group's steps. A pass covers ROWS_PER_PASS / 16 tiles of 16 tokens (1 for head_dim
    // 128, 2 for 64); a wave's rows lie in one of them, tile st_tile of the pass.
    constexpr int CPR = D * 2 / 16;  // 16-byte chunks per K/V row (as T)
    constexpr int LPT = kPfStep * CPR / kPfGroupThreads;  // chunks per thread per tensor per step
    static_assert(LPT * kPfGroupThreads == kPfStep * CPR, "staging split");
    const int gtid = tid - grp * kPfGroupThreads;
    const int st_c = gtid % CPR;
    const int st_r = gtid / CPR;
    constexpr int ROWS_PER_PASS = kPfGroupThreads / CPR;
    static_assert(ROWS_PER_PASS % 16 == 0 && kWave / CPR <= 16, "a wave's rows in one tile");
    const int st_tile = ROWS_PER_PASS > 16 ? __builtin_amdgcn_readfirstlane(st_r / 16) : 0;
    const int st_row = st_r % 16;
    raw_t kst[LPT], vst[LPT];
#pragma unroll
    for (int j = 0; j < LPT; ++j) kst[j] = vst[j] = KV::keep_if(raw_t{}, false);
    // A step's row j * 16 + r is row r of its 16-token tile j; block_size % 16 == 0 puts a
    // tile in one page, so the page lookup and the tile's base offset are the same for
    // every lane (scalar), and a lane only adds its constant in-tile offset. Each tile is
    // read through a buffer descriptor whose size ends at the last row below hi_all (rows
    // past it, and tiles that are holes, read as zeros).
    const uint32_t st_off = static_cast<uint32_t>((st_row * p.slot_stride + st_c * 8) * EB);
    // The page ids of a step's tiles are read from the window ahead of the loads (plan),
    // so the LDS latency of the lookups is not paid in front of each tile's loads.
    auto plan = [&](int step, int (&phys)[LPT]) {
#pragma unroll
      for (int j = 0; j < LPT; ++j)
        phys[j] = s_pg[page_of(step * kPfStep + ROWS_PER_PASS * j + 16 * st_tile) - pg_base];
    };
    auto issue = [&](int step, const int (&phys_planned)[LPT]) {
#pragma unroll
      for (int j = 0; j < LPT; ++j) {
        const int t0 = step * kPfStep + ROWS_PER_PASS * j + 16 * st_tile;  // the wave's tile
        const int pg = page_of(t0);
        const int phys = __builtin_amdgcn_readfirstlane(phys_planned[j]);
        const int rows_valid = min(16, hi_all - t0);
        const bool tile_in = phys >= 0 && rows_valid > 0 && t0 + 16 > lo_all;
        const int64_t tbase = tile_in ? static_cast<int64_t>(phys) * p.blk_stride +
                                            static_cast<int64_t>(t0 - pg * p.bs) * p.slot_stride +
                                            static_cast<int64_t>(kvh) * p.head_stride
                                      : 0;
        const int nbytes = tile_in ? static_cast<int>((rows_valid - 1) * row_bytes + D * EB) : 0;
        kst[j] = KV::template load<0>(tile_rsrc(kbase + tbase, nbytes), st_off);
        vst[j] = KV::template load<0>(tile_rsrc(vbase + tbase, nbytes), st_off);
        if (t0 < lo_all) {  // a window's first tile: rows below it are zeros too
          const bool keep = t0 + st_row >= lo_all;
          kst[j] = KV::keep_if(kst[j], keep);
          vst[j] = KV::keep_if(vst[j], keep);
        }
      }
    };
    auto stage = [&](int buf) {  // the registers loaded by issue() into LDS buffer `buf`
      uint16_t* const kb = buf ? &s_k1[grp][0] : &s_k0[grp][0];
      uint16_t* const vb = buf ? &s_v1[grp][0] : &s_v0[grp][0];
#pragma unroll
      for (int j = 0; j < LPT; ++j) {
        const int r = st_r + ROWS_PER_PASS * j;
        *reinterpret_cast<uint4*>(kb + r * RSK + st_c * 8) = KV::operand(kst[j]);
        *reinterpret_cast<uint4*>(vb + r * RSV + st_c * 8) = KV::operand(vst[j]);
      }
    };
    auto compute = [&](int step, int buf) {
      uint16_t* const kb = buf ? &s_k1[grp][0] : &s_k0[grp][0];
      uint16_t* const vb = buf ? &s_v1[grp][0] : &s_v0[grp][0];
      using J0 = std::integral_constant<int, 0>;
      using J1 = std::integral_constant<int, 1>;
      mf_f32x16 sv[2];
      auto ka_of = [&](int tl, int j) {
        return *reinterpret_cast<const uint4*>(kb + (32 * tl + cc) * RSK + 16 * j + 8 * hh);
      };
      if constexpr (MSATTN_PF_PRIO) __builtin_amdgcn_s_setprio(1);
      scores(ka_of, sv, J0{});
      scores(ka_of, sv, J1{});
      if constexpr (MSATTN_PF_PRIO) __builtin_amdgcn_s_setprio(0);
      if (!step_full(step)) {
        mask_scores(step, sv, J0{});
        mask_scores(step, sv, J1{});
      }
      // Half-step by half-step: the same order of operations as the copy path
      // (bit-identical results).
      auto va_of = [&](int ks, int c2, int t) {
        uint16_t* lo = vb + (32 * ks + 16 * c2 + 4 * hh + tr_tok) * RSV + 32 * t + tr_dim;
        return tr_pair(lo, lo + 8 * RSV);
      };
      static_for<2>([&](auto kc) {
        softmax_fast(sv, kc);
        softmax_end(sv, kc);
        if constexpr (MSATTN_PF_PRIO) __builtin_amdgcn_s_setprio(1);
        pv(va_of, kc);
        if constexpr (MSATTN_PF_PRIO) __builtin_amdgcn_s_setprio(0);
      });
    };

    // Group grp takes steps step_first + grp + 2i (i = 0, 1, ...) from its own pair of
    // buffers; both groups meet at one barrier per pair of steps.
    const int s_first = step_first + grp;
    if (step_first < step_end) {
      ensure_pages(step_first, min(step_first + 3, step_end - 1));
      int ph[LPT];
      if (s_first < step_end) {
        plan(s_first, ph);
        issue(s_first, ph);
      }
      stage(0);
      if (s_first + 2 < step_end) {
        plan(s_first + 2, ph);
        issue(s_first + 2, ph);
      }
    }
    // Everything loaded before the loop (query rows, the first steps) has landed: the
    // loop then only waits for its own staging loads, not for every load in flight.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int npairs = ceil_div(step_end - step_first, 2);
    for (int i = 0; i < npairs; ++i) {
      const int step = s_first + 2 * i;
      const int buf = i & 1;
      // The page ids of this iteration's prefetch (step + 4) are read before the compute.
      const int pair_next = step_first + 2 * i + 4;  // the next prefetch, uniform over groups
      int ph_next[LPT];
      if (pair_next < step_end) {
        ensure_pages(pair_next, min(pair_next + 1, step_end - 1));
        if (step + 4 < step_end) plan(step + 4, ph_next);
      }
      if (step < step_end) compute(step, buf);
      if (step + 2 < step_end) stage(buf ^ 1);  // its readers finished before the last barrier
      if (step + 4 < step_end) issue(step + 4, ph_next);
      __syncthreads();  // buf ^ 1 is written; buf's reads are done
    }
  }

  // ---- combine the two key groups (same rows, same lane layout), normalise, store ----
  // Group 1 hands its (acc, m, l) through LDS (the K slots hold the accumulators' dim
  // tiles, NDH of them each, the first V slot m and l; all free after the loop): lane l of
  // group 0's wave w reads exactly what lane l of group 1's wave w wrote. float4 i of dim
  // tile t holds the row's dims 32 t + 8 i + 4 hh .. + 3.
  constexpr int NDH = ND / 2;
  static_assert(NDH >= 1 && sizeof(s_k0) >= kPfWaves * NDH * 4 * kWave * 16, "combine space");
  static_assert(sizeof(s_v0) >= kPfWaves * kWave * 8, "combine space");
  float4* const s_acc0 = reinterpret_cast<float4*>(&s_k0[0][0]);
  float4* const s_acc1 = reinterpret_cast<float4*>(&s_k1[0][0]);
  float2* const s_ml = reinterpret_cast<float2*>(&s_v0[0][0]);
  auto s_slot = [&](int t, int i) {
    return (t < NDH ? s_acc0 : s_acc1) + ((w * NDH + t % NDH) * 4 + i) * kWave + lane;
  };
  if (grp == 1) {
#pragma unroll
    for (int t = 0; t < ND; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *s_slot(t, i) = make_float4(acc[t][4 * i], acc[t][4 * i + 1], acc[t][4 * i + 2], acc[t][4 * i + 3]);
    s_ml[w * kWave + lane] = make_float2(m_run, l_run);
  }
  __syncthreads();
  if (grp == 0) {
    const float2 ml1 = s_ml[w * kWave + lane];
    const float M = fmaxf(m_run, ml1.x);
    const float a0 = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - M);
    const float a1 = M == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml1.x - M);
    float l = l_run * a0 + ml1.y * a1;
    l = halves_sum(l);
    // the two groups' unnormalised sums of float4 i of dim tile t
    auto merged = [&](int t, int i) {
      const float4 o1 = *s_slot(t, i);
      return make_float4(acc[t][4 * i] * a0 + o1.x * a1, acc[t][4 * i + 1] * a0 + o1.y * a1,
                         acc[t][4 * i + 2] * a0 + o1.z * a1, acc[t][4 * i + 3] * a0 + o1.w * a1);
    };
    if constexpr (PX) {  // unnormalised partial of this (row, key partition)
      if (row_ok) {
        const int64_t slot = out_row() * p.npart + blockIdx.y;
        if (hh == 0) *reinterpret_cast<float2*>(p.pml + slot * 2) = make_float2(M, l);
#pragma unroll
        for (int t = 0; t < ND; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            *reinterpret_cast<float4*>(p.pacc + slot * D + 32 * t + 8 * i + 4 * hh) = merged(t, i);
      }
    } else if (!full) {  // stream-K share of a split task: its unnormalised partial
      if (row_ok) {
        const int rs = (2 * sk_share + (seg == 0 ? 0 : 1)) * kPfRows + (w * WROWS + cc);
        if (hh == 0) *reinterpret_cast<float2*>(p.sk_ml + static_cast<int64_t>(rs) * 2) = make_float2(M, l);
        float* const pa = p.sk_acc + static_cast<int64_t>(rs) * D + 4 * hh;
#pragma unroll
        for (int t = 0; t < ND; ++t)
#pragma unroll
          for (int i = 0; i < 4; ++i) *reinterpret_cast<float4*>(pa + 32 * t + 8 * i) = merged(t, i);
      }
    } else if (row_ok) {
      const float inv = l > 0.0f ? 1.0f / l : 0.0f;
      T* op = static_cast<T*>(p.out) + out_row() * D + 4 * hh;
#pragma unroll
      for (int t = 0; t < ND; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 o = merged(t, i);
          *reinterpret_cast<uint2*>(op + 32 * t + 8 * i) =
              make_uint2(Pack2<T>::pack(o.x * inv, o.y * inv), Pack2<T>::pack(o.z * inv, o.w * inv));
        }
    }
  }
  __syncthreads();  // this task's LDS reads are done before the next task's copies
  }  // task loop
}
// The stream-K schedule's fold launch: for each task split between shares, the merge of
// its shares' partials (m_j, l_j, acc_j) per row into the normalised output, with
// M = max m_j and w_j = 2^(m_j - M): out = sum_j w_j acc_j / sum_j w_j l_j (partials with
// m = -inf carry no weight; a row with no key at all gets zeros). A workgroup takes
// kPfFoldRows(D) rows of one task, D / 4 threads a row, 4 dims a thread, so that the
// partials of a task are read by many CUs at once. Tasks one share took whole were written
// by the prefill kernel; their workgroups return at once.
constexpr int kPfFoldThreads = 256;
template <int D>
constexpr int pf_fold_rows() { return kPfFoldThreads / (D / 4); }

template <typename T, int D>
__global__ __launch_bounds__(kPfFoldThreads) void prefill_sk_fold_kernel(const PrefillParams p) {
  constexpr int TPR = D / 4;                    // threads per row
  constexpr int FR = pf_fold_rows<D>();         // rows per workgroup
  constexpr int PER_TASK = kPfRows / FR;        // workgroups per task
  static_assert(kWave % TPR == 0 && kPfRows % FR == 0, "a row's threads in one wave");
  const unsigned task = blockIdx.x / PER_TASK;
  if (task >= static_cast<unsigned>(p.ntasks)) return;
  // the task's head starts at pv, its pairs at p0 (the shares' partial slots count from pv)
  const int pv = p.sk_pre[task], p1 = p.sk_pre[task + 1], total = p.sk_pre[p.ntasks];
  const int p0 = pv + p.sk_pre[p.ntasks + 1];
  if (p1 <= p0 || total <= 0) return;
  const int G = pf_sk_shares(p.sk_groups, total);
  const int l_lo = pf_sk_owner(p0, total, G), l_hi = pf_sk_owner(p1 - 1, total, G);
  if (l_lo == l_hi) return;  // one share's: written whole
  const unsigned per_b = static_cast<unsigned>(p.rblocks) * static_cast<unsigned>(p.KVH);
  const int b = static_cast<int>(task / per_b);
  const unsigned bx = task - static_cast<unsigned>(b) * per_b;
  const int rblock = p.rblocks - 1 - static_cast<int>(bx % static_cast<unsigned>(p.rblocks));
  const int kvh = static_cast<int>(bx / static_cast<unsigned>(p.rblocks));
  const int row0 = rblock * kPfRows;
  const int rows_here = min(kPfRows, p.rows_per_kvh - row0);
  const int j = static_cast<int>(threadIdx.x) % TPR;
  const int r = static_cast<int>(blockIdx.x % PER_TASK) * FR + static_cast<int>(threadIdx.x) / TPR;
  if (r >= rows_here) return;  // (the row's TPR threads leave together)
  // The row's M and L: thread j takes shares l_lo + j, l_lo + j + TPR, ...; then the row's
  // threads combine theirs.
  float M = -INFINITY, L = 0.0f;
  for (int l = l_lo + j; l <= l_hi; l += TPR) {
    const int rs = pf_sk_partial_slot(l, pv, total, G) * kPfRows + r;
    const float2 ml = *reinterpret_cast<const float2*>(p.sk_ml + static_cast<int64_t>(rs) * 2);
    if (ml.x == -INFINITY) continue;  // no key of this row in that share
    const float Mn = fmaxf(M, ml.x);
    L = L * __builtin_amdgcn_exp2f(M - Mn) + ml.y * __builtin_amdgcn_exp2f(ml.x - Mn);
    M = Mn;  // (2^(M - Mn) is 0 while M = -inf)
  }
#pragma unroll
  for (int o = 1; o < TPR; o <<= 1) {
    const float Mo = __shfl_xor(M, o, kWave);
    const float Lo = __shfl_xor(L, o, kWave);
    const float Mn = fmaxf(M, Mo);
    if (Mn != -INFINITY) {
      L = L * __builtin_amdgcn_exp2f(M - Mn) + Lo * __builtin_amdgcn_exp2f(Mo - Mn);
      M = Mn;
    }
  }
  float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll 4
  for (int l = l_lo; l <= l_hi; ++l) {
    const int64_t rs = static_cast<int64_t>(pf_sk_partial_slot(l, pv, total, G)) * kPfRows + r;
    const float m = p.sk_ml[rs * 2];
    const float4 v = *reinterpret_cast<const float4*>(p.sk_acc + rs * D + 4 * j);
    const float w = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - M);
    a.x = fmaf(v.x, w, a.x);
    a.y = fmaf(v.y, w, a.y);
    a.z = fmaf(v.z, w, a.z);
    a.w = fmaf(v.w, w, a.w);
  }
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  const int row = row0 + r;
  const int i = row / p.G;
  const int64_t orow = (static_cast<int64_t>(b) * p.q_len + i) * p.H + kvh * p.G + (row - i * p.G);
  *reinterpret_cast<uint2*>(static_cast<T*>(p.out) + orow * D + 4 * j) =
      make_uint2(Pack2<T>::pack(a.x * inv, a.y * inv), Pack2<T>::pack(a.z * inv, a.w * inv));
}

template <typename T, typename KT>
hipError_t launch_prefill_mfma_impl(const PrefillParams& p, int D, hipStream_t stream,
                                    bool* supported) {
  *supported = D == 64 || D == 128;
  if (!*supported) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(p.sk_groups > 0 ? p.sk_groups : kXcds * p.xcd_per));
  if (D == 128)
    hipLaunchKernelGGL((prefill_mfma_kernel<T, KT, 128, kPfRB, false>), grid, dim3(kPfThreads), 0,
                       stream, p);
  else
    hipLaunchKernelGGL((prefill_mfma_kernel<T, KT, 64, kPfRB, false>), grid, dim3(kPfThreads), 0,
                       stream, p);
  if (p.sk_groups > 0) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (D == 128)
      hipLaunchKernelGGL((prefill_sk_fold_kernel<T, 128>),
                         dim3(static_cast<unsigned>(p.ntasks * (kPfRows / pf_fold_rows<128>()))),
                         dim3(kPfFoldThreads), 0, stream, p);
    else
      hipLaunchKernelGGL((prefill_sk_fold_kernel<T, 64>),
                         dim3(static_cast<unsigned>(p.ntasks * (kPfRows / pf_fold_rows<64>()))),
                         dim3(kPfFoldThreads), 0, stream, p);
  }
  return hipGetLastError();
}

template <typename T, typename KT>
hipError_t launch_prefix_partials_impl(const PrefillParams& p, int D, hipStream_t stream,
                                       bool* supported) {
  *supported = D == 64 || D == 128;
  if (!*supported) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(p.rblocks * p.KVH), static_cast<unsigned>(p.npart), 1);
  if (D == 128)
    hipLaunchKernelGGL((prefill_mfma_kernel<T, KT, 128, kPfRB, true>), grid, dim3(kPfThreads), 0,
                       stream, p);
  else
    hipLaunchKernelGGL((prefill_mfma_kernel<T, KT, 64, kPfRB, true>), grid, dim3(kPfThreads), 0,
                       stream, p);
  return hipGetLastError();
}

// Launch for T in {bf16_t, _Float16} over a cache of T or of fp8 e4m3 (defined in
// prefill_mfma.hip and prefill_mfma_fp8.hip, the translation units compiled with the
// MFMA-in-VGPR option); *supported = false unless head_dim is 64 or 128.
template <typename T, typename KT>
hipError_t launch_prefill_mfma(const PrefillParams& p, int D, hipStream_t stream, bool* supported);
// The shared-prefix partials pass (PX kernels), same types.
template <typename T, typename KT>
hipError_t launch_prefix_partials(const PrefillParams& p, int D, hipStream_t stream,
                                  bool* supported);

#define MSATTN_DECLARE_PF(T, KT)                                                               \
  template <>                                                                                  \
  hipError_t launch_prefill_mfma<T, KT>(const PrefillParams& p, int D, hipStream_t stream,     \
                                        bool* supported);                                      \
  template <>                                                                                  \
  hipError_t launch_prefix_partials<T, KT>(const PrefillParams& p, int D, hipStream_t stream,  \
                                           bool* supported);
MSATTN_DECLARE_PF(bf16_t, bf16_t)
MSATTN_DECLARE_PF(_Float16, _Float16)
MSATTN_DECLARE_PF(bf16_t, fp8_t)
MSATTN_DECLARE_PF(_Float16, fp8_t)
MSATTN_DECLARE_PF(bf16_t, float)
MSATTN_DECLARE_PF(_Float16, float)
#undef MSATTN_DECLARE_PF

#define MSATTN_DEFINE_PF(T, KT)                                                                \
  template <>                                                                                  \
  hipError_t launch_prefill_mfma<T, KT>(const PrefillParams& p, int D, hipStream_t stream,     \
                                        bool* supported) {                                     \
    return launch_prefill_mfma_impl<T, KT>(p, D, stream, supported);                           \
  }                                                                                            \
  template <>                                                                                  \
  hipError_t launch_prefix_partials<T, KT>(const PrefillParams& p, int D, hipStream_t stream,  \
                                           bool* supported) {                                  \
    return launch_prefix_partials_impl<T, KT>(p, D, stream, supported);                        \
  }

}  // namespace msattn
