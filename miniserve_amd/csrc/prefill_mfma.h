// Chunked-prefill paged attention on MFMA (gfx950): q_len > 1, bf16/fp16, head_dim 128.
//
// One workgroup (4 waves) owns 64 query rows of one (sequence b, KV head): rows are
// the (query token i, GQA head g) pairs r = i * group + g, 16 per wave. It walks the
// keys its rows may see in steps of 64 tokens (four 16-token page slices):
//   * the step's K and V rows are staged through LDS (row-major, padded), loaded
//     one step ahead into registers;
//   * S^T = K Q^T on v_mfma_f32_16x16x32: A = K rows read from LDS, B = the wave's
//     query rows kept in registers, so lane (g = l/16, n = l%16) holds the scores
//     of query row n for tokens 4g .. 4g+3 of each 16-token slice;
//   * online softmax per row (fp32, base 2), causal / window masks per key;
//   * O^T += V^T P^T on the same MFMA: B = P^T comes straight from the score
//     registers (bf16), A = V^T is read transposed from the row-major V rows with
//     ds_read_b64_tr_b16 (each lane names 4 dims of one token; lane i of a
//     16-lane group receives dim i of four tokens). Lane (g, n) accumulates
//     O[row n][dims 16t + 4g + r], so the softmax rescale stays in the lane.
// The rows' outputs are normalised and written directly (no split-K partials).
//
// Semantics: PagedAttention.forward with q_len > 1 (miniserve/attention.py:205-250,
// mask :135-153; the trailing query positions q_pos = len - q_len + i, :146).
#pragma once

#include "decode_mfma.h"

namespace msattn {

constexpr int kPfWaves = 4;
constexpr int kPfThreads = kPfWaves * kWave;
constexpr int kPfRows = 16 * kPfWaves;  // query rows per workgroup
constexpr int kPfStep = 64;             // key tokens per step
constexpr int kPfPageChunk = 512;       // page ids cached in LDS at a time

typedef short pf_s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) pf_s4 lds_s4;  // an LDS pointer target

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
};

typedef float pf_f2 __attribute__((ext_vector_type(2)));
typedef __bf16 pf_bf2 __attribute__((ext_vector_type(2)));
typedef _Float16 pf_h2 __attribute__((ext_vector_type(2)));

// Two fp32 values -> one packed 16-bit pair (v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32,
// round to nearest even).
template <typename T> struct Pack2;
template <> struct Pack2<bf16_t> {
  __device__ static uint32_t pack(float a, float b) {
    const pf_f2 x = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, pf_bf2));
  }
};
template <> struct Pack2<_Float16> {
  __device__ static uint32_t pack(float a, float b) {
    const pf_f2 x = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, pf_h2));
  }
};

template <typename T, int D>
__global__ __launch_bounds__(kPfThreads) void prefill_mfma_kernel(const PrefillParams p) {
  static_assert(D == 128, "prefill MFMA kernel handles head_dim 128");
  constexpr int JD = D / 32;              // k-steps of S^T
  constexpr int ND = D / 16;              // 16-dim tiles of O^T
  constexpr int RS = D + 8;               // LDS row stride (elements): 16 B of padding
  constexpr int CPR = D * 2 / 16;         // 16-byte chunks per K/V row
  constexpr int LPT = kPfStep * CPR / kPfThreads;  // chunks per thread per tensor per step
  static_assert(LPT * kPfThreads == kPfStep * CPR, "staging split");

  __shared__ __attribute__((aligned(16))) uint16_t s_k[kPfStep * RS];
  __shared__ __attribute__((aligned(16))) uint16_t s_v[kPfStep * RS];
  __shared__ int s_pg[kPfPageChunk];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int g = lane >> 4;
  const int n = lane & 15;

  // Larger (later) row blocks first: they see the most keys under a causal mask.
  const unsigned bx = blockIdx.x;
  const int rblock = p.rblocks - 1 - static_cast<int>(bx % static_cast<unsigned>(p.rblocks));
  const int kvh = static_cast<int>(bx / static_cast<unsigned>(p.rblocks));
  const int b = blockIdx.z;

  int ctx = p.lens[b];
  ctx = ctx < 0 ? 0 : (ctx > p.max_ctx ? p.max_ctx : ctx);
  const int row0 = rblock * kPfRows;
  const int rows_here = min(kPfRows, p.rows_per_kvh - row0);

  // Key range of the block (query index grows with the row).
  const int i_first = row0 / p.G;
  const int i_last = (row0 + rows_here - 1) / p.G;
  const int lo_all = p.window > 0 ? max(0, ctx - p.q_len + i_first - p.window + 1) : 0;
  const int hi_all = p.causal ? min(ctx, ctx - p.q_len + i_last + 1) : ctx;

  // This lane's query row (MFMA column n of the wave's 16 rows).
  const int row = row0 + w * 16 + n;
  const bool row_ok = row < p.rows_per_kvh;
  int lo_n = 0, hi_n = 0;
  int64_t orow = 0;
  if (row_ok) {
    const int i = row / p.G;
    const int qpos = ctx - p.q_len + i;
    hi_n = p.causal ? min(ctx, qpos + 1) : ctx;
    lo_n = p.window > 0 ? max(0, qpos - p.window + 1) : 0;
    if (hi_n < lo_n) hi_n = lo_n;
    orow = (static_cast<int64_t>(b) * p.q_len + i) * p.H + kvh * p.G + (row - i * p.G);
  }
  // Keys every row of this wave sees: [wave_lo, wave_hi) (rows grow with the query).
  int wave_lo = 0, wave_hi = 0;
  {
    const int wr0 = row0 + w * 16;
    const int wr1 = min(wr0 + 16, p.rows_per_kvh) - 1;
    if (wr1 >= wr0) {
      const int qa = ctx - p.q_len + wr0 / p.G;  // first row's query position
      const int qb_ = ctx - p.q_len + wr1 / p.G; // last row's
      wave_hi = p.causal ? min(ctx, qa + 1) : ctx;
      wave_lo = p.window > 0 ? max(0, qb_ - p.window + 1) : 0;
    }
  }
  uint4 qb[JD];
  {
    const T* qp = static_cast<const T*>(p.q);
#pragma unroll
    for (int j = 0; j < JD; ++j) {
      qb[j] = make_uint4(0u, 0u, 0u, 0u);
      if (row_ok) qb[j] = *reinterpret_cast<const uint4*>(qp + orow * D + 32 * j + 8 * g);
    }
  }

  mf_f32x4 acc[ND];
#pragma unroll
  for (int t = 0; t < ND; ++t) acc[t] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;
  float l_run = 0.0f;

  const T* kbase = static_cast<const T*>(p.k);
  const T* vbase = static_cast<const T*>(p.v);
  const int step_first = hi_all > lo_all ? lo_all / kPfStep : 0;
  const int step_end = hi_all > lo_all ? ceil_div(hi_all, kPfStep) : 0;

  // Staging: thread tid loads chunk c of token rows tr + (kPfThreads / CPR) * j.
  const int st_c = tid % CPR;
  const int st_r = tid / CPR;
  constexpr int ROWS_PER_PASS = kPfThreads / CPR;
  uint4 kst[LPT], vst[LPT];
  int pg_chunk = -1;

  auto load_pages = [&](int chunk) {  // all threads; caller brackets with barriers
    for (int j = tid; j < kPfPageChunk; j += kPfThreads) {
      const int pg = chunk * kPfPageChunk + j;
      int phys = -1;
      if (pg < p.W) {
        phys = p.table[static_cast<int64_t>(b) * p.W + pg];
        if (phys < 0 || phys >= p.num_blocks) phys = -1;
      }
      s_pg[j] = phys;
    }
  };
  auto issue = [&](int step) {
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int tok = step * kPfStep + st_r + ROWS_PER_PASS * j;
      const int pg = tok / p.bs;
      const int phys = (tok < hi_all && tok >= lo_all) ? s_pg[pg - pg_chunk * kPfPageChunk] : -1;
      kst[j] = make_uint4(0u, 0u, 0u, 0u);
      vst[j] = make_uint4(0u, 0u, 0u, 0u);
      if (phys >= 0) {
        const int64_t off = static_cast<int64_t>(phys) * p.blk_stride +
                            static_cast<int64_t>(tok - pg * p.bs) * p.slot_stride +
                            static_cast<int64_t>(kvh) * p.head_stride + st_c * 8;
        kst[j] = *reinterpret_cast<const uint4*>(kbase + off);
        vst[j] = *reinterpret_cast<const uint4*>(vbase + off);
      }
    }
  };
  // The page ids a step needs lie in one chunk when kPfStep divides the chunk's tokens.
  auto ensure_pages = [&](int step) {
    const int chunk = (step * kPfStep) / p.bs / kPfPageChunk;
    if (chunk != pg_chunk) {
      __syncthreads();
      load_pages(chunk);
      pg_chunk = chunk;
      __syncthreads();
    }
  };

  if (step_first < step_end) {
    ensure_pages(step_first);
    issue(step_first);
  }
  for (int step = step_first; step < step_end; ++step) {
    __syncthreads();  // the previous step's LDS reads are done
#pragma unroll
    for (int j = 0; j < LPT; ++j) {
      const int r = st_r + ROWS_PER_PASS * j;
      *reinterpret_cast<uint4*>(&s_k[r * RS + st_c * 8]) = kst[j];
      *reinterpret_cast<uint4*>(&s_v[r * RS + st_c * 8]) = vst[j];
    }
    if (step + 1 < step_end) {
      ensure_pages(step + 1);
      issue(step + 1);
    }
    __syncthreads();  // this step's K/V rows are in LDS

    const int t_base = step * kPfStep;
    // Keys of this step all visible to every row of the wave: no per-key mask.
    const bool full = t_base >= wave_lo && t_base + kPfStep <= wave_hi;
    // ---- S^T for the wave's 16 rows: 4 slices of 16 tokens ----
    float sc[4][4];
    float mt = -INFINITY;
    mf_f32x4 sv[4];
#pragma unroll
    for (int sl = 0; sl < 4; ++sl) sv[sl] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
    // k-step outer, slices inner: four independent LDS reads, then four MFMAs
#pragma unroll
    for (int j = 0; j < JD; ++j) {
      uint4 ka[4];
#pragma unroll
      for (int sl = 0; sl < 4; ++sl)
        ka[sl] = *reinterpret_cast<const uint4*>(&s_k[(16 * sl + n) * RS + 32 * j + 8 * g]);
#pragma unroll
      for (int sl = 0; sl < 4; ++sl) sv[sl] = Mfma16<T>::mac(ka[sl], qb[j], sv[sl]);
    }
#pragma unroll
    for (int sl = 0; sl < 4; ++sl) {
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[sl][r] = sv[sl][r] * p.scale_log2;
      if (!full) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = t_base + 16 * sl + 4 * g + r;
          sc[sl][r] = (tok >= lo_n && tok < hi_n) ? sc[sl][r] : -INFINITY;
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) mt = fmaxf(mt, sc[sl][r]);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 16, kWave));
    mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
    const float m_new = fmaxf(m_run, mt);
    const bool live = m_new != -INFINITY;
    const float alpha = live ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
    float psum = 0.0f;
    uint4 pb[2];  // P^T as the B operand of the two 32-token k-steps
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      float pr[8];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float x = live ? __builtin_amdgcn_exp2f(sc[2 * ks + h][r] - m_new) : 0.0f;
          pr[4 * h + r] = x;
          psum += x;
        }
      pb[ks] = make_uint4(Pack2<T>::pack(pr[0], pr[1]), Pack2<T>::pack(pr[2], pr[3]),
                          Pack2<T>::pack(pr[4], pr[5]), Pack2<T>::pack(pr[6], pr[7]));
    }
    l_run = fmaf(l_run, alpha, psum);
    m_run = m_new;
    if (__any(alpha != 1.0f)) {  // alpha is exactly 1 for rows whose max did not move
#pragma unroll
      for (int t = 0; t < ND; ++t) acc[t] *= alpha;
    }

    // ---- O^T += V^T P^T: A = V^T via transposed LDS reads ----
    // Lane s of a 16-lane group names 4 dims (4 * (s & 3) ..) of token (s >> 2) + base;
    // lane i then receives dim i of those four tokens.
    const int tr_tok = lane >> 2 & 3;   // (s >> 2) within the group
    const int tr_dim = 4 * (lane & 3);  // 4 * (s & 3)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int tok0 = 32 * ks + 4 * g + tr_tok;        // e = 0..3: slice 2ks
      const int tok1 = 32 * ks + 16 + 4 * g + tr_tok;   // e = 4..7: slice 2ks + 1
      uint4 va[ND];  // all eight dim tiles' operands first, then the MFMAs
#pragma unroll
      for (int t = 0; t < ND; ++t) {
        const pf_s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s4*)(&s_v[tok0 * RS + 16 * t + tr_dim]));
        const pf_s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s4*)(&s_v[tok1 * RS + 16 * t + tr_dim]));
        const uint2 lo2 = __builtin_bit_cast(uint2, lo);
        const uint2 hi2 = __builtin_bit_cast(uint2, hi);
        va[t] = make_uint4(lo2.x, lo2.y, hi2.x, hi2.y);
      }
#pragma unroll
      for (int t = 0; t < ND; ++t) acc[t] = Mfma16<T>::mac(va[t], pb[ks], acc[t]);
    }
  }

  // ---- normalise and store: lane (g, n) holds O[row n][dims 16t + 4g + r] ----
  l_run += __shfl_xor(l_run, 16, kWave);
  l_run += __shfl_xor(l_run, 32, kWave);
  if (row_ok) {
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    T* op = static_cast<T*>(p.out) + orow * D;
#pragma unroll
    for (int t = 0; t < ND; ++t) {
      const uint2 pk = make_uint2(Pack2<T>::pack(acc[t][0] * inv, acc[t][1] * inv),
                                  Pack2<T>::pack(acc[t][2] * inv, acc[t][3] * inv));
      *reinterpret_cast<uint2*>(op + 16 * t + 4 * g) = pk;
    }
  }
}

template <typename T>
hipError_t launch_prefill_mfma(const PrefillParams& p, int D, hipStream_t stream, bool* supported) {
  *supported = D == 128;
  if (!*supported) return hipSuccess;
  const dim3 grid(static_cast<unsigned>(p.rblocks * p.KVH), 1, static_cast<unsigned>(p.batch));
  hipLaunchKernelGGL((prefill_mfma_kernel<T, 128>), grid, dim3(kPfThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace msattn
