// Log-sum-exp merge of split-K partials (one workgroup per output row).
//
// A row's partials sit in workspace slots 0, 1, ... up to the first end marker
// (l = -1) or the last slot. With M = max_j m_j and w_j = 2^(m_j - M):
//   out = sum_j w_j acc_j / sum_j w_j l_j
// which is the merge of kernels/paged_attn_triton.py:_merge_kernel (:250-284)
// and of flash_decode_reference's running update (:155-170), in base 2. Slots
// with m = -inf (no visible key) carry no weight. Rows with no key at all
// (context 0, or fully masked) get zeros, the value flash_decode_reference
// returns for L <= 0 (:143-144).
#include "kernels.h"

namespace msattn {

constexpr int kMergeThreads = 256;
constexpr int kMergeWaves = kMergeThreads / kWave;

template <typename QT>
__global__ __launch_bounds__(kMergeThreads) void merge_kernel(const MergeParams p) {
  __shared__ float s_w[kMergeThreads];
  __shared__ float s_red[kMergeThreads * 4];
  __shared__ float s_wave[kMergeWaves];
  __shared__ int s_end[kMergeWaves];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wv = tid / kWave;
  const int64_t row = blockIdx.x;
  const float* ml = p.ml + row * p.max_parts * 2;
  const float* acc = p.acc + row * p.max_parts * p.D;

  // Number of filled slots: index of the first end marker.
  int first_end = p.max_parts;
  for (int j = tid; j < p.max_parts; j += kMergeThreads)
    if (ml[2 * j + 1] == -1.0f) first_end = min(first_end, j);
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) first_end = min(first_end, __shfl_xor(first_end, o, kWave));
  if (lane == 0) s_end[wv] = first_end;
  __syncthreads();
  int n = s_end[0];
#pragma unroll
  for (int i = 1; i < kMergeWaves; ++i) n = min(n, s_end[i]);

  float m = -INFINITY;
  for (int j = tid; j < n; j += kMergeThreads) m = fmaxf(m, ml[2 * j]);
  m = group_max<kWave>(m);
  if (lane == 0) s_wave[wv] = m;
  __syncthreads();
  float M = s_wave[0];
#pragma unroll
  for (int i = 1; i < kMergeWaves; ++i) M = fmaxf(M, s_wave[i]);

  const int DV = p.D / 4;               // float4 columns per row
  const int PS = kMergeThreads / DV;    // slots handled side by side
  const int ps = tid / DV;
  const int d4 = tid - ps * DV;
  float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
  float L = 0.0f;
  for (int base = 0; base < n; base += kMergeThreads) {
    const int cnt = min(kMergeThreads, n - base);
    __syncthreads();
    if (tid < cnt) {
      const float mp = ml[2 * (base + tid)];
      const float lp = ml[2 * (base + tid) + 1];
      const float wgt = (mp == -INFINITY) ? 0.0f : exp2f(mp - M);
      s_w[tid] = wgt;
      L = fmaf(wgt, lp, L);
    }
    __syncthreads();
    if (ps < PS) {
      for (int j = ps; j < cnt; j += PS) {
        const float wgt = s_w[j];
        if (wgt != 0.0f) {
          const float4 x =
              *reinterpret_cast<const float4*>(acc + static_cast<int64_t>(base + j) * p.D + 4 * d4);
          a.x = fmaf(wgt, x.x, a.x);
          a.y = fmaf(wgt, x.y, a.y);
          a.z = fmaf(wgt, x.z, a.z);
          a.w = fmaf(wgt, x.w, a.w);
        }
      }
    }
  }
  L = group_sum<kWave>(L);
  __syncthreads();
  if (lane == 0) s_wave[wv] = L;
  if (ps < PS) {
    s_red[ps * p.D + 4 * d4 + 0] = a.x;
    s_red[ps * p.D + 4 * d4 + 1] = a.y;
    s_red[ps * p.D + 4 * d4 + 2] = a.z;
    s_red[ps * p.D + 4 * d4 + 3] = a.w;
  }
  __syncthreads();
  float Lt = 0.0f;
#pragma unroll
  for (int i = 0; i < kMergeWaves; ++i) Lt += s_wave[i];
  const float inv = Lt > 0.0f ? 1.0f / Lt : 0.0f;
  QT* out = static_cast<QT*>(p.out) + row * p.D;
  for (int d = tid; d < p.D; d += kMergeThreads) {
    float s = 0.0f;
    for (int i = 0; i < PS; ++i) s += s_red[i * p.D + d];
    Elt<QT>::store(out + d, s * inv);
  }
}

template <typename QT>
static hipError_t launch_merge_t(const MergeParams& p, hipStream_t stream) {
  hipLaunchKernelGGL(merge_kernel<QT>, dim3(static_cast<unsigned>(p.rows)), dim3(kMergeThreads), 0,
                     stream, p);
  return hipGetLastError();
}

hipError_t launch_merge(const MergeParams& p, int q_dtype, hipStream_t stream, bool* supported) {
  *supported = true;
  switch (q_dtype) {
    case 0: return launch_merge_t<float>(p, stream);
    case 1: return launch_merge_t<_Float16>(p, stream);
    case 2: return launch_merge_t<bf16_t>(p, stream);
    default: break;
  }
  *supported = false;
  return hipSuccess;
}

}  // namespace msattn
