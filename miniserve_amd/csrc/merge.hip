// Log-sum-exp merge of split-K partials into the attention output.
//
// One wave per output row (4 rows per workgroup). The workspace header says how
// the partials kernel laid its partials out:
//   kind 0 (partition kernels): a row's partials sit in its slots 0, 1, ... up to
//     the first end marker (l = -1) or the last slot;
//   kind 1 (stream-K decode): a decode row (b, h) belongs to unit u = rtile * KVH + kvh
//     (rtile = (h % G) / RT), unit group ug = u / UG; its segment ug * B + b spans
//     positions [ug * sumT + P_b, ... + T_b) of the chunked work list, and the chunk r
//     holding a piece of it stored that piece at id r + ug * B + b.
// The slot arithmetic is merge_slot_range (merge_slots.h), which reads only slots the
// workspace holds whatever its header says.
// With running max M and weights w_j = 2^(m_j - M):
//   out = sum_j w_j acc_j / sum_j w_j l_j
// which is the merge of kernels/paged_attn_triton.py:_merge_kernel (:250-284) and
// of flash_decode_reference's running update (:155-170), in base 2. Partials with
// m = -inf carry no weight; rows with no key at all get zeros (the value
// flash_decode_reference returns for L <= 0, :143-144). A cascade decode adds a second
// source: the npp partials per row of its shared-prefix pass, all slots written.
#include "kernels.h"

namespace msattn {

constexpr int kMergeThreads = 256;
constexpr int kMergeWaves = kMergeThreads / kWave;
constexpr int kMergeMaxDims = 4;  // dims per lane: head_dim <= 256
#ifndef MSATTN_MERGE_BATCH
#define MSATTN_MERGE_BATCH 8
#endif
constexpr int kMergeBatch = MSATTN_MERGE_BATCH;  // acc rows loaded together
// The same for a cascade decode's shared-prefix partials, which fill every slot (32 per
// row on C4): one round of loads where the decode source's batch would take four.
#ifndef MSATTN_MERGE_PREFIX_BATCH
#define MSATTN_MERGE_PREFIX_BATCH 32
#endif
constexpr int kMergePrefixBatch = MSATTN_MERGE_PREFIX_BATCH;

// DPL: dims per lane (head_dim <= 64 * DPL), so the acc rows in flight take only the
// registers the head size needs.
template <typename QT, int DPL>
__global__ __launch_bounds__(kMergeThreads) void merge_kernel(const MergeParams p) {
  constexpr int kMergeMaxDims = DPL;
  const int lane = threadIdx.x & (kWave - 1);
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kMergeWaves + w;
  if (row >= p.rows) return;
  const int D = p.D;

  // Header and this row's prefix entries are read up front, in one round trip (skipped
  // when the caller knows the partition layout was used: its slots need no header).
  // merge_slot_range checks every word it uses and keeps the slots it names inside the
  // workspace, whatever the header holds.
  const bool known0 = p.kind_hint == 0;
  int hv[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const int64_t bq = row / p.H;  // the sequence when q_len == 1
  const int bh = bq < p.batch ? static_cast<int>(bq) : p.batch - 1;  // batch + 1 prefixes
  int pb = 0, pe = 0;
  if (!known0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) hv[i] = p.hdr[i];
    pb = p.hdr[kHdrPrefix + bh];
    pe = p.hdr[kHdrPrefix + bh + 1];
  }
  // Partial j of this row sits at slot base + j * stride, j < n.
  const SlotRange sr = merge_slot_range(hv, pb, pe, row, p.batch, p.H, p.KVH, p.G, p.max_parts,
                                        p.slots, p.kind_hint);

  float acc[kMergeMaxDims];
#pragma unroll
  for (int k = 0; k < kMergeMaxDims; ++k) acc[k] = 0.0f;
  float M = -INFINITY;
  float L = 0.0f;
  // 64 partials at a time: lane j loads (m, l) of partial j0 + j, the wave takes their
  // max and weights, then folds the acc rows kMergeBatch at a time with all of a batch's
  // loads in flight together. The first batch's acc rows do not depend on (m, l) and are
  // loaded together with them.
  auto fold_source = [&](auto batch_c, const float* src_ml, const float* src_acc, int64_t base,
                         int64_t stride, int64_t n, bool markers) {
    constexpr int kMergeBatch = decltype(batch_c)::value;
    for (int64_t j0 = 0; j0 < n; j0 += kWave) {
      const int64_t j = j0 + lane;
      const int cmax = static_cast<int>(n - j0 < kWave ? n - j0 : kWave);
      float m = -INFINITY, l = 0.0f;
      if (j < n) {
        const float2 v = *reinterpret_cast<const float2*>(src_ml + (base + j * stride) * 2);
        m = v.x;
        l = v.y;
      }
      auto load_batch = [&](int i0, float (&x)[kMergeBatch][kMergeMaxDims]) {
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) {
          const int i = i0 + u < cmax ? i0 + u : cmax - 1;  // stays on a real slot
          const float* arow = src_acc + (base + (j0 + i) * stride) * D;
#pragma unroll
          for (int k = 0; k < kMergeMaxDims; ++k) {
            const int d = lane + kWave * k;
            x[u][k] = d < D ? arow[d] : 0.0f;
          }
        }
      };
      float x0[kMergeBatch][kMergeMaxDims];
      load_batch(0, x0);
      int cnt = cmax;
      bool end = false;
      if (markers) {  // the first end marker (l = -1) closes the row
        const uint64_t mk = __ballot(j < n && l == -1.0f);
        if (mk) {
          cnt = __builtin_ctzll(mk);
          end = true;
        }
      }
      if (lane >= cnt) m = -INFINITY;
      const float mb = group_max<kWave>(m);
      if (mb != -INFINITY) {
        const float Mn = fmaxf(M, mb);
        const float a = __builtin_amdgcn_exp2f(M - Mn);  // 0 while M = -inf
        const float wj = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - Mn);
        L = L * a + group_sum<kWave>(wj * l);
#pragma unroll
        for (int k = 0; k < kMergeMaxDims; ++k) acc[k] *= a;
        auto fold = [&](int i0, const float (&x)[kMergeBatch][kMergeMaxDims]) {
#pragma unroll
          for (int u = 0; u < kMergeBatch; ++u) {
            const int i = i0 + u < cnt ? i0 + u : cnt - 1;
            const float wv = i0 + u < cnt ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                                      __builtin_bit_cast(int, wj), i))
                                          : 0.0f;
#pragma unroll
            for (int k = 0; k < kMergeMaxDims; ++k)  // weight 0: partial without keys
              acc[k] += wv != 0.0f ? wv * x[u][k] : 0.0f;
          }
        };
        fold(0, x0);
        for (int i0 = kMergeBatch; i0 < cnt; i0 += kMergeBatch) {
          float x[kMergeBatch][kMergeMaxDims];
          load_batch(i0, x);
          fold(i0, x);
        }
        M = Mn;
      }
      if (end) break;
    }
  };
  fold_source(std::integral_constant<int, kMergeBatch>{}, p.ml, p.acc, sr.base, sr.stride, sr.n,
              sr.markers);
  if (p.npp > 0) {
    const SlotRange pr = clamp_slots(SlotRange{row * p.npp, 1, p.npp, false}, p.pslots);
    fold_source(std::integral_constant<int, kMergePrefixBatch>{}, p.pml, p.pacc, pr.base, 1,
                pr.n, false);
  }

  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  QT* out = static_cast<QT*>(p.out) + row * D;
#pragma unroll
  for (int k = 0; k < kMergeMaxDims; ++k) {
    const int d = lane + kWave * k;
    if (d < D) Elt<QT>::store(out + d, acc[k] * inv);
  }
}

template <typename QT, int DPL>
static hipError_t launch_merge_d(const MergeParams& p, hipStream_t stream) {
  const unsigned blocks = static_cast<unsigned>((p.rows + kMergeWaves - 1) / kMergeWaves);
  hipLaunchKernelGGL((merge_kernel<QT, DPL>), dim3(blocks), dim3(kMergeThreads), 0, stream, p);
  return hipGetLastError();
}

template <typename QT>
static hipError_t launch_merge_t(const MergeParams& p, hipStream_t stream) {
  if (p.D <= kWave) return launch_merge_d<QT, 1>(p, stream);
  if (p.D <= 2 * kWave) return launch_merge_d<QT, 2>(p, stream);
  return launch_merge_d<QT, kMergeMaxDims>(p, stream);
}

hipError_t launch_merge(const MergeParams& p, int q_dtype, hipStream_t stream, bool* supported) {
  *supported = p.D <= kWave * kMergeMaxDims;
  if (!*supported) return hipSuccess;
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
