// KV-cache scatter (write_kv) and block-table gather kernels.
#include "kernels.h"

namespace msattn {

constexpr int kOpsThreads = 256;

// Resolve (row b, absolute position pos) to an element offset of the token's
// [head 0, dim 0] in the cache, or -1 for a hole / out-of-table position.
__device__ __forceinline__ int64_t token_offset(const int32_t* table, int b, int pos, int bs,
                                                int W, int num_blocks, int64_t blk_stride,
                                                int64_t slot_stride) {
  if (pos < 0) return -1;
  const int pg = pos / bs;
  if (pg >= W) return -1;
  const int phys = table[static_cast<int64_t>(b) * W + pg];
  if (phys < 0 || phys >= num_blocks) return -1;
  return static_cast<int64_t>(phys) * blk_stride + static_cast<int64_t>(pos - pg * bs) * slot_stride;
}

// write_kv: cache[table[b, pos/bs], pos%bs, h, d] = convert(src[b, t, h, d]),
// pos = starts[b] + t (miniserve/attention.py:111-133). One thread per element.
template <typename ST, typename DT>
__global__ __launch_bounds__(kOpsThreads) void write_kv_kernel(const WriteKVParams p) {
  const int64_t total = static_cast<int64_t>(p.batch) * p.tokens * p.KVH * p.D;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kOpsThreads + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * kOpsThreads) {
    const int d = static_cast<int>(idx % p.D);
    int64_t rest = idx / p.D;
    const int h = static_cast<int>(rest % p.KVH);
    rest /= p.KVH;
    const int t = static_cast<int>(rest % p.tokens);
    const int b = static_cast<int>(rest / p.tokens);
    const int64_t off = token_offset(p.table, b, p.starts[b] + p.start_offset + t, p.bs, p.W, p.num_blocks,
                                     p.blk_stride, p.slot_stride);
    if (off < 0) continue;
    const int64_t dst = off + static_cast<int64_t>(h) * p.head_stride + d;
    Elt<DT>::store(static_cast<DT*>(p.k_cache) + dst, Elt<ST>::load(static_cast<const ST*>(p.k) + idx));
    Elt<DT>::store(static_cast<DT*>(p.v_cache) + dst, Elt<ST>::load(static_cast<const ST*>(p.v) + idx));
  }
}

// Same-dtype scatter: raw element copy (bit-exact, NaN payloads included).
template <typename T>
__global__ __launch_bounds__(kOpsThreads) void write_kv_copy_kernel(const WriteKVParams p) {
  const int64_t total = static_cast<int64_t>(p.batch) * p.tokens * p.KVH * p.D;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kOpsThreads + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * kOpsThreads) {
    const int d = static_cast<int>(idx % p.D);
    int64_t rest = idx / p.D;
    const int h = static_cast<int>(rest % p.KVH);
    rest /= p.KVH;
    const int t = static_cast<int>(rest % p.tokens);
    const int b = static_cast<int>(rest / p.tokens);
    const int64_t off = token_offset(p.table, b, p.starts[b] + p.start_offset + t, p.bs, p.W, p.num_blocks,
                                     p.blk_stride, p.slot_stride);
    if (off < 0) continue;
    const int64_t dst = off + static_cast<int64_t>(h) * p.head_stride + d;
    static_cast<T*>(p.k_cache)[dst] = static_cast<const T*>(p.k)[idx];
    static_cast<T*>(p.v_cache)[dst] = static_cast<const T*>(p.v)[idx];
  }
}

// Vector form of both scatters: one thread per E consecutive elements of a row (E * the
// source element = 16 bytes, or 4 fp32 elements), loaded with one load and stored with one
// store (E elements of the cache type), the table looked up once per thread. Used when
// head_dim is a multiple of E and the cache pointer and strides sit on the store's
// alignment; the same conversions as the element kernels (same-type: the bits copied).
template <int N>
struct alignas(N) RawN {
  unsigned char b[N];
};

template <typename ST, typename DT, int E>
__global__ __launch_bounds__(kOpsThreads) void write_kv_vec_kernel(const WriteKVParams p) {
  const int CPR = p.D / E;  // chunks per row
  const int64_t total = static_cast<int64_t>(p.batch) * p.tokens * p.KVH * CPR;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kOpsThreads + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * kOpsThreads) {
    const int c = static_cast<int>(idx % CPR);
    int64_t rest = idx / CPR;
    const int h = static_cast<int>(rest % p.KVH);
    rest /= p.KVH;
    const int t = static_cast<int>(rest % p.tokens);
    const int b = static_cast<int>(rest / p.tokens);
    const int64_t off = token_offset(p.table, b, p.starts[b] + p.start_offset + t, p.bs, p.W, p.num_blocks,
                                     p.blk_stride, p.slot_stride);
    if (off < 0) continue;
    const int64_t src = idx * E;  // [b, t, h, c * E] of the contiguous source
    const int64_t dst = off + static_cast<int64_t>(h) * p.head_stride + static_cast<int64_t>(c) * E;
#pragma unroll
    for (int which = 0; which < 2; ++which) {
      const ST* sp = static_cast<const ST*>(which ? p.v : p.k) + src;
      DT* dp = static_cast<DT*>(which ? p.v_cache : p.k_cache) + dst;
      if constexpr (std::is_same<ST, DT>::value) {
        *reinterpret_cast<RawN<E * sizeof(ST)>*>(dp) =
            *reinterpret_cast<const RawN<E * sizeof(ST)>*>(sp);
      } else {
        const RawN<E * sizeof(ST)> in = *reinterpret_cast<const RawN<E * sizeof(ST)>*>(sp);
        RawN<E * sizeof(DT)> o;
#pragma unroll
        for (int e = 0; e < E; ++e)
          Elt<DT>::store(reinterpret_cast<DT*>(o.b) + e,
                         Elt<ST>::load(reinterpret_cast<const ST*>(in.b) + e));
        *reinterpret_cast<RawN<E * sizeof(DT)>*>(dp) = o;
      }
    }
  }
}

static unsigned grid_for(int64_t total) {
  int64_t blocks = (total + kOpsThreads - 1) / kOpsThreads;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  return static_cast<unsigned>(blocks);
}

// Whether the vector form with E elements per thread applies: head_dim a multiple of E,
// the source (contiguous) on E source elements' alignment, the caches and their strides
// on E cache elements' alignment.
template <typename ST, typename DT, int E>
static bool wkv_vec_ok(const WriteKVParams& p) {
  const uintptr_t sa = E * sizeof(ST), da = E * sizeof(DT);
  auto al = [](const void* q, uintptr_t a) { return reinterpret_cast<uintptr_t>(q) % a == 0; };
  return p.D % E == 0 && al(p.k, sa) && al(p.v, sa) && al(p.k_cache, da) && al(p.v_cache, da) &&
         (p.blk_stride * sizeof(DT)) % da == 0 && (p.slot_stride * sizeof(DT)) % da == 0 &&
         (p.head_stride * sizeof(DT)) % da == 0;
}

template <typename ST, typename DT>
static hipError_t launch_wkv(const WriteKVParams& p, hipStream_t stream) {
  constexpr int E = sizeof(ST) >= 4 || sizeof(DT) >= 4 ? 4 : 8;
  if (wkv_vec_ok<ST, DT, E>(p)) {
    const int64_t total = static_cast<int64_t>(p.batch) * p.tokens * p.KVH * (p.D / E);
    hipLaunchKernelGGL((write_kv_vec_kernel<ST, DT, E>), dim3(grid_for(total)), dim3(kOpsThreads),
                       0, stream, p);
    return hipGetLastError();
  }
  const int64_t total = static_cast<int64_t>(p.batch) * p.tokens * p.KVH * p.D;
  hipLaunchKernelGGL((write_kv_kernel<ST, DT>), dim3(grid_for(total)), dim3(kOpsThreads), 0,
                     stream, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_wkv_copy(const WriteKVParams& p, hipStream_t stream) {
  constexpr int E = 16 / sizeof(T);
  if (wkv_vec_ok<T, T, E>(p)) {
    const int64_t total = static_cast<int64_t>(p.batch) * p.tokens * p.KVH * (p.D / E);
    hipLaunchKernelGGL((write_kv_vec_kernel<T, T, E>), dim3(grid_for(total)), dim3(kOpsThreads),
                       0, stream, p);
    return hipGetLastError();
  }
  const int64_t total = static_cast<int64_t>(p.batch) * p.tokens * p.KVH * p.D;
  hipLaunchKernelGGL(write_kv_copy_kernel<T>, dim3(grid_for(total)), dim3(kOpsThreads), 0, stream,
                     p);
  return hipGetLastError();
}

template <typename ST>
static hipError_t launch_wkv_src(const WriteKVParams& p, int dst_dtype, hipStream_t stream,
                                 bool* supported) {
  switch (dst_dtype) {
    case 0: return launch_wkv<ST, float>(p, stream);
    case 1: return launch_wkv<ST, _Float16>(p, stream);
    case 2: return launch_wkv<ST, bf16_t>(p, stream);
    case 3: return launch_wkv<ST, fp8_t>(p, stream);
    default: break;
  }
  *supported = false;
  return hipSuccess;
}

hipError_t launch_write_kv(const WriteKVParams& p, int src_dtype, int dst_dtype,
                           hipStream_t stream, bool* supported) {
  *supported = true;
  if (src_dtype == dst_dtype) {
    switch (src_dtype) {
      case 0: return launch_wkv_copy<uint32_t>(p, stream);
      case 1:
      case 2: return launch_wkv_copy<uint16_t>(p, stream);
      case 3: return launch_wkv_copy<uint8_t>(p, stream);
      default: break;
    }
    *supported = false;
    return hipSuccess;
  }
  switch (src_dtype) {
    case 0: return launch_wkv_src<float>(p, dst_dtype, stream, supported);
    case 1: return launch_wkv_src<_Float16>(p, dst_dtype, stream, supported);
    case 2: return launch_wkv_src<bf16_t>(p, dst_dtype, stream, supported);
    default: break;
  }
  *supported = false;
  return hipSuccess;
}

// Gather: out[b, pos, h, d] = cache[blk, pos % bs, h, d] with blk = table[b, pos / bs]
// for pos < len[b] and blk = 0 for pos >= len[b] (miniserve/attention.py:163-171).
// Holes give zeros.
template <typename T>
__global__ __launch_bounds__(kOpsThreads) void gather_kernel(const GatherParams p) {
  const int64_t total = static_cast<int64_t>(p.batch) * p.max_ctx * p.KVH * p.D;
  for (int64_t idx = static_cast<int64_t>(blockIdx.x) * kOpsThreads + threadIdx.x; idx < total;
       idx += static_cast<int64_t>(gridDim.x) * kOpsThreads) {
    const int d = static_cast<int>(idx % p.D);
    int64_t rest = idx / p.D;
    const int h = static_cast<int>(rest % p.KVH);
    rest /= p.KVH;
    const int pos = static_cast<int>(rest % p.max_ctx);
    const int b = static_cast<int>(rest / p.max_ctx);
    int64_t off;
    if (pos < p.lens[b]) {
      off = token_offset(p.table, b, pos, p.bs, p.W, p.num_blocks, p.blk_stride, p.slot_stride);
    } else {
      off = static_cast<int64_t>(pos % p.bs) * p.slot_stride;  // page 0
    }
    T val = T(0);
    if (off >= 0) val = static_cast<const T*>(p.cache)[off + static_cast<int64_t>(h) * p.head_stride + d];
    static_cast<T*>(p.out)[idx] = val;
  }
}

hipError_t launch_gather(const GatherParams& p, int elt_bytes, hipStream_t stream) {
  const int64_t total = static_cast<int64_t>(p.batch) * p.max_ctx * p.KVH * p.D;
  const dim3 grid(grid_for(total));
  switch (elt_bytes) {
    case 4: hipLaunchKernelGGL(gather_kernel<uint32_t>, grid, dim3(kOpsThreads), 0, stream, p); break;
    case 2: hipLaunchKernelGGL(gather_kernel<uint16_t>, grid, dim3(kOpsThreads), 0, stream, p); break;
    default: hipLaunchKernelGGL(gather_kernel<uint8_t>, grid, dim3(kOpsThreads), 0, stream, p); break;
  }
  return hipGetLastError();
}

}  // namespace msattn
