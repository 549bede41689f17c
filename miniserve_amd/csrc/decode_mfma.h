// Paged decode partials with MFMA scores (gfx950): a bf16/fp16 query over a cache of its
// type, of fp8 e4m3 or of fp32 (converted to the query type in registers), head_dim 64
// or 128.
//
// Same contract and workspace output as split_kernel (split_kernel.h): one
// workgroup per (sequence b, KV head, row tile, context partition), writing the
// partial (m, l, acc) of each query row over the partition's keys.
//
// Differences from split_kernel, which make this the fast path:
//  * Tiles of 16 tokens (one page slice) are processed with an online softmax;
//    each wave owns a contiguous run of tiles and keeps the next tile's K and V
//    loads in flight while it computes the current one (no block barrier until
//    the final combine).
//  * S = K Q^T for a tile is D/32 v_mfma_f32_16x16x32 instructions: the K rows
//    are the A operand straight from their 16-byte global loads (lane l holds
//    K[token pi(l%16)][dims 8*(4j + l/16) .. +8] for MFMA j) and the packed query
//    rows are the B operand (lane l holds Q[row l%16][the same dims]). Lane
//    (g = l/16, n = l%16) receives the scores of query row n for the tile tokens
//    pi(4g + r), r = 0..3.
//  * pi is chosen so that the 16-lane row g that holds those scores is also the
//    row whose V lanes need them: V is loaded with LPR = D/8 lanes per token row,
//    and the tokens of V lanes in DPP row g are exactly {pi(4g + r)}. P.V then
//    takes P[n][token] from lane 16g + n through DPP row_newbcast, without LDS
//    traffic, two tokens at a time on v_dot2_f32 (pv_tile below).
//  * The 4 waves' (m, l, acc) are combined in LDS once at the end.
//
// Masking, key ranges and the partial format follow split_kernel and hence
// kernels/paged_attn_triton.py:176-248 and miniserve/attention.py:135-153.
#pragma once

#include <type_traits>
#include <utility>

#include "split_kernel.h"

// Tuning knobs (compile-time):
//   MSATTN_MFMA_WAVES  waves per workgroup;
//   MSATTN_LOAD_AUX    cache-policy bits of the stream-K kernel's K/V buffer loads
//                      (2 = nontemporal: the KV stream is read once);
//   MSATTN_LAZY_RESCALE skip the accumulator rescale when no row's max moved.
#ifndef MSATTN_MFMA_WAVES
#define MSATTN_MFMA_WAVES 4
#endif
// Tiles in flight per wave (ring depth), head_dim 128 / head_dim 64.
// 8-wave workgroups (two waves per SIMD): each wave posts the tiles it has consumed in LDS
// and runs at raised priority while it is not ahead of its SIMD partner (wave w ^ 4), as
// the stream-K kernel does, so that the younger wave is not starved of load issue and
// the two reach the workgroup's reduction together.
#ifndef MSATTN_PART_BALANCE
#define MSATTN_PART_BALANCE 1
#endif
// 1: the partition kernel's grid runs partition-major (SplitParams::part_major).
#ifndef MSATTN_PART_MAJOR
#define MSATTN_PART_MAJOR 1
#endif
#ifndef MSATTN_MFMA_DEPTH
#define MSATTN_MFMA_DEPTH 2
#endif
#ifndef MSATTN_MFMA_DEPTH_D64
#define MSATTN_MFMA_DEPTH_D64 2
#endif
#ifndef MSATTN_LOAD_AUX
#define MSATTN_LOAD_AUX 2
#endif
#ifndef MSATTN_LAZY_RESCALE
#define MSATTN_LAZY_RESCALE 1
#endif

namespace msattn {

typedef __bf16 mf_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 mf_f16x8 __attribute__((ext_vector_type(8)));
typedef float mf_f32x4 __attribute__((ext_vector_type(4)));

template <typename T> struct Mfma16;
template <> struct Mfma16<bf16_t> {
  __device__ static mf_f32x4 mac(const uint4& a, const uint4& b, mf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mf_bf16x8, a),
                                                   __builtin_bit_cast(mf_bf16x8, b), c, 0, 0, 0);
  }
};
template <> struct Mfma16<_Float16> {
  __device__ static mf_f32x4 mac(const uint4& a, const uint4& b, mf_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mf_f16x8, a),
                                                  __builtin_bit_cast(mf_f16x8, b), c, 0, 0, 0);
  }
};

// Eight fp32 values in two 16-byte halves: an fp32 cache's K/V chunk, and an fp32 query's.
struct F8 {
  uint4 lo, hi;
};
__device__ __forceinline__ void f8_unpack(const F8& x, float* o) {
  const uint32_t w[8] = {x.lo.x, x.lo.y, x.lo.z, x.lo.w, x.hi.x, x.hi.y, x.hi.z, x.hi.w};
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = __uint_as_float(w[e]);
}
__device__ __forceinline__ F8 f8_pack(const float* f) {
  return F8{make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                       __float_as_uint(f[3])),
            make_uint4(__float_as_uint(f[4]), __float_as_uint(f[5]), __float_as_uint(f[6]),
                       __float_as_uint(f[7]))};
}

// An fp32 query over an fp32 cache: a chunk's eight dims are eight k-steps of
// v_mfma_f32_16x16x4_f32, lane group g supplying k-index g of each (A[n][g] =
// K[token n][dim d0 + e], B[g][n] = Q[row n][dim d0 + e] with d0 the lane group's first
// dim). Summed over the eight steps this is the same 16 x 16 tile of dot products, with
// the layout of the 16x16x32 form, in fp32 products and sums (the reference computes
// in fp32 there: attention.py:240-249 with an fp32 query).
template <> struct Mfma16<float> {
  __device__ static mf_f32x4 mac(const F8& a, const F8& b, mf_f32x4 c) {
    float av[8], bv[8];
    f8_unpack(a, av);
    f8_unpack(b, bv);
#pragma unroll
    for (int e = 0; e < 8; ++e) c = __builtin_amdgcn_mfma_f32_16x16x4f32(av[e], bv[e], c, 0, 0, 0);
    return c;
  }
};

// The query's MFMA B-operand chunk (eight dims of one row) for a query type: one 16-byte
// load of bf16/fp16, two of fp32.
template <typename T> struct QChunk {
  typedef uint4 type;
  static constexpr int kWords = 4;
  __device__ static type zero() { return make_uint4(0u, 0u, 0u, 0u); }
  __device__ static type load(const T* p) { return *reinterpret_cast<const uint4*>(p); }
  __device__ static void unpack(const type& x, float* o) { Chunk<T>::unpack(x, o); }
  __device__ static type pack(const float* f) { return Chunk<T>::pack(f); }
  __device__ static void words(const type& x, uint32_t (&w)[kWords]) {
    w[0] = x.x; w[1] = x.y; w[2] = x.z; w[3] = x.w;
  }
  __device__ static type from_words(const uint32_t (&w)[kWords]) {
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
};
template <> struct QChunk<float> {
  typedef F8 type;
  static constexpr int kWords = 8;
  __device__ static type zero() { return F8{make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u)}; }
  __device__ static type load(const float* p) {
    return F8{reinterpret_cast<const uint4*>(p)[0], reinterpret_cast<const uint4*>(p)[1]};
  }
  __device__ static void unpack(const type& x, float* o) { f8_unpack(x, o); }
  __device__ static type pack(const float* f) { return f8_pack(f); }
  __device__ static void words(const type& x, uint32_t (&w)[kWords]) {
    w[0] = x.lo.x; w[1] = x.lo.y; w[2] = x.lo.z; w[3] = x.lo.w;
    w[4] = x.hi.x; w[5] = x.hi.y; w[6] = x.hi.z; w[7] = x.hi.w;
  }
  __device__ static type from_words(const uint32_t (&w)[kWords]) {
    return F8{make_uint4(w[0], w[1], w[2], w[3]), make_uint4(w[4], w[5], w[6], w[7])};
  }
};

// Value of `v` in lane 16 * (lane / 16) + N (DPP row_newbcast).
template <int N>
__device__ __forceinline__ float row_bcast(float v) {
  static_assert(N >= 0 && N < 16, "row_newbcast source lane");
  const int x = __float_as_int(v);
  return __int_as_float(__builtin_amdgcn_update_dpp(x, x, 0x150 + N, 0xF, 0xF, false));
}

template <int N>
__device__ __forceinline__ uint32_t row_bcast_u(uint32_t v) {
  static_assert(N >= 0 && N < 16, "row_newbcast source lane");
  const int x = static_cast<int>(v);
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(x, x, 0x150 + N, 0xF, 0xF, false));
}

// Two fp32 values rounded to T (nearest even) and packed, a in the low half.
typedef float mf_f2 __attribute__((ext_vector_type(2)));
typedef __bf16 mf_bf2 __attribute__((ext_vector_type(2)));
typedef _Float16 mf_h2 __attribute__((ext_vector_type(2)));
template <typename T> struct Pack2;
template <> struct Pack2<bf16_t> {
  __device__ static uint32_t pack(float a, float b) {
    const mf_f2 x = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, mf_bf2));
  }
};
template <> struct Pack2<_Float16> {
  __device__ static uint32_t pack(float a, float b) {
    const mf_f2 x = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, mf_h2));
  }
};

// c + a.lo * b.lo + a.hi * b.hi for packed T pairs, accumulated in fp32 (v_dot2_f32_*).
template <typename T> struct Dot2;
template <> struct Dot2<bf16_t> {
  __device__ static float dot(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(mf_bf2, a), __builtin_bit_cast(mf_bf2, b),
                                           c, false);
  }
};
template <> struct Dot2<_Float16> {
  __device__ static float dot(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(mf_h2, a), __builtin_bit_cast(mf_h2, b), c, false);
  }
};

template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Raw buffer loads through a per-tile descriptor: a tile whose descriptor has
// num_records = 0 (a hole, or a tile past the wave's range) reads zeros and
// moves no memory, so the tile loop needs no branch around its loads.
typedef unsigned int mf_u32x4 __attribute__((ext_vector_type(4)));
constexpr int kBufferRsrcWord3 = 0x00020000;  // gfx9-family raw buffer, 32-bit format

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), bytes,
                                           kBufferRsrcWord3);
}

template <int AUX = 0>
__device__ __forceinline__ uint4 buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  const mf_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(byte_off), 0, AUX);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Device-scope coherent accesses: agent-scope atomic loads and stores, vector memory
// instructions with cache policy SC1. A store is written through to the memory every XCD
// reads, and a load does not take a line that another XCD may have changed from this
// XCD's L2 (each XCD has its own L2, not coherent with the others). Partials exchanged
// between workgroups inside one launch go through these, so publishing them needs only
// their completion (s_waitcnt vmcnt(0)), not a writeback of the whole L2.
constexpr int kWaitVmcnt0 = 0x0F70;  // s_waitcnt vmcnt(0), expcnt and lgkmcnt not waited
#ifndef MSATTN_MERGE_ACQREL
#define MSATTN_MERGE_ACQREL 0
#endif

__device__ __forceinline__ void store2_device(float* p, float a, float b) {  // p: 8-byte aligned
  const uint64_t v = static_cast<uint64_t>(__float_as_uint(a)) |
                     (static_cast<uint64_t>(__float_as_uint(b)) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 load2_device(const float* p) {  // p: 8-byte aligned
  const uint64_t v = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float(static_cast<uint32_t>(v)),
                     __uint_as_float(static_cast<uint32_t>(v >> 32)));
}

typedef float mf_f32x2 __attribute__((ext_vector_type(2)));

// Eight consecutive K/V elements per lane. A cache of the compute type T loads 16
// bytes; an fp8 (OCP e4m3) cache loads 8 bytes, kept raw while in flight and
// widened once they arrive. The widening is exact (every e4m3 value is a bf16 and
// an fp16 value), so an fp8 cache gives the result of the same kernel run on the
// cache converted to T beforehand (miniserve/attention.py:168-170, then .to(q.dtype)).
template <typename T, typename KT> struct Kv8;
template <typename T> struct Kv8<T, T> {
  typedef uint4 raw_t;
  // MFMA k-chunk j (8 dims) of lane group g of the scores' K and Q operands starts at
  // dim 8 (4j + g).
  __host__ __device__ static constexpr int qk_dim0(int j, int g, int /*JD*/) {
    return 8 * (4 * j + g);
  }
  template <int AUX>
  __device__ static raw_t load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return buffer_load16<AUX>(r, off);
  }
  // A K row's chunks for lane group g (row_off: the row's byte offset in the tile).
  template <int AUX, int JD>
  __device__ static void load_k(__amdgpu_buffer_rsrc_t r, uint32_t row_off, int g,
                                raw_t (&kb)[JD]) {
#pragma unroll
    for (int j = 0; j < JD; ++j)
      kb[j] = buffer_load16<AUX>(r, row_off + static_cast<uint32_t>(qk_dim0(j, g, JD)) * 2u);
  }
  __device__ static uint4 operand(const raw_t& x) { return x; }         // 8 x T, packed
  // Dim e of two tokens' chunks as one packed T pair (token a low): o[e] = (a[e], b[e]).
  __device__ static void pairs(const raw_t& a, const raw_t& b, uint32_t (&o)[8]) {
    const uint32_t wa[4] = {a.x, a.y, a.z, a.w};
    const uint32_t wb[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      o[2 * k] = __builtin_amdgcn_perm(wb[k], wa[k], 0x05040100u);
      o[2 * k + 1] = __builtin_amdgcn_perm(wb[k], wa[k], 0x07060302u);
    }
  }
  __device__ static void unpack(const raw_t& x, float* o) { Chunk<T>::unpack(x, o); }
  __device__ static raw_t keep_if(const raw_t& x, bool keep) {
    return keep ? x : make_uint4(0u, 0u, 0u, 0u);
  }
};
template <typename T> struct Kv8<T, fp8_t> {
  typedef uint2 raw_t;
  // K/Q chunks 2h and 2h + 1 of lane group g are dims 64 h + 16 g .. + 15: one 16-byte
  // load per lane, and the four lane groups of a row cover its bytes 64 h .. 64 h + 63.
  // (The chunks of 8 (4j + g) would take JD 8-byte loads that each touch 16 rows for 32
  // bytes; the memory pipe's request count, not the bytes, then bounds the kernel.) The
  // dot product does not depend on which dims share an MFMA, as long as Q and K use the
  // same split.
  __host__ __device__ static constexpr int qk_dim0(int j, int g, int /*JD*/) {
    return 64 * (j >> 1) + 16 * g + 8 * (j & 1);
  }
  template <int AUX>
  __device__ static raw_t load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(off), 0, AUX);
    return make_uint2(v.x, v.y);
  }
  template <int AUX, int JD>
  __device__ static void load_k(__amdgpu_buffer_rsrc_t r, uint32_t row_off, int g,
                                raw_t (&kb)[JD]) {
    static_assert(JD % 2 == 0, "pairs of chunks per 16-byte load");
#pragma unroll
    for (int h = 0; h < JD / 2; ++h) {
      const uint4 x = buffer_load16<AUX>(
          r, row_off + static_cast<uint32_t>(qk_dim0(2 * h, g, JD)));
      kb[2 * h] = make_uint2(x.x, x.y);
      kb[2 * h + 1] = make_uint2(x.z, x.w);
    }
  }
  // bytes 0..7 -> fp32 pairs (v_cvt_pk_f32_fp8, OCP e4m3 on gfx950)
  __device__ static void unpack(const raw_t& x, float* o) {
    const mf_f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(x.x), false);
    const mf_f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(x.x), true);
    const mf_f32x2 c = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(x.y), false);
    const mf_f32x2 d = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(x.y), true);
    o[0] = a.x; o[1] = a.y; o[2] = b.x; o[3] = b.y;
    o[4] = c.x; o[5] = c.y; o[6] = d.x; o[7] = d.y;
  }
  // bytes 0..7 -> eight T values (v_cvt_scalef32_pk_{bf16,f16}_fp8 with scale 1: exact)
  __device__ static uint4 operand(const raw_t& x) {
    return make_uint4(widen2<false>(x.x), widen2<true>(x.x), widen2<false>(x.y),
                      widen2<true>(x.y));
  }
  // Dim e of two tokens' chunks widened to T and packed (token a low): the bytes of dims
  // 2m, 2m + 1 of both tokens are interleaved first, then each half is widened.
  __device__ static void pairs(const raw_t& a, const raw_t& b, uint32_t (&o)[8]) {
    const uint32_t wa[2] = {a.x, a.y};
    const uint32_t wb[2] = {b.x, b.y};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint32_t lo = __builtin_amdgcn_perm(wb[k], wa[k], 0x05010400u);  // a0 b0 a1 b1
      const uint32_t hi = __builtin_amdgcn_perm(wb[k], wa[k], 0x07030602u);  // a2 b2 a3 b3
      o[4 * k] = widen2<false>(lo);
      o[4 * k + 1] = widen2<true>(lo);
      o[4 * k + 2] = widen2<false>(hi);
      o[4 * k + 3] = widen2<true>(hi);
    }
  }
  template <bool HI>  // bytes 2, 3 of w when HI, else bytes 0, 1
  __device__ static uint32_t widen2(uint32_t w) {
    if constexpr (std::is_same<T, bf16_t>::value)
      return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
    else
      return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
  }
  __device__ static raw_t keep_if(const raw_t& x, bool keep) {
    return keep ? x : make_uint2(0u, 0u);
  }
};

// An fp32 cache read by a bf16/fp16 query: eight elements are 32 bytes (two 16-byte
// loads), kept raw while in flight and rounded to T (nearest even) once they arrive.
// That is the reference's cast of the gathered K/V to query.dtype
// (miniserve/attention.py:240-241) done in registers, so the result is that of the same
// kernel run on the cache converted to T beforehand. Chunks follow the split of a cache
// of T (dims 8 (4j + g)): the four lane groups of a row read 128 contiguous bytes per
// chunk index.
template <typename T> struct Kv8<T, float> {
  typedef F8 raw_t;
  __host__ __device__ static constexpr int qk_dim0(int j, int g, int /*JD*/) {
    return 8 * (4 * j + g);
  }
  template <int AUX>
  __device__ static raw_t load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return raw_t{buffer_load16<AUX>(r, off), buffer_load16<AUX>(r, off + 16u)};
  }
  template <int AUX, int JD>
  __device__ static void load_k(__amdgpu_buffer_rsrc_t r, uint32_t row_off, int g,
                                raw_t (&kb)[JD]) {
#pragma unroll
    for (int j = 0; j < JD; ++j)
      kb[j] = load<AUX>(r, row_off + static_cast<uint32_t>(qk_dim0(j, g, JD)) * 4u);
  }
  __device__ static float f(uint32_t w) { return __uint_as_float(w); }
  // eight fp32 values -> eight T values (nearest even), packed
  __device__ static uint4 operand(const raw_t& x) {
    return make_uint4(Pack2<T>::pack(f(x.lo.x), f(x.lo.y)), Pack2<T>::pack(f(x.lo.z), f(x.lo.w)),
                      Pack2<T>::pack(f(x.hi.x), f(x.hi.y)), Pack2<T>::pack(f(x.hi.z), f(x.hi.w)));
  }
  // Dim e of two tokens' chunks rounded to T and packed (token a low).
  __device__ static void pairs(const raw_t& a, const raw_t& b, uint32_t (&o)[8]) {
    const uint32_t wa[8] = {a.lo.x, a.lo.y, a.lo.z, a.lo.w, a.hi.x, a.hi.y, a.hi.z, a.hi.w};
    const uint32_t wb[8] = {b.lo.x, b.lo.y, b.lo.z, b.lo.w, b.hi.x, b.hi.y, b.hi.z, b.hi.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = Pack2<T>::pack(f(wa[e]), f(wb[e]));
  }
  // The values the MFMA operand holds, as fp32 (rounded to T).
  __device__ static void unpack(const raw_t& x, float* o) { Chunk<T>::unpack(operand(x), o); }
  __device__ static raw_t keep_if(const raw_t& x, bool keep) {
    return keep ? x : raw_t{make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u)};
  }
};

// A bf16/fp16 or fp8 cache read by an fp32 query: the loads and head-dim split of the
// cache's own kernels (Kv8<KT, KT>, Kv8<bf16_t, fp8_t>), widened exactly to fp32 once
// they arrive: the reference's .to(query.dtype) of the gathered rows
// (miniserve/attention.py:240-241), so the scores run on fp32 MFMAs (Mfma16<float>) and
// P.V on fp32 FMAs over the cache's own values.
template <typename KT> struct Kv8Widened
    : Kv8<typename std::conditional<std::is_same<KT, fp8_t>::value, bf16_t, KT>::type, KT> {
  typedef Kv8<typename std::conditional<std::is_same<KT, fp8_t>::value, bf16_t, KT>::type, KT> Base;
  typedef typename Base::raw_t raw_t;
  __device__ static F8 operand(const raw_t& x) {
    float o[8];
    Base::unpack(x, o);  // exact: every bf16, fp16 and e4m3 value is an fp32 value
    return f8_pack(o);
  }
};
template <> struct Kv8<float, bf16_t> : Kv8Widened<bf16_t> {};
template <> struct Kv8<float, _Float16> : Kv8Widened<_Float16> {};
template <> struct Kv8<float, fp8_t> : Kv8Widened<fp8_t> {};

// An fp32 cache read by an fp32 query: the loads of Kv8<T, float>, kept in fp32 (the
// reference's .to(query.dtype) is the identity there). The MFMA operand is the raw chunk
// (Mfma16<float>), and P.V runs on fp32 FMAs.
template <> struct Kv8<float, float> {
  typedef F8 raw_t;
  __host__ __device__ static constexpr int qk_dim0(int j, int g, int /*JD*/) {
    return 8 * (4 * j + g);
  }
  template <int AUX>
  __device__ static raw_t load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return raw_t{buffer_load16<AUX>(r, off), buffer_load16<AUX>(r, off + 16u)};
  }
  template <int AUX, int JD>
  __device__ static void load_k(__amdgpu_buffer_rsrc_t r, uint32_t row_off, int g,
                                raw_t (&kb)[JD]) {
#pragma unroll
    for (int j = 0; j < JD; ++j)
      kb[j] = load<AUX>(r, row_off + static_cast<uint32_t>(qk_dim0(j, g, JD)) * 4u);
  }
  __device__ static const F8& operand(const raw_t& x) { return x; }
  __device__ static void unpack(const raw_t& x, float* o) { f8_unpack(x, o); }
  __device__ static raw_t keep_if(const raw_t& x, bool keep) {
    return keep ? x : raw_t{make_uint4(0u, 0u, 0u, 0u), make_uint4(0u, 0u, 0u, 0u)};
  }
};

// A new K/V row's eight elements (type ST) as loaded for the fused append, and the raw
// chunk a cache of KT holds for them: each element cast as msattn_write_kv casts it
// (through fp32 with the cache type's rounding; the same type keeps its bits).
template <typename ST> struct alignas(16) SrcChunk {
  ST v[8];
};
template <typename KT> struct alignas(sizeof(KT) * 8 >= 16 ? 16 : 8) CacheChunk {
  KT v[8];
};
template <typename KT, typename ST, typename RAW>
__device__ __forceinline__ RAW append_raw(const SrcChunk<ST>& x) {
  static_assert(sizeof(RAW) == 8 * sizeof(KT), "a raw chunk holds eight cache elements");
  if constexpr (std::is_same<KT, ST>::value) {
    return __builtin_bit_cast(RAW, x);
  } else {
    CacheChunk<KT> c;
#pragma unroll
    for (int e = 0; e < 8; ++e) Elt<KT>::store(&c.v[e], Elt<ST>::load(&x.v[e]));
    return __builtin_bit_cast(RAW, c);
  }
}

#ifndef MSATTN_PV_DOT2
#define MSATTN_PV_DOT2 1
#endif
// P.V of an fp32 query over an fp32 cache at 16 query rows per tile on the matrix core
// (v_mfma_f32_16x16x4_f32) instead of fp32 FMAs: chunked prefill and G >= 16 decodes.
#ifndef MSATTN_PV_MFMA32
#define MSATTN_PV_MFMA32 1
#endif

// P.V of one 16-token tile on the VALU, for the decode kernels. Lane (g, n) holds the
// weights pr[r] of query row n for tokens tile_token(4g + r); V lane (va, vc) holds, for
// load j, dims 8 vc .. 8 vc + 7 of token TPI * j + va, whose weight for row rn sits in
// lane rn of the lane's own 16-lane row (DPP row_newbcast; with two token groups per row,
// APR = 2, the group va & 1 picks between two broadcasts). With MSATTN_PV_DOT2 the tokens
// of loads 2i and 2i + 1 are paired: their weights are rounded to T and packed, V is
// widened to T (exact for fp8), and one v_dot2_f32 adds both products to the fp32
// accumulator, which halves the multiply-adds and the broadcasts.
template <typename T, typename KT, int D, int RT>
__device__ __forceinline__ void pv_tile(float (&acc)[RT][8], const float (&pr)[4],
                                        const typename Kv8<T, KT>::raw_t (&vb)[D / 32], int va) {
  typedef Kv8<T, KT> KV;
  constexpr int LPR = D / 8;
  constexpr int TPI = 64 / LPR;
  constexpr int NJ = 16 / TPI;
  constexpr int APR = 16 / LPR;
  static_assert(NJ == D / 32, "V loads per tile");
  // An fp32 query keeps P and V in fp32: scalar FMAs.
  constexpr bool kDot2 = MSATTN_PV_DOT2 && !std::is_same<T, float>::value;
  if constexpr (kDot2) {
  static_assert(NJ % 2 == 0, "V loads pair up");
#pragma unroll
  for (int i = 0; i < NJ / 2; ++i) {
    uint32_t vp[8];
    KV::pairs(vb[2 * i], vb[2 * i + 1], vp);
    uint32_t pp[APR];
#pragma unroll
    for (int a = 0; a < APR; ++a)
      pp[a] = Pack2<T>::pack(pr[APR * (2 * i) + a], pr[APR * (2 * i + 1) + a]);
    static_for<RT>([&](auto nc) {
      constexpr int rn = decltype(nc)::value;
      uint32_t pb;
      if constexpr (APR == 1) {
        pb = row_bcast_u<rn>(pp[0]);
      } else {
        const uint32_t b0 = row_bcast_u<rn>(pp[0]);
        const uint32_t b1 = row_bcast_u<rn>(pp[1]);
        pb = (va & 1) ? b1 : b0;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[rn][e] = Dot2<T>::dot(pb, vp[e], acc[rn][e]);
    });
  }
  } else {
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    float vf[8];
    KV::unpack(vb[j], vf);
    static_for<RT>([&](auto nc) {
      constexpr int rn = decltype(nc)::value;
      float pb;
      if constexpr (APR == 1) {
        pb = row_bcast<rn>(pr[j]);
      } else {
        const float b0 = row_bcast<rn>(pr[APR * j]);
        const float b1 = row_bcast<rn>(pr[APR * j + 1]);
        pb = (va & 1) ? b1 : b0;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[rn][e] = fmaf(pb, vf[e], acc[rn][e]);
    });
  }
  }
}

// Workgroups of the partition kernel a CU may hold (0: as registers allow). Two on a CU
// run one after the other (the older one's loads win the memory pipe), so a third only
// lengthens that CU's queue while other CUs idle; capping residency through LDS leaves
// the later workgroups to the dispatcher, which starts them on whichever CU frees first.
#ifndef MSATTN_MFMA_WG_PER_CU
#define MSATTN_MFMA_WG_PER_CU 2
#endif
constexpr int kMfmaWgPerCu = MSATTN_MFMA_WG_PER_CU;
// Partition workgroups a CU may hold in a launch of many workgroups per CU at head_dim 64
// (the regular shape): there a third resident workgroup hides more of each one's memory
// round trips (128 x H14/KVH2 at 1-4k tokens: 42.1 -> 37.7 us), while in a launch of about
// one round it only lengthens a CU's queue (C2: 11.6 -> 13.5 us).
#ifndef MSATTN_MFMA_WG_PER_CU_DEEP
#define MSATTN_MFMA_WG_PER_CU_DEEP 3
#endif
constexpr int kMfmaWgPerCuDeep = MSATTN_MFMA_WG_PER_CU_DEEP;
constexpr int kCuLdsBytes = 160 * 1024;  // gfx950 LDS per CU
constexpr int kMfmaWaves = MSATTN_MFMA_WAVES;
constexpr int kMfmaThreads = kMfmaWaves * kWave;
constexpr int kMaxTilesPerWave = kPartMax / 16 / kMfmaWaves;  // partitions are <= kPartMax tokens
// The wide shape of the partition kernel: kWideWaves waves (two per SIMD) over partitions
// of up to kPartWide tokens, the same tiles per wave as the regular shape's longest
// partition. It serves decodes with few (sequence, KV head) pairs over long contexts,
// where partitions of that length still fill the chip with one workgroup per CU.
constexpr int kWideWaves = 8;
constexpr int kPartWide = kMaxTilesPerWave * 16 * kWideWaves;
// Partition of the fp32 16-row route (MFMA P.V) when it merges in-kernel over a large grid
// (chunked prefill): longer partitions spread each workgroup's start, epilogue and merge
// over more tiles. Its kernel unrolls this many tiles per wave.
#ifndef MSATTN_PART_LONG_F32
#define MSATTN_PART_LONG_F32 2048
#endif
constexpr int kPartLongF32 = MSATTN_PART_LONG_F32;
static_assert(kPartLongF32 % (16 * kMfmaWaves) == 0 && kPartLongF32 / (16 * kMfmaWaves) <= 64,
              "whole tiles per wave, page ids in one lane each");

// Token (within a 16-token tile) whose score lands in MFMA row i = 4g + r.
template <int D>
__host__ __device__ constexpr int tile_token(int i) {
  constexpr int LPR = D / 8;      // V lanes per token row
  constexpr int TPI = 64 / LPR;   // tokens per V load instruction
  constexpr int APR = 16 / LPR;   // token groups per 16-lane row
  const int g = i / 4, r = i % 4;
  return TPI * (r / APR) + g * APR + (r % APR);
}

// Rotate-half RoPE on one query row held as MFMA B-operand chunks: chunk j of lane
// group g holds dims Kv8<T, KT>::qk_dim0(j, g) .. +7, and its partner (dims -/+ D/2) is
// chunk j +/- JD/2 of the same lane (2-byte caches: dims 8 (4j + g); an fp8 cache at
// D = 128: dims 64 (j / 2) + 16 g + 8 (j % 2)), or, for an fp8 cache at D = 64 (dims
// 16 g + 8 j), chunk j of lane group g +/- 2, the lane 32 away, which one
// v_permlane32_swap brings over. The rotation is that of kernels/paged_attn_triton.py:211-220
// (fp32 tables, fp32 products and sum); the rotated row is then rounded back to T, as the
// matrix cores take a T operand: the result is (q * cos + rotate_half(q) * sin).to(T)
// (miniserve/attention.py:41-62 with fp32 tables), where the reference's Triton kernel and
// flash_decode_reference (:134-138) keep the rotated query in fp32. That one rounding of
// the query (relative 2^-9 for bf16) is the only difference. Lanes l and l ^ 32 (the same
// query row) are both active or both not.
template <typename T, typename KT, int D>
__device__ __forceinline__ void rope_chunks(typename QChunk<T>::type (&qb)[D / 32], const float* cs,
                                            const float* sn, int g) {
  constexpr int JD = D / 32;
  constexpr bool kCross = sizeof(KT) == 1 && D == 64;  // the partner is in the other half-wave
  float q[JD][8];
  float qp[JD][8];
#pragma unroll
  for (int j = 0; j < JD; ++j) QChunk<T>::unpack(qb[j], q[j]);
  if constexpr (kCross) {
    const bool lo = g < 2;
#pragma unroll
    for (int j = 0; j < JD; ++j) {
      constexpr int NW = QChunk<T>::kWords;
      uint32_t w[NW], o[NW];
      QChunk<T>::words(qb[j], w);
#pragma unroll
      for (int k = 0; k < NW; ++k) {
        const auto t = __builtin_amdgcn_permlane32_swap(w[k], w[k], false, false);
        o[k] = lo ? t[1] : t[0];
      }
      QChunk<T>::unpack(QChunk<T>::from_words(o), qp[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < JD; ++j) {
    const int d0 = Kv8<T, KT>::qk_dim0(j, g, JD);
    const float4 c0 = *reinterpret_cast<const float4*>(cs + d0);
    const float4 c1 = *reinterpret_cast<const float4*>(cs + d0 + 4);
    const float4 s0 = *reinterpret_cast<const float4*>(sn + d0);
    const float4 s1 = *reinterpret_cast<const float4*>(sn + d0 + 4);
    const float c[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float r;
      if constexpr (kCross)
        r = g < 2 ? -qp[j][e] : qp[j][e];
      else
        r = j < JD / 2 ? -q[j + JD / 2][e] : q[j - JD / 2][e];
      o[e] = rope_mix(q[j][e], r, c[e], sv[e]);
    }
    qb[j] = QChunk<T>::pack(o);
  }
}

template <typename T, typename KT, int D, int RT, int W = kMfmaWaves, int WPC = kMfmaWgPerCu,
          bool APPEND = false>
__global__ __launch_bounds__(W * kWave) void decode_mfma_kernel(const SplitParams p) {
  constexpr int kWaves = W;               // waves per workgroup
  constexpr int kThreads = W * kWave;
  typedef Kv8<T, KT> KV;
  typedef typename KV::raw_t raw_t;
  static_assert(D == 64 || D == 128, "MFMA decode handles head_dim 64 and 128");
  static_assert(RT >= 1 && RT <= 16, "at most 16 query rows per tile");
  constexpr int JD = D / 32;        // MFMAs per tile
  constexpr int LPR = D / 8;        // V lanes per token row
  constexpr int TPI = 64 / LPR;     // V tokens per load instruction
  constexpr int NJ = 16 / TPI;      // V load instructions per tile
  constexpr int APR = 16 / LPR;     // token groups per 16-lane row

  __shared__ float s_red[kWaves][RT][D];
  __shared__ float s_ml[kWaves][RT][2];
  constexpr bool kBalance = MSATTN_PART_BALANCE && kWaves > 4;
  __shared__ int s_prog[kWaves];  // tiles consumed per wave (kBalance)
  __shared__ int s_last;  // in-kernel merge: this workgroup arrived last
  // LDS reserved beyond s_red / s_ml so that at most WPC workgroups share a
  // CU (the store below never runs; it keeps the array allocated).
  constexpr int kLdsUsed = static_cast<int>(sizeof(s_red) + sizeof(s_ml));
  constexpr int kLdsWant = WPC > 0 ? kCuLdsBytes / (WPC + 1) + 2048 : 0;
  constexpr int kPadFloats = kLdsWant > kLdsUsed ? (kLdsWant - kLdsUsed) / 4 : 1;
  __shared__ float s_pad[kPadFloats];
  if (p.batch < 0) s_pad[threadIdx.x % kPadFloats] = 0.0f;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  // wave index, made visibly wave-uniform so loop control stays scalar
  const int w = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int g = lane >> 4;   // MFMA lane group
  const int n = lane & 15;   // MFMA column = query row of the tile
  const int va = lane / LPR; // V token group
  const int vc = lane % LPR; // V 16-byte chunk

  // In-kernel merge: the partition workgroups of a (sequence, KV head, row tile) count
  // themselves in on a header ticket; the last one folds every partial into the output.
  // A sequence of one partition writes its output directly.
  const bool fused = p.out != nullptr;
  if (tid == 0 && blockIdx.x == 0 && blockIdx.z == 0) {
    p.hdr[kHdrKind] = fused ? 2 : 0;
    p.hdr[kHdrPart] = p.part;
    p.hdr[kHdrWaves] = W;
    p.hdr[kHdrResidency] = WPC;
  }
  // The grid order (SplitParams::part_major): partition-major over one x index, or
  // blockIdx.x = kvh + KVH * (part + max_parts * rtile) with blockIdx.z = b.
  const unsigned bx = blockIdx.x;
  const int kvh = static_cast<int>(bx % static_cast<unsigned>(p.KVH));
  const unsigned rest = bx / static_cast<unsigned>(p.KVH);
  int part, rtile, b;
  if (p.part_major) {
    rtile = static_cast<int>(rest % static_cast<unsigned>(p.rtiles));
    const unsigned rb = rest / static_cast<unsigned>(p.rtiles);
    b = static_cast<int>(rb % static_cast<unsigned>(p.batch));
    part = static_cast<int>(rb / static_cast<unsigned>(p.batch));
  } else {
    part = static_cast<int>(rest % static_cast<unsigned>(p.max_parts));
    rtile = static_cast<int>(rest / static_cast<unsigned>(p.max_parts));
    b = blockIdx.z;
  }

  // Wave w owns a fixed run of the partition's tiles, so their page ids can be
  // requested together with the context length instead of after it.
  const int per_wave = p.part / (16 * kWaves);
  const int tw0 = part * (p.part / 16) + w * per_wave;
  int phys_pre = -1;
  if (lane < per_wave) {
    const int pg = ((tw0 + lane) * 16) / p.bs;
    if (pg < p.W) phys_pre = p.table[static_cast<int64_t>(b) * p.W + pg];
  }

  int ctx = p.lens[b];
  ctx = ctx < 0 ? 0 : (ctx > p.max_ctx ? p.max_ctx : ctx);
  const int nparts = ctx > 0 ? ceil_div(ctx, p.part) : 1;
  if (part >= nparts) return;

  const int row0 = rtile * RT;
  const int nrows = min(RT, p.rows_per_kvh - row0);

  // Key range of the tile's first and last rows (ranges grow with the query index).
  const int i_first = row0 / p.G;
  const int i_last = (row0 + nrows - 1) / p.G;
  const int lo_all = max(p.key_lo, p.window > 0 ? max(0, ctx - p.q_len + i_first - p.window + 1) : 0);
  const int hi_all = p.causal ? min(ctx, ctx - p.q_len + i_last + 1) : ctx;
  const int tok0 = part * p.part;
  const int a0 = max(tok0, lo_all);
  const int a1 = min(min(tok0 + p.part, ctx), hi_all);

  // Tiles [t_begin, t_end) of 16 absolute positions hold the keys; the wave's run is
  // tiles tw0 .. tw0 + nt - 1 of it (earlier ones, below a window, read nothing).
  const int t_begin = a0 / 16;
  const int t_end = ceil_div(a1, 16);
  const int nt = max(0, min(per_wave, t_end - tw0));

  // Lane k holds tile tw0 + k's element offset, or -1 for a hole (a table entry outside
  // [0, num_blocks), a page past the table, a tile outside the key range).
  int64_t my_base = -1;
  if (lane < nt && tw0 + lane >= t_begin && phys_pre >= 0 && phys_pre < p.num_blocks) {
    const int t = tw0 + lane;
    const int pg = (t * 16) / p.bs;
    const int slot0 = t * 16 - pg * p.bs;
    my_base = static_cast<int64_t>(phys_pre) * p.blk_stride +
              static_cast<int64_t>(slot0) * p.slot_stride +
              static_cast<int64_t>(kvh) * p.head_stride;
  }

  // Per-lane byte offsets inside a tile (32-bit: a tile spans 16 slots).
  constexpr int EB = static_cast<int>(sizeof(KT));
  const uint32_t k_row_off = static_cast<uint32_t>(tile_token<D>(n) * p.slot_stride * EB);
  uint32_t v_lane_off[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
    v_lane_off[j] = static_cast<uint32_t>(((TPI * j + va) * p.slot_stride + vc * 8) * EB);
  const int tile_bytes = static_cast<int>((15 * p.slot_stride + D) * EB);

  const KT* kbase = static_cast<const KT*>(p.k);
  const KT* vbase = static_cast<const KT*>(p.v);

  // P.V on the matrix core (fp32 query and cache, a full 16-row tile): O = P V as
  // v_mfma_f32_16x16x4_f32 steps. Step r takes, in lane (g, n), A = P[row n][token
  // tile_token(4g + r)] (the lane's own weight pr[r], where the scores landed) and
  // B = V[that token][dim]; lane (g, n) loads 16 bytes of that token's row, dims
  // 64 h + 4 n .. + 3, and element e of them feeds output block (h, e), whose column n
  // is dim 64 h + 4 n + e. Output lane (g', n') then holds rows 4 g' .. 4 g' + 3 of dims
  // 64 h + 4 n' + e: a float4 of consecutive dims per (row, h).
  constexpr bool kPvMfma = MSATTN_PV_MFMA32 && std::is_same<T, float>::value &&
                           std::is_same<KT, float>::value && RT == 16;
  constexpr int NH = D / 64;         // 16-byte V loads per token step
  constexpr int NVQ = 4 * NH;        // V loads per tile (MFMA P.V)
  constexpr int NOB = 4 * NH;        // 16x16 output blocks (MFMA P.V)
  uint32_t v_mfma_off[kPvMfma ? NVQ : 1];
  if constexpr (kPvMfma) {
    static_assert(NVQ == 2 * NJ, "the V ring holds the MFMA P.V loads");
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int h = 0; h < NH; ++h)
        v_mfma_off[r * NH + h] = static_cast<uint32_t>(
            (tile_token<D>(4 * g + r) * p.slot_stride + 64 * h + 4 * n) * EB);
  }
  // Element offset of the wave's tile k, or -1 (hole, or k >= nt).
  auto tile_base = [&](int k) -> int64_t __attribute__((always_inline)) {
    const uint32_t lo = static_cast<uint32_t>(
        __builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(my_base)), k));
    const int hi = __builtin_amdgcn_readlane(static_cast<int>(my_base >> 32), k);
    return static_cast<int64_t>(lo) | (static_cast<int64_t>(hi) << 32);
  };
  auto issue = [&](int64_t base, raw_t (&kb)[JD], raw_t (&vb)[NJ]) __attribute__((always_inline)) {
    const bool ok = base >= 0;
    const int64_t b0 = ok ? base : 0;
    const __amdgpu_buffer_rsrc_t rk = tile_rsrc(kbase + b0, ok ? tile_bytes : 0);
    const __amdgpu_buffer_rsrc_t rv = tile_rsrc(vbase + b0, ok ? tile_bytes : 0);
    KV::template load_k<0, JD>(rk, k_row_off, g, kb);
    if constexpr (kPvMfma) {
#pragma unroll
      for (int q = 0; q < NVQ; ++q) {
        const uint4 x = buffer_load16<0>(rv, v_mfma_off[q]);
        if (q % 2 == 0) vb[q / 2].lo = x;
        else vb[q / 2].hi = x;
      }
    } else {
#pragma unroll
      for (int j = 0; j < NJ; ++j) vb[j] = KV::template load<0>(rv, v_lane_off[j]);
    }
  };

  // A ring of DEPTH tiles: the loads of DEPTH - 1 tiles are in flight while one is
  // consumed. The sequence is fully unrolled (a wave owns at most kMaxT tiles) so
  // every wait for a tile's loads is exact; loads for tiles at or past nt read
  // nothing (their descriptors have no records).
  constexpr int DEPTH = D == 64 ? MSATTN_MFMA_DEPTH_D64 : MSATTN_MFMA_DEPTH;
  raw_t kr[DEPTH][JD], vr[DEPTH][NJ];
  int64_t br[DEPTH];
  // The first tiles' loads go out as soon as the context length is known, ahead of the
  // lanes' row set-up and the query load, which then run under their round trip.
  if (a1 > a0) {
    static_for<DEPTH - 1>([&](auto dc) {
      constexpr int d = decltype(dc)::value;
      br[d] = tile_base(d);
      issue(br[d], kr[d], vr[d]);
    });
  }
  // This lane's query row n: key range [lo_n, hi_n) and output row.
  int lo_n = 0, hi_n = 0;
  int64_t orow_n = 0;
  if (n < nrows) {
    const int gr = row0 + n;
    const int i = gr / p.G;
    const int qpos = ctx - p.q_len + i;
    hi_n = p.causal ? min(ctx, qpos + 1) : ctx;
    lo_n = max(p.key_lo, p.window > 0 ? max(0, qpos - p.window + 1) : 0);
    if (hi_n < lo_n) hi_n = lo_n;
    orow_n = (static_cast<int64_t>(b) * p.q_len + i) * p.H + (kvh * p.G + (gr - i * p.G));
  }

  const bool direct = fused && nparts == 1;
  constexpr int D4 = D / 4;
  auto out_row = [&](int r) -> int64_t __attribute__((always_inline)) {
    const int gr = row0 + r;
    const int i = gr / p.G;
    return (static_cast<int64_t>(b) * p.q_len + i) * p.H + (kvh * p.G + (gr - i * p.G));
  };
  auto store_out4 = [&](int64_t orow, int d, float4 a, float inv) __attribute__((always_inline)) {
    T* o = static_cast<T*>(p.out) + orow * D + d;
    Elt<T>::store(o + 0, a.x * inv);
    Elt<T>::store(o + 1, a.y * inv);
    Elt<T>::store(o + 2, a.z * inv);
    Elt<T>::store(o + 3, a.w * inv);
  };
  // The in-kernel merge's second half: wait for this workgroup's device-scope partial
  // stores, take the ticket, and if every other partition of the row tile is in, fold
  // the nparts partials (slots 0 .. nparts - 1 of each row) into the output and leave the
  // ticket at zero for the next call. The fold is the merge kernel's: running max M,
  // weights 2^(m_j - M), out = sum w_j acc_j / sum w_j l_j; partials with m = -inf
  // (no key) carry no weight and their acc is not read into the sum.
  auto fused_merge = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();
    if (tid == 0) {
      int* t = p.tickets + ((static_cast<int64_t>(b) * p.KVH + kvh) * p.rtiles + rtile);
      // MSATTN_MERGE_ACQREL = 0 (default): a relaxed ticket. The partials were stored
      // through with agent-scope (sc1) stores, whose completion the s_waitcnt above
      // awaits in every thread before the barrier, and the last workgroup reads them with
      // agent-scope (sc1) loads issued after its barrier, which follows the ticket's
      // return: on gfx950 no L2 writeback or invalidation is needed. 1: the same exchange
      // as a release / acquire pair under the HIP memory model (the compiler then writes
      // back and invalidates this XCD's L2 around the ticket), for comparison.
      const int old = __hip_atomic_fetch_add(t, 1, MSATTN_MERGE_ACQREL ? __ATOMIC_ACQ_REL
                                                                       : __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
      const int last = old == nparts - 1;
      if (last) __hip_atomic_store(t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = last;
    }
    __syncthreads();
    if (!s_last) return;
    for (int idx = tid; idx < nrows * D4; idx += kThreads) {
      const int r = idx / D4;
      const int d = (idx - r * D4) * 4;
      const int64_t orow = out_row(r);
      const float* mlr = p.ml + orow * p.max_parts * 2;
      const float* ar = p.acc + orow * p.max_parts * D + d;
      float M = -INFINITY, L = 0.0f;
      float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      constexpr int kBatch = 8;
      for (int j0 = 0; j0 < nparts; j0 += kBatch) {
        float2 xlo[kBatch], xhi[kBatch];
        float mv[kBatch], lv[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {  // slots past nparts repeat the last one, unused
          const int j = j0 + u < nparts ? j0 + u : nparts - 1;
          const float2 ml = load2_device(mlr + 2 * j);
          mv[u] = j0 + u < nparts ? ml.x : -INFINITY;
          lv[u] = ml.y;
          xlo[u] = load2_device(ar + static_cast<int64_t>(j) * D);
          xhi[u] = load2_device(ar + static_cast<int64_t>(j) * D + 2);
        }
        float mb = -INFINITY;
#pragma unroll
        for (int u = 0; u < kBatch; ++u) mb = fmaxf(mb, mv[u]);
        if (mb == -INFINITY) continue;
        const float Mn = fmaxf(M, mb);
        const float alpha = __builtin_amdgcn_exp2f(M - Mn);  // 0 while M = -inf
        L *= alpha;
        a.x *= alpha;
        a.y *= alpha;
        a.z *= alpha;
        a.w *= alpha;
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {  // selects, not branches (see the combine)
          const bool live = mv[u] != -INFINITY;
          const float wj = __builtin_amdgcn_exp2f(live ? mv[u] - Mn : 0.0f);
          L = live ? fmaf(wj, lv[u], L) : L;
          a.x = live ? fmaf(wj, xlo[u].x, a.x) : a.x;
          a.y = live ? fmaf(wj, xlo[u].y, a.y) : a.y;
          a.z = live ? fmaf(wj, xhi[u].x, a.z) : a.z;
          a.w = live ? fmaf(wj, xhi[u].y, a.w) : a.w;
        }
        M = Mn;
      }
      store_out4(orow, d, a, L > 0.0f ? 1.0f / L : 0.0f);
    }
  };

  if (a1 <= a0) {
    if (direct) {  // no key in the only partition: zeros
      for (int idx = tid; idx < nrows * D4; idx += kThreads) {
        const int r = idx / D4;
        store_out4(out_row(r), (idx - r * D4) * 4, make_float4(0.0f, 0.0f, 0.0f, 0.0f), 0.0f);
      }
      return;
    }
    if (fused) {
      if (tid < nrows) store2_device(p.ml + (orow_n * p.max_parts + part) * 2, -INFINITY, 0.0f);
      fused_merge();
      return;
    }
    if (tid < nrows) {
      float* ml = p.ml + (orow_n * p.max_parts + part) * 2;
      ml[0] = -INFINITY;
      ml[1] = 0.0f;
      if (part + 1 == nparts && nparts < p.max_parts) {  // end marker
        ml[2] = -INFINITY;
        ml[3] = -1.0f;
      }
    }
    return;
  }

  // Query rows as the MFMA B operand: lane (g, n) holds Q[row n][dims 8*(4j+g) .. +8].
  typename QChunk<T>::type qb[JD];

  // The query rows (after the first tiles' loads).
  {
    const T* qp = static_cast<const T*>(p.q);
#pragma unroll
    for (int j = 0; j < JD; ++j) {
      qb[j] = QChunk<T>::zero();
      if (n < nrows) qb[j] = QChunk<T>::load(qp + orow_n * D + KV::qk_dim0(j, g, JD));
    }
    if (p.rope_cos != nullptr && n < nrows) {
      const int64_t po = static_cast<int64_t>(rope_position(p, b)) * D;
      rope_chunks<T, KT, D>(qb, p.rope_cos + po, p.rope_sin + po, g);
    }
  }
  // Tiles a wave may own: partitions of the fp32 16-row route reach kPartLongF32 tokens.
  constexpr int kMaxT = kPvMfma ? kPartLongF32 / 16 / kWaves : kMaxTilesPerWave;
  mf_f32x4 acc_o[kPvMfma ? NOB : 1];
  if constexpr (kPvMfma) {
#pragma unroll
    for (int q = 0; q < NOB; ++q) acc_o[q] = mf_f32x4{0.f, 0.f, 0.f, 0.f};
  }

  float m_run = -INFINITY;
  float l_run = 0.0f;
  constexpr int RTA = kPvMfma ? 1 : RT;  // rows of the FMA accumulator
  float acc[RTA][8];
#pragma unroll
  for (int r = 0; r < RTA; ++r)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][e] = 0.0f;

  auto consume = [&](int k, const raw_t (&kb)[JD], const raw_t (&vb)[NJ], int64_t base) __attribute__((always_inline)) {
    mf_f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < JD; ++j) s = Mfma16<T>::mac(KV::operand(kb[j]), qb[j], s);
    const int t0 = (tw0 + k) * 16;
    const bool hole = base < 0;
    float sc[4];
    float mt = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int tok = t0 + tile_token<D>(4 * g + r);
      const bool ok = !hole && tok >= lo_n && tok < hi_n;
      sc[r] = ok ? s[r] * p.scale_log2 : -INFINITY;
      mt = fmaxf(mt, sc[r]);
    }
    mt = rows4_max(mt);
    const float m_new = fmaxf(m_run, mt);
    const bool live = m_new != -INFINITY;
    const float alpha = live ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
    float pr[4];
    float psum = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pr[r] = live ? __builtin_amdgcn_exp2f(sc[r] - m_new) : 0.0f;
      psum += pr[r];
    }
    l_run = fmaf(l_run, alpha, psum);
    m_run = m_new;

    // Rows outside the tile's key range (partial tiles) may hold anything, even
    // NaN: their values are replaced by zeros before the weights meet them.
    const bool partial = t0 < a0 || t0 + 16 > a1;
    if constexpr (kPvMfma) {
      // alpha of output rows 4g .. 4g + 3 (row rr's alpha sits in lane rr).
      if (!MSATTN_LAZY_RESCALE || __any(alpha != 1.0f)) {
        float al[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          al[i] = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * (4 * g + i), __float_as_int(alpha)));
#pragma unroll
        for (int q = 0; q < NOB; ++q)
#pragma unroll
          for (int i = 0; i < 4; ++i) acc_o[q][i] *= al[i];
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        bool keep = true;
        if (partial) {
          const int vtok = t0 + tile_token<D>(4 * g + r);
          keep = vtok >= a0 && vtok < a1;
        }
#pragma unroll
        for (int h = 0; h < NH; ++h) {
          const int q = r * NH + h;
          const uint4 x = q % 2 == 0 ? vb[q / 2].lo : vb[q / 2].hi;
          const float xv[4] = {keep ? __uint_as_float(x.x) : 0.0f, keep ? __uint_as_float(x.y) : 0.0f,
                               keep ? __uint_as_float(x.z) : 0.0f, keep ? __uint_as_float(x.w) : 0.0f};
#pragma unroll
          for (int e = 0; e < 4; ++e)
            acc_o[4 * h + e] = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[r], xv[e], acc_o[4 * h + e], 0, 0, 0);
        }
      }
      return;
    }
    // alpha is exactly 1 for every row whose running max did not move.
    if (!MSATTN_LAZY_RESCALE || __any(alpha != 1.0f)) {
      static_for<RTA>([&](auto nc) {
        constexpr int rn = decltype(nc)::value;
        const float al = row_bcast<rn>(alpha);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[rn][e] *= al;
      });
    }
    raw_t vm[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      vm[j] = vb[j];
      if (partial) {  // wave-uniform branch; per-lane selects inside
        const int vtok = t0 + TPI * j + va;
        vm[j] = KV::keep_if(vm[j], vtok >= a0 && vtok < a1);
      }
    }
    pv_tile<T, KT, D, RTA>(acc, pr, vm, va);
  };

  // Fused append (p.k_new set): the new
  // token's K/V rows go to cache position ctx - 1. The wave whose run holds that position
  // requests them with its tiles, writes them to the cache (cast to the cache type) and
  // puts the same values into the tile's registers in place of the row it loaded, so
  // this launch reads what msattn_write_kv followed by a decode would read. No other
  // workgroup reads that position (it lies in the last partition), so nothing waits for
  // the store.
  // (Built as its own instantiation, APPEND, for 2-byte queries at up to 8 rows per tile:
  // the chunks held for it take 16-36 registers, which cost the decode without it 0.5-2.6 %.)
  constexpr bool kAppendOk = APPEND && !kPvMfma && sizeof(T) == 2 && RT <= 8;
  const bool app = kAppendOk && p.k_new != nullptr && ctx > 0;
  const int k_app = app ? (ctx - 1) / 16 - tw0 : -1;  // run index of the new token's tile
  const bool app_here = k_app >= 0 && k_app < nt;      // wave-uniform
  const int r_new = (ctx - 1) & 15;                    // its row in the tile
  const bool k_lane = tile_token<D>(n) == r_new;       // lanes holding its K chunks
  const bool v_lane = va <= r_new && (r_new - va) % TPI == 0;  // and one of its V chunks
  SrcChunk<T> kn[JD], vn;
  if (app_here) {
    const int64_t row = (static_cast<int64_t>(b) * p.KVH + kvh) * D;
    if (k_lane) {
#pragma unroll
      for (int j = 0; j < JD; ++j)
        kn[j] = *reinterpret_cast<const SrcChunk<T>*>(static_cast<const T*>(p.k_new) + row +
                                                      KV::qk_dim0(j, g, JD));
    }
    if (v_lane)
      vn = *reinterpret_cast<const SrcChunk<T>*>(static_cast<const T*>(p.v_new) + row + vc * 8);
  }
  auto append_patch = [&](raw_t (&kb)[JD], raw_t (&vb)[NJ], int64_t base) __attribute__((always_inline)) {
    if (base < 0) return;  // a hole: write_kv writes nothing there either
    const int64_t rowoff = base + static_cast<int64_t>(r_new) * p.slot_stride;
    if (k_lane) {
#pragma unroll
      for (int j = 0; j < JD; ++j) {
        const raw_t x = append_raw<KT, T, raw_t>(kn[j]);
        kb[j] = x;
        *reinterpret_cast<raw_t*>(const_cast<KT*>(kbase) + rowoff + KV::qk_dim0(j, g, JD)) = x;
      }
    }
    if (v_lane) {
      const raw_t x = append_raw<KT, T, raw_t>(vn);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (TPI * j + va == r_new) vb[j] = x;
      *reinterpret_cast<raw_t*>(const_cast<KT*>(vbase) + rowoff + vc * 8) = x;
    }
  };

  if constexpr (kBalance) {  // the progress words start at zero (every wave reaches here)
    if (tid < kWaves) s_prog[tid] = 0;
    __syncthreads();
  }
  static_for<kMaxT>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    if (k >= nt) return;
    constexpr int nx = k + DEPTH - 1;  // the tile whose loads go out now
    if constexpr (nx < kMaxT) {
      br[nx % DEPTH] = tile_base(nx);
      issue(br[nx % DEPTH], kr[nx % DEPTH], vr[nx % DEPTH]);
    }
    if constexpr (kAppendOk) {
      if (app_here && k == k_app) append_patch(kr[k % DEPTH], vr[k % DEPTH], br[k % DEPTH]);
    }
    consume(k, kr[k % DEPTH], vr[k % DEPTH], br[k % DEPTH]);
    if constexpr (kBalance) {
      // Post this wave's progress; take priority while not ahead of the partner.
      if (lane == 0)
        __hip_atomic_store(&s_prog[w], k + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      const int other = __hip_atomic_load(&s_prog[w ^ (kWaves / 2)], __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_WORKGROUP);
      if (k + 1 <= __builtin_amdgcn_readfirstlane(other))
        __builtin_amdgcn_s_setprio(1);
      else
        __builtin_amdgcn_s_setprio(0);
    }
  });
  if constexpr (kBalance) __builtin_amdgcn_s_setprio(0);

  // Wave totals: l over the 4 lane groups, acc over the V token groups (lanes of equal
  // lane % LPR), reduce-scattered so a lane keeps two dims of each row: dims
  // vc * 8 + 2 * share + {0, 1}.
  l_run = rows4_sum(l_run);
  if (lane < RT) {
    s_ml[w][lane][0] = m_run;
    s_ml[w][lane][1] = l_run;
  }
  if constexpr (kPvMfma) {  // the matrix core summed the wave's tokens already
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<float4*>(&s_red[w][4 * g + i][64 * h + 4 * n]) =
            make_float4(acc_o[4 * h][i], acc_o[4 * h + 1][i], acc_o[4 * h + 2][i], acc_o[4 * h + 3][i]);
  } else {
    float red[RTA * 2];
    reduce_scatter<LPR>(acc, red);
    if (rs_owner<LPR>(lane)) {
      const int d0 = vc * 8 + 2 * rs_share<LPR>(lane);
#pragma unroll
      for (int r = 0; r < RTA; ++r)
        *reinterpret_cast<float2*>(&s_red[w][r][d0]) = make_float2(red[2 * r], red[2 * r + 1]);
    }
  }
  __syncthreads();

  // Combine the waves, four dims a thread: rescale each wave to the common max. A wave
  // without keys (m = -inf) takes weight 0 through selects, not branches, so that every
  // wave's LDS reads go out together (a branch per wave serialises them; C5-decode's
  // combine took 1.2 us that way).
  for (int idx = tid; idx < nrows * D4; idx += kThreads) {
    const int r = idx / D4;
    const int d = (idx - r * D4) * 4;
    float mw[kWaves];
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) {
      mw[ww] = s_ml[ww][r][0];
      M = fmaxf(M, mw[ww]);
    }
    float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float L = 0.0f;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) {
      const bool live = mw[ww] != -INFINITY;  // then M is finite too
      const float f = __builtin_amdgcn_exp2f(live ? mw[ww] - M : 0.0f);
      const float4 v = *reinterpret_cast<const float4*>(&s_red[ww][r][d]);
      const float lw = s_ml[ww][r][1];
      a.x = live ? fmaf(v.x, f, a.x) : a.x;
      a.y = live ? fmaf(v.y, f, a.y) : a.y;
      a.z = live ? fmaf(v.z, f, a.z) : a.z;
      a.w = live ? fmaf(v.w, f, a.w) : a.w;
      L = live ? fmaf(lw, f, L) : L;
    }
    const int64_t orow = out_row(r);
    if (direct) {  // the only partition: normalise and write the output
      store_out4(orow, d, a, L > 0.0f ? 1.0f / L : 0.0f);
    } else if (fused) {
      float* slot = p.acc + (orow * p.max_parts + part) * D + d;
      store2_device(slot, a.x, a.y);
      store2_device(slot + 2, a.z, a.w);
    } else {
      *reinterpret_cast<float4*>(p.acc + (orow * p.max_parts + part) * D + d) = a;
    }
  }
  if (direct) return;
  if (tid < nrows) {
    float mw[kWaves], lw[kWaves];
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) {
      mw[ww] = s_ml[ww][tid][0];
      lw[ww] = s_ml[ww][tid][1];
      M = fmaxf(M, mw[ww]);
    }
    float L = 0.0f;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) {
      const bool live = mw[ww] != -INFINITY;
      const float f = __builtin_amdgcn_exp2f(live ? mw[ww] - M : 0.0f);
      L = live ? fmaf(lw[ww], f, L) : L;
    }
    float* ml = p.ml + (orow_n * p.max_parts + part) * 2;
    if (fused) {
      store2_device(ml, M, L);
    } else {
      ml[0] = M;
      ml[1] = L;
      if (part + 1 == nparts && nparts < p.max_parts) {  // end marker
        ml[2] = -INFINITY;
        ml[3] = -1.0f;
      }
    }
  }
  if (fused) fused_merge();
}

template <typename T, typename KT, int D, int RT, int W = kMfmaWaves, int WPC = kMfmaWgPerCu>
hipError_t launch_decode_mfma_one(const SplitParams& p_in, hipStream_t stream) {
  // Partition-major order wherever the flat index fits: a launch's empty partitions (past
  // their sequence's length, which the grid cannot know) are then dispatched after every
  // workgroup with keys instead of among them.
  SplitParams p = p_in;
  const uint64_t flat = static_cast<uint64_t>(p.max_parts) * static_cast<uint64_t>(p.KVH) *
                        static_cast<uint64_t>(p.rtiles) * static_cast<uint64_t>(p.batch);
  p.part_major = MSATTN_PART_MAJOR && flat < (uint64_t(1) << 31) ? 1 : 0;
  const unsigned gx = p.part_major ? static_cast<unsigned>(flat)
                                   : static_cast<unsigned>(p.max_parts) * static_cast<unsigned>(p.KVH) *
                                         static_cast<unsigned>(p.rtiles);
  const dim3 grid(gx, 1, p.part_major ? 1u : static_cast<unsigned>(p.batch));
  // the fused append's instantiation (the host sets k_new only where it is built)
  if constexpr (sizeof(T) == 2 && RT <= 8) {
    if (p.k_new != nullptr) {
      hipLaunchKernelGGL((decode_mfma_kernel<T, KT, D, RT, W, WPC, true>), grid, dim3(W * kWave),
                         0, stream, p);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((decode_mfma_kernel<T, KT, D, RT, W, WPC>), grid, dim3(W * kWave), 0,
                     stream, p);
  return hipGetLastError();
}

// Launch for T in {bf16_t, _Float16} and a KV cache of T or of fp8_t;
// *supported = false when (D, RT) is not compiled.
template <typename T, typename KT>
hipError_t launch_decode_mfma(const SplitParams& p, int D, int RT, hipStream_t stream,
                              bool* supported);

#define MSATTN_DECLARE_MFMA_LAUNCHER(T, KT)                                                  \
  template <>                                                                                \
  hipError_t launch_decode_mfma<T, KT>(const SplitParams& p, int D, int RT, hipStream_t stream, \
                                       bool* supported);
MSATTN_DECLARE_MFMA_LAUNCHER(bf16_t, bf16_t)
MSATTN_DECLARE_MFMA_LAUNCHER(_Float16, _Float16)
MSATTN_DECLARE_MFMA_LAUNCHER(bf16_t, fp8_t)
MSATTN_DECLARE_MFMA_LAUNCHER(_Float16, fp8_t)
MSATTN_DECLARE_MFMA_LAUNCHER(bf16_t, float)
MSATTN_DECLARE_MFMA_LAUNCHER(_Float16, float)
MSATTN_DECLARE_MFMA_LAUNCHER(float, float)
MSATTN_DECLARE_MFMA_LAUNCHER(float, bf16_t)
MSATTN_DECLARE_MFMA_LAUNCHER(float, _Float16)
MSATTN_DECLARE_MFMA_LAUNCHER(float, fp8_t)
#undef MSATTN_DECLARE_MFMA_LAUNCHER

}  // namespace msattn
