// Shared device helpers for the msattn HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace msattn {

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

// ---------------------------------------------------------------------------
// Element types. Storage types only; all arithmetic is fp32.
//   float      fp32
//   _Float16   fp16 (IEEE binary16)
//   bf16_t     bfloat16 bits
//   fp8_t      OCP float8 e4m3fn bits (no infinities, 0x7f/0xff are NaN)
// ---------------------------------------------------------------------------
struct bf16_t { uint16_t bits; };
struct fp8_t { uint8_t bits; };

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h16) {
  return __uint_as_float(h16 << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits, NaN -> 0x7fc0 (torch's rule).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Exact decode of one e4m3fn byte.
__device__ __forceinline__ float fp8e4m3_to_f32(uint32_t x) {
  const uint32_t sign = (x & 0x80u) << 24;
  const uint32_t e = (x >> 3) & 0xfu;
  const uint32_t m = x & 0x7u;
  if (e == 0) {
    const float v = static_cast<float>(m) * 0x1p-9f;  // subnormal: m * 2^-9
    return __uint_as_float(__float_as_uint(v) | sign);
  }
  if (e == 15 && m == 7) return __uint_as_float(sign | 0x7fc00000u);
  return __uint_as_float(sign | ((e + 120u) << 23) | (m << 20));
}

// fp32 -> e4m3fn, round to nearest even; |x| >= 480 and NaN give NaN (0x7f|sign),
// which is the rule torch.Tensor.to(torch.float8_e4m3fn) applies.
__device__ __forceinline__ uint8_t f32_to_fp8e4m3(float f) {
  uint32_t u = __float_as_uint(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  u &= 0x7fffffffu;
  if (u >= 0x43f00000u) return static_cast<uint8_t>(sign | 0x7fu);  // >= 480 or NaN
  if (u < 0x3c800000u) {
    // below 2^-6: subnormal range, quantum 2^-9. Exact RNE through the fp32 adder:
    // adding 2^-9 * 2^23 * 2^... is avoided; scale by 2^9 and round to integer.
    const float a = __uint_as_float(u) * 512.0f;  // exact (power of two scale)
    const float r = __builtin_rintf(a);           // RNE to integer 0..8
    return static_cast<uint8_t>(sign | static_cast<uint32_t>(r));
  }
  // normal: keep 3 mantissa bits with RNE, rebias exponent 127 -> 7.
  const uint32_t mant_odd = (u >> 20) & 1u;
  u += 0x7ffffu + mant_odd;
  const uint32_t e = (u >> 23) - 120u;
  const uint32_t m = (u >> 20) & 0x7u;
  return static_cast<uint8_t>(sign | (e << 3) | m);
}

template <typename T> struct Elt;
template <> struct Elt<float> {
  static constexpr int kBytes = 4;
  static constexpr int kCode = 0;
  __device__ static float load(const float* p) { return *p; }
  __device__ static void store(float* p, float v) { *p = v; }
};
template <> struct Elt<_Float16> {
  static constexpr int kBytes = 2;
  static constexpr int kCode = 1;
  __device__ static float load(const _Float16* p) { return static_cast<float>(*p); }
  __device__ static void store(_Float16* p, float v) { *p = static_cast<_Float16>(v); }
};
template <> struct Elt<bf16_t> {
  static constexpr int kBytes = 2;
  static constexpr int kCode = 2;
  __device__ static float load(const bf16_t* p) { return bf16_bits_to_f32(p->bits); }
  __device__ static void store(bf16_t* p, float v) { p->bits = f32_to_bf16_bits(v); }
};
template <> struct Elt<fp8_t> {
  static constexpr int kBytes = 1;
  static constexpr int kCode = 3;
  __device__ static float load(const fp8_t* p) { return fp8e4m3_to_f32(p->bits); }
  __device__ static void store(fp8_t* p, float v) { p->bits = f32_to_fp8e4m3(v); }
};

// Round an fp32 value to T's precision and back (identity for float).
template <typename T> __device__ __forceinline__ float round_to(float v) {
  T t;
  Elt<T>::store(&t, v);
  return Elt<T>::load(&t);
}

// K/V as a query of type QT sees them. The reference casts the gathered K/V to the
// query dtype before attending (miniserve/attention.py:240-241): a widening cast (fp8 or
// a 2-byte type to fp32, fp8 to a 2-byte type) is exact and leaves the value alone; a
// narrowing one (fp32 to bf16/fp16, bf16 <-> fp16) rounds to nearest even, as
// torch.Tensor.to does.
template <typename QT, typename KT> struct KvCast {
  static constexpr bool kRounds = !std::is_same<QT, float>::value &&
                                  !std::is_same<QT, KT>::value &&
                                  !std::is_same<KT, fp8_t>::value;
  template <int N>
  __device__ static void apply(float (&x)[N]) {
    if constexpr (kRounds) {
#pragma unroll
      for (int e = 0; e < N; ++e) x[e] = round_to<QT>(x[e]);
    }
  }
};

// Unpack one 16-byte chunk (four dwords) of KV elements into fp32.
template <typename T> struct Chunk;
template <> struct Chunk<float> {
  static constexpr int kElems = 4;
  __device__ static void unpack(const uint4& c, float* o) {
    o[0] = __uint_as_float(c.x); o[1] = __uint_as_float(c.y);
    o[2] = __uint_as_float(c.z); o[3] = __uint_as_float(c.w);
  }
};
template <> struct Chunk<bf16_t> {
  static constexpr int kElems = 8;
  __device__ static void unpack(const uint4& c, float* o) {
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = __uint_as_float(w[i] << 16);
      o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  // Eight fp32 values to one chunk, rounded like Elt<bf16_t>::store.
  __device__ static uint4 pack(const float* f) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = static_cast<uint32_t>(f32_to_bf16_bits(f[2 * i])) |
             (static_cast<uint32_t>(f32_to_bf16_bits(f[2 * i + 1])) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
};
template <> struct Chunk<_Float16> {
  static constexpr int kElems = 8;
  __device__ static void unpack(const uint4& c, float* o) {
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t lo = static_cast<uint16_t>(w[i] & 0xffffu);
      const uint16_t hi = static_cast<uint16_t>(w[i] >> 16);
      o[2 * i] = static_cast<float>(__builtin_bit_cast(_Float16, lo));
      o[2 * i + 1] = static_cast<float>(__builtin_bit_cast(_Float16, hi));
    }
  }
  __device__ static uint4 pack(const float* f) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f[2 * i]))) |
             (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(f[2 * i + 1]))) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
};
template <> struct Chunk<fp8_t> {
  static constexpr int kElems = 16;
  __device__ static void unpack(const uint4& c, float* o) {
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) o[4 * i + j] = fp8e4m3_to_f32((w[i] >> (8 * j)) & 0xffu);
    }
  }
};

// Max over the four 16-lane rows of the wave (lanes n, n + 16, n + 32, n + 48, for
// each n), every lane receiving it. gfx950's row swaps exchange rows 2k <-> 2k + 1
// (v_permlane16_swap) and the halves (v_permlane32_swap) of a register pair in the
// VALU, without the LDS round trip of a lane shuffle. Called with the same value twice,
// the pair returned holds each lane's own row value and its partner row's value.
#ifndef MSATTN_ROW_SWAPS
#define MSATTN_ROW_SWAPS 1
#endif
__device__ __forceinline__ float rows4_max(float v) {
#if MSATTN_ROW_SWAPS
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
#else
  v = fmaxf(v, __shfl_xor(v, 16, kWave));
  return fmaxf(v, __shfl_xor(v, 32, kWave));
#endif
}

// Sum over the four 16-lane rows, as rows4_max; every lane adds in the same order.
__device__ __forceinline__ float rows4_sum(float v) {
#if MSATTN_ROW_SWAPS
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
#else
  v += __shfl_xor(v, 16, kWave);
  return v + __shfl_xor(v, 32, kWave);
#endif
}

// ---------------------------------------------------------------------------
// Cross-lane reductions over aligned groups of `Width` lanes (power of two), every
// lane of a group receiving the result. Within a 16-lane row they run on DPP lane
// permutes (VALU): quad_perm [1,0,3,2] and [2,3,0,1] pair lanes i ^ 1 and i ^ 2,
// row_half_mirror then pairs the two quads of an 8-lane half (lane i with 7 - i) and
// row_mirror the two halves of the row (lane i with 15 - i); wider groups add the row
// swaps of rows4_max / rows4_sum. (MSATTN_ROW_SWAPS=0: lane shuffles throughout.)
// ---------------------------------------------------------------------------
template <int Ctrl>
__device__ __forceinline__ float dpp_mov(float v) {
  const int x = __float_as_int(v);
  return __int_as_float(__builtin_amdgcn_update_dpp(x, x, Ctrl, 0xF, 0xF, false));
}

template <int Width>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(Width >= 1 && Width <= 64 && (Width & (Width - 1)) == 0, "power-of-two width");
#if MSATTN_ROW_SWAPS
  if constexpr (Width >= 2) x += dpp_mov<0xB1>(x);   // quad_perm [1,0,3,2]
  if constexpr (Width >= 4) x += dpp_mov<0x4E>(x);   // quad_perm [2,3,0,1]
  if constexpr (Width >= 8) x += dpp_mov<0x141>(x);  // row_half_mirror
  if constexpr (Width >= 16) x += dpp_mov<0x140>(x); // row_mirror
  if constexpr (Width >= 32) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  }
  if constexpr (Width >= 64) {
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(b[0]) + __uint_as_float(b[1]);
  }
#else
#pragma unroll
  for (int o = Width / 2; o > 0; o >>= 1) x += __shfl_xor(x, o, kWave);
#endif
  return x;
}

template <int Width>
__device__ __forceinline__ float group_max(float x) {
  static_assert(Width >= 1 && Width <= 64 && (Width & (Width - 1)) == 0, "power-of-two width");
#if MSATTN_ROW_SWAPS
  if constexpr (Width >= 2) x = fmaxf(x, dpp_mov<0xB1>(x));
  if constexpr (Width >= 4) x = fmaxf(x, dpp_mov<0x4E>(x));
  if constexpr (Width >= 8) x = fmaxf(x, dpp_mov<0x141>(x));
  if constexpr (Width >= 16) x = fmaxf(x, dpp_mov<0x140>(x));
  if constexpr (Width >= 32) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  }
  if constexpr (Width >= 64) {
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
  }
#else
#pragma unroll
  for (int o = Width / 2; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, kWave));
#endif
  return x;
}

// Inclusive prefix sum over the wave (lane i receives x_0 + ... + x_i): DPP row shifts
// (lane i reads lane i - n of its 16-lane row; lanes without a source read 0) scan each
// row, then every row adds the totals of the rows below it.
__device__ __forceinline__ int wave_inclusive_sum(int x) {
#if MSATTN_ROW_SWAPS
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);  // row_shr:8
  const int r0 = __builtin_amdgcn_readlane(x, 15);
  const int r1 = __builtin_amdgcn_readlane(x, 31);
  const int r2 = __builtin_amdgcn_readlane(x, 47);
  const int row = static_cast<int>(__lane_id()) >> 4;
  return x + (row > 0 ? r0 : 0) + (row > 1 ? r1 : 0) + (row > 2 ? r2 : 0);
#else
  const int lane = static_cast<int>(__lane_id());
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int y = __shfl_up(x, o, kWave);
    if (lane >= o) x += y;
  }
  return x;
#endif
}

// ---------------------------------------------------------------------------
// Strided reduce-scatter: sums R x E values per lane over the lanes of equal
// lane % Stride (Stride a power of two, 1..64), leaving each lane a 1/P share of the
// totals, P = rs_parts(Stride) (4 below 32, 2 at 32, 1 at 64). A lane of share s =
// rs_share<Stride>(lane) ends with out[i] = sum of acc[i / per][s * per + i % per],
// per = E / P, i < R * per: a run of per consecutive elements of each row.
//
// A row swap of two different registers exchanges half of each: v_permlane32_swap(a, b)
// leaves (a_lo, b_lo) and (a_hi, b_hi), so their sum holds a's total over the halves in
// lanes 0-31 and b's in lanes 32-63, and v_permlane16_swap does the same for rows
// 2k / 2k + 1. One swap and one add thus fold two values where an all-lanes reduction
// needs two swaps, two copies and two adds; after both swaps row rho holds input value
// 4i + (rho bit-reversed). Strides below 16 finish with DPP row rotations inside a row.
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int rs_parts(int stride) {
  return stride >= 64 ? 1 : (stride == 32 ? 2 : 4);
}

template <int Stride>
__device__ __forceinline__ int rs_share(int lane) {
  constexpr int P = rs_parts(Stride);
  if constexpr (P == 4) {
    const int rho = lane >> 4;
    return ((rho & 1) << 1) | (rho >> 1);
  } else if constexpr (P == 2) {
    return lane >> 5;
  } else {
    return 0;
  }
}

// True for the lanes whose shares are distinct: below stride 16 the lanes of a row
// that differ only above lane % Stride hold copies.
template <int Stride>
__device__ __forceinline__ bool rs_owner(int lane) {
  if constexpr (Stride >= 16) return true;
  else return (lane & 15) < Stride;
}

template <int Stride, int R, int E>
__device__ __forceinline__ void reduce_scatter(const float (&acc)[R][E],
                                               float (&out)[R * E / rs_parts(Stride)]) {
  static_assert(Stride >= 1 && Stride <= 64 && (Stride & (Stride - 1)) == 0, "stride 1..64");
  constexpr int P = rs_parts(Stride);
  static_assert(E % P == 0, "row length must split into the shares");
  constexpr int per = E / P;
  constexpr int N = R * E;
  float x[N];
#pragma unroll
  for (int i = 0; i < N / P; ++i)
#pragma unroll
    for (int s = 0; s < P; ++s) x[P * i + s] = acc[i / per][s * per + i % per];
#if MSATTN_ROW_SWAPS
  if constexpr (P >= 2) {
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
      const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(x[2 * j]),
                                                      __float_as_uint(x[2 * j + 1]), false, false);
      x[j] = __uint_as_float(t[0]) + __uint_as_float(t[1]);
    }
  }
  if constexpr (P == 4) {
#pragma unroll
    for (int j = 0; j < N / 4; ++j) {
      const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(x[2 * j]),
                                                      __float_as_uint(x[2 * j + 1]), false, false);
      x[j] = __uint_as_float(t[0]) + __uint_as_float(t[1]);
    }
  }
  if constexpr (Stride < 16) {
#pragma unroll
    for (int j = 0; j < N / P; ++j) {
      if constexpr (Stride <= 1) x[j] += dpp_mov<0x121>(x[j]);  // row_ror:1
      if constexpr (Stride <= 2) x[j] += dpp_mov<0x122>(x[j]);  // row_ror:2
      if constexpr (Stride <= 4) x[j] += dpp_mov<0x124>(x[j]);  // row_ror:4
      x[j] += dpp_mov<0x128>(x[j]);                             // row_ror:8
    }
  }
#pragma unroll
  for (int j = 0; j < N / P; ++j) out[j] = x[j];
#else
  const int s = rs_share<Stride>(__lane_id());
#pragma unroll
  for (int j = 0; j < N; ++j)
#pragma unroll
    for (int o = Stride; o < kWave; o <<= 1) x[j] += __shfl_xor(x[j], o, kWave);
#pragma unroll
  for (int i = 0; i < N / P; ++i) {
    float v = x[P * i];
#pragma unroll
    for (int t = 1; t < P; ++t) v = s == t ? x[P * i + t] : v;
    out[i] = v;
  }
#endif
}

__host__ __device__ constexpr int next_pow2(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}

__host__ __device__ constexpr int ceil_div(int a, int b) { return (a + b - 1) / b; }

}  // namespace msattn
