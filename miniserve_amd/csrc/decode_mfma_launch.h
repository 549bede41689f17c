// Launcher bodies of the MFMA partition decode kernel, one per (query type, KV
// type), expanded by the instantiation files.
#pragma once

#include "decode_mfma.h"

namespace msattn {
template <typename T, typename KT>
constexpr bool kWideOk = sizeof(T) == 2 && sizeof(KT) <= 2;
}  // namespace msattn

// The wide (8-wave) shape is compiled for 4 and 8 rows per tile under a 2-byte query
// (a 16-bit or fp8 cache); p.mfma_waves selects it.
// p.mfma_deep selects, at head_dim 64 and 4 or 8 rows per tile, the regular shape with the
// deeper residency (kMfmaWgPerCuDeep workgroups a CU).
#define MSATTN_MFMA_RT(T, KT, D)                                                          \
  switch (RT) {                                                                           \
    case 1: return launch_decode_mfma_one<T, KT, D, 1>(p, stream);                        \
    case 2: return launch_decode_mfma_one<T, KT, D, 2>(p, stream);                        \
    case 4:                                                                               \
      if constexpr (kWideOk<T, KT>)                                                       \
        if (p.mfma_waves == kWideWaves) return launch_decode_mfma_one<T, KT, D, 4, kWideWaves>(p, stream); \
      if constexpr (D == 64 && sizeof(T) == 2)                                            \
        if (p.mfma_deep) return launch_decode_mfma_one<T, KT, D, 4, kMfmaWaves, kMfmaWgPerCuDeep>(p, stream); \
      return launch_decode_mfma_one<T, KT, D, 4>(p, stream);                              \
    case 8:                                                                               \
      if constexpr (kWideOk<T, KT>)                                                       \
        if (p.mfma_waves == kWideWaves) return launch_decode_mfma_one<T, KT, D, 8, kWideWaves>(p, stream); \
      if constexpr (D == 64 && sizeof(T) == 2)                                            \
        if (p.mfma_deep) return launch_decode_mfma_one<T, KT, D, 8, kMfmaWaves, kMfmaWgPerCuDeep>(p, stream); \
      return launch_decode_mfma_one<T, KT, D, 8>(p, stream);                              \
    case 16: return launch_decode_mfma_one<T, KT, D, 16>(p, stream);                      \
    default: break;                                                                       \
  }

#define MSATTN_MFMA_LAUNCHER(T, KT)                                                          \
  template <>                                                                                \
  hipError_t launch_decode_mfma<T, KT>(const SplitParams& p, int D, int RT, hipStream_t stream, \
                                       bool* supported) {                                    \
    *supported = true;                                                                       \
    if (D == 64) { MSATTN_MFMA_RT(T, KT, 64) }                                               \
    if (D == 128) { MSATTN_MFMA_RT(T, KT, 128) }                                             \
    *supported = false;                                                                      \
    return hipSuccess;                                                                       \
  }
