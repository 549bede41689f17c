// Split-K partial kernels instantiated for query bf16_t, KV cache bf16_t.
// Head dims compiled: 16, 24, 32, 64, 96, 128, 256; rows per tile 1, 2, 4, 8.
#include "split_kernel.h"

namespace msattn {

template <>
hipError_t launch_split<bf16_t, bf16_t>(const SplitParams& p, int D, int RT, hipStream_t stream,
                                    bool* supported) {
  *supported = true;
  switch (D) {
    case 16:
      MSATTN_SPLIT_RT(bf16_t, bf16_t, 16)
      break;
    case 24:
      MSATTN_SPLIT_RT(bf16_t, bf16_t, 24)
      break;
    case 32:
      MSATTN_SPLIT_RT(bf16_t, bf16_t, 32)
      break;
    case 64:
      MSATTN_SPLIT_RT(bf16_t, bf16_t, 64)
      break;
    case 96:
      MSATTN_SPLIT_RT(bf16_t, bf16_t, 96)
      break;
    case 128:
      MSATTN_SPLIT_RT(bf16_t, bf16_t, 128)
      break;
    case 256:
      MSATTN_SPLIT_RT(bf16_t, bf16_t, 256)
      break;
    default:
      break;
  }
  *supported = false;
  return hipSuccess;
}

}  // namespace msattn
