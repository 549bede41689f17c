// Split-K partial kernels instantiated for query float, KV cache float.
// Head dims compiled: 16, 24, 32, 64, 96, 128, 256; rows per tile 1, 2, 4, 8.
#include "split_kernel.h"

namespace msattn {

template <>
hipError_t launch_split<float, float>(const SplitParams& p, int D, int RT, hipStream_t stream,
                                    bool* supported) {
  *supported = true;
  switch (D) {
    case 16:
      MSATTN_SPLIT_RT(float, float, 16)
      break;
    case 24:
      MSATTN_SPLIT_RT(float, float, 24)
      break;
    case 32:
      MSATTN_SPLIT_RT(float, float, 32)
      break;
    case 64:
      MSATTN_SPLIT_RT(float, float, 64)
      break;
    case 96:
      MSATTN_SPLIT_RT(float, float, 96)
      break;
    case 128:
      MSATTN_SPLIT_RT(float, float, 128)
      break;
    case 256:
      MSATTN_SPLIT_RT(float, float, 256)
      break;
    default:
      break;
  }
  *supported = false;
  return hipSuccess;
}

}  // namespace msattn
