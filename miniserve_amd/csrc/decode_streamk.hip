// Stream-K decode instantiated for bf16 and fp16 KV, head_dim 64 and 128,
// row tiles of 1, 2, 4, 8 and 16 query rows.
#include "decode_streamk.h"

namespace msattn {

#define MSATTN_SK_RT(T, D)                                                    \
  switch (RT) {                                                               \
    case 1: return launch_decode_streamk_one<T, D, 1>(p, grid, stream);       \
    case 2: return launch_decode_streamk_one<T, D, 2>(p, grid, stream);       \
    case 4: return launch_decode_streamk_one<T, D, 4>(p, grid, stream);       \
    case 8: return launch_decode_streamk_one<T, D, 8>(p, grid, stream);       \
    case 16: return launch_decode_streamk_one<T, D, 16>(p, grid, stream);     \
    default: break;                                                           \
  }

#define MSATTN_SK_LAUNCHER(T)                                                                     \
  template <>                                                                                     \
  hipError_t launch_decode_streamk<T>(const SplitParams& p, int D, int RT, int grid,             \
                                      hipStream_t stream, bool* supported) {                      \
    *supported = true;                                                                            \
    if (D == 64) { MSATTN_SK_RT(T, 64) }                                                          \
    if (D == 128) { MSATTN_SK_RT(T, 128) }                                                        \
    *supported = false;                                                                           \
    return hipSuccess;                                                                            \
  }

MSATTN_SK_LAUNCHER(bf16_t)
MSATTN_SK_LAUNCHER(_Float16)

}  // namespace msattn
