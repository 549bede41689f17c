// Generic split-K partial kernels for a fp32 query over a fp32 KV cache:
// K/V read as stored.
#include "split_kernel.h"

namespace msattn {

MSATTN_SPLIT_LAUNCHER(float, float)

}  // namespace msattn
