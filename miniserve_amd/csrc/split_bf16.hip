// Generic split-K partial kernels for a bf16 query over a bf16 KV cache:
// K/V read as stored.
#include "split_kernel.h"

namespace msattn {

MSATTN_SPLIT_LAUNCHER(bf16_t, bf16_t)

}  // namespace msattn
