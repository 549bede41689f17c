// Generic split-K partial kernels for a fp16 query over a fp16 KV cache:
// K/V read as stored.
#include "split_kernel.h"

namespace msattn {

MSATTN_SPLIT_LAUNCHER(_Float16, _Float16)

}  // namespace msattn
