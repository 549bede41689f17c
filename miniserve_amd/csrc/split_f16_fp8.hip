// Generic split-K partial kernels for a fp16 query over a fp8 e4m3 KV cache:
// K/V widened exactly to the query type.
#include "split_kernel.h"

namespace msattn {

MSATTN_SPLIT_LAUNCHER(_Float16, fp8_t)

}  // namespace msattn
