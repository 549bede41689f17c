// Generic split-K partial kernels for a bf16 query over a fp16 KV cache:
// K/V rounded to the query type (nearest even) as loaded, the reference's
// .to(query.dtype) of the gathered rows (miniserve/attention.py:240-241).
#include "split_kernel.h"

namespace msattn {

MSATTN_SPLIT_LAUNCHER(bf16_t, _Float16)

}  // namespace msattn
