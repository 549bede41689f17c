// Stream-K decode over an fp32 KV cache read by a bf16 or fp16 query: each K/V element
// is rounded to the query type in registers (the reference's cast of the gathered rows
// to query.dtype, miniserve/attention.py:240-241).
#include "decode_streamk.h"

namespace msattn {

MSATTN_SK_LAUNCHER(bf16_t, float)
MSATTN_SK_LAUNCHER(_Float16, float)

}  // namespace msattn
