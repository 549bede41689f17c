// Stream-K decode over an fp8 (OCP e4m3) KV cache read by a bf16 or fp16 query:
// the cache is widened to the query type in registers.
#include "decode_streamk.h"

namespace msattn {

MSATTN_SK_LAUNCHER(bf16_t, fp8_t)
MSATTN_SK_LAUNCHER(_Float16, fp8_t)

}  // namespace msattn
