// MFMA decode partials over an fp8 (OCP e4m3) KV cache read by a bf16 or fp16
// query: the cache is widened to the query type in registers.
#include "decode_mfma_launch.h"

namespace msattn {

MSATTN_MFMA_LAUNCHER(bf16_t, fp8_t)
MSATTN_MFMA_LAUNCHER(_Float16, fp8_t)

}  // namespace msattn
