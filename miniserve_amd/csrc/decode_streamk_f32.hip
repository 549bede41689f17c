// Stream-K decode for an fp32 query over an fp32 KV cache: scores on
// v_mfma_f32_16x16x4_f32 (fp32 products and sums), P.V on fp32 FMAs -- the reference
// runner's default types (miniserve/model_runner.py:122-123 allocates fp32 caches).
#include "decode_streamk.h"

namespace msattn {

MSATTN_SK_LAUNCHER(float, float)

}  // namespace msattn
