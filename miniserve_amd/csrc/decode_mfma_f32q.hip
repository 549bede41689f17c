// MFMA decode partials for an fp32 query over a bf16, fp16 or fp8 (e4m3) KV cache: the
// cache's rows load as that type and widen exactly to fp32 in registers (the reference
// casts the gathered K/V to query.dtype, miniserve/attention.py:240-241); scores on
// v_mfma_f32_16x16x4_f32, P.V on fp32 FMAs. The reference runner's fp32 model over a
// lower-precision cache (miniserve/attention.py:151-152 takes an fp8 kv_dtype).
#include "decode_mfma_launch.h"

namespace msattn {

MSATTN_MFMA_LAUNCHER(float, bf16_t)
MSATTN_MFMA_LAUNCHER(float, _Float16)
MSATTN_MFMA_LAUNCHER(float, fp8_t)

}  // namespace msattn
