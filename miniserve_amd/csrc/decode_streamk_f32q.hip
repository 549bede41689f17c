// Stream-K decode for an fp32 query over a bf16, fp16 or fp8 (e4m3) KV cache: the
// cache's rows load as that type and widen exactly to fp32 in registers (the reference
// casts the gathered K/V to query.dtype, miniserve/attention.py:240-241); scores on
// v_mfma_f32_16x16x4_f32, P.V on fp32 FMAs.
#include "decode_streamk.h"

namespace msattn {

MSATTN_SK_LAUNCHER(float, bf16_t)
MSATTN_SK_LAUNCHER(float, _Float16)
MSATTN_SK_LAUNCHER(float, fp8_t)

}  // namespace msattn
