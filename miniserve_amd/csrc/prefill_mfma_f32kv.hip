// Chunked-prefill MFMA kernel for bf16 and fp16 queries over an fp32 cache: the K/V
// chunks are loaded as fp32 and rounded to the query type as they are staged into LDS
// (the reference's cast of the gathered rows to query.dtype,
// miniserve/attention.py:240-241), so the arithmetic is that of the same kernel on the
// cache converted beforehand. Compiled with the MFMA results in ordinary VGPRs, as
// prefill_mfma.hip.
#include "prefill_mfma.h"

namespace msattn {

MSATTN_DEFINE_PF(bf16_t, float)
MSATTN_DEFINE_PF(_Float16, float)

}  // namespace msattn
