// Chunked-prefill MFMA kernel for bf16 and fp16 queries over an fp8 e4m3 cache, head_dim
// 128: the K/V chunks are loaded as bytes and widened exactly to the query type as they
// are staged into LDS, so the arithmetic is that of the same kernel on the dequantized
// cache. Compiled with the MFMA results in ordinary VGPRs, as prefill_mfma.hip.
#include "prefill_mfma.h"

namespace msattn {

MSATTN_DEFINE_PF(bf16_t, fp8_t)
MSATTN_DEFINE_PF(_Float16, fp8_t)

}  // namespace msattn
