// Chunked-prefill MFMA kernel instantiated for bf16 and fp16 queries over a cache of the
// same type, head_dim 128 (fp8 caches: prefill_mfma_fp8.hip). This translation unit is
// compiled with the MFMA results in ordinary VGPRs (see build.py): the kernel fits in 256
// of them, and the accumulator-register form would copy every score and accumulator
// between register files on each step.
#include "prefill_mfma.h"

namespace msattn {

MSATTN_DEFINE_PF(bf16_t, bf16_t)
MSATTN_DEFINE_PF(_Float16, _Float16)

}  // namespace msattn
