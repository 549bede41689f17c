// MFMA decode partials instantiated for bf16 and fp16 KV read by a query of the
// same type (fp8 KV: decode_mfma_fp8.hip), head_dim 64 and 128, row tiles of 1, 2,
// 4, 8 and 16 query rows.
#include "decode_mfma_launch.h"

namespace msattn {

MSATTN_MFMA_LAUNCHER(bf16_t, bf16_t)
MSATTN_MFMA_LAUNCHER(_Float16, _Float16)

}  // namespace msattn
