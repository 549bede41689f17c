// Stream-K decode instantiated for bf16 and fp16 KV read by a query of the same
// type (fp8 KV: decode_streamk_fp8.hip), head_dim 64 and 128, row tiles of 1, 2, 4,
// 8 and 16 query rows.
#include "decode_streamk.h"

namespace msattn {

MSATTN_SK_LAUNCHER(bf16_t, bf16_t)
MSATTN_SK_LAUNCHER(_Float16, _Float16)

}  // namespace msattn
