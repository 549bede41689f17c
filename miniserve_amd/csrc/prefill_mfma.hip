// Chunked-prefill MFMA kernel instantiated for bf16 and fp16, head_dim 128. This
// translation unit is compiled with the MFMA results in ordinary VGPRs (see build.py):
// the kernel fits in 256 of them, and the accumulator-register form would copy every
// score and accumulator between register files on each step.
#include "prefill_mfma.h"

namespace msattn {

template <>
hipError_t launch_prefill_mfma<bf16_t>(const PrefillParams& p, int D, hipStream_t stream,
                                       bool* supported) {
  return launch_prefill_mfma_impl<bf16_t>(p, D, stream, supported);
}

template <>
hipError_t launch_prefill_mfma<_Float16>(const PrefillParams& p, int D, hipStream_t stream,
                                         bool* supported) {
  return launch_prefill_mfma_impl<_Float16>(p, D, stream, supported);
}

template <>
hipError_t launch_prefix_partials<bf16_t>(const PrefillParams& p, int D, hipStream_t stream,
                                          bool* supported) {
  return launch_prefix_partials_impl<bf16_t>(p, D, stream, supported);
}

template <>
hipError_t launch_prefix_partials<_Float16>(const PrefillParams& p, int D, hipStream_t stream,
                                            bool* supported) {
  return launch_prefix_partials_impl<_Float16>(p, D, stream, supported);
}

}  // namespace msattn
