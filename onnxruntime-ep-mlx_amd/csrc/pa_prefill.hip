// pa_prefill.hip — chunked-prefill attention over the paged cache.
//
// Until the LDS-shared prefill kernel lands, multi-token queries run on the split-K MFMA decode
// kernel, which parallelises over 16-row groups of (query token, head) rows and skips key tiles
// outside every row's causal range.
#include "pa_device.hpp"

namespace pa {

bool prefill_mfma_supported(int, pa_dtype, pa_dtype) { return false; }

hipError_t launch_prefill_mfma(const AttnParams&, pa_dtype, pa_dtype, hipStream_t) {
  return hipErrorNotSupported;
}

}  // namespace pa
