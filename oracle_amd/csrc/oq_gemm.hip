// Prefill / verify GEMM (m >= 16) on matrix cores: placeholder until the MFMA kernel lands;
// every m is served by the small-batch kernels meanwhile.
#include "oq_common.h"

namespace oq {

bool gemm_mfma_supported(const DeviceMatrix&, int) { return false; }

hipError_t launch_gemm_q4k_mfma(const DeviceMatrix&, int, const uint8_t*, float*, hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace oq
