// Instantiates the K-quant decode GEMV / small-batch kernels of oq_gemv_kq.h for one weight type
// and one activation form (F32 rows quantized to Q8_K inside the kernels, or Q8_K blocks).
// oracle_amd/build.py compiles this file once per (OQ_KQ_TYPE, OQ_KQ_FUSED) pair, so the six
// instantiation sets compile in parallel; oq_gemv_kq.hip dispatches to them.
#include "oq_gemv_kq.h"

#if !defined(OQ_KQ_TYPE) || !defined(OQ_KQ_FUSED)
#error "compile with -DOQ_KQ_TYPE=<12|13|14> -DOQ_KQ_FUSED=<0|1>"
#endif

namespace oq {

template <uint32_t TYPE, bool FUSED>
hipError_t launch_kq(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y, hipStream_t s) {
    return kq::launch_m<TYPE, FUSED>(w, m, x, q8k, y, s);
}

template <uint32_t TYPE, bool FUSED>
hipError_t launch_kq_argmax(const DeviceMatrix& w, const float* x, const uint8_t* q8k, float* y, ArgmaxPart* parts,
                            uint32_t max_parts, uint32_t* nparts, hipStream_t s) {
    return kq::launch_argmax_iters<TYPE, FUSED>(w, x, q8k, y, parts, max_parts, nparts, s);
}

template <uint32_t TYPE, bool FUSED>
hipError_t launch_kq_window(const DeviceMatrix& w, int m, const float* x, const uint8_t* q8k, float* y,
                            uint32_t pass0, uint32_t npass, int accumulate, hipStream_t s) {
    if (m <= 1) return kq::launch_window<TYPE, 1, FUSED>(w, m, x, q8k, y, pass0, npass, accumulate, s);
    if (m <= 2) return kq::launch_window<TYPE, 2, FUSED>(w, m, x, q8k, y, pass0, npass, accumulate, s);
    return hipErrorInvalidValue;
}

template hipError_t launch_kq<OQ_KQ_TYPE, (OQ_KQ_FUSED != 0)>(const DeviceMatrix&, int, const float*, const uint8_t*,
                                                               float*, hipStream_t);
template hipError_t launch_kq_argmax<OQ_KQ_TYPE, (OQ_KQ_FUSED != 0)>(const DeviceMatrix&, const float*,
                                                                      const uint8_t*, float*, ArgmaxPart*, uint32_t,
                                                                      uint32_t*, hipStream_t);
template hipError_t launch_kq_window<OQ_KQ_TYPE, (OQ_KQ_FUSED != 0)>(const DeviceMatrix&, int, const float*,
                                                                      const uint8_t*, float*, uint32_t, uint32_t, int,
                                                                      hipStream_t);

}  // namespace oq
