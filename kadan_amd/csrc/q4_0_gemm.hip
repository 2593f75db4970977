// Prefill Q4_0 GEMM (placeholder until the MFMA kernel lands).
#include "kdq_common.hpp"
extern "C" int kdq_quantize_q8(const uint16_t*, size_t, size_t, int8_t*, float*, void*) {
    return KDQ_ERR_UNSUPPORTED;
}
extern "C" int kdq_gemm_q4_0(const void*, size_t, size_t, const uint16_t*, size_t, uint16_t*, void*) {
    return KDQ_ERR_UNSUPPORTED;
}
