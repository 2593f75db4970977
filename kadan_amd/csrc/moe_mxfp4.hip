// MXFP4 MoE layer (placeholder until the kernels land).
#include "kdq_common.hpp"
extern "C" int kdq_moe_route(const float*, size_t, size_t, size_t, int32_t*, float*, int32_t*, int32_t*, void*) {
    return KDQ_ERR_UNSUPPORTED;
}
extern "C" int kdq_mxfp4_dequantize(const uint8_t*, const uint8_t*, size_t, size_t, float*, unsigned*, void*) {
    return KDQ_ERR_UNSUPPORTED;
}
extern "C" int kdq_moe_mxfp4(const uint16_t*, const float*, size_t, size_t, size_t, size_t, size_t,
                             const uint8_t*, const uint8_t*, const uint8_t*, const uint8_t*,
                             const uint8_t*, const uint8_t*, float*, int32_t*, float*, int32_t*,
                             int32_t*, void*) {
    return KDQ_ERR_UNSUPPORTED;
}
