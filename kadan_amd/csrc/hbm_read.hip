// The HBM read ceiling: a plain streaming read of a device buffer, the yardstick the
// GEMV's bandwidth is judged against.  It does the least a reader can do (16-byte
// non-temporal loads, eight in flight per lane, an xor fold), so its best time over
// launch shapes for a buffer of a given size is what any kernel that must read that many
// bytes once can hope for on this device.  Two forms: every workgroup stores its fold
// (as a kernel that produces output must store something), or a workgroup stores only
// when its fold equals `match` (a read with no output on the critical path; the
// measured difference is the latency of a kernel's final stores).
#include "kdq_common.hpp"

namespace {

using u32x4 = unsigned __attribute__((ext_vector_type(4)));
constexpr int kInFlight = 8;

template <int kThreads, bool kStoreAll>
__global__ __launch_bounds__(kThreads) void hbm_read_kernel(const u32x4* __restrict__ src,
                                                            size_t units, size_t per,
                                                            unsigned* __restrict__ sink,
                                                            unsigned match) {
    // workgroup b reads units [b * per, min(units, (b + 1) * per)) of 16 bytes
    const size_t first = size_t(blockIdx.x) * per;
    const size_t end = first + per < units ? first + per : units;
    u32x4 acc = {0u, 0u, 0u, 0u};
    // every pass issues all kInFlight loads before the first is used; lanes past `end`
    // load nothing (a partial last pass costs no extra round trip)
    for (size_t i = first + threadIdx.x; i < end; i += kInFlight * kThreads) {
        u32x4 v[kInFlight];
#pragma unroll
        for (int k = 0; k < kInFlight; ++k) {
            const size_t at = i + size_t(k) * kThreads;
            v[k] = at < end ? __builtin_nontemporal_load(src + at) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int k = 0; k < kInFlight; ++k)
            acc ^= v[k];
    }
    unsigned r = acc.x ^ acc.y ^ acc.z ^ acc.w;
    for (int off = 32; off; off >>= 1)
        r ^= __shfl_xor(r, off);
    __shared__ unsigned folded[kThreads / 64];
    if (threadIdx.x % 64 == 0)
        folded[threadIdx.x / 64] = r;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned all = 0;
        for (int w = 0; w < kThreads / 64; ++w)
            all ^= folded[w];
        if (kStoreAll || all == match)
            sink[blockIdx.x] = all;
    }
}

}  // namespace

extern "C" int kdq_hbm_read(const void* src, size_t bytes, unsigned* sink, size_t workgroups,
                            int threads, int store_all, unsigned match, void* stream) {
    if (!src || !sink || !bytes || !workgroups || workgroups > (size_t(1) << 20))
        return KDQ_ERR_ARGUMENT;
    if (threads != 256 && threads != 1024)
        return KDQ_ERR_UNSUPPORTED;
    if (bytes % 16)
        return KDQ_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(src) % 16)
        return KDQ_ERR_ALIGNMENT;
    const size_t units = bytes / 16;
    // shares of whole KiB (64 units), so every workgroup's span starts KiB-aligned
    const size_t per = ((units + workgroups - 1) / workgroups + 63) / 64 * 64;
    const auto* units16 = static_cast<const u32x4*>(src);
    const auto st = static_cast<hipStream_t>(stream);
    const dim3 grid{unsigned(workgroups)}, block{unsigned(threads)};
    if (threads == 256 && store_all)
        hipLaunchKernelGGL((hbm_read_kernel<256, true>), grid, block, 0, st, units16, units, per,
                           sink, match);
    else if (threads == 256)
        hipLaunchKernelGGL((hbm_read_kernel<256, false>), grid, block, 0, st, units16, units,
                           per, sink, match);
    else if (store_all)
        hipLaunchKernelGGL((hbm_read_kernel<1024, true>), grid, block, 0, st, units16, units,
                           per, sink, match);
    else
        hipLaunchKernelGGL((hbm_read_kernel<1024, false>), grid, block, 0, st, units16, units,
                           per, sink, match);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}
