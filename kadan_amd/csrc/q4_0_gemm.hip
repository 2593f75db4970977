// Prefill Q4_0 GEMM for gfx950: Y[m, n] (fp16) = sum_k X[m, k] W[n, k].
//
// Semantics (include/kadan_amd.h): activations fp16 quantized per 32 values to int8
// codes with an fp32 scale exactly as ggml's x86 quantize_row_q8_0 does
// (G/src/ggml-cpu/arch/x86/quants.c:302-398: d = amax/127, id = 127/amax, codes
// round-half-even(x*id); G = IW/third_party/ggml), then the Q4_0 x Q8 product of
// ggml_vec_dot_q4_0_q8_0 (G/src/ggml-cpu/quants.c:225-260) with fp32 accumulation.
//
// Kernels:
//   quantize_kernel  one wavefront per 64 values: the int8 codes and scales, and the
//                    dequantised activation fp16(code * d) that the GEMM consumes
//   gemm_kernel      128x128 output tile per 256-thread workgroup (4 wavefronts of
//                    64x64), k in steps of 64 staged through double-buffered LDS:
//                    fp16 activations copied, Q4_0 weights dequantised once per tile
//                    to fp16 ((q-8)*d rounded once, packed-fp16 arithmetic), products on
//                    v_mfma_f32_32x32x16_f16 with fp32 accumulation; workgroups are
//                    ordered so the four M tiles of one weight tile share an XCD (L2).
#include "kdq_common.hpp"

namespace kdq {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// --------------------------------------------------------------- quantizer

// Thread t of the grid handles 8 consecutive values; 4 threads share one block.
__global__ __launch_bounds__(256) void quantize_kernel(const uint16_t* __restrict__ x,
                                                       size_t count, int8_t* __restrict__ q,
                                                       float* __restrict__ d,
                                                       uint16_t* __restrict__ dequant) {
    const size_t t = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t e = t * 8;
    float v[8] = {};
    if (e < count) {
        const u32x4 raw = *reinterpret_cast<const u32x4*>(x + e);
        const unsigned w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = half_hw(w[i] & 0xffffu);
            v[2 * i + 1] = half_hw(w[i] >> 16);
        }
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    if (e >= count)
        return;
    const float scale = __fdiv_rn(amax, 127.0f);
    const float inv = amax != 0.f ? __fdiv_rn(127.0f, amax) : 0.f;
    unsigned packed[2] = {0, 0};
    unsigned halves[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int c = __float2int_rn(__fmul_rn(v[i], inv));  // round half to even
        packed[i / 4] |= (unsigned(c) & 255u) << (8 * (i % 4));
        const _Float16 h = _Float16(__fmul_rn(float(c), scale));
        halves[i / 2] |= unsigned(__builtin_bit_cast(uint16_t, h)) << (16 * (i % 2));
    }
    *reinterpret_cast<uint2*>(q + e) = make_uint2(packed[0], packed[1]);
    if (dequant)
        *reinterpret_cast<uint4*>(dequant + e) = make_uint4(halves[0], halves[1], halves[2], halves[3]);
    if ((t & 3) == 0)
        d[e / 32] = scale;
}

// ------------------------------------------------------------------- GEMM

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int kPitch = BK + 8;  // fp16 per LDS row (144 bytes: conflict-free fragment reads)

// 32 Q4_0 values (one block) -> 16 fp16x2 words of round((q - 8) * d).
// `codes` are the 16 code bytes as four dwords; values j and j+16 share byte j.
__device__ __forceinline__ void dequant_q4_0(const unsigned codes[4], unsigned d_bits,
                                             unsigned out[16]) {
    const f16x2 scale = __builtin_bit_cast(f16x2, d_bits | (d_bits << 16));
    const f16x2 bias = __builtin_bit_cast(f16x2, 0x64086408u);  // (1032, 1032)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const unsigned w = codes[i];
        // bytes (b0, b1) -> positions (0, 16) and (b2, b3) -> (0, 16)
        const unsigned lo01 = __builtin_amdgcn_perm(0u, w, 0x0c010c00u);
        const unsigned lo23 = __builtin_amdgcn_perm(0u, w, 0x0c030c02u);
        const unsigned q[4] = {(lo01 & 0x000f000fu) | 0x64006400u,
                               (lo23 & 0x000f000fu) | 0x64006400u,
                               ((lo01 >> 4) & 0x000f000fu) | 0x64006400u,
                               ((lo23 >> 4) & 0x000f000fu) | 0x64006400u};
        f16x2 r[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            r[k] = (__builtin_bit_cast(f16x2, q[k]) - bias) * scale;  // exact (q-8), one rounding
        // values: 4i, 4i+1 (lo01), 4i+2, 4i+3 (lo23), 16+4i.. (high nibbles)
        out[2 * i] = __builtin_bit_cast(unsigned, r[0]);
        out[2 * i + 1] = __builtin_bit_cast(unsigned, r[1]);
        out[8 + 2 * i] = __builtin_bit_cast(unsigned, r[2]);
        out[8 + 2 * i + 1] = __builtin_bit_cast(unsigned, r[3]);
    }
}

struct Stage {
    u32x4 a[4];     // 32 activation values (fp16)
    unsigned w[5];  // 20 bytes covering one Q4_0 block
};

__global__ __launch_bounds__(256) void gemm_kernel(const uint16_t* __restrict__ a,
                                                   const uint8_t* __restrict__ w, unsigned m,
                                                   unsigned n, unsigned k,
                                                   uint16_t* __restrict__ y) {
    __shared__ __align__(16) uint16_t lds_a[2][BM * kPitch];
    __shared__ __align__(16) uint16_t lds_b[2][BN * kPitch];

    // XCD-aware tile order: the M tiles of one N tile run back to back on one XCD.
    const unsigned m_tiles = (m + BM - 1) / BM, n_tiles = (n + BN - 1) / BN;
    const unsigned id = blockIdx.x, xcd = id % 8, local = id / 8;
    const unsigned per_xcd = (n_tiles * m_tiles + 7) / 8;
    const unsigned linear = xcd * per_xcd + local;  // contiguous chunk per XCD
    if (local >= per_xcd || linear >= n_tiles * m_tiles)
        return;
    const unsigned n_tile = linear / m_tiles, m_tile = linear % m_tiles;
    const unsigned m0 = m_tile * BM, n0 = n_tile * BN;

    const unsigned tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    const size_t row_bytes = size_t(k / 32) * 18;

    // global -> register staging: thread t copies activation row t/2, values
    // 32*(t%2) .. +31 of the 64-value step, and dequantises block t%2 of weight row t/2.
    const unsigned ar = tid / 2, ah = tid % 2;
    const bool a_ok = m0 + ar < m, b_ok = n0 + ar < n;
    const uint16_t* a_src = a + size_t(m0 + (a_ok ? ar : 0)) * k + 32 * ah;
    const uint8_t* b_src = w + size_t(n0 + (b_ok ? ar : 0)) * row_bytes + (ah ? 16 : 0);

    auto load = [&](unsigned step, Stage& s) {
        const uint16_t* pa = a_src + size_t(step) * BK;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            s.a[i] = a_ok ? *reinterpret_cast<const u32x4*>(pa + 8 * i) : u32x4{0, 0, 0, 0};
        const uint8_t* p = b_src + size_t(step) * 36;
        if (b_ok) {
            const u32x4 v = load16(p);
            s.w[0] = v.x, s.w[1] = v.y, s.w[2] = v.z, s.w[3] = v.w;
            s.w[4] = load4(p + 16);
        } else {
            s.w[0] = s.w[1] = s.w[2] = s.w[3] = s.w[4] = 0;
        }
    };
    auto store = [&](unsigned buf, const Stage& s) {
        uint16_t* da = lds_a[buf] + ar * kPitch + 32 * ah;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<u32x4*>(da + 8 * i) = s.a[i];
        unsigned codes[4], d_bits;
        if (ah == 0) {  // block at byte 0: d in bytes 0-1, codes at bytes 2..17
            d_bits = s.w[0] & 0xffffu;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                codes[i] = __builtin_amdgcn_alignbyte(s.w[i + 1], s.w[i], 2);
        } else {  // loaded from byte 16: d in bytes 18-19, codes at bytes 20..35
            d_bits = s.w[0] >> 16;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                codes[i] = s.w[i + 1];
        }
        unsigned vals[16];
        dequant_q4_0(codes, d_bits, vals);
        uint16_t* db = lds_b[buf] + ar * kPitch + 32 * ah;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<u32x4*>(db + 8 * i) =
                u32x4{vals[4 * i], vals[4 * i + 1], vals[4 * i + 2], vals[4 * i + 3]};
    };

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
            acc[i][j] = f32x16{};

    const unsigned wm = (wave / 2) * 64, wn = (wave % 2) * 64;
    const unsigned frag_row = lane % 32, frag_k = 8 * (lane / 32);
    const unsigned steps = k / BK;

    Stage s;
    load(0, s);
    store(0, s);
    __syncthreads();

    for (unsigned step = 0; step < steps; ++step) {
        const unsigned buf = step & 1;
        const bool more = step + 1 < steps;
        if (more)
            load(step + 1, s);
#pragma unroll
        for (unsigned ks = 0; ks < BK; ks += 16) {
            f16x8 af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                af[i] = *reinterpret_cast<const f16x8*>(
                    lds_a[buf] + (wm + 32 * i + frag_row) * kPitch + ks + frag_k);
                bf[i] = *reinterpret_cast<const f16x8*>(
                    lds_b[buf] + (wn + 32 * i + frag_row) * kPitch + ks + frag_k);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (more)
            store(buf ^ 1, s);
        __syncthreads();
    }

    // C fragment: lane holds column lane%32, rows 8*(v/4) + 4*(lane/32) + v%4.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const unsigned col = n0 + wn + 32 * j + lane % 32;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const unsigned row = m0 + wm + 32 * i + 8 * (v / 4) + 4 * (lane / 32) + v % 4;
                if (row < m && col < n)
                    y[size_t(row) * n + col] = __builtin_bit_cast(uint16_t, _Float16(acc[i][j][v]));
            }
        }
}

int launch_quantize(const uint16_t* x, size_t m, size_t k, int8_t* q, float* d,
                    uint16_t* dequant, hipStream_t stream) {
    const size_t threads = m * k / 8;
    hipLaunchKernelGGL(quantize_kernel, dim3(unsigned((threads + 255) / 256)), dim3(256), 0,
                       stream, x, m * k, q, d, dequant);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}

}  // namespace
}  // namespace kdq

using namespace kdq;

extern "C" int kdq_quantize_q8(const uint16_t* x_f16, size_t m, size_t k, int8_t* q, float* d,
                               void* stream) {
    if (!x_f16 || !q || !d || !m || !k)
        return KDQ_ERR_ARGUMENT;
    if (k % 32 || mul_overflows(m, k) || m * k / 8 > 0x7fffffffull * 256)
        return KDQ_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(x_f16) % 16 || reinterpret_cast<uintptr_t>(q) % 8)
        return KDQ_ERR_ALIGNMENT;
    return launch_quantize(x_f16, m, k, q, d, nullptr, static_cast<hipStream_t>(stream));
}

extern "C" int kdq_gemm_q4_0(const void* weights, size_t n, size_t k, const uint16_t* x_f16,
                             size_t m, uint16_t* y_f16, void* stream) {
    if (!weights || !x_f16 || !y_f16 || !m || !n || !k)
        return KDQ_ERR_ARGUMENT;
    if (k % 256 || m > 0xffffffu || n > 0xffffffu || k > 0xffffffu)
        return KDQ_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(x_f16) % 16 || reinterpret_cast<uintptr_t>(weights) % 4)
        return KDQ_ERR_ALIGNMENT;
    if (overlaps(y_f16, m * n * 2, x_f16, m * k * 2) ||
        overlaps(y_f16, m * n * 2, weights, n * (k / 32) * 18))
        return KDQ_ERR_ALIAS;
    // workspace: int8 codes, fp32 scales, fp16 dequantised activations
    int rc;
    const size_t codes = (m * k + 255) & ~size_t(255), scales = (m * k / 32 * 4 + 255) & ~size_t(255);
    auto* base = static_cast<uint8_t*>(workspace(codes + scales + m * k * 2, &rc));
    if (rc)
        return rc;
    auto st = static_cast<hipStream_t>(stream);
    rc = launch_quantize(x_f16, m, k, reinterpret_cast<int8_t*>(base),
                         reinterpret_cast<float*>(base + codes),
                         reinterpret_cast<uint16_t*>(base + codes + scales), st);
    if (rc)
        return rc;
    const unsigned tiles = unsigned(((m + BM - 1) / BM) * ((n + BN - 1) / BN));
    const unsigned grid = (tiles + 7) / 8 * 8;
    hipLaunchKernelGGL(gemm_kernel, dim3(grid), dim3(256), 0, st,
                       reinterpret_cast<const uint16_t*>(base + codes + scales),
                       static_cast<const uint8_t*>(weights), unsigned(m), unsigned(n),
                       unsigned(k), y_f16);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}
