// GGUF block-quantized decode and decode-time products for gfx950: Q8_0, Q4_0, Q4_K on
// every kernel below; Q3_K, Q6_K, IQ4_NL, IQ4_XS and the lattice encodings IQ3_XXS, IQ3_S,
// IQ2_S on decode_kernel, exact_gemv and mfma_gemv; BF16 on decode_kernel and
// exact_gemv.  Replaces the reference's gguf_decode_kernel and gguf_matvec_kernel
// (IW/src/cuda/h3_compute.cu:76-95,165-240; IW = services/hikari/inference_worker)
// behind the C ABI of include/kadan_amd.h.
//
// Kernels:
//   decode_kernel   exact decode of packed rows to fp32 (one thread per run of 8)
//   exact_gemv      exactly decoded weights x fp32 inputs, fp32 FMA chain, one
//                   wavefront per output (the reference semantics, wave64)
//   fast_gemv       HBM-streaming product: 1024-thread workgroups stage the
//                   activation rows in LDS as 16-bit block fixed point (two int8
//                   planes per 32 values), every lane owns 64 consecutive weights of
//                   a row (one Q4_K sub-block pair, or two Q8_0/Q4_0 blocks), loads
//                   them with 16-byte loads, multiplies with v_dot4_i32_i8 and
//                   applies the per-32 weight and activation scales in fp32.
#include "kdq_common.hpp"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <type_traits>
#include <vector>

namespace kdq {
namespace {

#include "kdq_decode.hpp"

template <int ENC>
__global__ __launch_bounds__(256) void decode_kernel(const uint8_t* packed, size_t row_bytes,
                                                     size_t rows, size_t in, float* out,
                                                     unsigned* status) {
    using F = Format<ENC>;
    const size_t runs = in / 8;
    const size_t t = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    bool bad = false;
    if (t < rows * runs) {
        const size_t row = t / runs, e0 = (t % runs) * 8;
        float v[8];
        decode_run<ENC>(packed + row * row_bytes + (e0 / F::values) * F::bytes,
                        unsigned(e0 % F::values), v);
        float4* o = reinterpret_cast<float4*>(out + row * in + e0);
        o[0] = make_float4(v[0], v[1], v[2], v[3]);
        o[1] = make_float4(v[4], v[5], v[6], v[7]);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            bad |= !isfinite(v[i]);
    }
    if (status && __any(bad) && (threadIdx.x % 64) == 0)
        atomicOr(status, 1u);
}

// ------------------------------------------------------------- exact GEMV

// `index` (optional): the weights start at weights + min(*index, index_limit - 1) *
// index_stride (the expert a device-side routing chose); a job whose index is negative
// is skipped (an unused item of a grouped launch sized for the most items).
template <int ENC, int ROWS>
__global__ __launch_bounds__(256) void exact_gemv(const uint8_t* weights, size_t row_bytes,
                                                  const float* x, unsigned rows, unsigned in,
                                                  unsigned out, float* y, size_t stride,
                                                  unsigned* status, const int32_t* index,
                                                  size_t index_stride, unsigned index_limit,
                                                  size_t x_step, size_t y_step, unsigned x_every) {
    using F = Format<ENC>;
    const unsigned column = blockIdx.x * 4 + threadIdx.x / 64;
    const unsigned lane = threadIdx.x % 64;
    if (column >= out)
        return;
    // job blockIdx.y of an affine batch: its input (every x_every jobs), output and expert
    // index step along
    x += (blockIdx.y / x_every) * x_step;
    y += blockIdx.y * y_step;
    if (index) {
        const int e = index[blockIdx.y];
        if (e < 0)
            return;
        weights += size_t(min(unsigned(e), index_limit - 1)) * index_stride;
    }
    const uint8_t* row = weights + size_t(column) * row_bytes;
    float sums[ROWS] = {};
    bool finite = true;
    for (unsigned i = lane * 8; i < in; i += 64 * 8) {
        float w[8];
        decode_run<ENC>(row + size_t(i / F::values) * F::bytes, i % F::values, w);
#pragma unroll
        for (int k = 0; k < 8; ++k)
            finite = finite && isfinite(w[k]);
#pragma unroll
        for (unsigned r = 0; r < ROWS; ++r)
            if (ROWS == 1 || r < rows) {
                const float* xr = x + size_t(r) * in + i;
                float s = sums[r];
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    s = fmaf(w[k], xr[k], s);
                sums[r] = s;
            }
    }
    if (status && __any(!finite) && lane == 0)
        atomicOr(status, 1u);
#pragma unroll
    for (unsigned r = 0; r < ROWS; ++r) {
        if (ROWS > 1 && r >= rows)
            break;
        const float s = wave_sum(sums[r]);
        if (lane == 0)
            y[size_t(r) * stride + column] = s;
    }
}

// -------------------------------------------------------------- fast GEMV

constexpr int kThreads = 1024, kWaves = 16;
constexpr int kSlot = 64;         // weights per lane per row step
constexpr int kWindow = 64 * kSlot;  // weights per wavefront per row step
// LDS bytes per staged slot: 128 bytes of hi/lo planes padded to 144, so that 16-byte
// reads by consecutive lanes (stride 144 = 36 banks) touch every bank once per pass,
// plus the slot's 16 bytes of scales and sums.
constexpr int kXPitch = 144;
constexpr int kSlotLds = kXPitch + 16;

// LDS byte offset, inside one 128-byte slot, of the (hi, lo) dword pair holding the
// four activation values that start at position p (p % 4 == 0) of the slot.  The
// pairing follows how each format's packed dwords expand: pair m holds values A
// (read against the low nibbles / first dword) and B (high nibbles / second dword).
template <int ENC> __device__ __forceinline__ unsigned pair_offset(unsigned p) {
    unsigned m, which;
    if constexpr (ENC == KDQ_Q4_K) {  // sub-block pair: A = first 32, B = second 32
        which = p >= 32;
        m = (p % 32) / 4;
    } else if constexpr (ENC == KDQ_Q4_0) {  // per block: A = values 0..15, B = 16..31
        const unsigned q = p % 32;
        which = q >= 16;
        m = (p / 32) * 4 + (q % 16) / 4;
    } else {  // Q8_0: A, B = consecutive dwords of codes
        m = p / 8;
        which = (p / 4) % 2;
    }
    return m * 16 + which * 8;
}

// Quantizes R activation rows into LDS:
//   xq[(r*slots + slot)*kXPitch + ...]  hi/lo int8 planes in pair order
//   xs[r*slots + slot] = (s0, sum0, s1, sum1) for the slot's two 32-value groups
// x_q = round(x * 32639 / amax) split as x_q = 256*hi + lo, hi, lo in int8.
// A unit is 8 consecutive values of one row; unit u is row u / (in/8).
struct XUnit {
    float4 a, b;
};

__device__ __forceinline__ void load_unit(const float* x, unsigned in, unsigned u, XUnit& v) {
    const unsigned r = u / (in / 8), e = (u % (in / 8)) * 8;
    const float4* src = reinterpret_cast<const float4*>(x + size_t(r) * in + e);
    v.a = src[0];
    v.b = src[1];
}

// Every thread of a group of four (one 32-value group) must call this together.
template <int ENC>
__device__ __forceinline__ void stage_unit(unsigned in, unsigned u, const XUnit& xu,
                                           uint8_t* xq, float* xs) {
    const unsigned slots = in / kSlot;
    const unsigned r = u / (in / 8), e = (u % (in / 8)) * 8;
    const float v[8] = {xu.a.x, xu.a.y, xu.a.z, xu.a.w, xu.b.x, xu.b.y, xu.b.z, xu.b.w};
    float amax = 0.f, sum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        amax = fmaxf(amax, fabsf(v[i]));
        sum += v[i];
    }
    bool finite = true;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        finite = finite && isfinite(v[i]);
    // four consecutive threads (one DPP quad) hold one 32-value group
    amax = fmaxf(amax, quad_xor1(amax));
    amax = fmaxf(amax, quad_xor2(amax));
    sum += quad_xor1(sum);
    sum += quad_xor2(sum);
    int ok = finite;
    ok &= quad_xor1(ok);
    ok &= quad_xor2(ok);
    finite = ok != 0;
    const float inv = amax > 0.f ? 32639.0f / amax : 0.f;
    const float scale = finite ? amax / 32639.0f : __builtin_nanf("");
    unsigned hi[2] = {0, 0}, lo[2] = {0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        int q = __float2int_rn(v[i] * inv);
        q = min(32639, max(-32639, q));
        const int h = (q + 128) >> 8;
        const int l = q - h * 256;
        hi[i / 4] |= (unsigned(h) & 255u) << (8 * (i % 4));
        lo[i / 4] |= (unsigned(l) & 255u) << (8 * (i % 4));
    }
    const unsigned slot = e / kSlot, p = e % kSlot;
    uint8_t* base = xq + (size_t(r) * slots + slot) * kXPitch;
    *reinterpret_cast<uint2*>(base + pair_offset<ENC>(p)) = make_uint2(hi[0], lo[0]);
    *reinterpret_cast<uint2*>(base + pair_offset<ENC>(p + 4)) = make_uint2(hi[1], lo[1]);
    if ((u & 3u) == 0)
        *reinterpret_cast<float2*>(xs + (size_t(r) * slots + slot) * 4 + (p / 32) * 2) =
            make_float2(scale, sum);
}

// Packed weights of one lane for one row step.  Ordinary loads: in the row-major
// layout the two code loads of a lane each use half of the same 128-byte lines, and the
// non-temporal policy would drop the lines between them (measured 9.4 -> 12.4 us at C2).
struct Lane {
    unsigned w[19];
};

template <int ENC>
__device__ __forceinline__ void load_lane(const uint8_t* row, unsigned slot, Lane& L) {
    if constexpr (ENC == KDQ_Q4_K) {
        const uint8_t* block = row + size_t(slot / 4) * 144;
        const unsigned pair = slot % 4;
        const u32x4 h = load16(block);
        const u32x4 q0 = load16(block + 16 + 32 * pair);
        const u32x4 q1 = load16(block + 32 + 32 * pair);
        L.w[0] = h.x, L.w[1] = h.y, L.w[2] = h.z, L.w[3] = h.w;
        L.w[4] = q0.x, L.w[5] = q0.y, L.w[6] = q0.z, L.w[7] = q0.w;
        L.w[8] = q1.x, L.w[9] = q1.y, L.w[10] = q1.z, L.w[11] = q1.w;
    } else if constexpr (ENC == KDQ_Q4_0) {
        const uint8_t* p = row + size_t(slot) * 36;
        const u32x4 a = load16(p), b = load16(p + 16);
        L.w[0] = a.x, L.w[1] = a.y, L.w[2] = a.z, L.w[3] = a.w;
        L.w[4] = b.x, L.w[5] = b.y, L.w[6] = b.z, L.w[7] = b.w;
        L.w[8] = load4(p + 32);
    } else {
        const uint8_t* p = row + size_t(slot) * 68;
        const u32x4 a = load16(p), b = load16(p + 16), c = load16(p + 32), d = load16(p + 48);
        L.w[0] = a.x, L.w[1] = a.y, L.w[2] = a.z, L.w[3] = a.w;
        L.w[4] = b.x, L.w[5] = b.y, L.w[6] = b.z, L.w[7] = b.w;
        L.w[8] = c.x, L.w[9] = c.y, L.w[10] = c.z, L.w[11] = c.w;
        L.w[12] = d.x, L.w[13] = d.y, L.w[14] = d.z, L.w[15] = d.w;
        L.w[16] = load4(p + 64);
    }
}

// IQ4_XS (136-byte super-block: d, scales_h, scales_l[4], qs[128]; G/src/ggml-common.h
// block_iq4_xs): chunk G is blocks 2G, 2G+1, whose indices lie as Q4_0's codes (16 bytes
// a block, positions 0..15 low nibbles, 16..31 high).  Image: w[0..3], w[4..7] = the two
// blocks' 16 index bytes, w[8] = d | scales_h << 16, w[9] = scales_l.
__device__ __forceinline__ void load_lane_iq4xs(const uint8_t* row, unsigned group, unsigned G,
                                                Lane& L) {
    const uint8_t* block = row + size_t(group) * 136;
    const u32x4 a = load16(block + 8 + 32 * G), b = load16(block + 24 + 32 * G);
    const uint2 h = *reinterpret_cast<const uint2*>(block);
    L.w[0] = a.x, L.w[1] = a.y, L.w[2] = a.z, L.w[3] = a.w;
    L.w[4] = b.x, L.w[5] = b.y, L.w[6] = b.z, L.w[7] = b.w;
    L.w[8] = h.x, L.w[9] = h.y;
}

// Q3_K (110-byte super-block: hmask[32], qs[64], 12 packed 6-bit scales, f16 d;
// G/src/ggml-common.h block_q3_K).  Position 128n + 32j + l holds 2-bit field j of
// qs[32n + l] and bit 4n + j of hmask[l], scale 8n + 2j + l/16.  MFMA chunk G = 2n + p
// takes fields j = 2p (block 0) and 2p + 1 (block 1), scales 4G .. 4G+3.  Image:
// w[0..7] = qs[32n .. 32n+31], w[8..15] = hmask, w[16] = scale bytes 4p .. 4p+3 (low
// nibbles of scales 4G.. when n = 0, high nibbles when n = 1), w[17] = scale bytes 8..11
// (the high bit pairs), w[18] = bytes 106..109 (d in the high half; a load ending inside
// the block).
__device__ __forceinline__ void load_lane_q3k(const uint8_t* row, unsigned group, unsigned G,
                                              Lane& L) {
    const uint8_t* block = row + size_t(group) * 110;
    const unsigned n = G / 2, p = G % 2;
    const u32x4 a = load16_a2(block + 32 + 32 * n), b = load16_a2(block + 48 + 32 * n);
    const u32x4 c = load16_a2(block), d = load16_a2(block + 16);
    L.w[0] = a.x, L.w[1] = a.y, L.w[2] = a.z, L.w[3] = a.w;
    L.w[4] = b.x, L.w[5] = b.y, L.w[6] = b.z, L.w[7] = b.w;
    L.w[8] = c.x, L.w[9] = c.y, L.w[10] = c.z, L.w[11] = c.w;
    L.w[12] = d.x, L.w[13] = d.y, L.w[14] = d.z, L.w[15] = d.w;
    L.w[16] = load4_a2(block + 96 + 4 * p);
    L.w[17] = load4_a2(block + 104);
    L.w[18] = load4_a2(block + 106);
}

// IQ3_XXS (98-byte super-block: f16 d, 64 grid-index bytes, 8 sign-and-scale words;
// G/src/ggml-common.h block_iq3_xxs).  Block k (32 values) has index bytes 8k .. 8k+7
// (byte i: positions 4i .. 4i+3) and word k of the tail: four 7-bit sign sets (set i:
// positions 8i .. 8i+7, eighth sign their parity) and a 4-bit scale on top.  MFMA chunk
// G is blocks 2G, 2G+1.  Image: w[0..3] = the two blocks' index bytes, w[4], w[5] = their
// words, w[6] = bytes 0..3 (d in the low half).
__device__ __forceinline__ void load_lane_iq3xxs(const uint8_t* row, unsigned group, unsigned G,
                                                 Lane& L) {
    const uint8_t* block = row + size_t(group) * 98;
    const u32x4 a = load16_a2(block + 2 + 16 * G);
    const uint2 s = load8_a2(block + 66 + 8 * G);
    L.w[0] = a.x, L.w[1] = a.y, L.w[2] = a.z, L.w[3] = a.w;
    L.w[4] = s.x, L.w[5] = s.y;
    L.w[6] = load4_a2(block);
}

// IQ3_S (110-byte super-block: f16 d, qs[64] low index bits, qh[8], signs[32], scales[4];
// G/src/ggml-common.h block_iq3_s).  Block k has index bytes 8k .. 8k+7 (byte i:
// positions 4i .. 4i+3, bit 8 of the index in bit i of qh[k]), sign bytes 4k .. 4k+3
// (byte i: positions 8i .. 8i+7) and scale nibble k (low nibble of scales[k/2] for even
// k).  Image for chunk G: w[0..3] = the two blocks' index bytes, w[4], w[5] = their sign
// bytes, w[6] = bytes 0..3 (d low), w[7] = bytes 66+2G .. 69+2G (their qh bytes low),
// w[8] = the four scale bytes.
__device__ __forceinline__ void load_lane_iq3s(const uint8_t* row, unsigned group, unsigned G,
                                               Lane& L) {
    const uint8_t* block = row + size_t(group) * 110;
    const u32x4 a = load16_a2(block + 2 + 16 * G);
    const uint2 s = load8_a2(block + 74 + 8 * G);
    L.w[0] = a.x, L.w[1] = a.y, L.w[2] = a.z, L.w[3] = a.w;
    L.w[4] = s.x, L.w[5] = s.y;
    L.w[6] = load4_a2(block);
    L.w[7] = load4_a2(block + 66 + 2 * G);
    L.w[8] = load4_a2(block + 106);
}

// IQ2_S (82-byte super-block: f16 d, qs[32] low index bits, signs[32], qh[8], scales[8];
// G/src/ggml-common.h block_iq2_s).  Block k has index bytes 4k .. 4k+3 (byte i:
// positions 8i .. 8i+7, bits 8, 9 of the index in bits 2i, 2i+1 of qh[k]), sign bytes
// 32 + 4k .. (byte i: positions 8i .. 8i+7) and scales[k] (low nibble: positions 0..15,
// high: 16..31).  Image for chunk G: w[0], w[1] = the two blocks' index bytes, w[2],
// w[3] = their sign bytes, w[4] = bytes 66+2G .. (their qh bytes low), w[5] = scale bytes
// 74 + 4(G/2) .. (theirs at byte 2(G%2)), w[6] = bytes 0..3 (d low).  Every load ends
// inside the super-block.
__device__ __forceinline__ void load_lane_iq2s(const uint8_t* row, unsigned group, unsigned G,
                                               Lane& L) {
    const uint8_t* block = row + size_t(group) * 82;
    const uint2 q = load8_a2(block + 2 + 8 * G), s = load8_a2(block + 34 + 8 * G);
    L.w[0] = q.x, L.w[1] = q.y, L.w[2] = s.x, L.w[3] = s.y;
    L.w[4] = load4_a2(block + 66 + 2 * G);
    L.w[5] = load4_a2(block + 74 + 4 * (G / 2));
    L.w[6] = load4_a2(block);
}

// Four IQ4 indices (bits 0-3 of each byte of n; bits 4-7 ignored) -> their int8 grid
// values: v_perm looks up indices 0-7 and 8-15 in the grid's four words, a third v_perm
// keeps per byte the one its index's bit 3 names.
__device__ __forceinline__ unsigned iq4_grid4(unsigned n) {
    const unsigned sel = n & 0x07070707u;
    const unsigned lo = __builtin_amdgcn_perm(0xf6eaddcfu, 0xbfad9881u, sel);
    const unsigned hi = __builtin_amdgcn_perm(0x71594535u, 0x26190d01u, sel);
    return __builtin_amdgcn_perm(hi, lo, 0x03020100u | ((n >> 1) & 0x04040404u));
}

// Q6_K (210-byte super-block: ql[128] low nibbles, qh[64] high bit pairs, 16 int8
// scales, f16 d; G/src/ggml-common.h block_q6_K).  MFMA chunk G = 2h + p of super-block
// `group` takes both nibbles of ql[32G .. 32G+31]: its block 0 is super-block positions
// 128h + 32p + t (low nibble, qh[32h + t] bits 2p, 2p+1; scales 8h + 2p + t/16), its
// block 1 positions 128h + 64 + 32p + t (high nibble, qh bits 4 + 2p, 5 + 2p; scales
// 8h + 4 + 2p + t/16).  Image: w[0..7] = the lane's 32 ql bytes, w[8..15] = qh[32h ..
// 32h+31], w[16..17] = scales 8h .. 8h+7, w[18] = bytes 206..209 (d in the high half).
__device__ __forceinline__ void load_lane_q6k(const uint8_t* row, unsigned group, unsigned G,
                                              Lane& L) {
    const uint8_t* block = row + size_t(group) * 210;
    const unsigned h = G / 2;
    const u32x4 a = load16_a2(block + 32 * G), b = load16_a2(block + 32 * G + 16);
    const u32x4 c = load16_a2(block + 128 + 32 * h), d = load16_a2(block + 144 + 32 * h);
    const uint2 sc = load8_a2(block + 192 + 8 * h);
    L.w[0] = a.x, L.w[1] = a.y, L.w[2] = a.z, L.w[3] = a.w;
    L.w[4] = b.x, L.w[5] = b.y, L.w[6] = b.z, L.w[7] = b.w;
    L.w[8] = c.x, L.w[9] = c.y, L.w[10] = c.z, L.w[11] = c.w;
    L.w[12] = d.x, L.w[13] = d.y, L.w[14] = d.z, L.w[15] = d.w;
    L.w[16] = sc.x, L.w[17] = sc.y;
    L.w[18] = load4_a2(block + 206);
}

struct XSlot {
    u32x4 q[8];
    float4 s;
};

__device__ __forceinline__ void load_x(const uint8_t* xq, const float* xs, size_t index,
                                       XSlot& X) {
    const u32x4* q = reinterpret_cast<const u32x4*>(xq + index * kXPitch);
#pragma unroll
    for (int m = 0; m < 8; ++m)
        X.q[m] = q[m];
    X.s = reinterpret_cast<const float4*>(xs)[index];
}

// Contribution of one lane's 64 weights against one activation slot; sets `bad`
// when a block scale is not finite (then some decoded weight is not finite).
template <int ENC>
__device__ __forceinline__ float lane_dot(const Lane& L, unsigned slot, const XSlot& X,
                                          bool& bad) {
    if constexpr (ENC == KDQ_Q4_K) {
        const float d = half_hw(L.w[0] & 0xffffu), dmin = half_hw(L.w[0] >> 16);
        bad |= !isfinite(d) || !isfinite(dmin);
        // sub-blocks ga = 2*pair and gb = 2*pair + 1 of the block
        const unsigned pair = slot % 4;
        const unsigned shift = 8 * ((2 * pair) & 3);
        const unsigned b1 = L.w[1] >> shift, b2 = L.w[2] >> shift, b3 = L.w[3] >> shift;
        unsigned sca, ma, scb, mb;
        if (pair < 2) {
            sca = b1 & 63u, ma = b2 & 63u;
            scb = (b1 >> 8) & 63u, mb = (b2 >> 8) & 63u;
        } else {
            sca = (b3 & 15u) | ((b1 >> 2) & 48u);
            ma = ((b3 >> 4) & 15u) | ((b2 >> 2) & 48u);
            scb = ((b3 >> 8) & 15u) | ((b1 >> 10) & 48u);
            mb = ((b3 >> 12) & 15u) | ((b2 >> 10) & 48u);
        }
        int ah = 0, al = 0, bh = 0, bl = 0;
#pragma unroll
        for (int m = 0; m < 8; ++m) {
            const unsigned q = L.w[4 + m];
            const unsigned lo4 = q & 0x0f0f0f0fu, hi4 = (q >> 4) & 0x0f0f0f0fu;
            ah = sdot4(lo4, X.q[m].x, ah);
            al = sdot4(lo4, X.q[m].y, al);
            bh = sdot4(hi4, X.q[m].z, bh);
            bl = sdot4(hi4, X.q[m].w, bl);
        }
        const float A = float(ah * 256 + al), B = float(bh * 256 + bl);
        const float fa = d * float(sca), fb = d * float(scb);
        const float oa = dmin * float(ma), ob = dmin * float(mb);
        float acc = fa * (X.s.x * A);
        acc = fmaf(fb, X.s.z * B, acc);
        acc = fmaf(-oa, X.s.y, acc);
        return fmaf(-ob, X.s.w, acc);
    } else if constexpr (ENC == KDQ_Q4_0) {
        const float d0 = half_hw(L.w[0] & 0xffffu), d1 = half_hw(L.w[4] >> 16);
        bad |= !isfinite(d0) || !isfinite(d1);
        int h0 = 0, l0 = 0, h1 = 0, l1 = 0;
#pragma unroll
        for (int m = 0; m < 4; ++m) {  // block 0 codes start 2 bytes into dword 0
            const unsigned q = __builtin_amdgcn_alignbyte(L.w[m + 1], L.w[m], 2);
            const unsigned lo4 = q & 0x0f0f0f0fu, hi4 = (q >> 4) & 0x0f0f0f0fu;
            h0 = sdot4(lo4, X.q[m].x, h0);
            l0 = sdot4(lo4, X.q[m].y, l0);
            h0 = sdot4(hi4, X.q[m].z, h0);
            l0 = sdot4(hi4, X.q[m].w, l0);
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {  // block 1 codes are dword aligned
            const unsigned q = L.w[5 + m];
            const unsigned lo4 = q & 0x0f0f0f0fu, hi4 = (q >> 4) & 0x0f0f0f0fu;
            h1 = sdot4(lo4, X.q[4 + m].x, h1);
            l1 = sdot4(lo4, X.q[4 + m].y, l1);
            h1 = sdot4(hi4, X.q[4 + m].z, h1);
            l1 = sdot4(hi4, X.q[4 + m].w, l1);
        }
        // sum (q - 8) x = s * sum q x_q - 8 * sum x
        const float t0 = fmaf(X.s.x, float(h0 * 256 + l0), -8.f * X.s.y);
        const float t1 = fmaf(X.s.z, float(h1 * 256 + l1), -8.f * X.s.w);
        return fmaf(d1, t1, d0 * t0);
    } else {
        const float d0 = half_hw(L.w[0] & 0xffffu), d1 = half_hw(L.w[8] >> 16);
        bad |= !isfinite(d0) || !isfinite(d1);
        int h0 = 0, l0 = 0, h1 = 0, l1 = 0;
#pragma unroll
        for (int m = 0; m < 4; ++m) {  // block 0 codes start 2 bytes into dword 0
            const unsigned a = __builtin_amdgcn_alignbyte(L.w[2 * m + 1], L.w[2 * m], 2);
            const unsigned b = __builtin_amdgcn_alignbyte(L.w[2 * m + 2], L.w[2 * m + 1], 2);
            h0 = sdot4(a, X.q[m].x, h0);
            l0 = sdot4(a, X.q[m].y, l0);
            h0 = sdot4(b, X.q[m].z, h0);
            l0 = sdot4(b, X.q[m].w, l0);
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {  // block 1 codes are dwords 9..16
            const unsigned a = L.w[9 + 2 * m], b = L.w[10 + 2 * m];
            h1 = sdot4(a, X.q[4 + m].x, h1);
            l1 = sdot4(a, X.q[4 + m].y, l1);
            h1 = sdot4(b, X.q[4 + m].z, h1);
            l1 = sdot4(b, X.q[4 + m].w, l1);
        }
        return fmaf(d1 * X.s.z, float(h1 * 256 + l1), d0 * X.s.x * float(h0 * 256 + l0));
    }
}

// Rows whose packed weights are loaded before any of them is reduced.
template <int R> constexpr int rows_in_flight = R == 1 ? 4 : 2;

// Packed weights of the rows base, base + stride, ... (kRows of them, those below r1).
template <int ENC, int kRows>
__device__ __forceinline__ void load_rows(const uint8_t* weights, size_t row_bytes,
                                          unsigned base, unsigned stride, unsigned r1,
                                          unsigned slot, bool active, Lane (&L)[kRows]) {
#pragma unroll
    for (int u = 0; u < kRows; ++u) {
        const unsigned n = base + u * stride;
        if (active && n < r1)
            load_lane<ENC>(weights + size_t(n) * row_bytes, slot, L[u]);
    }
}

// Workgroup: 16 wavefronts, one workgroup per compute unit.  The row is cut into `nw`
// windows of 4096 values (nw divides 16); wavefront w takes window w % nw of the rows
// r0 + w/nw, r0 + w/nw + 16/nw, ...  in [r0, r0 + rows_per_wg).  With nw > 1 the window
// partials meet in LDS and are summed in window order.  The first rows' packed weights
// are requested before the activations are staged, so their HBM latency overlaps the
// staging instead of following it.
template <int ENC, int R>
__global__ __launch_bounds__(kThreads) void fast_gemv(const uint8_t* __restrict__ weights,
                                                      size_t row_bytes, const float* x,
                                                      unsigned in, unsigned out,
                                                      float* __restrict__ y, size_t stride,
                                                      unsigned* status, unsigned rows_per_wg,
                                                      unsigned nw) {
    extern __shared__ __align__(16) uint8_t lds[];
    const unsigned slots = in / kSlot;
    uint8_t* xq = lds;
    float* xs = reinterpret_cast<float*>(lds + size_t(R) * slots * kXPitch);
    float* partial = xs + size_t(R) * slots * 4;

    const unsigned wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const unsigned window = wave % nw, groups = kWaves / nw, group = wave / nw;
    const unsigned slot = window * 64 + lane;
    const bool active = slot < slots;
    const unsigned r0 = blockIdx.x * rows_per_wg;
    const unsigned r1 = min(out, r0 + rows_per_wg);
    constexpr int kRowsInFlight = rows_in_flight<R>;
    bool bad = false;

    // Load order: this thread's first activation unit, then the first rows' packed
    // weights, then the staging that uses the activations.  Both load sets are issued
    // by every lane unconditionally (indices past the end are clamped to valid data),
    // so the wait before the staging counts exactly the weight loads and does not wait
    // for them.
    const unsigned units = R * in / 8;
    XUnit first_unit;
    load_unit(x, in, min(unsigned(threadIdx.x), units - 1), first_unit);
    asm volatile("" ::: "memory");  // x is not restrict: its loads stay before this point
    __builtin_amdgcn_sched_barrier(0);
    Lane L[kRowsInFlight];
    unsigned base = r0 + group;
#pragma unroll
    for (int u = 0; u < kRowsInFlight; ++u)
        load_lane<ENC>(weights + size_t(min(base + u * groups, r1 - 1)) * row_bytes,
                       min(slot, slots - 1), L[u]);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    if (threadIdx.x < units)
        stage_unit<ENC>(in, threadIdx.x, first_unit, xq, xs);
    for (unsigned u = threadIdx.x + kThreads; u < units; u += kThreads) {
        XUnit more;
        load_unit(x, in, u, more);
        stage_unit<ENC>(in, u, more, xq, xs);
    }
    __syncthreads();

    XSlot X[1];  // single-row passes keep the activation slot in registers
    if constexpr (R == 1) {
        if (active)
#pragma unroll
            for (int r = 0; r < R; ++r)
                load_x(xq, xs, size_t(r) * slots + slot, X[r]);
    }

    for (bool first = true; base < r1; base += kRowsInFlight * groups, first = false) {
        if (!first)
            load_rows<ENC, kRowsInFlight>(weights, row_bytes, base, groups, r1, slot, active, L);
#pragma unroll
        for (int u = 0; u < kRowsInFlight; ++u) {
            const unsigned n = base + u * groups;
            if (n >= r1)
                break;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float v = 0.f;
                if (active) {
                    if constexpr (R == 1) {
                        v = lane_dot<ENC>(L[u], slot, X[0], bad);
                    } else {
                        XSlot Xr;
                        load_x(xq, xs, size_t(r) * slots + slot, Xr);
                        v = lane_dot<ENC>(L[u], slot, Xr, bad);
                    }
                }
                v = wave_total(v);
                if (lane == 0) {
                    if (nw == 1)
                        y[size_t(r) * stride + n] = v;
                    else
                        partial[(size_t(n - r0) * R + r) * nw + window] = v;
                }
            }
        }
    }
    if (status && __any(bad) && lane == 0)
        atomicOr(status, 1u);
    if (nw > 1) {
        __syncthreads();
        const unsigned count = (r1 > r0 ? r1 - r0 : 0) * R;
        for (unsigned t = threadIdx.x; t < count; t += kThreads) {
            float s = 0.f;
            for (unsigned w = 0; w < nw; ++w)
                s += partial[size_t(t) * nw + w];
            const unsigned n = r0 + t / R, r = t % R;
            y[size_t(r) * stride + n] = s;
        }
    }
}

// -------------------------------------------------------------- MFMA GEMV
//
// The product on v_mfma_i32_16x16x64_i8.  One MFMA multiplies a 16 x 64 activation
// operand A by a 64 x 16 weight operand B: the 16 columns of B are 16 weight rows (a
// tile), and its 64 k values are four lane groups G of 16, where group G carries the
// 64-value chunk G of a 256-value group g of the row (Q4_K: the sub-block pair G of the
// super-block; Q8_0 / Q4_0: the block pair 2G, 2G+1).  Within a chunk, block (or
// sub-block) b = 0, 1 holds positions t = 0..31, and MFMA m (0..3) takes positions
// 8m..8m+7 of both: B element e of group G is position 8m + e%8 of block e/8.
// A is block-diagonal: row 4G + 2b + plane carries, in group G's k values of block b,
// the activation codes of plane `plane` (0: high byte, 1: low byte of the 16-bit code);
// so C row 4G + v (v = 2b + plane) of column j is the exact integer sum of block b of
// chunk G of weight row j against one byte plane.  Every lane of C holds useful sums:
// lane l = 16G + j has rows 4G..4G+3 of column j.  Weight scales are applied to those
// integers in fp32, per lane, from the lane's own row header; the 64 per-(row, chunk)
// partials meet in LDS at the end of a pass and are summed in a fixed order.

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kAGroup = 1024;     // LDS bytes of A operands per 256-value group
constexpr int kPartialPitch = 17; // floats per lane in the pass partials (bank spread)

// Tiles of 16 rows per pass, and units (tile, 256-value group) in flight per wavefront:
// two for one activation row (with all of a wavefront's units requested at once, the
// memory system answers them in its own order and the in-order waits make the first
// MFMA wait for most of them).
template <int R> constexpr int mfma_tiles = R >= 4 ? 1 : 4 / R;
template <int ENC, int R>
constexpr int mfma_units = R == 1 ? 2 : (R == 2 ? 2 : 1);

// LDS layout of mfma_gemv (bytes):
//   [0, 1024)                                       zeros (A operand of non-carrier lanes)
//   A table, per batch row r and group g:           kAGroup bytes, entry (m*16 + 4G + v)
//       is the 16-byte A register of MFMA m for lane 16G + 4G + v (v = 2b + plane):
//       bytes 8b..8b+7 hold plane `plane` of positions 8m..8m+7 of block b of chunk
//       4g + G; the other 8 bytes are zero
//   block table, per batch row r and 32-value block: float4 (s, sum x, sum of codes as
//       int bits, sum of the codes of its first 16 values as int bits)
//   partials [R][mats * tiles][64 lanes][kPartialPitch] floats (mats = 2 for paired jobs:
//       the gate tiles, then the up tiles)
//   lookup tables of the lattice encodings (mfma_table_bytes; none for the others)
struct MfmaLds {
    size_t a, blocks, partial, table, total;
};

// The lattice encodings' grids and sign sets: IQ3_XXS 256 entries of 4 values and
// 7-bit sign sets (the eighth sign their parity), IQ3_S 512 entries of 4 values and
// 8-bit sign bytes, IQ2_S 1024 entries of 8 values and 8-bit sign bytes.
__host__ __device__ constexpr unsigned lattice_entries(int encoding) {
    return encoding == KDQ_IQ3_XXS ? 256 : (encoding == KDQ_IQ3_S ? 512 : 1024);
}
__host__ __device__ constexpr unsigned lattice_signs(int encoding) {
    return encoding == KDQ_IQ3_XXS ? 128 : 256;
}
__host__ __device__ constexpr unsigned lattice_width(int encoding) {
    return encoding == KDQ_IQ2_S ? 8 : 4;
}
__host__ __device__ constexpr bool lattice(int encoding) {
    return encoding == KDQ_IQ3_XXS || encoding == KDQ_IQ3_S || encoding == KDQ_IQ2_S;
}

// LDS lookup tables of the lattice encodings: per grid entry its magnitude bytes then
// their negations (8 bytes for 4 values, 16 for 8), then per sign set a pair of v_perm
// selectors (8 bytes).
__host__ __device__ constexpr size_t mfma_table_bytes(int encoding) {
    return lattice(encoding) ? size_t(lattice_entries(encoding)) * 2 * lattice_width(encoding) +
                                   size_t(lattice_signs(encoding)) * 8
                             : 0;
}

__host__ __device__ inline MfmaLds mfma_layout(unsigned batch, unsigned in, unsigned mats = 1,
                                               size_t table = 0) {
    const size_t tiles = (batch >= 4 ? 1 : 4 / batch) * mats;
    MfmaLds l;
    l.a = 1024;
    l.blocks = l.a + size_t(batch) * (in / 256) * kAGroup;
    l.partial = l.blocks + size_t(batch) * (in / 32) * 16;
    l.table = l.partial + size_t(batch) * tiles * 64 * kPartialPitch * 4;
    l.total = l.table + table;
    return l;
}

// The MFMA chunk G and block b (of the chunk) that carry 32-value block k (0..7) of a
// 256-value group: chunk G is blocks 2G, 2G+1, except for Q6_K, whose chunk G = 2h + p
// is blocks 4h + p and 4h + 2 + p (the two nibbles of one run of ql bytes).
template <int ENC> __host__ __device__ __forceinline__ unsigned chunk_of(unsigned k) {
    return ENC == KDQ_Q6_K ? 2 * (k / 4) + k % 2 : k / 2;
}
template <int ENC> __host__ __device__ __forceinline__ unsigned half_of(unsigned k) {
    return ENC == KDQ_Q6_K ? (k / 2) % 2 : k % 2;
}
template <int ENC> __host__ __device__ __forceinline__ unsigned block_of(unsigned G, unsigned b) {
    return ENC == KDQ_Q6_K ? 4 * (G / 2) + 2 * b + G % 2 : 2 * G + b;
}

// Quantizes one unit of 8 activation values (the 16-bit block code of stage_unit) into
// the A table and the block table.  The four threads of a DPP quad hold one block.
template <int ENC>
__device__ __forceinline__ void mstage_unit(unsigned in, unsigned u, const XUnit& xu,
                                            uint8_t* atab, float4* blocks) {
    const unsigned r = u / (in / 8), e0 = (u % (in / 8)) * 8;
    const unsigned k = (e0 % 256) / 32;
    const unsigned g = e0 / 256, G = chunk_of<ENC>(k), b = half_of<ENC>(k), m = (e0 % 32) / 8;
    const float v[8] = {xu.a.x, xu.a.y, xu.a.z, xu.a.w, xu.b.x, xu.b.y, xu.b.z, xu.b.w};
    float amax = 0.f, sum = 0.f;
    int ok = 1;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        amax = fmaxf(amax, fabsf(v[i]));
        sum += v[i];
        ok &= int(isfinite(v[i]));
    }
    amax = fmaxf(amax, quad_xor1(amax));
    amax = fmaxf(amax, quad_xor2(amax));
    sum += quad_xor1(sum);
    sum += quad_xor2(sum);
    ok &= quad_xor1(ok);
    ok &= quad_xor2(ok);
    const float inv = amax > 0.f ? 32639.0f / amax : 0.f;
    const float scale = ok ? amax / 32639.0f : __builtin_nanf("");
    unsigned hi[2] = {0, 0}, lo[2] = {0, 0};
    int codes = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        int q = __float2int_rn(v[i] * inv);
        q = min(32639, max(-32639, q));
        codes += q;
        const int h = (q + 128) >> 8;
        const int l = q - h * 256;
        hi[i / 4] |= (unsigned(h) & 255u) << (8 * (i % 4));
        lo[i / 4] |= (unsigned(l) & 255u) << (8 * (i % 4));
    }
    codes += quad_xor1(codes);
    const int first16 = codes;  // quad threads 0, 1: the block's first 16 values
    codes += quad_xor2(codes);
    uint8_t* entry = atab + (size_t(r) * (in / 256) + g) * kAGroup + (m * 16 + 4 * G + 2 * b) * 16;
    *reinterpret_cast<uint4*>(entry) = b ? make_uint4(0, 0, hi[0], hi[1]) : make_uint4(hi[0], hi[1], 0, 0);
    *reinterpret_cast<uint4*>(entry + 16) =
        b ? make_uint4(0, 0, lo[0], lo[1]) : make_uint4(lo[0], lo[1], 0, 0);
    if (m == 0)
        blocks[size_t(r) * (in / 32) + e0 / 32] =
            make_float4(scale, sum, __int_as_float(codes), __int_as_float(first16));
}

// Tile-packed weights (kdq_gguf_pack), this library's resident GGUF layout.  Rows are
// taken 16 at a time (tile T = rows 16T .. 16T+15, zero rows past the end); the unit of
// tile T and 256-value group g sits at (T * groups + g) * unit bytes and holds, for lane
// l = 16G + s (row slot s = row % 16, 64-value chunk G of the group):
//   code piece p (p < pieces): the 16 bytes at p * 1024 + 16 l
//     Q4_K  pieces 0, 1: code bytes 0..15, 16..31 of sub-block pair G
//     Q4_0  piece c: the 16 code bytes of block 2G + c of the group
//     Q8_0  piece 2c + h: code bytes 16h .. 16h+15 of block 2G + c
//     Q6_K  pieces 0, 1: ql bytes 32G .. 32G+15, 32G+16 .. 32G+31 (chunk G = 2h + p,
//           mfma_gemv's Q6_K chunk map); piece 2: the chunk's qh bit pairs, dword m for
//           positions 8m..8m+7: byte i holds, for position 8m+i in its high nibble and
//           8m+4+i in its low nibble, (block-0 bits) | (block-1 bits) << 2
//   side data at pieces * 1024:
//     Q4_K  the 16-byte block header (d, dmin, scales) of row slot s at + 16 s
//     Q4_0, Q8_0  one dword at + 4 l: d of block 2G | d of block 2G + 1 << 16
//     Q6_K  one dword at + 4 l: the chunk's scales 8h+2p, 8h+2p+1, 8h+4+2p, 8h+5+2p;
//           then at + 256 + 4 (s/2): d of row slots s & ~1 | d of s | 1 << 16
// A wavefront's load of one piece is 1 KB contiguous; the bytes are the row bytes
// reordered (unit = 16 rows x one group's bytes), nothing is added or converted (Q6_K's
// qh bit pairs are regrouped within the unit so that no two lanes load the same byte).
template <int ENC> struct PackedFormat;
template <> struct PackedFormat<KDQ_Q4_K> {
    static constexpr int pieces = 2, unit = 2304;
};
template <> struct PackedFormat<KDQ_Q4_0> {
    static constexpr int pieces = 2, unit = 2304;
};
template <> struct PackedFormat<KDQ_Q8_0> {
    static constexpr int pieces = 4, unit = 4352;
};
template <> struct PackedFormat<KDQ_Q6_K> {
    static constexpr int pieces = 3, unit = 3360;
};

// One lane's chunk from a packed unit, in the register image the packed operand
// functions read: Q4_K exactly as load_lane (w[0..3] header, w[4..11] codes); Q4_0 and
// Q8_0 code pieces in w[0 .. 4*pieces) and the scale dword in w[4*pieces].  The code
// pieces are requested first: the MFMAs need them before the scales.  Non-temporal
// loads: one C2 launch streams 33 MB once (measured 8.44 -> 7.89 us with the nt policy).
template <int ENC>
__device__ __forceinline__ void load_packed(const uint8_t* unit, unsigned G, unsigned s, Lane& L) {
    constexpr int P = PackedFormat<ENC>::pieces;
    const unsigned l = 16 * G + s;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const u32x4 q = stream16(unit + p * 1024 + 16 * l);
        const int at = ENC == KDQ_Q4_K ? 4 + 4 * p : 4 * p;
        L.w[at] = q.x, L.w[at + 1] = q.y, L.w[at + 2] = q.z, L.w[at + 3] = q.w;
    }
    if constexpr (ENC == KDQ_Q4_K) {
        const u32x4 h = stream16(unit + P * 1024 + 16 * s);
        L.w[0] = h.x, L.w[1] = h.y, L.w[2] = h.z, L.w[3] = h.w;
    } else {
        L.w[4 * P] = stream4(unit + P * 1024 + 4 * l);
        if constexpr (ENC == KDQ_Q6_K)
            L.w[4 * P + 1] = stream4(unit + P * 1024 + 256 + 4 * (s / 2));
    }
}

// Magnitude of level index i (0..7) of a lattice encoding's grid.
template <int ENC> __device__ __forceinline__ unsigned lattice_level(unsigned i) {
    if constexpr (ENC == KDQ_IQ3_XXS)
        return i == 7 ? 62u : 8u * i + 4u;
    else if constexpr (ENC == KDQ_IQ3_S)
        return 2u * i + 1u;
    else
        return i == 0 ? 8u : (i == 1 ? 25u : 43u);
}

// The grid entry of index i (lane b, the level index of value b, at bits [w*b, w*b + w),
// w = 3, or 2 for IQ2_S).
template <int ENC> __device__ __forceinline__ unsigned lattice_entry(unsigned i) {
    if constexpr (ENC == KDQ_IQ3_XXS)
        return kIq3xxsGrid[i];
    else if constexpr (ENC == KDQ_IQ3_S)
        return kIq3sGrid[i];
    else
        return kIq2sGrid[i];
}

// Entries of the grid each thread of a kThreads workgroup converts into the LDS table.
template <int ENC, unsigned kThreads>
constexpr unsigned lattice_per_thread = (lattice_entries(ENC) + kThreads - 1) / kThreads;

// Fills a lattice encoding's LDS tables (mfma_table_bytes): thread t converts grid entries
// t, t + kThreads, .. (already read into `entry`) and sign set t.  A selector byte i picks
// byte i of the magnitudes (i) or of their negations (i + 4).
template <int ENC, unsigned kThreads>
__device__ __forceinline__ void lattice_table(uint8_t* table,
                                              const unsigned (&entry)[lattice_per_thread<ENC, kThreads>]) {
    constexpr unsigned E = lattice_entries(ENC), S = lattice_signs(ENC);
    constexpr unsigned bits = ENC == KDQ_IQ2_S ? 2 : 3;
    const unsigned t = threadIdx.x;
#pragma unroll
    for (unsigned k = 0; k < lattice_per_thread<ENC, kThreads>; ++k) {
        const unsigned i = t + k * kThreads;
        if (i >= E)
            break;
        unsigned pos[2] = {0, 0}, neg[2] = {0, 0};
#pragma unroll
        for (unsigned b = 0; b < lattice_width(ENC); ++b) {
            const unsigned level = lattice_level<ENC>((entry[k] >> (bits * b)) & ((1u << bits) - 1));
            pos[b / 4] |= level << (8 * (b % 4));
            neg[b / 4] |= ((256u - level) & 255u) << (8 * (b % 4));
        }
        if constexpr (lattice_width(ENC) == 8)
            reinterpret_cast<uint4*>(table)[i] = make_uint4(pos[0], pos[1], neg[0], neg[1]);
        else
            reinterpret_cast<uint2*>(table)[i] = make_uint2(pos[0], neg[0]);
    }
    uint2* sels = reinterpret_cast<uint2*>(table + size_t(E) * 2 * lattice_width(ENC));
    for (unsigned i = t; i < S; i += kThreads) {
        const unsigned s = ENC == KDQ_IQ3_XXS ? i | ((__builtin_popcount(i) & 1u) << 7) : i;
        unsigned lo = 0, hi = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            lo |= (unsigned(b) + 4u * ((s >> b) & 1u)) << (8 * b);
            hi |= (unsigned(b) + 4u * ((s >> (4 + b)) & 1u)) << (8 * b);
        }
        sels[i] = make_uint2(lo, hi);
    }
}

// B operand of MFMA m from one lane's packed chunk (load_lane layout, or load_packed's
// when PACKED).  `table`: the encoding's LDS lookup tables (IQ3_XXS).
template <int ENC, bool PACKED = false>
__device__ __forceinline__ i32x4 b_operand(const Lane& L, int m, unsigned q6_shift,
                                           const uint8_t* table = nullptr) {
    if constexpr (lattice(ENC)) {
        // positions 8m .. 8m+7 of block b: one 8-value grid entry (IQ2_S) or two 4-value
        // ones, and sign set m; v_perm takes per byte the magnitude or its negation
        const uint2* sels = reinterpret_cast<const uint2*>(
            table + size_t(lattice_entries(ENC)) * 2 * lattice_width(ENC));
        unsigned v[4];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if constexpr (ENC == KDQ_IQ2_S) {
                // index byte m of the block | its qh bits 2m, 2m+1 as bits 8, 9
                const unsigned i = ((L.w[b] >> (8 * m)) & 255u) |
                                   (((L.w[4] >> (8 * b + 2 * m)) & 3u) << 8);
                const uint2 sel = sels[(L.w[2 + b] >> (8 * m)) & 255u];
                const uint4 g = reinterpret_cast<const uint4*>(table)[i];
                v[2 * b] = __builtin_amdgcn_perm(g.z, g.x, sel.x);
                v[2 * b + 1] = __builtin_amdgcn_perm(g.w, g.y, sel.y);
            } else {
                // index bytes 2m, 2m+1 (four positions each); IQ3_S adds their qh bits
                // 2m, 2m+1 as bit 8
                const unsigned idx = L.w[2 * b + m / 2] >> (16 * (m % 2));
                unsigned i0 = idx & 255u, i1 = (idx >> 8) & 255u, sign;
                if constexpr (ENC == KDQ_IQ3_S) {
                    const unsigned qh = L.w[7] >> (8 * b + 2 * m);
                    i0 |= (qh & 1u) << 8;
                    i1 |= (qh & 2u) << 7;
                    sign = (L.w[4 + b] >> (8 * m)) & 255u;
                } else {
                    sign = (L.w[4 + b] >> (7 * m)) & 127u;
                }
                const uint2* grid = reinterpret_cast<const uint2*>(table);
                const uint2 sel = sels[sign];
                const uint2 g0 = grid[i0], g1 = grid[i1];
                v[2 * b] = __builtin_amdgcn_perm(g0.y, g0.x, sel.x);
                v[2 * b + 1] = __builtin_amdgcn_perm(g1.y, g1.x, sel.y);
            }
        }
        return i32x4{int(v[0]), int(v[1]), int(v[2]), int(v[3])};
    } else if constexpr (PACKED && ENC == KDQ_Q6_K) {
        // the qh pairs of positions 8m+i sit in bits 4-7 of byte i of w[8+m], those of
        // 8m+4+i in bits 0-3 (block 0 bits low, block 1 bits high in each nibble)
        const unsigned l0 = L.w[2 * m], l1 = L.w[2 * m + 1], h = L.w[8 + m];
        return i32x4{int((l0 & 0x0f0f0f0fu) | (h & 0x30303030u)),
                     int((l1 & 0x0f0f0f0fu) | ((h << 4) & 0x30303030u)),
                     int(((l0 >> 4) & 0x0f0f0f0fu) | ((h >> 2) & 0x30303030u)),
                     int(((l1 >> 4) & 0x0f0f0f0fu) | ((h << 2) & 0x30303030u))};
    } else if constexpr (ENC == KDQ_Q3_K) {
        // unsigned codes q + 4 (0..7) of positions 8m..8m+7: field 2p (block 0) or 2p+1
        // (block 1) of the qs bytes, hmask bit 2G (or 2G+1) above them; q6_shift = G
        const unsigned G = q6_shift, sq = 4 * (G % 2), sh = 2 * G;
        const unsigned q0 = L.w[2 * m], q1 = L.w[2 * m + 1];
        const unsigned h0 = L.w[8 + 2 * m], h1 = L.w[9 + 2 * m];
        auto code = [](unsigned q, unsigned h, unsigned fq, unsigned fh) {
            return ((q >> fq) & 0x03030303u) | (((h >> fh) & 0x01010101u) << 2);
        };
        return i32x4{int(code(q0, h0, sq, sh)), int(code(q1, h1, sq, sh)),
                     int(code(q0, h0, sq + 2, sh + 1)), int(code(q1, h1, sq + 2, sh + 1))};
    } else if constexpr (ENC == KDQ_IQ4_XS) {
        // the grid values (int8) of the indices of positions 8m..8m+7 of both blocks
        const int k = 2 * (m % 2);
        const unsigned shift = m >= 2 ? 4 : 0;
        return i32x4{int(iq4_grid4(L.w[k] >> shift)), int(iq4_grid4(L.w[k + 1] >> shift)),
                     int(iq4_grid4(L.w[4 + k] >> shift)), int(iq4_grid4(L.w[5 + k] >> shift))};
    } else if constexpr (ENC == KDQ_IQ4_NL) {
        // Q4_0's row-major image (18-byte blocks: d, 16 index bytes), grid values
        const int k = 2 * (m % 2);
        const unsigned shift = m >= 2 ? 4 : 0;
        const unsigned a0 = __builtin_amdgcn_alignbyte(L.w[k + 1], L.w[k], 2);
        const unsigned a1 = __builtin_amdgcn_alignbyte(L.w[k + 2], L.w[k + 1], 2);
        return i32x4{int(iq4_grid4(a0 >> shift)), int(iq4_grid4(a1 >> shift)),
                     int(iq4_grid4(L.w[5 + k] >> shift)), int(iq4_grid4(L.w[6 + k] >> shift))};
    } else if constexpr (ENC == KDQ_Q6_K) {
        // the 6-bit codes (0..63) of positions 8m..8m+7: low nibble | qh bits 2p, 2p+1
        // (block 0), high nibble | qh bits 4+2p, 5+2p (block 1); q6_shift = 2p
        const unsigned l0 = L.w[2 * m], l1 = L.w[2 * m + 1];
        const unsigned h0 = L.w[8 + 2 * m], h1 = L.w[9 + 2 * m];
        const unsigned up = 4 - q6_shift;
        return i32x4{int((l0 & 0x0f0f0f0fu) | ((h0 << up) & 0x30303030u)),
                     int((l1 & 0x0f0f0f0fu) | ((h1 << up) & 0x30303030u)),
                     int(((l0 >> 4) & 0x0f0f0f0fu) | ((h0 >> q6_shift) & 0x30303030u)),
                     int(((l1 >> 4) & 0x0f0f0f0fu) | ((h1 >> q6_shift) & 0x30303030u))};
    } else if constexpr (PACKED && ENC == KDQ_Q8_0) {
        // block 0 codes in w[0..7], block 1 in w[8..15]
        return i32x4{int(L.w[2 * m]), int(L.w[2 * m + 1]), int(L.w[8 + 2 * m]),
                     int(L.w[9 + 2 * m])};
    } else if constexpr (PACKED && ENC == KDQ_Q4_0) {
        // block 0 code bytes in w[0..3], block 1 in w[4..7]; positions 0..15 are low
        // nibbles, 16..31 high nibbles
        const int k = 2 * (m % 2);
        const int shift = m >= 2 ? 4 : 0;
        return i32x4{int((L.w[k] >> shift) & 0x0f0f0f0fu), int((L.w[k + 1] >> shift) & 0x0f0f0f0fu),
                     int((L.w[4 + k] >> shift) & 0x0f0f0f0fu),
                     int((L.w[5 + k] >> shift) & 0x0f0f0f0fu)};
    } else if constexpr (ENC == KDQ_Q4_K) {
        // code bytes 8m..8m+7 of the pair: low nibbles are sub-block 2G (kept as 0..15),
        // high nibbles sub-block 2G+1, kept in place as 16q - 128 (one bit operation)
        const unsigned w0 = L.w[4 + 2 * m], w1 = L.w[5 + 2 * m];
        return i32x4{int(w0 & 0x0f0f0f0fu), int(w1 & 0x0f0f0f0fu),
                     int((w0 & 0xf0f0f0f0u) ^ 0x80808080u),
                     int((w1 & 0xf0f0f0f0u) ^ 0x80808080u)};
    } else if constexpr (ENC == KDQ_Q8_0) {
        // block 0 codes start 2 bytes into dword 0, block 1 codes at dword 9
        return i32x4{int(__builtin_amdgcn_alignbyte(L.w[2 * m + 1], L.w[2 * m], 2)),
                     int(__builtin_amdgcn_alignbyte(L.w[2 * m + 2], L.w[2 * m + 1], 2)),
                     int(L.w[9 + 2 * m]), int(L.w[10 + 2 * m])};
    } else {
        // positions 0..15 are low nibbles of code bytes 0..15, 16..31 high nibbles
        const int k = 2 * (m % 2);
        const unsigned a0 = __builtin_amdgcn_alignbyte(L.w[k + 1], L.w[k], 2);
        const unsigned a1 = __builtin_amdgcn_alignbyte(L.w[k + 2], L.w[k + 1], 2);
        const unsigned c0 = L.w[5 + k], c1 = L.w[6 + k];
        const int shift = m >= 2 ? 4 : 0;
        return i32x4{int((a0 >> shift) & 0x0f0f0f0fu), int((a1 >> shift) & 0x0f0f0f0fu),
                     int((c0 >> shift) & 0x0f0f0f0fu), int((c1 >> shift) & 0x0f0f0f0fu)};
    }
}

// Per-lane constants of the Q4_K scale decode for sub-blocks 2G, 2G+1.
struct ScaleSel {
    unsigned shift;
    bool high;
};

// The chunk's contribution from the four integer sums of this lane (c.x, c.y: block 0
// high and low planes; c.z, c.w: block 1) with the activation block entries x0, x1.
template <int ENC, bool PACKED = false>
__device__ __forceinline__ float chunk_value(const Lane& L, ScaleSel sel, i32x4 c, i32x4 c2,
                                             float4 x0, float4 x1, bool& bad) {
    if constexpr (ENC == KDQ_Q3_K) {
        // scales 4G + t (t = 2b + half): low 4 bits from w[16] (nibble n), high 2 bits
        // from w[17]; sum (q + 4 - 4) x_q per 16 values exact, then (scale - 32) and d
        const unsigned G = sel.shift;
        const float d = half_hw(L.w[18] >> 16);
        bad |= !isfinite(d);
        const unsigned lo = L.w[16] >> (4 * (G / 2)), hi = L.w[17] >> (2 * G);
        auto scale = [&](unsigned t) {
            return float(int(((lo >> (8 * t)) & 15u) | (((hi >> (8 * t)) & 3u) << 4)) - 32);
        };
        const int f0 = __float_as_int(x0.w), f1 = __float_as_int(x1.w);
        const int t0 = __float_as_int(x0.z) - f0, t1 = __float_as_int(x1.z) - f1;
        const float a00 = float(c.x * 256 + c.y - 4 * f0), a01 = float(c2.x * 256 + c2.y - 4 * t0);
        const float a10 = float(c.z * 256 + c.w - 4 * f1), a11 = float(c2.z * 256 + c2.w - 4 * t1);
        const float b0 = fmaf(scale(1), a01, scale(0) * a00);
        const float b1 = fmaf(scale(3), a11, scale(2) * a10);
        return d * fmaf(x1.x, b1, x0.x * b0);
    } else if constexpr (ENC == KDQ_IQ4_NL) {
        const float d0 = half_hw(L.w[0] & 0xffffu), d1 = half_hw(L.w[4] >> 16);
        bad |= !isfinite(d0) || !isfinite(d1);
        const float A0 = float(c.x * 256 + c.y), A1 = float(c.z * 256 + c.w);
        return fmaf(d1 * x1.x, A1, d0 * x0.x * A0);
    } else if constexpr (ENC == KDQ_IQ3_XXS) {
        // block scales d * (0.5 + s) / 2 = d * (2s + 1) / 4, s = bits 28..31 of the
        // block's word
        const float d = half_hw(L.w[6] & 0xffffu);
        bad |= !isfinite(d);
        const float f0 = 0.25f * d * float(2 * (L.w[4] >> 28) + 1);
        const float f1 = 0.25f * d * float(2 * (L.w[5] >> 28) + 1);
        const float A0 = float(c.x * 256 + c.y), A1 = float(c.z * 256 + c.w);
        return fmaf(f1 * x1.x, A1, f0 * x0.x * A0);
    } else if constexpr (ENC == KDQ_IQ3_S) {
        // block scales d * (1 + 2s), s = nibble 2G (block 0), 2G+1 (block 1) of the scale
        // bytes (sel.shift = G)
        const float d = half_hw(L.w[6] & 0xffffu);
        bad |= !isfinite(d);
        const unsigned sc = L.w[8] >> (8 * sel.shift);
        const float f0 = d * float(2 * (sc & 15u) + 1), f1 = d * float(2 * ((sc >> 4) & 15u) + 1);
        const float A0 = float(c.x * 256 + c.y), A1 = float(c.z * 256 + c.w);
        return fmaf(f1 * x1.x, A1, f0 * x0.x * A0);
    } else if constexpr (ENC == KDQ_IQ2_S) {
        // scales d * (0.5 + s) / 4 = d * (2s + 1) / 8 per 16 values: c holds positions
        // 0..15 of each block, c2 16..31; the block's scale byte is byte 2(G%2) + b of w[5]
        const float d = half_hw(L.w[6] & 0xffffu);
        bad |= !isfinite(d);
        const unsigned sc = L.w[5] >> (16 * (sel.shift % 2));
        const float e = 0.125f * d;
        auto f = [&](unsigned n) { return e * float(2 * (n & 15u) + 1); };
        const float a00 = float(c.x * 256 + c.y), a01 = float(c2.x * 256 + c2.y);
        const float a10 = float(c.z * 256 + c.w), a11 = float(c2.z * 256 + c2.w);
        const float b0 = fmaf(f(sc >> 4), a01, f(sc) * a00);
        const float b1 = fmaf(f(sc >> 12), a11, f(sc >> 8) * a10);
        return fmaf(x1.x, b1, x0.x * b0);
    } else if constexpr (ENC == KDQ_IQ4_XS) {
        // block scales d * (ls - 32), ls = 4 bits of scales_l | 2 bits of scales_h << 4
        // (sel.shift = G: blocks 2G, 2G+1)
        const float d = half_hw(L.w[8] & 0xffffu);
        bad |= !isfinite(d);
        const unsigned G = sel.shift, sl = L.w[9] >> (8 * G), sh = L.w[8] >> (16 + 4 * G);
        const int ls0 = int((sl & 15u) | ((sh & 3u) << 4)) - 32;
        const int ls1 = int(((sl >> 4) & 15u) | (((sh >> 2) & 3u) << 4)) - 32;
        const float A0 = float(c.x * 256 + c.y), A1 = float(c.z * 256 + c.w);
        return fmaf(d * float(ls1) * x1.x, A1, d * float(ls0) * x0.x * A0);
    } else if constexpr (ENC == KDQ_Q6_K) {
        // c: positions 0..15 of each block, c2: 16..31; sum (q - 32) x_q per 16 values is
        // an exact integer below 2^24 in magnitude, then the int8 scales and d in fp32
        // row-major image: scales 8h..8h+7 in w[16..17], d high in w[18]; packed: the
        // chunk's four scales in w[12], the d pair of the lane's row slots in w[13]
        // (sel.high: odd row slot)
        const float d = PACKED ? half_hw(L.w[13] >> (sel.high ? 16 : 0)) : half_hw(L.w[18] >> 16);
        bad |= !isfinite(d);
        const unsigned s0 = PACKED ? L.w[12] : L.w[16] >> (8 * sel.shift);
        const unsigned s1 = PACKED ? L.w[12] >> 16 : L.w[17] >> (8 * sel.shift);
        const int f0 = __float_as_int(x0.w), f1 = __float_as_int(x1.w);
        const int t0 = __float_as_int(x0.z) - f0, t1 = __float_as_int(x1.z) - f1;
        const float a00 = float(c.x * 256 + c.y - 32 * f0), a01 = float(c2.x * 256 + c2.y - 32 * t0);
        const float a10 = float(c.z * 256 + c.w - 32 * f1), a11 = float(c2.z * 256 + c2.w - 32 * t1);
        const float b0 = fmaf(float(int8_t(s0 >> 8)), a01, float(int8_t(s0)) * a00);
        const float b1 = fmaf(float(int8_t(s1 >> 8)), a11, float(int8_t(s1)) * a10);
        return d * fmaf(x1.x, b1, x0.x * b0);
    } else if constexpr (PACKED && ENC != KDQ_Q4_K) {
        // the two block scales share one dword after the code pieces
        const unsigned sc = L.w[4 * PackedFormat<ENC>::pieces];
        const float d0 = half_hw(sc & 0xffffu), d1 = half_hw(sc >> 16);
        bad |= !isfinite(d0) || !isfinite(d1);
        const float A0 = float(c.x * 256 + c.y), A1 = float(c.z * 256 + c.w);
        if constexpr (ENC == KDQ_Q4_0) {
            const float t0 = fmaf(x0.x, A0, -8.f * x0.y);
            const float t1 = fmaf(x1.x, A1, -8.f * x1.y);
            return fmaf(d1, t1, d0 * t0);
        } else {
            return fmaf(d1 * x1.x, A1, d0 * x0.x * A0);
        }
    }
    const float A0 = float(c.x * 256 + c.y);
    if constexpr (ENC == KDQ_Q4_K) {
        const float d = half_hw(L.w[0] & 0xffffu), dmin = half_hw(L.w[0] >> 16);
        bad |= !isfinite(d) || !isfinite(dmin);
        const unsigned b1 = L.w[1] >> sel.shift, b2 = L.w[2] >> sel.shift,
                       b3 = L.w[3] >> sel.shift;
        unsigned sca, ma, scb, mb;
        if (!sel.high) {
            sca = b1 & 63u, ma = b2 & 63u;
            scb = (b1 >> 8) & 63u, mb = (b2 >> 8) & 63u;
        } else {
            sca = (b3 & 15u) | ((b1 >> 2) & 48u);
            ma = ((b3 >> 4) & 15u) | ((b2 >> 2) & 48u);
            scb = ((b3 >> 8) & 15u) | ((b1 >> 10) & 48u);
            mb = ((b3 >> 12) & 15u) | ((b2 >> 10) & 48u);
        }
        // block 1 codes entered as 16q - 128: sum q x = (sum (16q - 128) x + 128 sum x) / 16
        const float A1 = float((c.z * 256 + c.w + 128 * __float_as_int(x1.z)) >> 4);
        const float fa = d * float(sca), fb = d * float(scb);
        const float oa = dmin * float(ma), ob = dmin * float(mb);
        float acc = fa * (x0.x * A0);
        acc = fmaf(fb, x1.x * A1, acc);
        acc = fmaf(-oa, x0.y, acc);
        return fmaf(-ob, x1.y, acc);
    } else if constexpr (ENC == KDQ_Q4_0) {
        const float d0 = half_hw(L.w[0] & 0xffffu), d1 = half_hw(L.w[4] >> 16);
        bad |= !isfinite(d0) || !isfinite(d1);
        const float A1 = float(c.z * 256 + c.w);
        // sum (q - 8) x = s * sum q x_q - 8 * sum x
        const float t0 = fmaf(x0.x, A0, -8.f * x0.y);
        const float t1 = fmaf(x1.x, A1, -8.f * x1.y);
        return fmaf(d1, t1, d0 * t0);
    } else {
        const float d0 = half_hw(L.w[0] & 0xffffu), d1 = half_hw(L.w[8] >> 16);
        bad |= !isfinite(d0) || !isfinite(d1);
        const float A1 = float(c.z * 256 + c.w);
        return fmaf(d1 * x1.x, A1, d0 * x0.x * A0);
    }
}

// Sum over each aligned group of 16 lanes (DPP row), returned to every lane of it.
__device__ __forceinline__ float row16_total(float v) {
    v += dpp_read<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]
    v += dpp_read<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]
    v += dpp_read<0x141, 0xf>(v);  // row_half_mirror
    v += dpp_read<0x140, 0xf>(v);  // row_mirror
    return v;
}

// A wavefront's position in its unit sequence: group g = wave + W q, tile t.
struct UnitCursor {
    unsigned g, t;
    __device__ __forceinline__ void next(unsigned tiles, unsigned waves) {
        if (++t == tiles) {
            t = 0;
            g += waves;
        }
    }
};

// Up to kMaxFused products of one shape (encoding, batch rows, in) in one launch: job
// blockIdx.y, output rows blockIdx.x * rows_per_wg .. + rows_per_wg (workgroups past a
// job's rows exit at once).  The table travels in the kernel arguments and is indexed by
// blockIdx.y, so its fields load in the kernel's first round of argument loads (the
// reference runs every job of a submission in one launch per format,
// IW/src/cuda/h3_compute.cu:336-382).
constexpr int kMaxFused = 8;
struct MfmaJob {  // one job's fields together
    const uint8_t* weights;
    const float* x;
    float* y;
    unsigned* status;
    size_t row_bytes, stride;
    unsigned out, index_limit;
    // optional: the weights start at weights + min(*index, index_limit - 1) * index_stride;
    // a negative index skips the job (the whole workgroup returns before any barrier)
    const int32_t* index;
    size_t index_stride;
    // paired launches: the second matrix (same shape, same expert offset); y = silu(W x) * (up x)
    const uint8_t* up;
};
struct MfmaJobs {
    MfmaJob job[kMaxFused];
    unsigned count, columns, in, rows_per_wg;
    // affine batch: `count` jobs all described by job[0], job j's x, y and index advanced
    // by (j / x_every) * x_step, j * y_step and j
    unsigned affine, x_every;
    size_t x_step, y_step;
    // 2 when every job of the launch is paired (a launch-wide shape: the LDS layout
    // depends on it), else 1
    unsigned mats;
};

// Workgroup: W wavefronts (W <= 16), rows [r0, r1) of its job, processed in passes of up
// to kTiles tiles.  In a pass, wavefront w takes the units (g, t) for g = w, w + W, ... and every
// tile t, kUnits at a time.  Loads are issued by every lane
// unconditionally (rows past r1 and units past the wavefront's last are clamped to valid
// data and their results discarded), so waits count exactly.  Order: this thread's first
// activation unit, the first units' packed weights, then the staging.
//
// FORM 0 is the general kernel.  PLAIN launches (FORM 1, 2 and 3: no device-side expert
// index, no affine batch, no pairing: every decode product of kdq_gemv / kdq_gemv_batch)
// take job blockIdx.y as it stands; the MoE forms carry those fields (measured: the plain
// C2 launch 8.29 -> 7.77 us without them).  FORM 2, for inputs of more than 8 values a
// thread, requests a thread's second activation unit together with its first, before the
// weights (C2 down 14336 -> 4096: 9.54 -> 9.29 us; the same test in FORM 1's code made
// the one-unit launches 0.1-0.3 us slower, hence a form of its own).  FORM 3, for
// workgroups of several row tiles: every wavefront's activation request is issued before
// any wavefront's weight requests (one barrier between them), so the staging's data does
// not return behind other wavefronts' weights (C2 4096 -> 14336: 7.95 -> 7.77 us; with
// one tile a workgroup, C1, it measured 0.35 us slower).
//
// mfma_gemv_body is the workgroup (bx, by) of that grid; `routed` >= 0 stands in for the
// job's device index (the fused MoE decode, which selects the experts itself).  COHERENT
// stores y at device scope (written through to where every XCD reads it), for another
// workgroup to read after this one's completion count.  A `late` functor (anything but
// EarlyRoute) gives the expert only after the activation loads are in flight, just before
// the first weight loads (the fused decode routes there, every thread calling it).
struct EarlyRoute {};
template <int ENC, int R, int W, bool PACKED, int FORM, bool COHERENT = false,
          class LateRoute = EarlyRoute>
__device__ __forceinline__ void mfma_gemv_body(const MfmaJobs& jobs, unsigned bx,
                                               unsigned by, int routed,
                                               const LateRoute& late = LateRoute{}) {
    constexpr bool PLAIN = FORM > 0, X2 = FORM == 2, XFIRST = FORM == 3;
    constexpr bool LATE = !std::is_same_v<LateRoute, EarlyRoute>;
    const bool affine = !PLAIN && jobs.affine;
    const unsigned jid = affine ? 0 : by, step = affine ? by : 0;
    const MfmaJob& jb = jobs.job[jid];
    const unsigned mats = !PLAIN && jobs.mats == 2 ? 2 : 1;
    const uint8_t* __restrict__ weights = jb.weights;
    const uint8_t* __restrict__ up = mats == 2 ? jb.up : weights;
    auto place = [&](int chosen) {  // the expert slice's weights
        const size_t expert =
            !PLAIN && jb.index
                ? size_t(min(unsigned(chosen), jb.index_limit - 1)) * jb.index_stride
                : 0;
        weights = jb.weights + expert;
        up = mats == 2 ? jb.up + expert : weights;
    };
    if constexpr (!LATE) {
        const int chosen = routed >= 0 ? routed : (!PLAIN && jb.index ? jb.index[step] : 0);
        if (chosen < 0)
            return;
        place(chosen);
    }
    const size_t row_bytes = jb.row_bytes, stride = jb.stride;
    const float* x = jb.x + (affine ? step / jobs.x_every : 0) * jobs.x_step;
    float* __restrict__ y = jb.y + (affine ? step * jobs.y_step : 0);
    unsigned* status = jb.status;
    const unsigned in = jobs.in, out = jb.out, rows_per_wg = jobs.rows_per_wg;
    constexpr int kTiles = mfma_tiles<R>;
    constexpr int kUnits = mfma_units<ENC, R>;
    constexpr int kRowUnroll = R <= 2 ? R : 1;  // larger batches: one row's operands at a time
    constexpr unsigned kThreads = W * 64;
    extern __shared__ __align__(16) uint8_t lds[];
    const MfmaLds layout = mfma_layout(R, in, mats, mfma_table_bytes(ENC));
    const unsigned groups = in / 256;
    uint8_t* atab = lds + layout.a;
    uint8_t* table = lds + layout.table;
    float4* blocks = reinterpret_cast<float4*>(lds + layout.blocks);
    float* partial = reinterpret_cast<float*>(lds + layout.partial);

    const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const unsigned lane = threadIdx.x % 64;
    const unsigned j = lane % 16, G = lane / 16;
    // A operand base: carrier lanes (row j of A lies in their group) read their table
    // entry, the others a zero region; MFMA m adds m * 256 bytes
    const bool carrier = j / 4 == G;
    // Q4_K: the scale bytes of sub-blocks 2G, 2G+1; Q6_K: 2p for chunk G = 2h + p
    const ScaleSel sel = ENC == KDQ_Q6_K     ? ScaleSel{2 * (G % 2), (j & 1) != 0}
                         : ENC == KDQ_IQ4_XS || ENC == KDQ_Q3_K || lattice(ENC) ? ScaleSel{G, false}
                                             : ScaleSel{8 * ((2 * G) & 3), G >= 2};
    // every argument in one round of scalar loads, then the exit test
    if constexpr (LATE)
        asm volatile("" ::"s"(x), "s"(y), "s"(status), "s"(row_bytes), "s"(stride), "s"(in),
                     "s"(out), "s"(rows_per_wg));
    else
        asm volatile("" ::"s"(weights), "s"(up), "s"(x), "s"(y), "s"(status), "s"(row_bytes),
                     "s"(stride), "s"(in), "s"(out), "s"(rows_per_wg));
    const unsigned r0 = bx * rows_per_wg, r1 = min(out, r0 + rows_per_wg);
    if (r0 >= out)
        return;  // the whole workgroup, before any barrier
    bool bad = false;

    for (unsigned t = threadIdx.x; t < 256; t += kThreads)
        reinterpret_cast<uint32_t*>(lds)[t] = 0u;

    auto pass_tiles = [&](unsigned p0) { return min(unsigned(kTiles), (r1 - p0 + 15) / 16); };
    // cursor tile t < tiles is row tile t of `weights`, t >= tiles row tile t - tiles of `up`
    auto load_units = [&](unsigned p0, UnitCursor cur, Lane(&L)[kUnits]) {
        const unsigned tiles = pass_tiles(p0);
#pragma unroll
        for (int k = 0; k < kUnits; ++k) {
            const bool valid = cur.g < groups;
            const unsigned g = valid ? cur.g : wave % groups, t = valid ? cur.t : 0;
            const bool second = t >= tiles;
            const uint8_t* w = second ? up : weights;
            const unsigned n = min(p0 + 16 * (second ? t - tiles : t) + j, r1 - 1);
            if constexpr (PACKED)
                load_packed<ENC>(w + (size_t(n / 16) * groups + g) * PackedFormat<ENC>::unit,
                                 G, n % 16, L[k]);
            else if constexpr (ENC == KDQ_Q6_K)
                load_lane_q6k(w + size_t(n) * row_bytes, g, G, L[k]);
            else if constexpr (ENC == KDQ_IQ4_XS)
                load_lane_iq4xs(w + size_t(n) * row_bytes, g, G, L[k]);
            else if constexpr (ENC == KDQ_Q3_K)
                load_lane_q3k(w + size_t(n) * row_bytes, g, G, L[k]);
            else if constexpr (ENC == KDQ_IQ3_XXS)
                load_lane_iq3xxs(w + size_t(n) * row_bytes, g, G, L[k]);
            else if constexpr (ENC == KDQ_IQ3_S)
                load_lane_iq3s(w + size_t(n) * row_bytes, g, G, L[k]);
            else if constexpr (ENC == KDQ_IQ2_S)
                load_lane_iq2s(w + size_t(n) * row_bytes, g, G, L[k]);
            else if constexpr (ENC == KDQ_IQ4_NL)  // Q4_0's block size and layout
                load_lane<KDQ_Q4_0>(w + size_t(n) * row_bytes, 4 * g + G, L[k]);
            else
                load_lane<ENC>(w + size_t(n) * row_bytes, 4 * g + G, L[k]);
            cur.next(tiles * mats, W);
        }
    };

    const unsigned units_x = R * in / 8;
    XUnit first_unit, second_unit;
    load_unit(x, in, min(unsigned(threadIdx.x), units_x - 1), first_unit);
    if constexpr (X2)
        load_unit(x, in, min(unsigned(threadIdx.x) + kThreads, units_x - 1), second_unit);
    // the lattice grid entries this thread converts, requested before the weights (the
    // staging waits for them)
    unsigned entry[lattice(ENC) ? lattice_per_thread<ENC, kThreads> : 1];
    if constexpr (lattice(ENC)) {
#pragma unroll
        for (unsigned k = 0; k < lattice_per_thread<ENC, kThreads>; ++k)
            entry[k] = lattice_entry<ENC>(min(threadIdx.x + k * kThreads, lattice_entries(ENC) - 1));
    }
    asm volatile("" ::: "memory");  // x is not restrict: its loads stay before this point
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XFIRST) {
        __builtin_amdgcn_s_barrier();  // every wavefront's x request ahead of any weight request
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (LATE)
        place(late());
    Lane L[kUnits];
    load_units(r0, UnitCursor{wave, 0}, L);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (lattice(ENC))
        lattice_table<ENC, kThreads>(table, entry);
    if (threadIdx.x < units_x)
        mstage_unit<ENC>(in, threadIdx.x, first_unit, atab, blocks);
    if (X2 && threadIdx.x + kThreads < units_x)
        mstage_unit<ENC>(in, threadIdx.x + kThreads, second_unit, atab, blocks);
    for (unsigned u = threadIdx.x + (X2 ? 2 : 1) * kThreads; u < units_x; u += kThreads) {
        XUnit more;
        load_unit(x, in, u, more);
        mstage_unit<ENC>(in, u, more, atab, blocks);
    }
    __syncthreads();

    bool first = true;
    for (unsigned p0 = r0; p0 < r1; p0 += 16 * kTiles) {
        const unsigned tiles = pass_tiles(p0);
        // partial[((r*kTiles + t)*64 + lane)*kPartialPitch + wave] belongs to this thread
        float* mine = partial + size_t(lane) * kPartialPitch + wave;
        for (unsigned i = 0; i < R * kTiles * mats; ++i)
            mine[size_t(i) * 64 * kPartialPitch] = 0.f;
        for (UnitCursor cur{wave, 0}; cur.g < groups;) {
            if (!first)
                load_units(p0, cur, L);
            first = false;
#pragma unroll
            for (int k = 0; k < kUnits; ++k) {
                if (cur.g >= groups)
                    break;
                const unsigned b0 = 8 * cur.g + block_of<ENC>(G, 0);
                const unsigned b1 = 8 * cur.g + block_of<ENC>(G, 1);
#pragma unroll kRowUnroll
                for (int r = 0; r < R; ++r) {
                    const uint8_t* a = carrier ? atab + (size_t(r) * groups + cur.g) * kAGroup +
                                                     (4 * G + j % 4) * 16
                                               : lds;
                    // Q6_K keeps positions 0..15 (MFMAs 0, 1) and 16..31 (2, 3) of each
                    // block apart: its scales change every 16 values
                    i32x4 c = {0, 0, 0, 0}, c2 = {0, 0, 0, 0};
#pragma unroll
                    for (int m = 0; m < 4; ++m) {
                        const i32x4 av = *reinterpret_cast<const i32x4*>(a + m * 256);
                        const i32x4 bv = b_operand<ENC, PACKED>(L[k], m, sel.shift, table);
                        if ((ENC == KDQ_Q6_K || ENC == KDQ_Q3_K || ENC == KDQ_IQ2_S) && m >= 2)
                            c2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, c2, 0, 0, 0);
                        else
                            c = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bv, c, 0, 0, 0);
                    }
                    const float4* xb = blocks + size_t(r) * (in / 32);
                    // partial slot of (matrix, row tile): m * kTiles + tile
                    const unsigned slot = cur.t < tiles ? cur.t : kTiles + cur.t - tiles;
                    mine[size_t(r * kTiles * mats + slot) * 64 * kPartialPitch] +=
                        chunk_value<ENC, PACKED>(L[k], sel, c, c2, xb[b0], xb[b1], bad);
                }
                cur.next(tiles * mats, W);
            }
        }
        first = false;  // a wavefront without units in the first pass never used its loads
        __syncthreads();
        // output o = (r*tiles + t)*16 + jj: 16 threads (one DPP row), thread k < W sums
        // wavefront k's four lane groups, then the row of 16 is summed
        const unsigned outputs = R * tiles * 16;
        for (unsigned o = threadIdx.x / 16; o < outputs; o += kThreads / 16) {
            const unsigned k = threadIdx.x % 16;
            const unsigned jj = o % 16, t = (o / 16) % tiles, r = o / (16 * tiles);
            const float* src =
                partial + (size_t(r * kTiles * mats + t) * 64 + jj) * kPartialPitch + k;
            float v = k < W ? ((src[0] + src[16 * kPartialPitch]) + src[32 * kPartialPitch]) +
                                  src[48 * kPartialPitch]
                            : 0.f;
            v = row16_total(v);
            if (mats == 2) {  // the up row of the same output, kTiles slots on
                const float* us = src + size_t(kTiles) * 64 * kPartialPitch;
                float u = k < W ? ((us[0] + us[16 * kPartialPitch]) + us[32 * kPartialPitch]) +
                                      us[48 * kPartialPitch]
                                : 0.f;
                v = silu_of(v) * row16_total(u);
            }
            const unsigned n = p0 + 16 * t + jj;
            if (k == 0 && n < r1) {
                if constexpr (COHERENT)
                    __hip_atomic_store(&y[size_t(r) * stride + n], v, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                else
                    y[size_t(r) * stride + n] = v;
            }
        }
        __syncthreads();
    }
    if (status && __any(bad) && lane == 0)
        atomicOr(status, 1u);
}

template <int ENC, int R, int W, bool PACKED, int FORM>
__global__ __launch_bounds__(W * 64) void mfma_gemv(const MfmaJobs jobs) {
    mfma_gemv_body<ENC, R, W, PACKED, FORM>(jobs, blockIdx.x, blockIdx.y, -1);
}

// ----------------------------------------------------------------- host side

template <int ENC>
int launch_decode(const void* packed, size_t row_bytes, size_t rows, size_t in, float* out,
                  unsigned* status, hipStream_t stream) {
    const size_t threads = rows * (in / 8);
    const size_t grid = (threads + 255) / 256;
    if (grid > 0x7fffffffu)
        return KDQ_ERR_UNSUPPORTED;
    hipLaunchKernelGGL((decode_kernel<ENC>), dim3(unsigned(grid)), dim3(256), 0, stream,
                       static_cast<const uint8_t*>(packed), row_bytes, rows, in, out, status);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}

template <int ENC>
int launch_exact(const void* w, size_t row_bytes, const float* x, size_t rows, size_t in,
                 size_t out, float* y, size_t stride, unsigned* status, hipStream_t stream,
                 const int32_t* index = nullptr, size_t index_stride = 0,
                 unsigned index_limit = 1, unsigned batch = 1, size_t x_step = 0,
                 size_t y_step = 0, unsigned x_every = 1) {
    const dim3 grid(unsigned((out + 3) / 4), batch);
    for (size_t first = 0; first < rows; first += 8) {
        const unsigned group = unsigned(std::min<size_t>(8, rows - first));
        if (group == 1)
            hipLaunchKernelGGL((exact_gemv<ENC, 1>), grid, dim3(256), 0, stream,
                               static_cast<const uint8_t*>(w), row_bytes, x + first * in, 1u,
                               unsigned(in), unsigned(out), y + first * stride, stride, status,
                               index, index_stride, index_limit, x_step, y_step, x_every);
        else
            hipLaunchKernelGGL((exact_gemv<ENC, 8>), grid, dim3(256), 0, stream,
                               static_cast<const uint8_t*>(w), row_bytes, x + first * in, group,
                               unsigned(in), unsigned(out), y + first * stride, stride, status,
                               index, index_stride, index_limit, x_step, y_step, x_every);
        KDQ_HIP(hipGetLastError());
    }
    return KDQ_OK;
}

struct FastPlan {
    unsigned nw, rows_per_wg, grid, batch;
    size_t lds;
};

// Window count (power of two dividing 16), rows per workgroup, batch rows per pass.
bool plan_fast(size_t rows, size_t in, size_t out, FastPlan& p) {
    const size_t windows = (in + kWindow - 1) / kWindow;
    unsigned nw = 1;
    while (nw < windows)
        nw *= 2;
    if (nw > 16)
        return false;
    // batch rows per pass: the staged activations (2.5 bytes per value) must fit
    unsigned batch = 1;
    while (batch < 8 && batch < rows && size_t(batch * 2) * (in / kSlot) * kSlotLds <= 96 * 1024)
        batch *= 2;
    // one workgroup per compute unit: every wavefront's rows are requested up front
    const size_t rows_per_wg = std::max<size_t>(1, (out + compute_units() - 1) / compute_units());
    p.nw = nw;
    p.batch = batch;
    p.rows_per_wg = unsigned(rows_per_wg);
    p.grid = unsigned((out + rows_per_wg - 1) / rows_per_wg);
    p.lds = size_t(batch) * (in / kSlot) * kSlotLds + (nw > 1 ? rows_per_wg * batch * nw * 4 : 0);
    return p.lds <= 160 * 1024;
}

template <int ENC, int R>
int launch_fast_pass(const FastPlan& p, const void* w, size_t row_bytes, const float* x,
                     size_t in, size_t out, float* y, size_t stride, unsigned* status,
                     hipStream_t stream) {
    static bool configured = false;  // one attribute call per instantiation
    if (!configured) {
        KDQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&fast_gemv<ENC, R>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        configured = true;
    }
    hipLaunchKernelGGL((fast_gemv<ENC, R>), dim3(p.grid), dim3(kThreads), p.lds, stream,
                       static_cast<const uint8_t*>(w), row_bytes, x, unsigned(in),
                       unsigned(out), y, stride, status, p.rows_per_wg, p.nw);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}

template <int ENC>
int launch_fast(const void* w, size_t row_bytes, const float* x, size_t rows, size_t in,
                size_t out, float* y, size_t stride, unsigned* status, hipStream_t stream) {
    FastPlan p;
    if (!plan_fast(rows, in, out, p))
        return KDQ_ERR_UNSUPPORTED;
    for (size_t first = 0; first < rows;) {
        const size_t left = rows - first;
        unsigned r = p.batch;
        while (r > left)
            r /= 2;
        FastPlan q = p;
        q.lds = size_t(r) * (in / kSlot) * kSlotLds +
                (p.nw > 1 ? size_t(p.rows_per_wg) * r * p.nw * 4 : 0);
        int rc;
        const float* xs = x + first * in;
        float* ys = y + first * stride;
        switch (r) {
        case 1:
            rc = launch_fast_pass<ENC, 1>(q, w, row_bytes, xs, in, out, ys, stride, status, stream);
            break;
        case 2:
            rc = launch_fast_pass<ENC, 2>(q, w, row_bytes, xs, in, out, ys, stride, status, stream);
            break;
        case 4:
            rc = launch_fast_pass<ENC, 4>(q, w, row_bytes, xs, in, out, ys, stride, status, stream);
            break;
        default:
            rc = launch_fast_pass<ENC, 8>(q, w, row_bytes, xs, in, out, ys, stride, status, stream);
            break;
        }
        if (rc)
            return rc;
        first += r;
    }
    return KDQ_OK;
}

// LDS bytes of mfma_gemv for `batch` rows (mats = 2: paired jobs).
size_t mfma_lds(size_t batch, size_t in, unsigned mats = 1, size_t table = 0) {
    return mfma_layout(unsigned(batch), unsigned(in), mats, table).total;
}

struct MfmaPlan {
    unsigned rows_per_wg, grid, batch, waves;
};

// Batch rows per pass as the LDS allows (at most 8); `waves` wavefronts per workgroup and
// ceil(total_out / workgroup slots) rows per workgroup, total_out summed over the jobs of
// one launch (paired jobs: mats = 2, each output row two rows of work).  Over packed
// weights the rows per workgroup are a multiple of 8, so every 128-byte line of a unit
// (8 row slots of one chunk) belongs to one workgroup.
bool plan_mfma(size_t rows, size_t in, size_t total_out, MfmaPlan& p, bool packed = false,
               unsigned mats = 1, size_t table = 0) {
    constexpr size_t limit = 160 * 1024;
    if (in % 256 || mfma_lds(1, in, mats, table) > limit)
        return false;
    unsigned batch = 1;
    while (batch < 8 && batch < rows && mfma_lds(batch * 2, in, mats, table) <= limit)
        batch *= 2;
    // A wavefront takes the 256-value groups w, w + W, ...: narrow products (the MoE
    // experts' 768 / 2048 inputs) use 4 or 8 wavefronts, and correspondingly more
    // workgroups per compute unit (as many as the LDS holds, up to 16 wavefronts).
    const size_t groups = in / 256;
    unsigned waves = groups <= 4 ? 4 : (groups <= 8 ? 8 : 16);
    size_t per_cu = 16 / waves;
    while (per_cu > 1 && per_cu * mfma_lds(batch, in, mats, table) > limit)
        per_cu /= 2;
    const size_t slots = compute_units() * per_cu;
    size_t rows_per_wg = std::max<size_t>(1, (total_out * mats + slots - 1) / slots / mats);
    // narrow products (the MoE experts' 768 / 1024 inputs): at least one pass of whole
    // tiles per workgroup, so the per-workgroup costs (expert index, activation staging,
    // reduction) are paid over 16 * kTiles rows (Qwen3 MoE decode: 48.3 -> 42.9 us; 128
    // rows, or the same for 2048 inputs, measured slower)
    if (groups <= 4)
        rows_per_wg = std::max<size_t>(rows_per_wg, 16 * size_t(batch >= 4 ? 1 : 4 / batch));
    else if (groups <= 8)  // and at least one whole tile (Qwen3 MoE, 4 tokens: 75.8 -> 70.8 us)
        rows_per_wg = std::max<size_t>(rows_per_wg, 16);
    if (packed)
        rows_per_wg = (rows_per_wg + 7) & ~size_t(7);
    p.batch = batch;
    p.waves = waves;
    p.rows_per_wg = unsigned(rows_per_wg);
    p.grid = unsigned((total_out + rows_per_wg - 1) / rows_per_wg);
    return true;
}

// Sets rows_per_wg and the grid columns (workgroups of the largest job) of `jobs`
// (count, out[] set).
void number_workgroups(MfmaJobs& jobs, unsigned rows_per_wg) {
    jobs.rows_per_wg = rows_per_wg;
    jobs.columns = 0;
    for (unsigned k = 0; k < (jobs.affine ? 1u : jobs.count); ++k)
        jobs.columns = std::max(jobs.columns, (jobs.job[k].out + rows_per_wg - 1) / rows_per_wg);
}

template <int ENC, int R, int W, bool PACKED, int FORM>
int launch_mfma_form(const MfmaJobs& jobs, hipStream_t stream) {
    static bool configured = false;  // one attribute call per instantiation
    if (!configured) {
        KDQ_HIP(hipFuncSetAttribute(
            reinterpret_cast<const void*>(&mfma_gemv<ENC, R, W, PACKED, FORM>),
            hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        configured = true;
    }
    hipLaunchKernelGGL((mfma_gemv<ENC, R, W, PACKED, FORM>), dim3(jobs.columns, jobs.count),
                       dim3(W * 64), mfma_lds(R, jobs.in, jobs.mats == 2 ? 2 : 1, mfma_table_bytes(ENC)),
                       stream, jobs);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}

// Plain launches (no job with a device index, not affine, not paired) run the lean form:
// with 16 wavefronts and more than 8 input values a thread its two-unit staging, with
// 16 wavefronts and workgroups of 32 rows or more its activation-first form (not Q6_K,
// which measured 0.1-0.2 us slower with it).
template <int ENC, int R, int W, bool PACKED>
int launch_mfma_shape(const MfmaJobs& jobs, hipStream_t stream) {
    bool plain = !jobs.affine && jobs.mats != 2;
    for (unsigned k = 0; plain && k < jobs.count; ++k)
        plain = jobs.job[k].index == nullptr;
    if (!plain)
        return launch_mfma_form<ENC, R, W, PACKED, 0>(jobs, stream);
    if constexpr (W == 16) {
        if (size_t(R) * jobs.in / 8 > size_t(W) * 64)
            return launch_mfma_form<ENC, R, W, PACKED, 2>(jobs, stream);
        if constexpr (ENC != KDQ_Q6_K)
            if (jobs.rows_per_wg >= 32)
                return launch_mfma_form<ENC, R, W, PACKED, 3>(jobs, stream);
    }
    return launch_mfma_form<ENC, R, W, PACKED, 1>(jobs, stream);
}

template <int ENC, int R, bool PACKED>
int launch_mfma_pass(unsigned waves, const MfmaJobs& jobs, hipStream_t stream) {
    switch (waves) {
    case 4:
        return launch_mfma_shape<ENC, R, 4, PACKED>(jobs, stream);
    case 8:
        return launch_mfma_shape<ENC, R, 8, PACKED>(jobs, stream);
    default:
        return launch_mfma_shape<ENC, R, 16, PACKED>(jobs, stream);
    }
}

template <int ENC, bool PACKED>
int launch_mfma_rows(unsigned r, unsigned waves, const MfmaJobs& jobs, hipStream_t stream) {
    switch (r) {
    case 1:
        return launch_mfma_pass<ENC, 1, PACKED>(waves, jobs, stream);
    case 2:
        return launch_mfma_pass<ENC, 2, PACKED>(waves, jobs, stream);
    case 4:
        return launch_mfma_pass<ENC, 4, PACKED>(waves, jobs, stream);
    default:
        return launch_mfma_pass<ENC, 8, PACKED>(waves, jobs, stream);
    }
}

// `rows` activation rows in passes of the plan's batch (the largest power of two that
// fits what is left).  `row_bytes` is unused over packed weights.
template <int ENC, bool PACKED>
int launch_mfma(const void* w, size_t row_bytes, const float* x, size_t rows, size_t in,
                size_t out, float* y, size_t stride, unsigned* status, hipStream_t stream) {
    MfmaPlan p;
    if (!plan_mfma(rows, in, out, p, PACKED, 1, mfma_table_bytes(ENC)))
        return KDQ_ERR_UNSUPPORTED;
    for (size_t first = 0; first < rows;) {
        const size_t left = rows - first;
        unsigned r = p.batch;
        while (r > left)
            r /= 2;
        MfmaJobs jobs{};
        jobs.count = 1;
        jobs.in = unsigned(in);
        jobs.job[0] = MfmaJob{static_cast<const uint8_t*>(w), x + first * in, y + first * stride,
                              status, row_bytes, stride, unsigned(out), 0};
        number_workgroups(jobs, p.rows_per_wg);
        const int rc = launch_mfma_rows<ENC, PACKED>(r, p.waves, jobs, stream);
        if (rc)
            return rc;
        first += r;
    }
    return KDQ_OK;
}

template <bool PACKED>
int launch_mfma_any(int encoding, const void* w, size_t row_bytes, const float* x, size_t rows,
                    size_t in, size_t out, float* y, size_t stride, unsigned* status,
                    hipStream_t s) {
    switch (encoding) {
    case KDQ_Q8_0:
        return launch_mfma<KDQ_Q8_0, PACKED>(w, row_bytes, x, rows, in, out, y, stride, status, s);
    case KDQ_Q4_0:
        return launch_mfma<KDQ_Q4_0, PACKED>(w, row_bytes, x, rows, in, out, y, stride, status, s);
    case KDQ_Q4_K:
        return launch_mfma<KDQ_Q4_K, PACKED>(w, row_bytes, x, rows, in, out, y, stride, status, s);
    case KDQ_Q6_K:
        return launch_mfma<KDQ_Q6_K, PACKED>(w, row_bytes, x, rows, in, out, y, stride, status, s);
    case KDQ_IQ4_XS:  // row-major only: no packed unit
        if constexpr (!PACKED)
            return launch_mfma<KDQ_IQ4_XS, false>(w, row_bytes, x, rows, in, out, y, stride,
                                                  status, s);
        return KDQ_ERR_UNSUPPORTED;
    case KDQ_IQ4_NL:
        if constexpr (!PACKED)
            return launch_mfma<KDQ_IQ4_NL, false>(w, row_bytes, x, rows, in, out, y, stride,
                                                  status, s);
        return KDQ_ERR_UNSUPPORTED;
    case KDQ_Q3_K:
        if constexpr (!PACKED)
            return launch_mfma<KDQ_Q3_K, false>(w, row_bytes, x, rows, in, out, y, stride,
                                                status, s);
        return KDQ_ERR_UNSUPPORTED;
    case KDQ_IQ3_XXS:
        if constexpr (!PACKED)
            return launch_mfma<KDQ_IQ3_XXS, false>(w, row_bytes, x, rows, in, out, y, stride,
                                                   status, s);
        return KDQ_ERR_UNSUPPORTED;
    case KDQ_IQ3_S:
        if constexpr (!PACKED)
            return launch_mfma<KDQ_IQ3_S, false>(w, row_bytes, x, rows, in, out, y, stride,
                                                 status, s);
        return KDQ_ERR_UNSUPPORTED;
    case KDQ_IQ2_S:
        if constexpr (!PACKED)
            return launch_mfma<KDQ_IQ2_S, false>(w, row_bytes, x, rows, in, out, y, stride,
                                                 status, s);
        return KDQ_ERR_UNSUPPORTED;
    default:
        return KDQ_ERR_UNSUPPORTED;
    }
}

// ------------------------------------------------------------- packing

size_t packed_unit(int encoding) {
    switch (encoding) {
    case KDQ_Q4_K:
        return PackedFormat<KDQ_Q4_K>::unit;
    case KDQ_Q4_0:
        return PackedFormat<KDQ_Q4_0>::unit;
    case KDQ_Q8_0:
        return PackedFormat<KDQ_Q8_0>::unit;
    case KDQ_Q6_K:
        return PackedFormat<KDQ_Q6_K>::unit;
    default:
        return 0;
    }
}

// Four bytes from any alignment, little-endian.
__device__ __forceinline__ unsigned bytes4(const uint8_t* p) {
    return unsigned(p[0]) | unsigned(p[1]) << 8 | unsigned(p[2]) << 16 | unsigned(p[3]) << 24;
}

__device__ __forceinline__ uint4 bytes16(const uint8_t* p) {
    return make_uint4(bytes4(p), bytes4(p + 4), bytes4(p + 8), bytes4(p + 12));
}

// One thread per (tile, group, lane): writes that lane's code pieces and side data of
// the unit (PackedFormat layout); rows past `out` are written as zeros.
template <int ENC>
__global__ __launch_bounds__(256) void pack_kernel(const uint8_t* __restrict__ raw,
                                                   size_t row_bytes, unsigned groups,
                                                   unsigned out, size_t lanes,
                                                   uint8_t* __restrict__ packed) {
    const size_t id = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (id >= lanes)
        return;
    constexpr int P = PackedFormat<ENC>::pieces;
    const unsigned l = unsigned(id % 64), G = l / 16, s = l % 16;
    const size_t unit_index = id / 64;
    const unsigned g = unsigned(unit_index % groups);
    const size_t n = (unit_index / groups) * 16 + s;
    uint8_t* unit = packed + unit_index * PackedFormat<ENC>::unit;
    const bool live = n < out;
    const uint8_t* row = raw + (live ? n : 0) * row_bytes;
    const uint4 zero = make_uint4(0, 0, 0, 0);
    if constexpr (ENC == KDQ_Q4_K) {
        const uint8_t* block = row + size_t(g) * 144;
#pragma unroll
        for (int p = 0; p < P; ++p)
            *reinterpret_cast<uint4*>(unit + p * 1024 + 16 * l) =
                live ? bytes16(block + 16 + 32 * G + 16 * p) : zero;
        if (G == 0)
            *reinterpret_cast<uint4*>(unit + P * 1024 + 16 * s) = live ? bytes16(block) : zero;
    } else if constexpr (ENC == KDQ_Q6_K) {
        const uint8_t* block = row + size_t(g) * 210;
        const unsigned h = G / 2, p = G % 2;
        *reinterpret_cast<uint4*>(unit + 16 * l) = live ? bytes16(block + 32 * G) : zero;
        *reinterpret_cast<uint4*>(unit + 1024 + 16 * l) = live ? bytes16(block + 32 * G + 16) : zero;
        // qh pairs of position t: block 0 bits 2p, 2p+1 and block 1 bits 4+2p, 5+2p of
        // qh[32h + t], as one nibble
        auto pairs = [&](unsigned t) {
            const unsigned q = block[128 + 32 * h + t];
            return ((q >> (2 * p)) & 3u) | (((q >> (4 + 2 * p)) & 3u) << 2);
        };
        uint4 x = zero;
        unsigned* xw = &x.x;
        if (live)
            for (unsigned m = 0; m < 4; ++m)
                for (unsigned i = 0; i < 4; ++i)
                    xw[m] |= ((pairs(8 * m + i) << 4) | pairs(8 * m + 4 + i)) << (8 * i);
        *reinterpret_cast<uint4*>(unit + 2048 + 16 * l) = x;
        const uint8_t* sc = block + 192 + 8 * h + 2 * p;
        *reinterpret_cast<unsigned*>(unit + 3072 + 4 * l) =
            live ? unsigned(sc[0]) | unsigned(sc[1]) << 8 | unsigned(sc[4]) << 16 |
                       unsigned(sc[5]) << 24
                 : 0u;
        if (G == 0) {  // this row slot's d, in the dword of its pair of slots
            const unsigned dh = live ? half_bits_at(block + 208) : 0u;
            reinterpret_cast<uint16_t*>(unit + 3328)[s] = uint16_t(dh);
        }
    } else {
        constexpr int bytes = Format<ENC>::bytes;
        const uint8_t* b0 = row + (size_t(g) * 8 + 2 * G) * bytes;
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const uint8_t* src = ENC == KDQ_Q4_0 ? b0 + p * bytes + 2
                                                 : b0 + (p / 2) * bytes + 2 + 16 * (p % 2);
            *reinterpret_cast<uint4*>(unit + p * 1024 + 16 * l) = live ? bytes16(src) : zero;
        }
        const unsigned side = live ? (half_bits_at(b0) | half_bits_at(b0 + bytes) << 16) : 0u;
        *reinterpret_cast<unsigned*>(unit + P * 1024 + 4 * l) = side;
    }
}

template <int ENC>
int launch_pack(const void* raw, size_t row_bytes, size_t in, size_t out, void* packed,
                hipStream_t stream) {
    const size_t groups = in / 256, tiles = (out + 15) / 16;
    const size_t lanes = tiles * groups * 64;
    const size_t grid = (lanes + 255) / 256;
    if (grid > 0x7fffffffu)
        return KDQ_ERR_UNSUPPORTED;
    hipLaunchKernelGGL((pack_kernel<ENC>), dim3(unsigned(grid)), dim3(256), 0, stream,
                       static_cast<const uint8_t*>(raw), row_bytes, unsigned(groups),
                       unsigned(out), lanes, static_cast<uint8_t*>(packed));
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}

bool aligned(const void* p, size_t a) {
    return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}

// Calls f(std::integral_constant<int, ENC>) for every encoding the decode and the
// exact product take; KDQ_ERR_UNSUPPORTED otherwise.
template <typename F>
int with_encoding(int encoding, F&& f) {
    switch (encoding) {
    case KDQ_Q8_0:
        return f(std::integral_constant<int, KDQ_Q8_0>{});
    case KDQ_Q4_0:
        return f(std::integral_constant<int, KDQ_Q4_0>{});
    case KDQ_Q4_K:
        return f(std::integral_constant<int, KDQ_Q4_K>{});
    case KDQ_Q3_K:
        return f(std::integral_constant<int, KDQ_Q3_K>{});
    case KDQ_Q6_K:
        return f(std::integral_constant<int, KDQ_Q6_K>{});
    case KDQ_IQ4_NL:
        return f(std::integral_constant<int, KDQ_IQ4_NL>{});
    case KDQ_IQ4_XS:
        return f(std::integral_constant<int, KDQ_IQ4_XS>{});
    case KDQ_BF16:
        return f(std::integral_constant<int, KDQ_BF16>{});
    case KDQ_IQ3_XXS:
        return f(std::integral_constant<int, KDQ_IQ3_XXS>{});
    case KDQ_IQ2_S:
        return f(std::integral_constant<int, KDQ_IQ2_S>{});
    case KDQ_IQ3_S:
        return f(std::integral_constant<int, KDQ_IQ3_S>{});
    case KDQ_F32:
        return f(std::integral_constant<int, KDQ_F32>{});
    case KDQ_F16:
        return f(std::integral_constant<int, KDQ_F16>{});
    default:
        return KDQ_ERR_UNSUPPORTED;
    }
}

// The encodings the streaming and MFMA products take over row-major weights (the packed
// layout: Q8_0, Q4_0, Q4_K).
bool streamed_encoding(int encoding) {
    return encoding == KDQ_Q8_0 || encoding == KDQ_Q4_0 || encoding == KDQ_Q4_K ||
           encoding == KDQ_Q6_K || encoding == KDQ_IQ4_XS || encoding == KDQ_IQ4_NL ||
           encoding == KDQ_Q3_K || lattice(encoding);
}

// The streaming kernels need whole 64-value lane slots, 4-byte aligned rows and packed
// rows of exactly the format's size (16-byte aligned for Q4_K); Q6_K (MFMA kernel only)
// 256-value groups and 2-byte aligned rows.
bool streams(int encoding, const void* weights, size_t row_bytes, size_t in) {
    // 210-, 110-, 98- and 82-byte super-blocks: 2-byte aligned rows
    if (encoding == KDQ_Q6_K || encoding == KDQ_Q3_K || lattice(encoding))
        return in % 256 == 0 && row_bytes % 2 == 0 && aligned(weights, 2);
    if (encoding == KDQ_IQ4_XS)  // 136-byte super-blocks: 8-byte aligned rows
        return in % 256 == 0 && row_bytes % 8 == 0 && aligned(weights, 8);
    return streamed_encoding(encoding) && in % 256 == 0 && row_bytes % 4 == 0 &&
           aligned(weights, 4) &&
           (encoding != KDQ_Q4_K || (row_bytes % 16 == 0 && aligned(weights, 16)));
}

// Shared argument checks of the product entry points.
int check_product(int encoding, const void* weights, size_t row_bytes, const float* x,
                  size_t rows, size_t in, size_t out, const float* y, size_t stride) {
    const size_t values = block_values(encoding);
    if (!values)
        return KDQ_ERR_UNSUPPORTED;
    if (!weights || !x || !y || !rows || !in || !out)
        return KDQ_ERR_ARGUMENT;
    if (in % values || in % 8 || row_bytes < in / values * block_bytes(encoding) ||
        stride < out || rows > 4096 || in > 0xffffffffu || out > 0xffffffffu)
        return KDQ_ERR_SHAPE;
    if (mul_overflows(out, row_bytes) || mul_overflows(rows, in) || mul_overflows(rows, stride))
        return KDQ_ERR_ARGUMENT;
    const size_t ybytes = ((rows - 1) * stride + out) * sizeof(float);
    if (overlaps(y, ybytes, weights, out * row_bytes) ||
        overlaps(y, ybytes, x, rows * in * sizeof(float)))
        return KDQ_ERR_ALIAS;
    if (!aligned(x, 16))
        return KDQ_ERR_ALIGNMENT;
    return KDQ_OK;
}

}  // namespace
}  // namespace kdq

using namespace kdq;

extern "C" int kdq_dequantize(int encoding, const void* packed, size_t row_bytes, size_t rows,
                              size_t in, float* out, unsigned* status, void* stream) {
    const size_t values = block_values(encoding);
    if (!values)
        return KDQ_ERR_UNSUPPORTED;
    if (!packed || !out || !rows || !in)
        return KDQ_ERR_ARGUMENT;
    if (in % values || row_bytes < in / values * block_bytes(encoding))
        return KDQ_ERR_SHAPE;
    if (mul_overflows(rows, in) || mul_overflows(rows, row_bytes))
        return KDQ_ERR_ARGUMENT;
    if (!aligned(out, 16))
        return KDQ_ERR_ALIGNMENT;
    if (overlaps(out, rows * in * sizeof(float), packed, rows * row_bytes))
        return KDQ_ERR_ALIAS;
    auto s = static_cast<hipStream_t>(stream);
    return with_encoding(encoding, [&](auto enc) {
        return launch_decode<decltype(enc)::value>(packed, row_bytes, rows, in, out, status, s);
    });
}

extern "C" int kdq_gemv_exact(int encoding, const void* weights, size_t row_bytes,
                              const float* x, size_t rows, size_t in, size_t out, float* y,
                              size_t stride, unsigned* status, void* stream) {
    int rc = check_product(encoding, weights, row_bytes, x, rows, in, out, y, stride);
    if (rc)
        return rc;
    auto s = static_cast<hipStream_t>(stream);
    return with_encoding(encoding, [&](auto enc) {
        return launch_exact<decltype(enc)::value>(weights, row_bytes, x, rows, in, out, y,
                                                  stride, status, s);
    });
}

extern "C" int kdq_gemv(int encoding, const void* weights, size_t row_bytes, const float* x,
                        size_t rows, size_t in, size_t out, float* y, size_t stride,
                        unsigned* status, void* stream) {
    int rc = check_product(encoding, weights, row_bytes, x, rows, in, out, y, stride);
    if (rc)
        return rc;
    auto s = static_cast<hipStream_t>(stream);
    // Shapes the streaming kernels do not take run on the exact kernel.
    const bool fast = streams(encoding, weights, row_bytes, in);
    if (fast) {
        rc = launch_mfma_any<false>(encoding, weights, row_bytes, x, rows, in, out, y, stride,
                                    status, s);
        if (rc != KDQ_ERR_UNSUPPORTED)
            return rc;
        switch (encoding) {
        case KDQ_Q8_0:
            rc = launch_fast<KDQ_Q8_0>(weights, row_bytes, x, rows, in, out, y, stride, status, s);
            break;
        case KDQ_Q4_0:
            rc = launch_fast<KDQ_Q4_0>(weights, row_bytes, x, rows, in, out, y, stride, status, s);
            break;
        case KDQ_Q4_K:
            rc = launch_fast<KDQ_Q4_K>(weights, row_bytes, x, rows, in, out, y, stride, status, s);
            break;
        default:
            rc = KDQ_ERR_UNSUPPORTED;
            break;
        }
        if (rc != KDQ_ERR_UNSUPPORTED)
            return rc;
    }
    return kdq_gemv_exact(encoding, weights, row_bytes, x, rows, in, out, y, stride, status,
                          stream);
}

extern "C" size_t kdq_gguf_packed_bytes(int encoding, size_t in, size_t out) {
    const size_t unit = packed_unit(encoding);
    if (!unit || !in || !out || in % 256 || in > 0xffffffffu || out > 0xffffffffu)
        return 0;
    const size_t units = (out + 15) / 16 * (in / 256);
    return mul_overflows(units, unit) ? 0 : units * unit;
}

extern "C" int kdq_gguf_pack(int encoding, const void* weights, size_t row_bytes, size_t in,
                             size_t out, void* packed, void* stream) {
    if (!block_values(encoding))
        return KDQ_ERR_UNSUPPORTED;
    if (!weights || !packed || !in || !out)
        return KDQ_ERR_ARGUMENT;
    const size_t bytes = kdq_gguf_packed_bytes(encoding, in, out);
    if (!bytes || row_bytes < in / block_values(encoding) * block_bytes(encoding))
        return KDQ_ERR_SHAPE;
    if (mul_overflows(out, row_bytes))
        return KDQ_ERR_ARGUMENT;
    if (!aligned(packed, 16))
        return KDQ_ERR_ALIGNMENT;
    if (overlaps(packed, bytes, weights, out * row_bytes))
        return KDQ_ERR_ALIAS;
    auto s = static_cast<hipStream_t>(stream);
    switch (encoding) {
    case KDQ_Q8_0:
        return launch_pack<KDQ_Q8_0>(weights, row_bytes, in, out, packed, s);
    case KDQ_Q4_0:
        return launch_pack<KDQ_Q4_0>(weights, row_bytes, in, out, packed, s);
    case KDQ_Q4_K:
        return launch_pack<KDQ_Q4_K>(weights, row_bytes, in, out, packed, s);
    case KDQ_Q6_K:
        return launch_pack<KDQ_Q6_K>(weights, row_bytes, in, out, packed, s);
    default:
        return KDQ_ERR_UNSUPPORTED;
    }
}

namespace kdq {
namespace {

// Argument checks of the packed product entry points (check_product with the packed
// size in place of out * row_bytes, and 16-byte aligned packed weights).
int check_packed(int encoding, const void* packed, const float* x, size_t rows, size_t in,
                 size_t out, const float* y, size_t stride) {
    if (!block_values(encoding))
        return KDQ_ERR_UNSUPPORTED;
    if (!packed || !x || !y || !rows || !in || !out)
        return KDQ_ERR_ARGUMENT;
    const size_t bytes = kdq_gguf_packed_bytes(encoding, in, out);
    if (!bytes || stride < out || rows > 4096)
        return KDQ_ERR_SHAPE;
    if (mul_overflows(rows, in) || mul_overflows(rows, stride))
        return KDQ_ERR_ARGUMENT;
    const size_t ybytes = ((rows - 1) * stride + out) * sizeof(float);
    if (overlaps(y, ybytes, packed, bytes) || overlaps(y, ybytes, x, rows * in * sizeof(float)))
        return KDQ_ERR_ALIAS;
    if (!aligned(x, 16) || !aligned(packed, 16))
        return KDQ_ERR_ALIGNMENT;
    return KDQ_OK;
}

}  // namespace
}  // namespace kdq

extern "C" int kdq_gemv_packed_supported(int encoding, size_t in) {
    MfmaPlan p;
    return kdq_gguf_packed_bytes(encoding, in, 16) != 0 && plan_mfma(1, in, 16, p, true) ? 1 : 0;
}

extern "C" int kdq_gemv_packed(int encoding, const void* packed, const float* x, size_t rows,
                               size_t in, size_t out, float* y, size_t stride,
                               unsigned* status, void* stream) {
    const int rc = check_packed(encoding, packed, x, rows, in, out, y, stride);
    if (rc)
        return rc;
    // no other kernel reads the packed layout: shapes beyond the MFMA kernel's LDS
    // (in above ~32K values) are unsupported here
    return launch_mfma_any<true>(encoding, packed, 0, x, rows, in, out, y, stride, status,
                                 static_cast<hipStream_t>(stream));
}

namespace kdq {
namespace {

// One fused MFMA launch for jobs[idx[0..n)] (same encoding, rows, in; checked).
template <bool PACKED>
int launch_fused(const kdq_matvec_job* jobs, const size_t* idx, size_t n, hipStream_t stream,
                 const IndexedJob* indexed = nullptr) {
    const kdq_matvec_job& j0 = jobs[idx[0]];
    size_t total = 0;
    for (size_t k = 0; k < n; ++k)
        total += jobs[idx[k]].columns;
    const unsigned mats = indexed && indexed[idx[0]].paired ? 2 : 1;  // one kind per launch
    MfmaPlan p;
    if (!plan_mfma(j0.rows, j0.in, total, p, PACKED, mats, mfma_table_bytes(j0.encoding)))
        return KDQ_ERR_UNSUPPORTED;
    MfmaJobs mj{};
    mj.count = unsigned(n);
    mj.in = j0.in;
    mj.mats = mats;
    for (size_t k = 0; k < n; ++k) {
        const kdq_matvec_job& j = jobs[idx[k]];
        mj.job[k] = MfmaJob{static_cast<const uint8_t*>(j.weights), j.input, j.output,
                            j.status, PACKED ? 0 : j.row_bytes, j.stride, j.columns, 0};
        if (indexed) {
            mj.job[k].index = indexed[idx[k]].index;
            mj.job[k].index_stride = indexed[idx[k]].index_stride;
            mj.job[k].index_limit = indexed[idx[k]].index_limit;
            mj.job[k].up = static_cast<const uint8_t*>(indexed[idx[k]].paired);
        }
    }
    number_workgroups(mj, p.rows_per_wg);
    switch (j0.encoding) {
    case KDQ_Q8_0:
        return launch_mfma_rows<KDQ_Q8_0, PACKED>(j0.rows, p.waves, mj, stream);
    case KDQ_Q4_0:
        return launch_mfma_rows<KDQ_Q4_0, PACKED>(j0.rows, p.waves, mj, stream);
    case KDQ_Q4_K:
        return launch_mfma_rows<KDQ_Q4_K, PACKED>(j0.rows, p.waves, mj, stream);
    case KDQ_Q6_K:
        return launch_mfma_rows<KDQ_Q6_K, PACKED>(j0.rows, p.waves, mj, stream);
    case KDQ_IQ4_XS:
        if constexpr (!PACKED)
            return launch_mfma_rows<KDQ_IQ4_XS, false>(j0.rows, p.waves, mj, stream);
        return KDQ_ERR_UNSUPPORTED;
    case KDQ_IQ4_NL:
        if constexpr (!PACKED)
            return launch_mfma_rows<KDQ_IQ4_NL, false>(j0.rows, p.waves, mj, stream);
        return KDQ_ERR_UNSUPPORTED;
    case KDQ_Q3_K:
        if constexpr (!PACKED)
            return launch_mfma_rows<KDQ_Q3_K, false>(j0.rows, p.waves, mj, stream);
        return KDQ_ERR_UNSUPPORTED;
    case KDQ_IQ3_XXS:
        if constexpr (!PACKED)
            return launch_mfma_rows<KDQ_IQ3_XXS, false>(j0.rows, p.waves, mj, stream);
        return KDQ_ERR_UNSUPPORTED;
    case KDQ_IQ3_S:
        if constexpr (!PACKED)
            return launch_mfma_rows<KDQ_IQ3_S, false>(j0.rows, p.waves, mj, stream);
        return KDQ_ERR_UNSUPPORTED;
    case KDQ_IQ2_S:
        if constexpr (!PACKED)
            return launch_mfma_rows<KDQ_IQ2_S, false>(j0.rows, p.waves, mj, stream);
        return KDQ_ERR_UNSUPPORTED;
    default:
        return KDQ_ERR_UNSUPPORTED;
    }
}

// Jobs the fused launch takes: shapes whose rows fit one pass of the MFMA kernel (1, 2,
// 4 or 8 rows, within its LDS batch), streaming ones when the weights are row-major.
bool fusable(const kdq_matvec_job& j, bool packed) {
    MfmaPlan p;
    return (packed || streams(j.encoding, j.weights, j.row_bytes, j.in)) &&
           (j.rows & (j.rows - 1)) == 0 &&
           plan_mfma(j.rows, j.in, j.columns, p, packed, 1, mfma_table_bytes(j.encoding)) &&
           p.batch >= j.rows;
}

// kdq_gemv_batch / kdq_gemv_packed_batch after validation: jobs of one shape (encoding,
// rows, in) run together, up to kMaxFused per launch, in submission order; the rest one
// launch each.
template <bool PACKED>
int run_batch(const kdq_matvec_job* jobs, size_t count, void* stream) {
    auto s = static_cast<hipStream_t>(stream);
    std::vector<char> done(count, 0);
    for (size_t i = 0; i < count; ++i) {
        if (done[i] || !fusable(jobs[i], PACKED))
            continue;
        size_t idx[kMaxFused], n = 0;
        for (size_t k = i; k < count && n < size_t(kMaxFused); ++k) {
            const auto& a = jobs[i];
            const auto& b = jobs[k];
            if (!done[k] && b.encoding == a.encoding && b.rows == a.rows && b.in == a.in &&
                fusable(b, PACKED))
                idx[n++] = k;
        }
        const int rc = launch_fused<PACKED>(jobs, idx, n, s);
        if (rc)
            return rc;
        for (size_t k = 0; k < n; ++k)
            done[idx[k]] = 1;
    }
    for (size_t i = 0; i < count; ++i) {
        if (done[i])
            continue;
        const auto& j = jobs[i];
        const int rc =
            PACKED ? kdq_gemv_packed(j.encoding, j.weights, j.input, j.rows, j.in, j.columns,
                                     j.output, j.stride, j.status, stream)
                   : kdq_gemv(j.encoding, j.weights, j.row_bytes, j.input, j.rows, j.in,
                              j.columns, j.output, j.stride, j.status, stream);
        if (rc)
            return rc;
    }
    return KDQ_OK;
}

}  // namespace

bool swiglu_pairable(const kdq_matvec_job& j, size_t count) {
    MfmaPlan p;
    return fusable(j, false) &&
           plan_mfma(j.rows, j.in, size_t(j.columns) * count, p, false, 2,
                     mfma_table_bytes(j.encoding)) &&
           p.batch >= j.rows;
}

int indexed_gemv_affine(const IndexedJob& first, unsigned count, size_t x_step,
                        size_t y_step, hipStream_t s, unsigned x_every) {
    const kdq_matvec_job& j = first.job;
    if (count > 65535 || !x_every)
        return KDQ_ERR_UNSUPPORTED;
    if (count == 1)
        return indexed_gemv_batch(&first, 1, s);
    const unsigned mats = first.paired ? 2 : 1;
    MfmaPlan p;  // planned over every job's rows, as launch_fused plans a fused group
    if (fusable(j, false) &&
        plan_mfma(j.rows, j.in, size_t(j.columns) * count, p, false, mats,
                  mfma_table_bytes(j.encoding)) &&
        p.batch >= j.rows) {
        MfmaJobs mj{};
        mj.count = count;
        mj.in = j.in;
        mj.affine = 1;
        mj.x_every = x_every;
        mj.mats = mats;
        mj.x_step = x_step;
        mj.y_step = y_step;
        mj.job[0] = MfmaJob{static_cast<const uint8_t*>(j.weights), j.input, j.output, j.status,
                            j.row_bytes, j.stride, j.columns, first.index ? first.index_limit : 0,
                            first.index, first.index_stride,
                            static_cast<const uint8_t*>(first.paired)};
        number_workgroups(mj, p.rows_per_wg);
        switch (j.encoding) {
        case KDQ_Q8_0:
            return launch_mfma_rows<KDQ_Q8_0, false>(j.rows, p.waves, mj, s);
        case KDQ_Q4_0:
            return launch_mfma_rows<KDQ_Q4_0, false>(j.rows, p.waves, mj, s);
        case KDQ_Q4_K:
            return launch_mfma_rows<KDQ_Q4_K, false>(j.rows, p.waves, mj, s);
        case KDQ_Q6_K:
            return launch_mfma_rows<KDQ_Q6_K, false>(j.rows, p.waves, mj, s);
        case KDQ_IQ4_XS:
            return launch_mfma_rows<KDQ_IQ4_XS, false>(j.rows, p.waves, mj, s);
        case KDQ_IQ4_NL:
            return launch_mfma_rows<KDQ_IQ4_NL, false>(j.rows, p.waves, mj, s);
        case KDQ_Q3_K:
            return launch_mfma_rows<KDQ_Q3_K, false>(j.rows, p.waves, mj, s);
        case KDQ_IQ3_XXS:
            return launch_mfma_rows<KDQ_IQ3_XXS, false>(j.rows, p.waves, mj, s);
        case KDQ_IQ3_S:
            return launch_mfma_rows<KDQ_IQ3_S, false>(j.rows, p.waves, mj, s);
        case KDQ_IQ2_S:
            return launch_mfma_rows<KDQ_IQ2_S, false>(j.rows, p.waves, mj, s);
        default:
            return KDQ_ERR_UNSUPPORTED;
        }
    }
    if (first.paired)
        return KDQ_ERR_UNSUPPORTED;  // the exact kernel has no paired form
    return with_encoding(j.encoding, [&](auto enc) {
        return launch_exact<decltype(enc)::value>(j.weights, j.row_bytes, j.input, j.rows, j.in,
                                                  j.columns, j.output, j.stride, j.status, s,
                                                  first.index, first.index_stride,
                                                  first.index ? first.index_limit : 1u, count,
                                                  x_step, y_step, x_every);
    });
}

int indexed_gemv_affine_packed(const IndexedJob& first, unsigned count, size_t x_step,
                               size_t y_step, hipStream_t s, unsigned x_every) {
    const kdq_matvec_job& j = first.job;
    const unsigned mats = first.paired ? 2 : 1;
    MfmaPlan p;
    if (count > 65535 || !x_every || !packed_unit(j.encoding) || j.columns % 16 ||
        (j.rows & (j.rows - 1)) != 0 ||
        !plan_mfma(j.rows, j.in, size_t(j.columns) * count, p, true, mats, 0) ||
        p.batch < j.rows)
        return KDQ_ERR_UNSUPPORTED;
    MfmaJobs mj{};
    mj.count = count;
    mj.in = j.in;
    mj.affine = 1;
    mj.x_every = x_every;
    mj.mats = mats;
    mj.x_step = x_step;
    mj.y_step = y_step;
    mj.job[0] = MfmaJob{static_cast<const uint8_t*>(j.weights), j.input, j.output, j.status,
                        0, j.stride, j.columns, first.index ? first.index_limit : 0,
                        first.index, first.index_stride,
                        static_cast<const uint8_t*>(first.paired)};
    number_workgroups(mj, p.rows_per_wg);
    switch (j.encoding) {
    case KDQ_Q8_0:
        return launch_mfma_rows<KDQ_Q8_0, true>(j.rows, p.waves, mj, s);
    case KDQ_Q4_0:
        return launch_mfma_rows<KDQ_Q4_0, true>(j.rows, p.waves, mj, s);
    case KDQ_Q4_K:
        return launch_mfma_rows<KDQ_Q4_K, true>(j.rows, p.waves, mj, s);
    case KDQ_Q6_K:
        return launch_mfma_rows<KDQ_Q6_K, true>(j.rows, p.waves, mj, s);
    default:
        return KDQ_ERR_UNSUPPORTED;
    }
}

int indexed_gemv_batch(const IndexedJob* jobs, size_t count, hipStream_t s) {
    std::vector<kdq_matvec_job> plain(count);
    for (size_t i = 0; i < count; ++i)
        plain[i] = jobs[i].job;
    std::vector<char> done(count, 0);
    for (size_t i = 0; i < count; ++i) {  // fused MFMA launches, as run_batch groups them
        if (done[i] || !fusable(plain[i], false))
            continue;
        size_t idx[kMaxFused], n = 0;
        for (size_t k = i; k < count && n < size_t(kMaxFused); ++k)
            if (!done[k] && plain[k].encoding == plain[i].encoding &&
                plain[k].rows == plain[i].rows && plain[k].in == plain[i].in &&
                !jobs[k].paired == !jobs[i].paired && fusable(plain[k], false))
                idx[n++] = k;
        const int rc = launch_fused<false>(plain.data(), idx, n, s, jobs);
        if (rc)
            return rc;
        for (size_t k = 0; k < n; ++k)
            done[idx[k]] = 1;
    }
    for (size_t i = 0; i < count; ++i) {
        if (done[i])
            continue;
        const IndexedJob& ij = jobs[i];
        const kdq_matvec_job& j = ij.job;
        if (ij.paired)
            return KDQ_ERR_UNSUPPORTED;  // the exact kernel has no paired form
        const int rc = with_encoding(j.encoding, [&](auto enc) {
            return launch_exact<decltype(enc)::value>(j.weights, j.row_bytes, j.input, j.rows,
                                                      j.in, j.columns, j.output, j.stride,
                                                      j.status, s, ij.index, ij.index_stride,
                                                      ij.index ? ij.index_limit : 1u);
        });
        if (rc)
            return rc;
    }
    return KDQ_OK;
}

// ----------------------------------------------------------------- fused MoE decode

namespace {

#include "kdq_route.hpp"

// The fused decode's device-wide state (one copy per GPU, zero at load): the epoch of the
// last completed call (the down launch advances it, so a call's up launch reads the same
// value in every workgroup, and a replayed graph of the launches still numbers each call
// anew), the router workgroups' completion count (the last one resets it) and, per
// (token, slot), the published selection: (epoch << 8) | expert.  Calls that overlap on
// one GPU race on them (and on the workspace), as on the rest of the library's scratch.
// Kernels take its address as an argument (DecodeRoute::state), not through the symbol.
constexpr unsigned kDecodeTokens = kFusedDecodeTokens;
struct DecodeState {
    unsigned epoch;
    unsigned router_arrived;
    unsigned routed_slot[kDecodeTokens * kMaxFused];  // token t's slot i at t * top_k + i
};
__device__ DecodeState g_decode_state;

// This call's epoch: one past the last completed call's, 24 bits, never 0 (the
// published words start at 0 and unused ones are cleared to 0).
__device__ __forceinline__ unsigned call_epoch(const DecodeState* state) {
    const unsigned e =
        (__hip_atomic_load(&state->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1) &
        0xffffffu;
    return e ? e : 1u;
}

struct DecodeRoute {
    const uint8_t* router;  // F32 rows [experts][row_bytes]
    size_t router_row_bytes;
    unsigned router_workgroups;  // the grid's first workgroups: one router row per wavefront
    DecodeState* state;          // this device's g_decode_state
    float* logits;
    unsigned experts, top_k, tokens;
    int32_t* idx;
    float* w;
    unsigned* counters;
    unsigned counter_count;
    // the shared expert's gate sigmoid(gate_vector . x), taken once for the down launch
    const float* gate_vector;
    const float* x;
    unsigned hidden;
    float* gate;
    unsigned* status;
};

// *out = sigmoid(v . x) over `hidden` values by threads 0..255 of the workgroup, in
// combine_kernel's order (a thread's float4 columns j, j + 256, ... with the four products
// of each fused in turn, an xor butterfly per wavefront, then (0 + 1) + (2 + 3)), so the
// fused and the separate decode take the same value; a non-finite entry of v sets bit 1
// of *status.  Every thread of the workgroup calls it.
__device__ __forceinline__ void shared_gate(const float* __restrict__ v,
                                            const float* __restrict__ x, unsigned hidden,
                                            float* out, unsigned* status) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    __shared__ float wave_sum[4];
    __shared__ int wave_bad[4];
    if (threadIdx.x < 256) {
        const f32x4* xr = reinterpret_cast<const f32x4*>(x);
        const f32x4* vr = reinterpret_cast<const f32x4*>(v);
        float s = 0.f;
        bool finite = true;
        for (unsigned q = threadIdx.x; q < hidden / 4; q += 256) {
            const f32x4 a = xr[q], b = vr[q];
            finite = finite && isfinite(b.x) && isfinite(b.y) && isfinite(b.z) && isfinite(b.w);
            s = fmaf(a.x, b.x, s);
            s = fmaf(a.y, b.y, s);
            s = fmaf(a.z, b.z, s);
            s = fmaf(a.w, b.w, s);
        }
        for (int m = 32; m >= 1; m /= 2)
            s += __shfl_xor(s, m, 64);
        const bool bad = __any(!finite);
        if (threadIdx.x % 64 == 0) {
            wave_sum[threadIdx.x / 64] = s;
            wave_bad[threadIdx.x / 64] = bad;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        *out = sigmoid_of((wave_sum[0] + wave_sum[1]) + (wave_sum[2] + wave_sum[3]));
        if (status && (wave_bad[0] | wave_bad[1] | wave_bad[2] | wave_bad[3]))
            atomicOr(status, 1u);
    }
}

// Bounded wait for the routing: about 2^20 sleeps of 64 clocks (tens of ms); past it
// the workgroup goes on with expert 0 and sets status bit 3 (a routing that never came).
constexpr unsigned kRouteSpinLimit = 1u << 20;

// Workgroups [0, router_workgroups): the router GEMV, one F32 row per wavefront in
// exact_gemv<KDQ_F32, 1>'s arithmetic (the same logits as the staged path), stored at
// device scope; the last of them to finish routes the tokens (route_select_wg, the whole
// workgroup, for one; route_select, a wavefront each, for several) and publishes each
// (token, slot)'s expert with this call's epoch.
// Then the experts' paired gate / up workgroups (job step = slot): their activation
// loads go out first, then thread 0 waits for the epoch and reads its slot's expert.
// Then the shared expert's paired gate / up; its first workgroup also takes the gate
// scalar.  The router workgroups come first in the grid, so they are dispatched before
// any workgroup that waits on them.
template <int EA, bool PA, int EB, int W>
__global__ __launch_bounds__(W * 64) void moe_decode_up_kernel(const MfmaJobs a,
                                                               const MfmaJobs b,
                                                               const DecodeRoute route) {
    __shared__ int chosen;
    __shared__ unsigned arrived;
    const unsigned wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    if (blockIdx.x < route.router_workgroups) {
        // x of every token staged in LDS (its first bytes; the routing's scratch later
        // reuses them)
        extern __shared__ __align__(16) uint8_t lds[];
        float4* xs = reinterpret_cast<float4*>(lds);
        const unsigned column = blockIdx.x * W + wave;
        const u32x4* row = reinterpret_cast<const u32x4*>(
            route.router + size_t(min(column, route.experts - 1)) * route.router_row_bytes);
        // chunks of 8 values a lane (hidden <= 4096: at most 8), four at a time: the four
        // chunks' loads all issued (at clamped, in-bounds addresses), then the products of
        // the lane's valid ones in exact_gemv's order, one chain per token
        constexpr int kChunks = 8, kBatch = 4;
        u32x4 wv[kBatch][2];
        auto load_batch = [&](int c0) {
#pragma unroll
            for (int c = 0; c < kBatch; ++c) {
                const unsigned i = min(lane * 8 + (c0 + c) * 512, a.in - 8);
                wv[c][0] = row[i / 4];
                wv[c][1] = row[i / 4 + 1];
            }
        };
        load_batch(0);
        for (unsigned q = threadIdx.x; q < route.tokens * a.in / 4; q += W * 64)
            xs[q] = reinterpret_cast<const float4*>(route.x)[q];
        __syncthreads();
        if (column < route.experts) {
            float sum[kDecodeTokens] = {};
            bool finite = true;
#pragma unroll
            for (int c0 = 0; c0 < kChunks; c0 += kBatch) {
                if (c0 * 512 >= a.in)
                    break;  // uniform: lane 0 has the lowest index
                if (c0 > 0)
                    load_batch(c0);
                // every value here (the compiler would otherwise sink each chunk's loads
                // into its guarded products: one memory round trip per chunk)
#pragma unroll
                for (int c = 0; c < kBatch; ++c)
                    asm volatile("" : "+v"(wv[c][0]), "+v"(wv[c][1]));
#pragma unroll
                for (int c = 0; c < kBatch; ++c) {
                    const unsigned i = lane * 8 + (c0 + c) * 512;
                    if (i >= a.in)
                        break;
                    float w[8];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        w[k] = __uint_as_float(wv[c][0][k]);
                        w[4 + k] = __uint_as_float(wv[c][1][k]);
                    }
#pragma unroll
                    for (int k = 0; k < 8; ++k)
                        finite = finite && isfinite(w[k]);
#pragma unroll
                    for (unsigned t = 0; t < kDecodeTokens; ++t) {
                        if (t >= route.tokens)
                            break;  // uniform
                        const float4 x0 = xs[(t * a.in + i) / 4], x1 = xs[(t * a.in + i) / 4 + 1];
                        const float xr[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                        for (int k = 0; k < 8; ++k)
                            sum[t] = fmaf(w[k], xr[k], sum[t]);
                    }
                }
            }
            if (route.status && __any(!finite) && lane == 0)
                atomicOr(route.status, 1u);
#pragma unroll
            for (unsigned t = 0; t < kDecodeTokens; ++t) {
                if (t >= route.tokens)
                    break;
                const float total = wave_sum(sum[t]);
                if (lane == 0)
                    __hip_atomic_store(&route.logits[size_t(t) * route.experts + column], total,
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the logits stored first
        __syncthreads();
        if (threadIdx.x == 0)
            arrived = atomicAdd(&route.state->router_arrived, 1u);
        __syncthreads();
        if (arrived != route.router_workgroups - 1)
            return;
        // the routing, its LDS the GEMV's, no longer used: one token by the whole
        // workgroup, several by a wavefront each; then each slot's word, this call's epoch
        // and its expert
        int e = 0;
        float we = 0.f;
        const unsigned epoch = call_epoch(route.state);
        auto publish = [&](unsigned token, unsigned slot) {
            const unsigned at = token * route.top_k + slot;
            __hip_atomic_store(&route.idx[at], e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&route.w[at], we, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&route.state->routed_slot[at], (epoch << 8) | unsigned(e),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        };
        // words past this call's slots: cleared, so an old word can never carry a later
        // call's epoch (the epoch wraps after 2^24 calls)
        for (unsigned i = route.tokens * route.top_k + threadIdx.x;
             i < kDecodeTokens * kMaxFused; i += W * 64)
            __hip_atomic_store(&route.state->routed_slot[i], 0u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        if (route.tokens == 1) {
            route_select_wg<W, kMaxFused, true>(route.logits, route.experts, route.top_k,
                                                *reinterpret_cast<RouteScratch*>(lds), e, we);
            if (threadIdx.x < route.top_k)
                publish(0, threadIdx.x);
        } else if (wave < route.tokens) {
            route_select<true>(route.logits, wave, route.experts, route.top_k, lane, e, we);
            if (lane < route.top_k)
                publish(wave, lane);
        }
        for (unsigned i = threadIdx.x; i < route.counter_count; i += W * 64)
            route.counters[i] = 0u;
        if (threadIdx.x == 0)
            route.state->router_arrived = 0u;
        return;
    }
    const unsigned a_workgroups = a.columns * a.count;
    const unsigned id = blockIdx.x - route.router_workgroups;
    if (id < a_workgroups) {
        const unsigned slot = id / a.columns;
        // the slot's expert, once the routing is published (the activation loads are in
        // flight meanwhile)
        auto late = [&]() -> int {
            if (threadIdx.x == 0) {
                const unsigned epoch = call_epoch(route.state);
                unsigned spins = 0, word;
                const unsigned* published = &route.state->routed_slot[slot];
                while (((word = __hip_atomic_load(published, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT)) >> 8) !=
                       epoch) {
                    if (++spins == kRouteSpinLimit) {
                        if (route.status)
                            atomicOr(route.status, 8u);
                        word = 0;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                chosen = int(word & 0xffu);
            }
            __syncthreads();
            return chosen;
        };
        mfma_gemv_body<EA, 1, W, PA, 0, false, decltype(late)>(a, id % a.columns, slot, -1,
                                                               late);
    } else {
        const unsigned k = id - a_workgroups;
        if (k < route.tokens) {  // token k's gate scalar
            shared_gate(route.gate_vector, route.x + size_t(k) * route.hidden, route.hidden,
                        route.gate + k, route.status);
            __syncthreads();  // its LDS words before the product's
        }
        mfma_gemv_body<EB, 1, W, false, 0>(b, k % b.columns, k / b.columns, -1);
    }
}

// y of each token = sum over its selections, in selection order, of down * weight, plus
// shared_down * sigmoid(gate_vector . x), as combine_kernel computes it.
struct DecodeCombine {
    const float* down;    // [tokens][top_k][hidden]
    const float* shared;  // [tokens][hidden]
    const float* w;       // [tokens][top_k]
    const float* gate;    // [tokens]: sigmoid(gate_vector . x), from the up launch
    unsigned top_k, hidden;
    float* y;             // [tokens][hidden]
    unsigned* counters;   // one per (token, row block), zero on entry
    DecodeState* state;   // its epoch advanced here, after every up workgroup has read it
};

// Workgroups [0, a.columns * a.count) run the experts' down rows (job step = token *
// top_k + slot), the rest the shared down (job step = token); both halves cut the hidden
// rows into the same blocks of a.rows_per_wg.  Each workgroup then counts itself into its
// token's row block; the last of the top_k + 1 to arrive (its fences make the others'
// stored rows visible) combines that block, so the layer needs no launch of its own for
// the combine.  The sum runs in the fixed selection order whichever workgroup is last.
template <int EA, bool PA, int EB, int W>
__global__ __launch_bounds__(W * 64) void moe_decode_down_kernel(const MfmaJobs a,
                                                                 const MfmaJobs b,
                                                                 const DecodeCombine c) {
    __shared__ unsigned arrived;
    if (blockIdx.x == 0 && threadIdx.x == 0)
        __hip_atomic_store(&c.state->epoch, call_epoch(c.state), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    const unsigned a_workgroups = a.columns * a.count;
    unsigned block, token;
    if (blockIdx.x < a_workgroups) {
        block = blockIdx.x % a.columns;
        const unsigned step = blockIdx.x / a.columns;
        token = step / c.top_k;
        mfma_gemv_body<EA, 1, W, PA, 0, true>(a, block, step, -1);
    } else {
        const unsigned k = blockIdx.x - a_workgroups;
        block = k % b.columns;
        token = k / b.columns;
        mfma_gemv_body<EB, 1, W, false, 0, true>(b, block, token, -1);
    }
    unsigned* counter = &c.counters[token * a.columns + block];
    // The rows went out as device-scope stores; once every one of them has completed
    // (the wait below, then the barrier) the count may announce them.  The combining
    // workgroup reads them with device-scope loads.  No cache-wide fence: one per
    // workgroup (an L2 write-back and invalidate each) cost more than the layer.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0)
        arrived = atomicAdd(counter, 1u);
    __syncthreads();
    if (arrived != c.top_k)
        return;  // the whole workgroup: another one combines this block

    const float gate = c.gate[token];
    const float* down = c.down + size_t(token) * c.top_k * c.hidden;
    const float* shared = c.shared + size_t(token) * c.hidden;
    const float* w = c.w + size_t(token) * c.top_k;
    float* y = c.y + size_t(token) * c.hidden;
    const unsigned r0 = block * a.rows_per_wg, r1 = min(c.hidden, r0 + a.rows_per_wg);
    auto coherent = [](const float* p) {
        return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    for (unsigned r = r0 + threadIdx.x; r < r1; r += W * 64) {
        // the row's top_k + 1 loads all issued (clamped to the last slot), then the sum
        float v[kMaxFused + 1];
#pragma unroll
        for (int i = 0; i < kMaxFused; ++i)
            v[i] = coherent(down + size_t(min(unsigned(i), c.top_k - 1)) * c.hidden + r);
        v[kMaxFused] = coherent(shared + r);
#pragma unroll
        for (int i = 0; i <= kMaxFused; ++i)
            asm volatile("" : "+v"(v[i]));
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < kMaxFused; ++i)
            if (unsigned(i) < c.top_k)
                sum += v[i] * w[i];
        y[r] = sum + v[kMaxFused] * gate;
    }
    if (threadIdx.x == 0)
        *counter = 0u;  // ready for the next layer call
}

// An affine launch over `count` slots of one token (job step = slot; x rows x_step apart,
// a new one every x_every slots; y rows y_step apart), as indexed_gemv_affine(_packed)
// builds it; false when the MFMA kernel does not take it.
bool decode_half(const IndexedJob& ij, unsigned count, size_t x_step, unsigned x_every,
                 size_t y_step, bool packed, MfmaJobs& mj, MfmaPlan& p) {
    const kdq_matvec_job& j = ij.job;
    const unsigned mats = ij.paired ? 2 : 1;
    if (j.rows != 1 || mfma_table_bytes(j.encoding) ||
        (packed ? (!packed_unit(j.encoding) || j.columns % 16) : !fusable(j, false)) ||
        !plan_mfma(1, j.in, size_t(j.columns) * count, p, packed, mats, 0))
        return false;
    mj = MfmaJobs{};
    mj.count = count;
    mj.in = j.in;
    mj.affine = count > 1 || ij.index ? 1 : 0;
    mj.x_every = x_every;
    mj.mats = mats;
    mj.x_step = x_step;
    mj.y_step = y_step;
    mj.job[0] = MfmaJob{static_cast<const uint8_t*>(j.weights), j.input, j.output, j.status,
                        packed ? 0 : j.row_bytes, j.stride, j.columns,
                        ij.index ? ij.index_limit : 0, ij.index, ij.index_stride,
                        static_cast<const uint8_t*>(ij.paired)};
    number_workgroups(mj, p.rows_per_wg);
    return true;
}

// the fused decode kernels keep a few static LDS words beside the dynamic area
constexpr int kDecodeDynamicLds = 159 * 1024;

template <int EA, bool PA, int EB, int W>
int launch_decode_up(const MfmaJobs& a, const MfmaJobs& b, const DecodeRoute& r, size_t lds,
                     hipStream_t s) {
    static bool configured = false;
    if (!configured) {
        KDQ_HIP(hipFuncSetAttribute(
            reinterpret_cast<const void*>(&moe_decode_up_kernel<EA, PA, EB, W>),
            hipFuncAttributeMaxDynamicSharedMemorySize, kDecodeDynamicLds));
        configured = true;
    }
    hipLaunchKernelGGL((moe_decode_up_kernel<EA, PA, EB, W>),
                       dim3(r.router_workgroups + a.columns * a.count + b.columns * b.count),
                       dim3(W * 64), lds, s, a, b, r);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}

template <int EA, bool PA, int EB>
int launch_decode_down(const MfmaJobs& a, const MfmaJobs& b, const DecodeCombine& c,
                       size_t lds, hipStream_t s) {
    static bool configured = false;
    if (!configured) {
        KDQ_HIP(hipFuncSetAttribute(
            reinterpret_cast<const void*>(&moe_decode_down_kernel<EA, PA, EB, 4>),
            hipFuncAttributeMaxDynamicSharedMemorySize, kDecodeDynamicLds));
        configured = true;
    }
    hipLaunchKernelGGL((moe_decode_down_kernel<EA, PA, EB, 4>),
                       dim3(a.columns * a.count + b.columns * b.count), dim3(256), lds, s, a,
                       b, c);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}

}  // namespace

int moe_decode_fused(const DecodeMoe& m, hipStream_t s, bool check_only) {
    const unsigned K = m.top_k, T = m.tokens, H = m.hidden;
    // the router's x rows are staged in LDS: at most 64 KB of them
    if (K == 0 || K > unsigned(kMaxFused) || T == 0 || T > kDecodeTokens ||
        m.experts > 256 || H % 4 || size_t(T) * H * 4 > 64 * 1024)
        return KDQ_ERR_UNSUPPORTED;
    MfmaJobs ua, ub, da, db;
    MfmaPlan pua, pub, pda, pdb;
    const size_t F = m.experts_up.job.columns, S = m.shared_up.job.columns;
    // slot j = token * K + i: the expert products read x row j / K and write g row j; the
    // shared ones read x row t and write row t
    if (m.experts_down.job.in != F || m.shared_down.job.in != S ||
        !decode_half(m.experts_up, T * K, H, K, F, m.up_packed, ua, pua) ||
        !decode_half(m.shared_up, T, H, 1, S, false, ub, pub) ||
        !decode_half(m.experts_down, T * K, F, 1, H, m.down_packed, da, pda) ||
        !decode_half(m.shared_down, T, S, 1, H, false, db, pdb))
        return KDQ_ERR_UNSUPPORTED;
    // both halves of a launch: one workgroup size; the down halves cut the hidden rows
    // alike (packed halves: rows per workgroup a multiple of 8)
    if (pua.waves != pub.waves || pua.waves < 8 || pdb.waves != 4 || pda.waves != 4 ||
        m.experts_down.job.columns != m.hidden || m.shared_down.job.columns != m.hidden ||
        !m.experts_up.paired || !m.shared_up.paired || m.experts_down.paired ||
        m.shared_down.paired)
        return KDQ_ERR_UNSUPPORTED;
    const unsigned rows = (std::max(da.rows_per_wg, db.rows_per_wg) + 7) & ~7u;
    number_workgroups(da, rows);
    number_workgroups(db, rows);
    // (the router's staged x and the routing's scratch lie in the same dynamic LDS)
    const size_t up_lds = std::max({mfma_lds(1, ua.in, 2), mfma_lds(1, ub.in, 2),
                                    sizeof(RouteScratch), size_t(T) * H * 4});
    const size_t down_lds = std::max(mfma_lds(1, da.in, 1), mfma_lds(1, db.in, 1));
    if (std::max(up_lds, down_lds) > size_t(kDecodeDynamicLds))
        return KDQ_ERR_UNSUPPORTED;
    const int ea = m.experts_up.job.encoding, eb = m.shared_up.job.encoding;
    const int da_enc = m.experts_down.job.encoding, db_enc = m.shared_down.job.encoding;
    // the instantiated pairs (the Q4_K / Q6_K / Q8_0 mixes of K-quant MoE checkpoints)
    const bool up_ok = ea == KDQ_Q4_K && (eb == KDQ_Q8_0 || eb == KDQ_Q4_K) &&
                       (pua.waves == 8 || pua.waves == 16);
    const bool down_ok = (da_enc == KDQ_Q6_K || da_enc == KDQ_Q4_K) &&
                         (db_enc == KDQ_Q4_K || db_enc == KDQ_Q6_K);
    if (!up_ok || !down_ok || da.columns != db.columns ||
        size_t(T) * da.columns > m.counter_count ||
        m.experts > 256 || m.hidden > 4096 ||
        m.router.encoding != KDQ_F32 || m.router.in != m.hidden ||
        m.router.columns != m.experts || m.router.row_bytes % 16 ||
        reinterpret_cast<uintptr_t>(m.router.weights) % 16 ||
        reinterpret_cast<uintptr_t>(m.x) % 16)
        return KDQ_ERR_UNSUPPORTED;
    constexpr int kDevices = 64;  // per-device state kept for devices 0..63
    int device = 0;
    KDQ_HIP(hipGetDevice(&device));
    if (device < 0 || device >= kDevices)
        return KDQ_ERR_UNSUPPORTED;
    if (check_only)
        return KDQ_OK;

    static std::atomic<DecodeState*> states[kDevices];  // g_decode_state's address
    DecodeState* state = states[device].load();
    if (!state) {
        void* address = nullptr;
        KDQ_HIP(hipGetSymbolAddress(&address, HIP_SYMBOL(g_decode_state)));
        state = static_cast<DecodeState*>(address);
        states[device].store(state);
    }
    const DecodeRoute route{static_cast<const uint8_t*>(m.router.weights),
                            m.router.row_bytes,
                            unsigned((m.experts + pua.waves - 1) / pua.waves),
                            state,
                            m.logits,
                            m.experts,
                            K,
                            T,
                            m.idx,
                            m.w,
                            m.counters,
                            T * da.columns,
                            m.gate_vector,
                            m.x,
                            m.hidden,
                            m.gate,
                            m.status};
    int rc;
    auto up = [&]<bool PA>() -> int {
        if (pua.waves == 8)
            return eb == KDQ_Q8_0 ? launch_decode_up<KDQ_Q4_K, PA, KDQ_Q8_0, 8>(ua, ub, route, up_lds, s)
                                  : launch_decode_up<KDQ_Q4_K, PA, KDQ_Q4_K, 8>(ua, ub, route, up_lds, s);
        return eb == KDQ_Q8_0 ? launch_decode_up<KDQ_Q4_K, PA, KDQ_Q8_0, 16>(ua, ub, route, up_lds, s)
                              : launch_decode_up<KDQ_Q4_K, PA, KDQ_Q4_K, 16>(ua, ub, route, up_lds, s);
    };
    if ((rc = m.up_packed ? up.template operator()<true>() : up.template operator()<false>()))
        return rc;
    const DecodeCombine comb{m.experts_down.job.output, m.shared_down.job.output, m.w, m.gate,
                             K, m.hidden, m.y, m.counters, state};
    auto down = [&]<bool PA>() -> int {
        if (da_enc == KDQ_Q6_K)
            return db_enc == KDQ_Q4_K ? launch_decode_down<KDQ_Q6_K, PA, KDQ_Q4_K>(da, db, comb, down_lds, s)
                                      : launch_decode_down<KDQ_Q6_K, PA, KDQ_Q6_K>(da, db, comb, down_lds, s);
        return db_enc == KDQ_Q4_K ? launch_decode_down<KDQ_Q4_K, PA, KDQ_Q4_K>(da, db, comb, down_lds, s)
                                  : launch_decode_down<KDQ_Q4_K, PA, KDQ_Q6_K>(da, db, comb, down_lds, s);
    };
    return m.down_packed ? down.template operator()<true>() : down.template operator()<false>();
}

}  // namespace kdq

extern "C" int kdq_gemv_batch(const kdq_matvec_job* jobs, size_t count, void* stream) {
    if (count && !jobs)
        return KDQ_ERR_ARGUMENT;
    // Validate the whole submission before the first launch.
    for (size_t i = 0; i < count; ++i) {
        const auto& j = jobs[i];
        const int rc = check_product(j.encoding, j.weights, j.row_bytes, j.input, j.rows, j.in,
                                     j.columns, j.output, j.stride);
        if (rc)
            return rc;
    }
    return run_batch<false>(jobs, count, stream);
}

extern "C" int kdq_gemv_packed_batch(const kdq_matvec_job* jobs, size_t count, void* stream) {
    if (count && !jobs)
        return KDQ_ERR_ARGUMENT;
    for (size_t i = 0; i < count; ++i) {
        const auto& j = jobs[i];
        const int rc = check_packed(j.encoding, j.weights, j.input, j.rows, j.in, j.columns,
                                    j.output, j.stride);
        if (rc)
            return rc;
    }
    return run_batch<true>(jobs, count, stream);
}
