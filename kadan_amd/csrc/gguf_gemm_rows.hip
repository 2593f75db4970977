// Prefill GEMM over row-major GGUF rows for gfx950, any encoding: Y[m, n] (fp32) =
// sum_k X[m, k] W[n, k], W as the file holds it (`row_bytes` per row).
//
// The reference runs prefill chunks by decoding a packed tile to fp32 and calling
// cublasSgemm (IW/src/cuda/h3_compute.cu:2201-2218,2451; IW =
// services/hikari/inference_worker), whatever the encoding.  The packed GEMM
// (gguf_gemm.hip) covers Q4_K, Q8_0 and Q6_K over the bank's tile-packed copy with
// dequantisation specialised per format; this kernel takes every other encoding (Q3_K,
// IQ4_XS, IQ4_NL, IQ3_XXS, IQ3_S, IQ2_S, BF16, Q4_0) through the one exact decoder the
// decode-time products use (decode_run, kdq_decode.hpp), so each weight byte is read once
// per workgroup tile instead of once per 8 activation rows.
//
//   stage_rows_kernel  one workgroup per token row (rows up to the next multiple of 128,
//                      past m zero): the row's power-of-two scale sigma (max|x| / sigma in
//                      [2^14, 2^15), 1 for a row whose maximum is below 2^-100, NaN for a
//                      non-finite row) and fp16(x / sigma) in natural order
//   rows_gemm_kernel   128 weight rows x 128 tokens per workgroup, four wavefronts each
//                      owning one 32-row weight operand and all 128 tokens (four 32-token
//                      blocks).  Per K group (256 values; 64 for BF16) the workgroup copies
//                      its rows' raw block bytes into LDS with 16-byte loads (one group
//                      ahead, double-buffered); per step of 32 values the activations pass
//                      through LDS (double-buffered, swizzled; loaded up to four steps
//                      ahead into a ring of registers); each lane decodes the 8
//                      values of its MFMA A operand (its row, its half of the 16-value
//                      sub-step) with decode_run from the LDS bytes, rounds them to fp16 and
//                      multiplies on v_mfma_f32_32x32x16_f16 with fp32 accumulation.  The
//                      epilogue undoes sigma and stores fp32 rows.  Outputs too narrow to
//                      give every compute unit two workgroups split K into slices whose
//                      fp32 tiles slice_sum_kernel adds in slice order.
//
// Roundings: the activation once to fp16 (after the exact power-of-two scale), each weight
// once, from its exact fp32 decode, to fp16.  *status |= 1 for a non-finite decoded
// weight, |= 2 for a weight past the fp16 range (the caller then takes the exact product).
#include "kdq_common.hpp"

#include <algorithm>
#include <utility>

namespace kdq {
namespace {

#include "kdq_decode.hpp"

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int RM = 128;  // tokens per workgroup: four 32-token blocks
constexpr int RN = 128;  // weight rows per workgroup: one 32-row operand per wavefront
constexpr int RK = 32;   // K values per step: two 16-value MFMA sub-steps
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;

// K values per staged group and the LDS bytes of one row's group: an odd number of 16-byte
// chunks, so the 32 rows a wavefront decodes at one offset spread over the banks (a
// 128-byte pitch put every row of a 16-byte read on the same banks: measured 55 % of the
// LDS cycles in bank conflicts for BF16).
template <int ENC> struct RowsGroup {
    static constexpr int values = Format<ENC>::values == 1 ? 64 : 256;
    static constexpr int bytes = values / Format<ENC>::values * Format<ENC>::bytes;
    static constexpr int pitch = ((bytes + 15) / 16 | 1) * 16;
    static constexpr int chunks = RN * pitch / 16;  // 16-byte copies per group
    static constexpr int per_thread = (chunks + kThreads - 1) / kThreads;
};

// The lattice encodings' grids as LDS tables: per grid entry its level magnitudes as
// bytes (IQ3_XXS 256 and IQ3_S 512 entries of 4, IQ2_S 1024 entries of 8).
template <int ENC> constexpr unsigned lattice_rows_entries =
    ENC == KDQ_IQ3_XXS ? 256 : ENC == KDQ_IQ3_S ? 512 : ENC == KDQ_IQ2_S ? 1024 : 0;
template <int ENC> constexpr unsigned lattice_rows_width = ENC == KDQ_IQ2_S ? 8 : 4;
template <int ENC> constexpr size_t lattice_rows_bytes =
    size_t(lattice_rows_entries<ENC>) * lattice_rows_width<ENC>;

template <int ENC> constexpr size_t rows_lds = 2 * size_t(RN) * RowsGroup<ENC>::pitch +
                                               2 * size_t(RM) * RK * 2 + lattice_rows_bytes<ENC>;

// Fills the LDS grid table (every thread of the workgroup; a barrier follows before use):
// entry i's level indices (3 or 2 bits each, as iq_grids.inc encodes them) as the levels
// themselves, kIq3xxsGridLevels / kIq3sGridLevels / kIq2sGridLevels, one byte each.
template <int ENC> __device__ __forceinline__ void lattice_rows_table(uint8_t* table) {
    constexpr unsigned E = lattice_rows_entries<ENC>, Wd = lattice_rows_width<ENC>;
    constexpr unsigned bits = ENC == KDQ_IQ2_S ? 2 : 3;
    for (unsigned i = threadIdx.x; i < E; i += kThreads) {
        const unsigned entry = ENC == KDQ_IQ3_XXS ? kIq3xxsGrid[i]
                               : ENC == KDQ_IQ3_S ? kIq3sGrid[i]
                                                  : kIq2sGrid[i];
        unsigned w[2] = {0u, 0u};
#pragma unroll
        for (unsigned b = 0; b < Wd; ++b) {
            const unsigned li = (entry >> (bits * b)) & ((1u << bits) - 1);
            const unsigned level = ENC == KDQ_IQ3_XXS ? kIq3xxsGridLevels[li]
                                   : ENC == KDQ_IQ3_S ? kIq3sGridLevels[li]
                                                      : kIq2sGridLevels[li];
            w[b / 4] |= level << (8 * (b % 4));
        }
        if constexpr (Wd == 8)
            reinterpret_cast<uint2*>(table)[i] = make_uint2(w[0], w[1]);
        else
            reinterpret_cast<unsigned*>(table)[i] = w[0];
    }
}

// ----------------------------------------------------------- operand decode

// A lane's 8 fp16 weights: fp16 of each value exactly as decode_run gives it (the same
// fp32 operations in the same order), from the row's raw group bytes in LDS.  The
// encodings below read whole code words and look values up four at a time; their range
// flags are taken once per call from the block scale: `nonfinite` for a non-finite
// scale, `wide` when the scale could take a weight past the fp16 range (the largest code
// times |scale| above 65504, as the packed GEMM checks it); their fp16 scales convert in
// hardware (exact for every finite half; a NaN stays a NaN).  Other encodings decode
// value by value and check each value; BF16 checks its bits.
struct RowFlags {
    bool nonfinite = false, wide = false;
    unsigned bf16_max = 0;  // BF16: the largest |bits| seen (two 16-bit lanes)
};

typedef unsigned u32x2_a8 __attribute__((ext_vector_type(2), aligned(8)));
typedef unsigned short us2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ unsigned lds_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}
// Eight bytes from a 2-byte aligned LDS address: three dword reads, realigned.
__device__ __forceinline__ u32x2_a8 lds_bytes8_a2(const uint8_t* p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const unsigned* w = reinterpret_cast<const unsigned*>(a & ~uintptr_t(3));
    const unsigned w0 = w[0], w1 = w[1], w2 = w[2];
    if (a & 2u)
        return u32x2_a8{__builtin_amdgcn_alignbyte(w1, w0, 2), __builtin_amdgcn_alignbyte(w2, w1, 2)};
    return u32x2_a8{w0, w1};
}
// Four IQ4 code points (the formats' fixed grid, as iq4_value holds it) for the four
// 4-bit indices in the bytes of `nib`, by two byte permutations and a select on bit 3.
__device__ __forceinline__ unsigned iq4_bytes(unsigned nib) {
    const unsigned sel = nib & 0x07070707u;
    const unsigned lo = __builtin_amdgcn_perm(0xf6eaddcfu, 0xbfad9881u, sel);  // entries 0..7
    const unsigned hi = __builtin_amdgcn_perm(0x71594535u, 0x26190d01u, sel);  // 8..15
    const unsigned mask = ((nib >> 3) & 0x01010101u) * 0xffu;
    return (hi & mask) | (lo & ~mask);
}
// step * (signed byte i of q, i = 0..3) into a[at..at+3]
__device__ __forceinline__ void scale_signed(f16x8& a, int at, float step, unsigned q) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
        a[at + i] = _Float16(mul_rn(step, float(int8_t(q >> (8 * i)))));
}

template <int ENC> struct RowsDecode {
    // every other encoding: decode_run, each value checked
    static __device__ __forceinline__ f16x8 run(const uint8_t* row, unsigned kk, RowFlags& f,
                                                const uint8_t*) {
        using F = Format<ENC>;
        float v[8];
        decode_run<ENC>(row + (kk / F::values) * F::bytes, kk % F::values, v);
        f16x8 a;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            f.nonfinite = f.nonfinite || !isfinite(v[i]);
            f.wide = f.wide || fabsf(v[i]) > 65504.f;
            a[i] = _Float16(v[i]);
        }
        return a;
    }
};

template <> struct RowsDecode<KDQ_IQ4_XS> {  // the group is one 136-byte super-block
    static __device__ __forceinline__ f16x8 run(const uint8_t* row, unsigned kk, RowFlags& f,
                                                const uint8_t*) {
        const unsigned g = kk / 32, at = kk % 32;
        const float d = half_hw(lds_u16(row));
        const unsigned high = lds_u16(row + 2);
        const int scale = int(((unsigned(row[4 + g / 2]) >> (4 * (g % 2))) & 15u) |
                              (((high >> (2 * g)) & 3u) << 4)) - 32;
        const float step = mul_rn(d, float(scale));
        f.nonfinite = f.nonfinite || !isfinite(step);
        f.wide = f.wide || 127.f * fabsf(step) > 65504.f;
        const u32x2_a8 b = *reinterpret_cast<const u32x2_a8*>(row + 8 + 16 * g + at % 16);
        const unsigned sh = at < 16 ? 0u : 4u;
        f16x8 a;
        scale_signed(a, 0, step, iq4_bytes((b.x >> sh) & 0x0f0f0f0fu));
        scale_signed(a, 4, step, iq4_bytes((b.y >> sh) & 0x0f0f0f0fu));
        return a;
    }
};

template <> struct RowsDecode<KDQ_IQ4_NL> {  // eight 18-byte blocks of 32 values
    static __device__ __forceinline__ f16x8 run(const uint8_t* row, unsigned kk, RowFlags& f,
                                                const uint8_t*) {
        const uint8_t* block = row + (kk / 32) * 18;
        const unsigned at = kk % 32;
        const float d = half_hw(lds_u16(block));
        f.nonfinite = f.nonfinite || !isfinite(d);
        f.wide = f.wide || 127.f * fabsf(d) > 65504.f;
        const u32x2_a8 b = lds_bytes8_a2(block + 2 + at % 16);
        const unsigned sh = at < 16 ? 0u : 4u;
        f16x8 a;
        scale_signed(a, 0, d, iq4_bytes((b.x >> sh) & 0x0f0f0f0fu));
        scale_signed(a, 4, d, iq4_bytes((b.y >> sh) & 0x0f0f0f0fu));
        return a;
    }
};

template <> struct RowsDecode<KDQ_Q4_0> {  // eight 18-byte blocks: (q - 8) * d
    static __device__ __forceinline__ f16x8 run(const uint8_t* row, unsigned kk, RowFlags& f,
                                                const uint8_t*) {
        const uint8_t* block = row + (kk / 32) * 18;
        const unsigned at = kk % 32;
        const float d = half_hw(lds_u16(block));
        f.nonfinite = f.nonfinite || !isfinite(d);
        f.wide = f.wide || 8.f * fabsf(d) > 65504.f;
        const u32x2_a8 b = lds_bytes8_a2(block + 2 + at % 16);
        const unsigned sh = at < 16 ? 0u : 4u;
        const unsigned n[2] = {(b.x >> sh) & 0x0f0f0f0fu, (b.y >> sh) & 0x0f0f0f0fu};
        f16x8 a;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            a[i] = _Float16(mul_rn(float(int((n[i / 4] >> (8 * (i % 4))) & 255u) - 8), d));
        return a;
    }
};

template <> struct RowsDecode<KDQ_Q8_0> {  // eight 34-byte blocks: q * d
    static __device__ __forceinline__ f16x8 run(const uint8_t* row, unsigned kk, RowFlags& f,
                                                const uint8_t*) {
        const uint8_t* block = row + (kk / 32) * 34;
        const float d = half_hw(lds_u16(block));
        f.nonfinite = f.nonfinite || !isfinite(d);
        f.wide = f.wide || 128.f * fabsf(d) > 65504.f;
        const u32x2_a8 b = lds_bytes8_a2(block + 2 + kk % 32);
        f16x8 a;
        scale_signed(a, 0, d, b.x);
        scale_signed(a, 4, d, b.y);
        return a;
    }
};

template <> struct RowsDecode<KDQ_Q4_K> {  // one 144-byte super-block
    static __device__ __forceinline__ f16x8 run(const uint8_t* row, unsigned kk, RowFlags& f,
                                                const uint8_t*) {
        const float d = half_hw(lds_u16(row)), dmin = half_hw(lds_u16(row + 2));
        const unsigned g = kk / 32;
        unsigned sc, m;
        q4k_scale_min(row + 4, g, sc, m);
        const float scaled = mul_rn(d, float(sc));
        const float offset = mul_rn(dmin, float(m));
        f.nonfinite = f.nonfinite || !isfinite(scaled) || !isfinite(offset);
        f.wide = f.wide || 15.f * fabsf(scaled) + fabsf(offset) > 65504.f;
        const u32x2_a8 b = *reinterpret_cast<const u32x2_a8*>(row + 16 + (kk / 64) * 32 + kk % 32);
        const unsigned sh = (g & 1u) ? 4u : 0u;
        const unsigned n[2] = {(b.x >> sh) & 0x0f0f0f0fu, (b.y >> sh) & 0x0f0f0f0fu};
        f16x8 a;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            a[i] = _Float16(sub_rn(mul_rn(scaled, float((n[i / 4] >> (8 * (i % 4))) & 255u)),
                                   offset));
        return a;
    }
};

template <> struct RowsDecode<KDQ_Q3_K> {  // one 110-byte super-block
    static __device__ __forceinline__ f16x8 run(const uint8_t* row, unsigned kk, RowFlags& f,
                                                const uint8_t*) {
        const float d = half_hw(lds_u16(row + 108));
        const unsigned g = kk / 16;
        const uint8_t* scales = row + 96;
        const unsigned low = g < 8 ? scales[g] & 15u : unsigned(scales[g - 8]) >> 4;
        const unsigned high = (unsigned(scales[8 + g % 4]) >> (2 * (g / 4))) & 3u;
        const float step = mul_rn(d, float(int(low | (high << 4)) - 32));
        f.nonfinite = f.nonfinite || !isfinite(step);
        f.wide = f.wide || 4.f * fabsf(step) > 65504.f;
        const unsigned shift = 2 * ((kk % 128) / 32), mask_bit = kk / 32;
        const u32x2_a8 c = *reinterpret_cast<const u32x2_a8*>(row + 32 + (kk / 128) * 32 + kk % 32);
        const u32x2_a8 h = *reinterpret_cast<const u32x2_a8*>(row + kk % 32);
        // code = 2-bit field - 4 unless the high-mask bit is set: (field | bit << 2) - 4
        const unsigned q[2] = {((c.x >> shift) & 0x03030303u) | (((h.x >> mask_bit) & 0x01010101u) << 2),
                               ((c.y >> shift) & 0x03030303u) | (((h.y >> mask_bit) & 0x01010101u) << 2)};
        f16x8 a;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            a[i] = _Float16(mul_rn(step, float(int((q[i / 4] >> (8 * (i % 4))) & 255u) - 4)));
        return a;
    }
};

// +-(scale * level byte i of m), sign bit i of `signs` (decode_run's signed_level: the
// product, then an exact sign change), into a[at..at+3]
__device__ __forceinline__ void signed_levels(f16x8& a, int at, float scale, unsigned m,
                                              unsigned signs) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float v = mul_rn(scale, float((m >> (8 * i)) & 255u));
        a[at + i] = _Float16((signs >> i) & 1u ? -v : v);
    }
}

template <> struct RowsDecode<KDQ_IQ3_XXS> {  // one 98-byte super-block
    static __device__ __forceinline__ f16x8 run(const uint8_t* row, unsigned kk, RowFlags& f,
                                                const uint8_t* table) {
        const unsigned g = kk / 32, pair = (kk % 32) / 8;
        const float d = half_hw(lds_u16(row));
        const unsigned aux = lds_u16(row + 66 + 4 * g) | (lds_u16(row + 68 + 4 * g) << 16);
        const float scale = mul_rn(mul_rn(d, 0.5f + float(aux >> 28)), 0.5f);
        f.nonfinite = f.nonfinite || !isfinite(scale);
        f.wide = f.wide || 62.f * fabsf(scale) > 65504.f;
        unsigned signs = (aux >> (7 * pair)) & 127u;
        signs |= (__builtin_popcount(signs) & 1u) << 7;
        const unsigned idx = lds_u16(row + 2 + 8 * g + 2 * pair);
        const unsigned* t = reinterpret_cast<const unsigned*>(table);
        f16x8 a;
        signed_levels(a, 0, scale, t[idx & 255u], signs);
        signed_levels(a, 4, scale, t[idx >> 8], signs >> 4);
        return a;
    }
};

template <> struct RowsDecode<KDQ_IQ3_S> {  // one 110-byte super-block
    static __device__ __forceinline__ f16x8 run(const uint8_t* row, unsigned kk, RowFlags& f,
                                                const uint8_t* table) {
        const unsigned g = kk / 32, q = (kk % 32) / 8;
        const float d = half_hw(lds_u16(row));
        const unsigned sb = row[106 + g / 2];
        const unsigned nibble = g % 2 ? sb >> 4 : sb & 15u;
        const float scale = mul_rn(d, float(int(1 + 2 * nibble)));
        f.nonfinite = f.nonfinite || !isfinite(scale);
        f.wide = f.wide || 15.f * fabsf(scale) > 65504.f;
        const unsigned high = row[66 + g], signs = row[74 + 4 * g + q];
        const unsigned idx = lds_u16(row + 2 + 8 * g + 2 * q);
        const unsigned* t = reinterpret_cast<const unsigned*>(table);
        f16x8 a;
        signed_levels(a, 0, scale, t[(idx & 255u) | ((high << (8 - 2 * q)) & 256u)], signs);
        signed_levels(a, 4, scale, t[(idx >> 8) | ((high << (7 - 2 * q)) & 256u)], signs >> 4);
        return a;
    }
};

template <> struct RowsDecode<KDQ_IQ2_S> {  // one 82-byte super-block
    static __device__ __forceinline__ f16x8 run(const uint8_t* row, unsigned kk, RowFlags& f,
                                                const uint8_t* table) {
        const unsigned g = kk / 32, q = (kk % 32) / 8;
        const float d = half_hw(lds_u16(row));
        const unsigned sb = row[74 + g];
        const unsigned nibble = q < 2 ? sb & 15u : sb >> 4;
        const float scale = mul_rn(mul_rn(d, 0.5f + float(nibble)), 0.25f);
        f.nonfinite = f.nonfinite || !isfinite(scale);
        f.wide = f.wide || 43.f * fabsf(scale) > 65504.f;
        const unsigned index = row[2 + 4 * g + q] | ((unsigned(row[66 + g]) << (8 - 2 * q)) & 0x300u);
        const uint2 m = reinterpret_cast<const uint2*>(table)[index];
        const unsigned signs = row[34 + 4 * g + q];
        f16x8 a;
        signed_levels(a, 0, scale, m.x, signs);
        signed_levels(a, 4, scale, m.y, signs >> 4);
        return a;
    }
};

template <> struct RowsDecode<KDQ_BF16> {  // 64 values of 2 bytes: exact, bits checked
    static __device__ __forceinline__ f16x8 run(const uint8_t* row, unsigned kk, RowFlags& f,
                                                const uint8_t*) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(row + 2 * kk);
        f16x8 a;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const unsigned m = w[i] & 0x7fff7fffu;  // |bits| of the two values
            f.bf16_max = __builtin_bit_cast(
                unsigned, __builtin_elementwise_max(__builtin_bit_cast(us2, f.bf16_max),
                                                    __builtin_bit_cast(us2, m)));
            a[2 * i] = _Float16(__uint_as_float(w[i] << 16));
            a[2 * i + 1] = _Float16(__uint_as_float(w[i] & 0xffff0000u));
        }
        return a;
    }
};

__device__ __forceinline__ float row_max(float v) {
    for (int s = 32; s >= 1; s /= 2)
        v = fmaxf(v, __shfl_xor(v, s, 64));
    return v;
}

// Row t of x (fp32, k values) -> its scale and fp16(x / sigma); rows t >= m are zeros
// with scale 1.  One 256-thread workgroup per row, and one more (blockIdx.x == m_pad)
// that copies the last K group of the final weight row into `tail`, zero-filled to
// `tail_size` bytes: the GEMM reads its 16-byte pieces there, so none runs past the end
// of the weights.
__global__ __launch_bounds__(256) void stage_rows_kernel(const float* __restrict__ x,
                                                         unsigned m, unsigned m_pad, unsigned k,
                                                         uint16_t* __restrict__ xs,
                                                         float* __restrict__ sigma,
                                                         const uint8_t* __restrict__ tail_src,
                                                         unsigned tail_bytes, unsigned tail_size,
                                                         uint8_t* __restrict__ tail) {
    __shared__ float wave_max[4];
    const unsigned t = blockIdx.x;
    if (t == m_pad) {
        for (unsigned i = threadIdx.x; i < tail_size; i += 256)
            tail[i] = i < tail_bytes ? tail_src[i] : uint8_t(0);
        return;
    }
    const bool live = t < m;
    const float4* src = reinterpret_cast<const float4*>(x + size_t(live ? t : 0) * k);
    float amax = 0.f;
    for (unsigned i = threadIdx.x; live && i < k / 4; i += 256) {
        const float4 v = src[i];
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        if (!(isfinite(v.x) && isfinite(v.y) && isfinite(v.z) && isfinite(v.w)))
            amax = INFINITY;
    }
    amax = row_max(amax);
    if (threadIdx.x % 64 == 0)
        wave_max[threadIdx.x / 64] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wave_max[0], wave_max[1]), fmaxf(wave_max[2], wave_max[3]));
    float scale = 1.f, inv = 1.f;
    if (isfinite(amax) && amax >= 0x1p-100f) {
        int e = 0;
        (void)frexpf(amax, &e);  // amax in [2^(e-1), 2^e)
        scale = ldexpf(1.f, e - 15);
        inv = ldexpf(1.f, 15 - e);
    } else if (!isfinite(amax)) {
        scale = __builtin_nanf("");  // a non-finite input poisons its row
    }
    if (threadIdx.x == 0)
        sigma[t] = scale;
    uint4* dst = reinterpret_cast<uint4*>(xs + size_t(t) * k);
    for (unsigned c = threadIdx.x; c < k / 8; c += 256) {
        unsigned words[4] = {0u, 0u, 0u, 0u};
        if (live) {
            const float4 a = src[2 * c], b = src[2 * c + 1];
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
                words[i] = unsigned(__builtin_bit_cast(uint16_t, _Float16(v[2 * i] * inv))) |
                           unsigned(__builtin_bit_cast(uint16_t, _Float16(v[2 * i + 1] * inv)))
                               << 16;
        }
        dst[c] = make_uint4(words[0], words[1], words[2], words[3]);
    }
}

// Grid: ceil(n / RN) * ceil(m_pad / RM) * slices workgroups, rounded up to a multiple of 8
// and ordered so that the token tiles of one weight tile (and K slice) run together on one
// XCD (its L2 serves the weight bytes to all of them).  xs holds m_pad = ceil(m / RM) * RM
// rows.  K slices (outputs too narrow to fill the compute units): slice `ks` runs groups
// [ks * per, (ks + 1) * per) and writes its fp32 tile to part[ks] (m x n, already scaled
// back by sigma, a power of two: exact), summed in slice order by slice_sum_kernel.
template <int ENC>
__global__ __launch_bounds__(kThreads, 2) void rows_gemm_kernel(
    const uint16_t* __restrict__ xs, const float* __restrict__ sigma,
    const uint8_t* __restrict__ w, size_t row_bytes, const uint8_t* __restrict__ tail,
    unsigned m, unsigned n, unsigned k, unsigned slices, unsigned per, float* __restrict__ y,
    float* __restrict__ part, unsigned* __restrict__ status) {
    using G = RowsGroup<ENC>;
    extern __shared__ __align__(16) uint8_t lds[];
    uint8_t* raw = lds;                        // [2][RN][pitch]
    uint8_t* xt = lds + 2 * RN * G::pitch;     // [2][RM][RK] fp16, 16-byte chunks swizzled
    uint8_t* table = xt + 2 * RM * RK * 2;     // lattice encodings: the grid's levels
    if constexpr (lattice_rows_entries<ENC> > 0)
        lattice_rows_table<ENC>(table);  // before the prologue's barrier

    const unsigned m_tiles = (m + RM - 1) / RM, n_tiles = (n + RN - 1) / RN;
    const unsigned id = blockIdx.x, xcd = id % 8, local = id / 8;
    const unsigned per_xcd = (m_tiles * n_tiles * slices + 7) / 8;
    const unsigned linear = xcd * per_xcd + local;
    if (local >= per_xcd || linear >= m_tiles * n_tiles * slices)
        return;  // the whole workgroup, before any barrier
    const unsigned n0 = (linear / (m_tiles * slices)) * RN;
    const unsigned slice = (linear / m_tiles) % slices, m0 = (linear % m_tiles) * RM;
    float* __restrict__ out_tile = slices > 1 ? part + size_t(slice) * m * n : y;

    const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const unsigned lane = threadIdx.x % 64, r = lane % 32, h = lane / 32;
    // this slice's groups [g0, g0 + groups) (slices = ceil(all groups / per): none empty)
    const unsigned g0 = slice * per, groups = min(k / G::values - g0, per);
    const unsigned per_group = G::values / RK, steps = groups * per_group;

    // raw copy: chunk c of the group buffer = LDS bytes 16c = row c / (pitch / 16), byte
    // 16 (c % (pitch / 16)) of that row's group; rows past n copy row n - 1.  A 16-byte
    // piece may run past its group into the next one (never read).  The final row's last
    // group is read from `tail` (its copy, zero-filled to a whole pitch), so no piece
    // passes the weights' end.
    const unsigned last_group = k / G::values - 1 - g0;  // in this slice's numbering
    const uint8_t* src[G::per_thread];
    unsigned dst[G::per_thread], tail_at[G::per_thread];
#pragma unroll
    for (int j = 0; j < G::per_thread; ++j) {
        const unsigned c = min(threadIdx.x + unsigned(j) * kThreads, unsigned(G::chunks) - 1);
        const unsigned row = c / (G::pitch / 16), at = 16 * (c % (G::pitch / 16));
        src[j] = w + size_t(min(n0 + row, n - 1)) * row_bytes + size_t(g0) * G::bytes + at;
        tail_at[j] = n0 + row + 1 >= n ? at : ~0u;
        dst[j] = row * G::pitch + at;
    }
    auto load_raw = [&](unsigned g, u32x4 (&v)[G::per_thread]) {
#pragma unroll
        for (int j = 0; j < G::per_thread; ++j)
            v[j] = load16_a2(g == last_group && tail_at[j] != ~0u ? tail + tail_at[j]
                                                                   : src[j] + size_t(g) * G::bytes);
    };
    // (threads past the last chunk hold the last chunk again and store the same bytes to
    // the same place: no per-lane condition, which made the compiler sink the load into
    // the store's branch and wait on it there)
    auto store_raw = [&](unsigned buf, const u32x4 (&v)[G::per_thread]) {
#pragma unroll
        for (int j = 0; j < G::per_thread; ++j)
            *reinterpret_cast<u32x4*>(raw + buf * RN * G::pitch + dst[j]) = v[j];
    };
    // activation copy: thread i moves 16-byte chunks i and i + 256 of the step's RM x 64 B;
    // chunk c of token t lands at t * 64 + 16 (c ^ swz(t)), swz(t) = ((t >> 1) ^ (t >> 3))
    // & 3: the 16-byte reads of 8 (or 16) consecutive tokens then cover distinct banks
    // whether a clock serves 128 or 256 bytes
    const uint8_t* xrow[2];
    unsigned xdst[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const unsigned q = threadIdx.x + unsigned(j) * kThreads, t = q / 4, c = q % 4;
        xrow[j] = reinterpret_cast<const uint8_t*>(xs) + size_t(m0 + t) * k * 2 +
                  size_t(g0) * G::values * 2 + 16 * c;
        xdst[j] = t * 64 + 16 * (c ^ (((t >> 1) ^ (t >> 3)) & 3u));
    }
    auto load_x = [&](unsigned s, u32x4 (&v)[2]) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
            v[j] = load16(xrow[j] + size_t(s) * RK * 2);
    };
    auto store_x = [&](unsigned buf, const u32x4 (&v)[2]) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
            *reinterpret_cast<u32x4*>(xt + buf * RM * RK * 2 + xdst[j]) = v[j];
    };

    f32x16 acc[4];
#pragma unroll
    for (int b = 0; b < 4; ++b)
        acc[b] = f32x16{};
    RowFlags flags;

    // Software pipeline, one barrier per step.  The top of step s refills the LDS buffers
    // that step s - 1 finished reading: activations of step s + 1 (from a register ring,
    // loaded kAhead steps earlier) and, on a group's last step, the raw bytes of the next
    // group (loaded a whole group earlier).  Each refill is followed at once by the load
    // that reuses its registers, so a store only ever waits on loads issued at least
    // kAhead steps (or one group) before.  The loop is unrolled by one turn of the ring, so
    // its register indices are constants; loads past the end re-read the last step or
    // group (never used).  The prologue's order is pinned (sched_barrier) so that at the
    // loop's entry the loads in flight stand in the same order as at its back edge: the
    // waits the compiler places at the loop's head then hold for both.
    constexpr int PG = G::values / RK;  // steps per group
    // (two for Q8_0 and Q6_K, whose decode holds more registers: four would spill)
    constexpr int kAhead = PG < 4 || ENC == KDQ_Q8_0 || ENC == KDQ_Q6_K ? 2 : 4;
    constexpr int kUnroll = kAhead;
    static_assert(PG % kAhead == 0, "a group is whole turns of the ring");
    u32x4 rv[G::per_thread], xv[kAhead][2];
    load_x(0, xv[0]);
    load_raw(0, rv);
#pragma unroll
    for (int a = 1; a < kAhead; ++a)
        load_x(min(unsigned(a), steps - 1), xv[a]);
    __builtin_amdgcn_sched_barrier(0);
    store_x(0, xv[0]);
    __builtin_amdgcn_sched_barrier(0);
    load_x(min(unsigned(kAhead), steps - 1), xv[0]);
    __builtin_amdgcn_sched_barrier(0);
    store_raw(0, rv);
    __builtin_amdgcn_sched_barrier(0);
    load_raw(min(1u, groups - 1), rv);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    const uint8_t* my_row0 = raw + (wave * 32 + r) * G::pitch;
    auto step = [&]<int U>(unsigned s) {  // U = s % kUnroll
        constexpr int slot = (U + 1) % kAhead;
        const unsigned g = s / PG, within = s % PG;
        store_x((s + 1) % 2, xv[slot]);
        load_x(min(s + 1 + kAhead, steps - 1), xv[slot]);
        if (within == PG - 1) {
            store_raw((g + 1) % 2, rv);
            load_raw(min(g + 2, groups - 1), rv);
        }
        const uint8_t* row = my_row0 + (g % 2) * RN * G::pitch;
        const uint8_t* xb = xt + (s % 2) * RM * RK * 2;
#pragma unroll
        for (int sub = 0; sub < 2; ++sub) {
            // this lane's 8 weights: values 16 sub + 8 h .. +7 of the step
            const unsigned kk = within * RK + 16 * sub + 8 * h;
            const f16x8 a = RowsDecode<ENC>::run(row, kk, flags, table);
            const unsigned c = 2 * sub + h;  // 16-byte chunk of the token's 64 bytes
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const unsigned t = 32 * b + r;
                const f16x8 xf =
                    *reinterpret_cast<const f16x8*>(xb + t * 64 +
                                                    16 * (c ^ (((t >> 1) ^ (t >> 3)) & 3u)));
                acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, xf, acc[b], 0, 0, 0);
            }
        }
        __syncthreads();
    };
    unsigned s = 0;
    do {  // steps >= PG: a do-while keeps the prologue's loads ahead of the loop, in order
        [&]<int... U>(std::integer_sequence<int, U...>) {
            (step.template operator()<U>(s + U), ...);
        }(std::make_integer_sequence<int, kUnroll>{});
        s += kUnroll;
    } while (s < steps);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the re-read prefetches

    // D of token block b: token 32 b + r, weight rows 8 (v / 4) + 4 h + v % 4 of the
    // wavefront's 32; scaled back by the token's sigma
    const bool vec = n % 4 == 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const unsigned tok = m0 + 32 * b + r;
        if (tok >= m)
            continue;
        const float sg = sigma[tok];
        float* out = out_tile + size_t(tok) * n;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const unsigned col = n0 + wave * 32 + 8 * q + 4 * h;
            if (vec && col + 3 < n) {
                *reinterpret_cast<float4*>(out + col) =
                    make_float4(acc[b][4 * q] * sg, acc[b][4 * q + 1] * sg,
                                acc[b][4 * q + 2] * sg, acc[b][4 * q + 3] * sg);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (col + i < n)
                        out[col + i] = acc[b][4 * q + i] * sg;
            }
        }
    }
    if (status) {
        if constexpr (ENC == KDQ_BF16) {  // |bits| 0x7f80 and up: inf / NaN; 0x4780 (65536) up
            const unsigned mx = max(flags.bf16_max & 0xffffu, flags.bf16_max >> 16);
            flags.nonfinite = mx >= 0x7f80u;
            flags.wide = mx >= 0x4780u && mx < 0x7f80u;
        }
        const unsigned f = (__any(flags.nonfinite) ? 1u : 0u) | (__any(flags.wide) ? 2u : 0u);
        if (f && lane == 0)
            atomicOr(status, f);
    }
}

// y = sum over the slices of part[s], in slice order; one thread per 4 outputs (m * n % 4
// == 0 when slices run).
__global__ __launch_bounds__(256) void slice_sum_kernel(const float* __restrict__ part,
                                                        size_t count, unsigned slices,
                                                        float* __restrict__ y) {
    const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= count / 4)
        return;
    float4 acc = reinterpret_cast<const float4*>(part)[i];
    for (unsigned s = 1; s < slices; ++s) {
        const float4 v = reinterpret_cast<const float4*>(part + s * count)[i];
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
    }
    reinterpret_cast<float4*>(y)[i] = acc;
}

// K slices: enough workgroups for about two per compute unit when the output tiles are
// fewer; whole groups, none empty, and only where m * n % 4 == 0.
struct RowsPlan {
    unsigned slices, per;
};

RowsPlan rows_plan(size_t m, size_t n, size_t groups) {
    const size_t tiles = (m + RM - 1) / RM * ((n + RN - 1) / RN);
    const size_t target = 2 * size_t(compute_units());
    size_t slices = (m * n) % 4 ? 1 : std::max<size_t>(1, target / tiles);
    slices = std::min(slices, groups);
    const size_t per = (groups + slices - 1) / slices;
    return RowsPlan{unsigned((groups + per - 1) / per), unsigned(per)};
}

struct RowsScratch {
    size_t m_pad, xs, sigma, tail, total;
};

constexpr unsigned kTailSize = 512;  // >= every RowsGroup pitch

RowsScratch rows_scratch(size_t m, size_t n, size_t k, size_t row_bytes, unsigned slices) {
    RowsScratch s;
    s.m_pad = (m + RM - 1) / RM * RM;
    s.xs = (s.m_pad * k * 2 + 255) / 256 * 256;
    s.sigma = (s.m_pad * 4 + 255) / 256 * 256;
    s.tail = kTailSize;
    s.total = s.xs + s.sigma + s.tail + (slices > 1 ? size_t(slices) * m * n * 4 : 0);
    return s;
}

template <int ENC>
int launch_rows(const uint8_t* w, size_t row_bytes, size_t n, size_t k, const float* x, size_t m,
                float* y, unsigned* status, uint8_t* scratch, hipStream_t st) {
    using G = RowsGroup<ENC>;
    if (k % G::values)
        return KDQ_ERR_SHAPE;
    static bool configured = false;  // one attribute call per instantiation
    if (!configured) {
        KDQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&rows_gemm_kernel<ENC>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize,
                                    int(rows_lds<ENC>)));
        configured = true;
    }
    const RowsPlan plan = rows_plan(m, n, k / G::values);
    const RowsScratch s = rows_scratch(m, n, k, row_bytes, plan.slices);
    auto* xs = reinterpret_cast<uint16_t*>(scratch);
    auto* sigma = reinterpret_cast<float*>(scratch + s.xs);
    uint8_t* tail = scratch + s.xs + s.sigma;
    auto* part = reinterpret_cast<float*>(tail + s.tail);
    static_assert(G::pitch <= int(kTailSize));
    const uint8_t* tail_src = w + (n - 1) * row_bytes + (k / G::values - 1) * G::bytes;
    hipLaunchKernelGGL(stage_rows_kernel, dim3(unsigned(s.m_pad) + 1), dim3(256), 0, st, x,
                       unsigned(m), unsigned(s.m_pad), unsigned(k), xs, sigma, tail_src,
                       unsigned(G::bytes), unsigned(G::pitch), tail);
    KDQ_HIP(hipGetLastError());
    const size_t tiles = (s.m_pad / RM) * ((n + RN - 1) / RN) * plan.slices;
    hipLaunchKernelGGL(rows_gemm_kernel<ENC>, dim3(unsigned((tiles + 7) / 8 * 8)),
                       dim3(kThreads), rows_lds<ENC>, st, xs, sigma, w, row_bytes, tail,
                       unsigned(m), unsigned(n), unsigned(k), plan.slices, plan.per, y, part,
                       status);
    KDQ_HIP(hipGetLastError());
    if (plan.slices > 1) {
        const size_t count = m * n;
        hipLaunchKernelGGL(slice_sum_kernel, dim3(unsigned((count / 4 + 255) / 256)), dim3(256),
                           0, st, part, count, plan.slices, y);
        KDQ_HIP(hipGetLastError());
    }
    return KDQ_OK;
}

int rows_gemm(int encoding, const uint8_t* w, size_t row_bytes, size_t n, size_t k,
              const float* x, size_t m, float* y, unsigned* status, uint8_t* scratch,
              hipStream_t st) {
    switch (encoding) {
    case KDQ_Q3_K:
        return launch_rows<KDQ_Q3_K>(w, row_bytes, n, k, x, m, y, status, scratch, st);
    case KDQ_IQ4_XS:
        return launch_rows<KDQ_IQ4_XS>(w, row_bytes, n, k, x, m, y, status, scratch, st);
    case KDQ_IQ4_NL:
        return launch_rows<KDQ_IQ4_NL>(w, row_bytes, n, k, x, m, y, status, scratch, st);
    case KDQ_IQ3_XXS:
        return launch_rows<KDQ_IQ3_XXS>(w, row_bytes, n, k, x, m, y, status, scratch, st);
    case KDQ_IQ3_S:
        return launch_rows<KDQ_IQ3_S>(w, row_bytes, n, k, x, m, y, status, scratch, st);
    case KDQ_IQ2_S:
        return launch_rows<KDQ_IQ2_S>(w, row_bytes, n, k, x, m, y, status, scratch, st);
    case KDQ_BF16:
        return launch_rows<KDQ_BF16>(w, row_bytes, n, k, x, m, y, status, scratch, st);
    case KDQ_Q4_0:
        return launch_rows<KDQ_Q4_0>(w, row_bytes, n, k, x, m, y, status, scratch, st);
    case KDQ_Q4_K:
        return launch_rows<KDQ_Q4_K>(w, row_bytes, n, k, x, m, y, status, scratch, st);
    case KDQ_Q8_0:
        return launch_rows<KDQ_Q8_0>(w, row_bytes, n, k, x, m, y, status, scratch, st);
    case KDQ_Q6_K:
        return launch_rows<KDQ_Q6_K>(w, row_bytes, n, k, x, m, y, status, scratch, st);
    default:
        return KDQ_ERR_UNSUPPORTED;
    }
}

}  // namespace
}  // namespace kdq

using namespace kdq;

extern "C" size_t kdq_gemm_rows_values(int encoding) {
    switch (encoding) {
    case KDQ_BF16:
        return 64;
    case KDQ_Q3_K: case KDQ_IQ4_XS: case KDQ_IQ4_NL: case KDQ_IQ3_XXS: case KDQ_IQ3_S:
    case KDQ_IQ2_S: case KDQ_Q4_0: case KDQ_Q4_K: case KDQ_Q8_0: case KDQ_Q6_K:
        return 256;
    default:
        return 0;
    }
}

extern "C" int kdq_gemm_rows(int encoding, const void* weights, size_t row_bytes, size_t n,
                             size_t k, const float* x, size_t m, float* y, unsigned* status,
                             void* stream) {
    const size_t values = kdq_gemm_rows_values(encoding);
    if (!values)
        return KDQ_ERR_UNSUPPORTED;
    if (!weights || !x || !y || !m || !n || !k)
        return KDQ_ERR_ARGUMENT;
    if (k % values || k > 65536 || m > 0xffffffu || n > 0xffffffu ||
        row_bytes < kdq_row_bytes(encoding, k) || row_bytes % 2)
        return KDQ_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(weights) % 2 ||
        reinterpret_cast<uintptr_t>(y) % 16)
        return KDQ_ERR_ALIGNMENT;
    if (mul_overflows(n, row_bytes) || mul_overflows(m, k) || mul_overflows(m, n))
        return KDQ_ERR_ARGUMENT;
    const size_t w_bytes = (n - 1) * row_bytes + kdq_row_bytes(encoding, k);
    if (overlaps(y, m * n * 4, x, m * k * 4) || overlaps(y, m * n * 4, weights, w_bytes))
        return KDQ_ERR_ALIAS;
    int rc;
    void* scratch = workspace(
        rows_scratch(m, n, k, row_bytes, rows_plan(m, n, k / values).slices).total, &rc);
    if (rc)
        return rc;
    return rows_gemm(encoding, static_cast<const uint8_t*>(weights), row_bytes, n, k, x, m, y,
                     status, static_cast<uint8_t*>(scratch), static_cast<hipStream_t>(stream));
}
