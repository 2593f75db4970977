// Exact decode of the GGUF block encodings, shared by the decode-time products
// (gguf_gemv.hip) and the prefill GEMM over row-major rows (gguf_gemm_rows.hip):
// decode_run<ENC> gives eight consecutive values of one block, each equal to the
// reference's single-value decode (IW/include/kadan/gguf_quantization.hpp:631-762; IW =
// services/hikari/inference_worker).  Included inside namespace kdq's anonymous
// namespace of each translation unit.
#pragma once

// ------------------------------------------------------------------ decode

template <int ENC> struct Format;
template <> struct Format<KDQ_Q8_0> {
    static constexpr int values = 32, bytes = 34;
};
template <> struct Format<KDQ_Q4_0> {
    static constexpr int values = 32, bytes = 18;
};
template <> struct Format<KDQ_Q4_K> {
    static constexpr int values = 256, bytes = 144;
};
template <> struct Format<KDQ_Q3_K> {
    static constexpr int values = 256, bytes = 110;
};
template <> struct Format<KDQ_Q6_K> {
    static constexpr int values = 256, bytes = 210;
};
template <> struct Format<KDQ_IQ4_NL> {
    static constexpr int values = 32, bytes = 18;
};
template <> struct Format<KDQ_IQ4_XS> {
    static constexpr int values = 256, bytes = 136;
};
template <> struct Format<KDQ_BF16> {
    static constexpr int values = 1, bytes = 2;
};
template <> struct Format<KDQ_F32> {
    static constexpr int values = 1, bytes = 4;
};
template <> struct Format<KDQ_F16> {
    static constexpr int values = 1, bytes = 2;
};
template <> struct Format<KDQ_IQ3_XXS> {
    static constexpr int values = 256, bytes = 98;
};
template <> struct Format<KDQ_IQ2_S> {
    static constexpr int values = 256, bytes = 82;
};
template <> struct Format<KDQ_IQ3_S> {
    static constexpr int values = 256, bytes = 110;
};

// IQ2_S / IQ3_XXS / IQ3_S lattice grids (the formats' tables, re-encoded as lane indices
// into their magnitude levels by gen_iq_grids.py).
#define IQ_GRID_TABLE static __device__ const
#include "iq_grids.inc"
#undef IQ_GRID_TABLE

__device__ __forceinline__ unsigned word_at(const uint8_t* p) {
    return unsigned(p[0]) | (unsigned(p[1]) << 8) | (unsigned(p[2]) << 16) |
           (unsigned(p[3]) << 24);
}

// v[i] = +-(scale * level): the sign is a separate product by -1 or 1, as the reference
// decode takes it.
__device__ __forceinline__ float signed_level(float scale, unsigned level, unsigned negative) {
    return mul_rn(mul_rn(scale, float(level)), negative ? -1.0f : 1.0f);
}

// The 16 IQ4 code points (IQ4_NL and IQ4_XS; the format's fixed non-linear grid,
// G/src/ggml-common.h:1120-1122), looked up two per nibble pair with v_perm.
__device__ __forceinline__ float iq4_value(unsigned index) {
    // bytes of the signed grid, four per word
    const unsigned words[4] = {0xbfad9881u, 0xf6eaddcfu, 0x26190d01u, 0x71594535u};
    const unsigned w = index < 8 ? (index < 4 ? words[0] : words[1])
                                 : (index < 12 ? words[2] : words[3]);
    return float(int8_t(w >> (8 * (index % 4))));
}

__device__ __forceinline__ unsigned half_bits_at(const uint8_t* p) {
    return unsigned(p[0]) | (unsigned(p[1]) << 8);
}

// Q4_K sub-block g: 6-bit scale and min from the 12 packed bytes at `s`.
__device__ __forceinline__ void q4k_scale_min(const uint8_t* s, unsigned g, unsigned& sc,
                                              unsigned& m) {
    if (g < 4) {
        sc = s[g] & 63u;
        m = s[g + 4] & 63u;
    } else {
        sc = (s[g + 4] & 15u) | ((unsigned(s[g - 4]) >> 6) << 4);
        m = (unsigned(s[g + 4]) >> 4) | ((unsigned(s[g]) >> 6) << 4);
    }
}

// Eight values from element `within` (a multiple of 8) of one block, each equal to
// the reference's single-value decode (IW/include/kadan/gguf_quantization.hpp:631-762;
// a run of eight never crosses a scale group).  BF16 runs read eight one-value blocks.
template <int ENC>
__device__ __forceinline__ void decode_run(const uint8_t* block, unsigned within, float* v) {
    if constexpr (ENC == KDQ_BF16) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v[i] = __uint_as_float(half_bits_at(block + 2 * i) << 16);
        return;
    } else if constexpr (ENC == KDQ_F32) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v[i] = __uint_as_float(half_bits_at(block + 4 * i) | (half_bits_at(block + 4 * i + 2) << 16));
        return;
    } else if constexpr (ENC == KDQ_F16) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v[i] = half_exact(half_bits_at(block + 2 * i));
        return;
    } else if constexpr (ENC == KDQ_Q3_K) {
        // 16 groups of 16 with 6-bit scales (low nibbles at 96.., high pairs at 104..),
        // 2-bit code fields, minus 4 unless the value's high-mask bit is set
        const float d = half_exact(half_bits_at(block + 108));
        const unsigned g = within / 16;
        const uint8_t* scales = block + 96;
        const unsigned low = g < 8 ? scales[g] & 15u : unsigned(scales[g - 8]) >> 4;
        const unsigned high = (unsigned(scales[8 + g % 4]) >> (2 * (g / 4))) & 3u;
        const float step = mul_rn(d, float(int(low | (high << 4)) - 32));
        const unsigned shift = 2 * ((within % 128) / 32), mask_bit = within / 32;
        const uint8_t* codes = block + 32 + (within / 128) * 32;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const unsigned lane = (within + i) % 32;
            const int code = int((unsigned(codes[lane]) >> shift) & 3u) -
                             ((unsigned(block[lane]) >> mask_bit) & 1u ? 0 : 4);
            v[i] = mul_rn(step, float(code));
        }
        return;
    } else if constexpr (ENC == KDQ_Q6_K) {
        // halves of 128: low nibble from ql, two high bits from qh, int8 scale per 16
        const float d = half_exact(half_bits_at(block + 208));
        const unsigned k = within / 128, off = within % 128, q = off / 32;
        const float step = mul_rn(d, float(int8_t(block[192 + 8 * k + (off % 32) / 16 + 2 * q])));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const unsigned lane = (off + i) % 32;
            const unsigned byte = block[64 * k + lane + 32 * (q & 1u)];
            const unsigned low = q < 2 ? byte & 15u : byte >> 4;
            const unsigned high = (unsigned(block[128 + 32 * k + lane]) >> (2 * q)) & 3u;
            v[i] = mul_rn(step, float(int(low | (high << 4)) - 32));
        }
        return;
    } else if constexpr (ENC == KDQ_IQ4_NL) {
        const float d = half_exact(half_bits_at(block));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const unsigned e = within + i, byte = block[2 + e % 16];
            v[i] = mul_rn(d, iq4_value(e < 16 ? byte & 15u : byte >> 4));
        }
        return;
    } else if constexpr (ENC == KDQ_IQ3_XXS) {
        // group word: four 7-bit sign sets (eighth sign = their parity), 4-bit scale on top
        const float d = half_exact(half_bits_at(block));
        const unsigned g = within / 32, pair = (within % 32) / 8;
        const unsigned aux = word_at(block + 66 + 4 * g);
        const float scale = mul_rn(mul_rn(d, 0.5f + float(aux >> 28)), 0.5f);
        unsigned signs = (aux >> (7 * pair)) & 127u;
        signs |= (__builtin_popcount(signs) & 1u) << 7;
        const unsigned e[2] = {kIq3xxsGrid[block[2 + 8 * g + 2 * pair]],
                               kIq3xxsGrid[block[2 + 8 * g + 2 * pair + 1]]};
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v[i] = signed_level(scale, kIq3xxsGridLevels[(e[i / 4] >> (3 * (i % 4))) & 7u],
                                (signs >> i) & 1u);
        return;
    } else if constexpr (ENC == KDQ_IQ2_S) {
        // quarter q of group g: grid index (10 bits), sign byte, 4-bit scale
        const float d = half_exact(half_bits_at(block));
        const unsigned g = within / 32, q = (within % 32) / 8;
        const unsigned nibble = q < 2 ? block[74 + g] & 15u : unsigned(block[74 + g]) >> 4;
        const float scale = mul_rn(mul_rn(d, 0.5f + float(nibble)), 0.25f);
        const unsigned index = block[2 + 4 * g + q] |
                               ((unsigned(block[66 + g]) << (8 - 2 * q)) & 0x300u);
        const unsigned e = kIq2sGrid[index], signs = block[34 + 4 * g + q];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v[i] = signed_level(scale, kIq2sGridLevels[(e >> (2 * i)) & 3u], (signs >> i) & 1u);
        return;
    } else if constexpr (ENC == KDQ_IQ3_S) {
        // quarter q of group g: two grid entries (9-bit indices), sign byte, scale 1 + 2s
        const float d = half_exact(half_bits_at(block));
        const unsigned g = within / 32, q = (within % 32) / 8;
        const unsigned nibble = g % 2 ? unsigned(block[106 + g / 2]) >> 4 : block[106 + g / 2] & 15u;
        const float scale = mul_rn(d, float(int(1 + 2 * nibble)));
        const unsigned high = block[66 + g], signs = block[74 + 4 * g + q];
        unsigned e[2];
#pragma unroll
        for (int h = 0; h < 2; ++h)
            e[h] = kIq3sGrid[block[2 + 8 * g + 2 * q + h] | ((high << (8 - 2 * q - h)) & 256u)];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v[i] = signed_level(scale, kIq3sGridLevels[(e[i / 4] >> (3 * (i % 4))) & 7u],
                                (signs >> i) & 1u);
        return;
    } else if constexpr (ENC == KDQ_IQ4_XS) {
        // 8 groups of 32 with 6-bit scales minus 32, indices laid out as IQ4_NL
        const float d = half_exact(half_bits_at(block));
        const unsigned g = within / 32, at = within % 32;
        const unsigned high = half_bits_at(block + 2);
        const int scale = int(((unsigned(block[4 + g / 2]) >> (4 * (g % 2))) & 15u) |
                              (((high >> (2 * g)) & 3u) << 4)) - 32;
        const float step = mul_rn(d, float(scale));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const unsigned e = at + i, byte = block[8 + 16 * g + e % 16];
            v[i] = mul_rn(step, iq4_value(e < 16 ? byte & 15u : byte >> 4));
        }
        return;
    }
    const float d = half_exact(half_bits_at(block));
    if constexpr (ENC == KDQ_Q8_0) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            v[i] = mul_rn(d, float(int8_t(block[2 + within + i])));
    } else if constexpr (ENC == KDQ_Q4_0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const unsigned e = within + i;
            const unsigned byte = block[2 + (e & 15u)];
            const int code = int(e < 16 ? (byte & 15u) : (byte >> 4)) - 8;
            v[i] = mul_rn(float(code), d);
        }
    } else {
        const float dmin = half_exact(half_bits_at(block + 2));
        const unsigned g = within / 32;
        unsigned sc, m;
        q4k_scale_min(block + 4, g, sc, m);
        const float scaled = mul_rn(d, float(sc));
        const float offset = mul_rn(dmin, float(m));
        const uint8_t* codes = block + 16 + (within / 64) * 32 + (within % 32);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const unsigned code = (g & 1u) ? (codes[i] >> 4) : (codes[i] & 15u);
            v[i] = sub_rn(mul_rn(scaled, float(code)), offset);
        }
    }
}
