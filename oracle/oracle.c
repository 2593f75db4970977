/*
 * CPU oracle for the quantized-weight matmul path: TEST INFRASTRUCTURE ONLY.
 * See oracle.h for the contract, the reference citations and the pinning of
 * every function.  Compile with -ffp-contract=off (oracle/Makefile does).
 */
#include "oracle.h"

#include <math.h>
#include <immintrin.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ scalars */

static float bits_to_float(uint32_t bits) {
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

static uint32_t float_to_bits(float f) {
    uint32_t bits;
    memcpy(&bits, &f, sizeof bits);
    return bits;
}

float kdo_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exponent = (h >> 10) & 0x1fu;
    const uint32_t mantissa = h & 0x3ffu;
    if (exponent == 0x1fu) /* inf / NaN: payload kept in the top mantissa bits */
        return bits_to_float(sign | 0x7f800000u | (mantissa << 13));
    if (exponent == 0) {
        /* zero or subnormal: mantissa * 2^-24 is exact in binary32 */
        const float magnitude = (float)mantissa * 0x1p-24f;
        return bits_to_float(sign | float_to_bits(magnitude));
    }
    return bits_to_float(sign | ((exponent + 112u) << 23) | (mantissa << 13));
}

uint16_t kdo_float_to_half(float value) {
    const uint32_t bits = float_to_bits(value);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const uint32_t magnitude = bits & 0x7fffffffu;
    if (magnitude >= 0x7f800000u) { /* inf or NaN (quiet bit forced for NaN) */
        if (magnitude == 0x7f800000u)
            return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t)((magnitude >> 13) & 0x3ffu);
    }
    if (magnitude >= 0x477ff000u) /* rounds to >= 65520 -> inf */
        return sign | 0x7c00u;
    if (magnitude < 0x38800000u) {
        /* result is a half subnormal (or zero): value / 2^-24 rounded to an integer */
        const float scaled = bits_to_float(magnitude) * 0x1p24f; /* exact */
        const float rounded = nearbyintf(scaled);               /* RNE */
        return sign | (uint16_t)rounded;
    }
    /* normal: rebias, round the 13 dropped bits to nearest even */
    uint32_t h = ((magnitude >> 13) - (112u << 10));
    const uint32_t dropped = magnitude & 0x1fffu;
    if (dropped > 0x1000u || (dropped == 0x1000u && (h & 1u)))
        h += 1u;
    return sign | (uint16_t)h;
}

float kdo_bf16_to_float(uint16_t bits) {
    return bits_to_float((uint32_t)bits << 16);
}

uint16_t kdo_float_to_bf16(float value) {
    uint32_t bits = float_to_bits(value);
    if ((bits & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)((bits >> 16) | 0x40u);
    bits += 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)(bits >> 16);
}

static uint16_t load_u16(const uint8_t* p) {
    return (uint16_t)(p[0] | (p[1] << 8));
}

/* ------------------------------------------------------------ block layouts */

int kdo_block_values(int encoding) {
    switch (encoding) {
    case KDO_F32:
    case KDO_F16:
    case KDO_BF16:
        return 1;
    case KDO_Q4_0:
    case KDO_Q8_0:
    case KDO_IQ4_NL:
        return 32;
    case KDO_Q3_K:
    case KDO_Q4_K:
    case KDO_Q6_K:
    case KDO_IQ4_XS:
    case KDO_IQ3_XXS:
    case KDO_IQ2_S:
    case KDO_IQ3_S:
        return 256;
    default:
        return 0;
    }
}

int kdo_block_bytes(int encoding) {
    switch (encoding) {
    case KDO_Q4_0:
        return 18; /* fp16 d + 16 bytes of nibbles */
    case KDO_Q8_0:
        return 34; /* fp16 d + 32 int8 */
    case KDO_Q4_K:
        return 144; /* fp16 d, fp16 dmin, 12 packed 6-bit scales, 128 bytes of nibbles */
    case KDO_Q3_K:
        return 110; /* 32 high-bit bytes, 64 bytes of 2-bit codes, 12 scale bytes, fp16 d */
    case KDO_Q6_K:
        return 210; /* 128 low-nibble bytes, 64 high-pair bytes, 16 int8 scales, fp16 d */
    case KDO_IQ4_NL:
        return 18; /* fp16 d + 16 bytes of table indices */
    case KDO_IQ4_XS:
        return 136; /* fp16 d, 16-bit high scale bits, 4 low scale bytes, 128 index bytes */
    case KDO_BF16:
    case KDO_F16:
        return 2;
    case KDO_F32:
        return 4;
    case KDO_IQ3_XXS:
        return 98; /* fp16 d, 64 grid bytes, 8 sign/scale words */
    case KDO_IQ2_S:
        return 82; /* fp16 d, 32 grid bytes, 32 sign bytes, 8 high-bit bytes, 8 scale bytes */
    case KDO_IQ3_S:
        return 110; /* fp16 d, 64 grid bytes, 8 high-bit bytes, 32 sign bytes, 4 scale bytes */
    default:
        return 0;
    }
}

/* IQ2_S / IQ3_XXS / IQ3_S lattice grids (format tables, re-encoded as lane indices into
 * their magnitude levels by kadan_amd/csrc/gen_iq_grids.py). */
#define IQ_GRID_TABLE static const
#include "../kadan_amd/csrc/iq_grids.inc"

static unsigned iq2s_level(unsigned index, unsigned lane) {
    return kIq2sGridLevels[(kIq2sGrid[index] >> (2 * lane)) & 3u];
}
static unsigned iq3xxs_level(unsigned index, unsigned lane) {
    return kIq3xxsGridLevels[(kIq3xxsGrid[index] >> (3 * lane)) & 7u];
}
static unsigned iq3s_level(unsigned index, unsigned lane) {
    return kIq3sGridLevels[(kIq3sGrid[index] >> (3 * lane)) & 7u];
}

static uint32_t load_u32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* IQ3_XXS: 8 groups of 32.  Group g's 32-bit word at 66 + 4g holds four 7-bit sign sets
 * (the eighth sign is their parity) and a 4-bit scale s in its top bits; the group's 8
 * grid bytes at 2 + 8g pick IQ3_XXS grid entries of 4 magnitudes each.
 * w = +-((d * (0.5 + s)) * 0.5) * magnitude, every product rounded. */
static void decode_iq3_xxs(const uint8_t* block, float* out) {
    const float d = kdo_half_to_float(load_u16(block));
    for (unsigned g = 0; g < 8; ++g) {
        const uint32_t aux = load_u32(block + 66 + 4 * g);
        const float scale = (d * (0.5f + (float)(aux >> 28))) * 0.5f;
        for (unsigned pair = 0; pair < 4; ++pair) {
            unsigned signs = (aux >> (7 * pair)) & 127u;
            const unsigned parity = (unsigned)__builtin_popcount(signs) & 1u;
            signs |= parity << 7;
            for (unsigned lane = 0; lane < 8; ++lane) {
                const unsigned index = block[2 + 8 * g + 2 * pair + lane / 4];
                const float magnitude = scale * (float)iq3xxs_level(index, lane % 4);
                out[32 * g + 8 * pair + lane] = magnitude * ((signs >> lane) & 1u ? -1.0f : 1.0f);
            }
        }
    }
}

/* IQ2_S: 8 groups of 32, quarters of 8.  Quarter q of group g: grid index = byte
 * 2 + 4g + q with bits 8..9 from byte 66 + g (bits 2q..2q+1), sign bits from byte
 * 34 + 4g + q, 4-bit scale from byte 74 + g (low nibble for q < 2).
 * w = +-((d * (0.5 + s)) * 0.25) * magnitude. */
static void decode_iq2_s(const uint8_t* block, float* out) {
    const float d = kdo_half_to_float(load_u16(block));
    for (unsigned g = 0; g < 8; ++g)
        for (unsigned q = 0; q < 4; ++q) {
            const unsigned nibble = q < 2 ? block[74 + g] & 15u : (unsigned)block[74 + g] >> 4;
            const float scale = (d * (0.5f + (float)nibble)) * 0.25f;
            const unsigned index = block[2 + 4 * g + q] | (((unsigned)block[66 + g] << (8 - 2 * q)) & 0x300u);
            const unsigned signs = block[34 + 4 * g + q];
            for (unsigned lane = 0; lane < 8; ++lane) {
                const float magnitude = scale * (float)iq2s_level(index, lane);
                out[32 * g + 8 * q + lane] = magnitude * ((signs >> lane) & 1u ? -1.0f : 1.0f);
            }
        }
}

/* IQ3_S: 8 groups of 32, quarters of 8 (two grid entries of 4 each).  Entry h of quarter
 * q of group g: index = byte 2 + 8g + 2q + h with bit 8 from byte 66 + g (bit 2q + h);
 * sign bits from byte 74 + 4g + q; scale d * (1 + 2s) with the 4-bit s of byte 106 + g/2
 * (low nibble for even g). */
static void decode_iq3_s(const uint8_t* block, float* out) {
    const float d = kdo_half_to_float(load_u16(block));
    for (unsigned g = 0; g < 8; ++g) {
        const unsigned nibble = g % 2 ? (unsigned)block[106 + g / 2] >> 4 : block[106 + g / 2] & 15u;
        const float scale = d * (float)(int)(1 + 2 * nibble);
        for (unsigned q = 0; q < 4; ++q) {
            const unsigned signs = block[74 + 4 * g + q];
            for (unsigned lane = 0; lane < 8; ++lane) {
                const unsigned h = lane / 4;
                const unsigned index = block[2 + 8 * g + 2 * q + h] |
                                       (((unsigned)block[66 + g] << (8 - 2 * q - h)) & 256u);
                const float magnitude = scale * (float)iq3s_level(index, lane % 4);
                out[32 * g + 8 * q + lane] = magnitude * ((signs >> lane) & 1u ? -1.0f : 1.0f);
            }
        }
    }
}

/* The 16 IQ4 code points (the non-linear 4-bit grid of IQ4_NL / IQ4_XS, fixed by the
 * format: G/src/ggml-common.h kvalues_iq4nl). */
static const int8_t iq4_grid[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                    1,    13,   25,  38,  53,  69,  89,  113};

/* Q3_K: 16 sub-blocks of 16 values with 6-bit signed scales (low 4 bits in bytes
 * 96..103 as nibbles, high 2 bits in bytes 104..107); value v of the block is the
 * 2-bit field (v % 128) / 32 of code byte 32 + (v / 128) * 32 + v % 32, minus 4 unless
 * bit v / 32 of high-bit byte v % 32 is set; w = (d * scale) * code. */
static void decode_q3_k(const uint8_t* block, float* out) {
    const float d = kdo_half_to_float(load_u16(block + 108));
    const uint8_t* scales = block + 96;
    for (unsigned s = 0; s < 16; ++s) {
        const unsigned low = s < 8 ? scales[s] & 15u : (unsigned)scales[s - 8] >> 4;
        const unsigned high = ((unsigned)scales[8 + s % 4] >> (2 * (s / 4))) & 3u;
        const float step = d * (float)((int)(low | (high << 4)) - 32); /* rounded */
        for (unsigned i = 0; i < 16; ++i) {
            const unsigned v = 16 * s + i, lane = v % 32;
            const unsigned bits = ((unsigned)block[32 + (v / 128) * 32 + lane] >> (2 * ((v % 128) / 32))) & 3u;
            const int code = (int)bits - ((block[lane] >> (v / 32)) & 1u ? 0 : 4);
            out[v] = step * (float)code; /* rounded */
        }
    }
}

/* Q6_K: two halves of 128; in half k, quarter q (32 values) of lane l takes the low
 * (q < 2) or high nibble of ql[64k + 32(q & 1) + l] and bits 2q..2q+1 of
 * qh[32k + l] as its top two bits; code - 32 scaled by int8 scale 8k + l/16 + 2q. */
static void decode_q6_k(const uint8_t* block, float* out) {
    const float d = kdo_half_to_float(load_u16(block + 208));
    for (unsigned k = 0; k < 2; ++k)
        for (unsigned q = 0; q < 4; ++q)
            for (unsigned l = 0; l < 32; ++l) {
                const unsigned byte = block[64 * k + 32 * (q & 1u) + l];
                const unsigned low = q < 2 ? byte & 15u : byte >> 4;
                const unsigned high = ((unsigned)block[128 + 32 * k + l] >> (2 * q)) & 3u;
                const int scale = (int8_t)block[192 + 8 * k + l / 16 + 2 * q];
                const float step = d * (float)scale; /* rounded */
                out[128 * k + 32 * q + l] = step * (float)((int)(low | (high << 4)) - 32);
            }
}

/* IQ4_NL: 32 values; value i < 16 is the low nibble of byte 2 + i, value i + 16 its
 * high nibble, each an index into the IQ4 grid; w = d * grid. */
static void decode_iq4_nl(const uint8_t* block, float* out) {
    const float d = kdo_half_to_float(load_u16(block));
    for (unsigned i = 0; i < 16; ++i) {
        out[i] = d * (float)iq4_grid[block[2 + i] & 15u];
        out[i + 16] = d * (float)iq4_grid[block[2 + i] >> 4];
    }
}

/* IQ4_XS: 8 sub-blocks of 32 with 6-bit scales (low nibble from byte 4 + s/2, high two
 * bits from the 16-bit word at byte 2), offset by 32; sub-block s holds 16 index bytes
 * at 8 + 16s laid out as IQ4_NL; w = (d * scale) * grid. */
static void decode_iq4_xs(const uint8_t* block, float* out) {
    const float d = kdo_half_to_float(load_u16(block));
    const unsigned high = load_u16(block + 2);
    for (unsigned s = 0; s < 8; ++s) {
        const unsigned low = ((unsigned)block[4 + s / 2] >> (4 * (s % 2))) & 15u;
        const int scale = (int)(low | (((high >> (2 * s)) & 3u) << 4)) - 32;
        const float step = d * (float)scale; /* rounded */
        for (unsigned i = 0; i < 16; ++i) {
            const unsigned byte = block[8 + 16 * s + i];
            out[32 * s + i] = step * (float)iq4_grid[byte & 15u];
            out[32 * s + 16 + i] = step * (float)iq4_grid[byte >> 4];
        }
    }
}

/* Q4_K sub-block g (0..7): 6-bit scale and min packed into 12 bytes. */
static void q4k_scale_min(const uint8_t* packed, unsigned g, unsigned* scale, unsigned* min) {
    if (g < 4) {
        *scale = packed[g] & 0x3fu;
        *min = packed[g + 4] & 0x3fu;
    } else {
        *scale = (packed[g + 4] & 0x0fu) | ((unsigned)(packed[g - 4] >> 6) << 4);
        *min = (unsigned)(packed[g + 4] >> 4) | ((unsigned)(packed[g] >> 6) << 4);
    }
}

static void decode_block(int encoding, const uint8_t* block, float* out) {
    switch (encoding) {
    case KDO_Q3_K:
        return decode_q3_k(block, out);
    case KDO_Q6_K:
        return decode_q6_k(block, out);
    case KDO_IQ4_NL:
        return decode_iq4_nl(block, out);
    case KDO_IQ4_XS:
        return decode_iq4_xs(block, out);
    case KDO_BF16:
        out[0] = kdo_bf16_to_float(load_u16(block));
        return;
    case KDO_F32:
        out[0] = bits_to_float(load_u32(block));
        return;
    case KDO_F16:
        out[0] = kdo_half_to_float(load_u16(block));
        return;
    case KDO_IQ3_XXS:
        return decode_iq3_xxs(block, out);
    case KDO_IQ2_S:
        return decode_iq2_s(block, out);
    case KDO_IQ3_S:
        return decode_iq3_s(block, out);
    default:
        break;
    }
    const float d = kdo_half_to_float(load_u16(block));
    if (encoding == KDO_Q8_0) {
        for (int i = 0; i < 32; ++i)
            out[i] = d * (float)(int8_t)block[2 + i];
    } else if (encoding == KDO_Q4_0) {
        for (int i = 0; i < 16; ++i) {
            const uint8_t byte = block[2 + i];
            out[i] = (float)((int)(byte & 0x0f) - 8) * d;
            out[i + 16] = (float)((int)(byte >> 4) - 8) * d;
        }
    } else { /* Q4_K */
        const float dmin = kdo_half_to_float(load_u16(block + 2));
        const uint8_t* packed = block + 4;
        const uint8_t* nibbles = block + 16;
        for (unsigned g = 0; g < 8; ++g) {
            unsigned sc, m;
            q4k_scale_min(packed, g, &sc, &m);
            const float step = d * (float)sc;     /* rounded */
            const float offset = dmin * (float)m; /* rounded */
            const uint8_t* bytes = nibbles + (g / 2) * 32;
            for (unsigned i = 0; i < 32; ++i) {
                const unsigned code = (g & 1u) ? (bytes[i] >> 4) : (bytes[i] & 0x0fu);
                const float scaled = step * (float)code; /* rounded */
                out[g * 32 + i] = scaled - offset;       /* rounded, never fused */
            }
        }
    }
}

int kdo_dequantize_row(int encoding, const uint8_t* row, size_t in, float* out) {
    const int values = kdo_block_values(encoding);
    if (!values || in % (size_t)values)
        return -1;
    const int bytes = kdo_block_bytes(encoding);
    for (size_t b = 0; b < in / (size_t)values; ++b)
        decode_block(encoding, row + b * (size_t)bytes, out + b * (size_t)values);
    return 0;
}

int kdo_gemv(int encoding, const uint8_t* weights, size_t row_bytes, const float* x,
             size_t rows, size_t in, size_t out, float* y, size_t stride) {
    float* decoded = (float*)malloc((in ? in : 1) * sizeof(float));
    if (!decoded)
        return -2;
    for (size_t c = 0; c < out; ++c) {
        if (kdo_dequantize_row(encoding, weights + c * row_bytes, in, decoded)) {
            free(decoded);
            return -1;
        }
        for (size_t r = 0; r < rows; ++r) {
            double sum = 0.0;
            const float* xr = x + r * in;
            for (size_t k = 0; k < in; ++k)
                sum += (double)decoded[k] * (double)xr[k];
            y[r * stride + c] = (float)sum;
        }
    }
    free(decoded);
    return 0;
}

/* ------------------------------------------------------ activation quantizers */

static float block_absmax(const float* x, size_t n) {
    float amax = 0.0f;
    for (size_t j = 0; j < n; ++j) {
        const float a = fabsf(x[j]);
        amax = a > amax ? a : amax;
    }
    return amax;
}

void kdo_quantize_row_q8_0(const float* x, size_t k, int8_t* qs, uint16_t* d_half) {
    for (size_t b = 0; b < k / 32; ++b) {
        const float* xb = x + b * 32;
        const float amax = block_absmax(xb, 32);
        d_half[b] = kdo_float_to_half(amax / 127.0f);
        const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
        for (int j = 0; j < 32; ++j)
            qs[b * 32 + j] = (int8_t)(int)nearbyintf(xb[j] * id); /* round half even */
    }
}

void kdo_quantize_q8_f16(const uint16_t* x, size_t m, size_t k, int8_t* qs, float* d) {
    float block[32];
    for (size_t r = 0; r < m; ++r)
        for (size_t b = 0; b < k / 32; ++b) {
            for (int j = 0; j < 32; ++j)
                block[j] = kdo_half_to_float(x[r * k + b * 32 + j]);
            const float amax = block_absmax(block, 32);
            d[r * (k / 32) + b] = amax / 127.0f;
            const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
            for (int j = 0; j < 32; ++j)
                qs[r * k + b * 32 + j] = (int8_t)(int)nearbyintf(block[j] * id);
        }
}

/* G/src/ggml-quants.c:621-626 nearest_int: round half to even via the 1.5*2^23 trick. */
static int nearest_even(float v) {
    return (int)nearbyintf(v);
}

void kdo_quantize_row_q8_K(const float* x, size_t k, int8_t* qs, float* d, int16_t* bsums) {
    for (size_t b = 0; b < k / 256; ++b) {
        const float* xb = x + b * 256;
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 256; ++j) {
            const float a = fabsf(xb[j]);
            if (a > amax) {
                amax = a;
                max = xb[j];
            }
        }
        int8_t* q = qs + b * 256;
        if (amax == 0.0f) {
            d[b] = 0.0f;
            memset(q, 0, 256);
            memset(bsums + b * 16, 0, 16 * sizeof(int16_t));
            continue;
        }
        const float iscale = -127.0f / max;
        for (int j = 0; j < 256; ++j) {
            const int v = nearest_even(iscale * xb[j]);
            q[j] = (int8_t)(v < 127 ? v : 127);
        }
        for (int g = 0; g < 16; ++g) {
            int sum = 0;
            for (int i = 0; i < 16; ++i)
                sum += q[g * 16 + i];
            bsums[b * 16 + g] = (int16_t)sum;
        }
        d[b] = 1.0f / iscale;
    }
}

/* --------------------------------------------------------------- CPU dots */

float kdo_vec_dot_q8_0_q8_0(size_t k, const uint8_t* w, const int8_t* xq, const uint16_t* xd) {
    float total = 0.0f;
    for (size_t b = 0; b < k / 32; ++b) {
        const uint8_t* block = w + b * 34;
        int dot = 0;
        for (int j = 0; j < 32; ++j)
            dot += (int)(int8_t)block[2 + j] * (int)xq[b * 32 + j];
        total += (float)dot * (kdo_half_to_float(load_u16(block)) * kdo_half_to_float(xd[b]));
    }
    return total;
}

float kdo_vec_dot_q4_0_q8_0(size_t k, const uint8_t* w, const int8_t* xq, const uint16_t* xd) {
    float total = 0.0f;
    for (size_t b = 0; b < k / 32; ++b) {
        const uint8_t* block = w + b * 18;
        const int8_t* q = xq + b * 32;
        int dot = 0;
        for (int j = 0; j < 16; ++j) {
            dot += ((int)(block[2 + j] & 0x0f) - 8) * (int)q[j];
            dot += ((int)(block[2 + j] >> 4) - 8) * (int)q[j + 16];
        }
        total += (float)dot * kdo_half_to_float(load_u16(block)) * kdo_half_to_float(xd[b]);
    }
    return total;
}

float kdo_vec_dot_q4_K_q8_K(size_t k, const uint8_t* w, const int8_t* xq, const float* xd,
                            const int16_t* bsums) {
    float total = 0.0f;
    for (size_t b = 0; b < k / 256; ++b) {
        const uint8_t* block = w + b * 144;
        const int8_t* q = xq + b * 256;
        int scaled = 0, offset = 0;
        for (unsigned g = 0; g < 8; ++g) {
            unsigned sc, m;
            q4k_scale_min(block + 4, g, &sc, &m);
            const uint8_t* bytes = block + 16 + (g / 2) * 32;
            int dot = 0;
            for (unsigned i = 0; i < 32; ++i) {
                const int code = (g & 1u) ? (bytes[i] >> 4) : (bytes[i] & 0x0f);
                dot += code * (int)q[g * 32 + i];
            }
            scaled += (int)sc * dot;
            offset += (int)m * ((int)bsums[b * 16 + 2 * g] + (int)bsums[b * 16 + 2 * g + 1]);
        }
        const float d = kdo_half_to_float(load_u16(block)) * xd[b];
        const float dmin = kdo_half_to_float(load_u16(block + 2)) * xd[b];
        total += d * (float)scaled - dmin * (float)offset;
    }
    return total;
}

/* ----------------------------------------------------- threaded CPU matvec */

typedef struct {
    int encoding;
    const uint8_t* weights;
    size_t row_bytes, rows, in, out;
    const int8_t* xq;
    const void* xd; /* uint16_t* (q8_0) or float* (q8_K) */
    const int16_t* bsums;
    float* y;
    atomic_size_t next;
} matvec_work;

enum { UNIT_COLUMNS = 64 };

static void* matvec_worker(void* arg) {
    matvec_work* m = (matvec_work*)arg;
    const size_t units = (m->out + UNIT_COLUMNS - 1) / UNIT_COLUMNS;
    for (;;) {
        const size_t u = atomic_fetch_add(&m->next, 1);
        if (u >= units)
            break;
        const size_t end = (u + 1) * UNIT_COLUMNS < m->out ? (u + 1) * UNIT_COLUMNS : m->out;
        for (size_t c = u * UNIT_COLUMNS; c < end; ++c)
            for (size_t r = 0; r < m->rows; ++r) {
                const uint8_t* row = m->weights + c * m->row_bytes;
                const int8_t* q = m->xq + r * m->in;
                float v;
                if (m->encoding == KDO_Q4_K)
                    v = kdo_vec_dot_q4_K_q8_K(m->in, row, q, (const float*)m->xd + r * (m->in / 256),
                                              m->bsums + r * (m->in / 16));
                else if (m->encoding == KDO_Q8_0)
                    v = kdo_vec_dot_q8_0_q8_0(m->in, row, q, (const uint16_t*)m->xd + r * (m->in / 32));
                else
                    v = kdo_vec_dot_q4_0_q8_0(m->in, row, q, (const uint16_t*)m->xd + r * (m->in / 32));
                m->y[r * m->out + c] = v;
            }
    }
    return NULL;
}

int kdo_cpu_matvec(int encoding, const uint8_t* weights, size_t row_bytes, const float* x,
                   size_t rows, size_t in, size_t out, float* y, int threads) {
    if ((encoding != KDO_Q4_0 && encoding != KDO_Q8_0 && encoding != KDO_Q4_K) ||
        in % (size_t)kdo_block_values(encoding) || threads < 1)
        return -1;
    int8_t* xq = (int8_t*)malloc(rows * in + 1);
    void* xd = malloc(rows * (in / 16 + 1) * sizeof(float));
    int16_t* bsums = (int16_t*)malloc(rows * (in / 16 + 1) * sizeof(int16_t));
    if (!xq || !xd || !bsums) {
        free(xq), free(xd), free(bsums);
        return -2;
    }
    for (size_t r = 0; r < rows; ++r) {
        if (encoding == KDO_Q4_K)
            kdo_quantize_row_q8_K(x + r * in, in, xq + r * in, (float*)xd + r * (in / 256),
                                  bsums + r * (in / 16));
        else
            kdo_quantize_row_q8_0(x + r * in, in, xq + r * in, (uint16_t*)xd + r * (in / 32));
    }
    matvec_work work = {encoding, weights, row_bytes, rows, in, out, xq, xd, bsums, y, 0};
    pthread_t* pool = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    int started = 0;
    for (int t = 1; t < threads && pool; ++t)
        if (pthread_create(&pool[started], NULL, matvec_worker, &work) == 0)
            ++started;
    matvec_worker(&work); /* the caller is the last worker */
    for (int t = 0; t < started; ++t)
        pthread_join(pool[t], NULL);
    free(pool);
    free(xq), free(xd), free(bsums);
    return 0;
}

/* ------------------------------------------------------------ Q4_0 GEMM */

int kdo_gemm_q4_0_q8(const uint8_t* weights, size_t n_out, size_t k, const int8_t* xq,
                     const float* xd, size_t m, float* y) {
    if (k % 32)
        return -1;
    const size_t blocks = k / 32;
    for (size_t n = 0; n < n_out; ++n) {
        const uint8_t* row = weights + n * blocks * 18;
        for (size_t r = 0; r < m; ++r) {
            double sum = 0.0;
            for (size_t b = 0; b < blocks; ++b) {
                const uint8_t* block = row + b * 18;
                const int8_t* q = xq + r * k + b * 32;
                int dot = 0;
                for (int j = 0; j < 16; ++j) {
                    dot += ((int)(block[2 + j] & 0x0f) - 8) * (int)q[j];
                    dot += ((int)(block[2 + j] >> 4) - 8) * (int)q[j + 16];
                }
                sum += (double)dot * (double)kdo_half_to_float(load_u16(block)) *
                       (double)xd[r * blocks + b];
            }
            y[r * n_out + n] = (float)sum;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ MXFP4 */

float kdo_e2m1(uint8_t code) {
    /* sign bit 3; exponent bits 2..1; mantissa bit 0; subnormal step 0.5 */
    static const float magnitude[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    const float v = magnitude[code & 7u];
    return (code & 8u) ? -v : v;
}

/* One decoded row of MXFP4 weights; returns 0 or a negative error. */
static int mxfp4_row(const uint8_t* blocks, const uint8_t* scales, size_t cols, float* out) {
    for (size_t c = 0; c < cols; ++c) {
        const uint8_t scale = scales[c / 32];
        if (scale == 255)
            return -2;
        const uint8_t code = (uint8_t)((blocks[c / 2] >> (4 * (c % 2))) & 15u);
        const double value = ldexp((double)kdo_e2m1(code), (int)scale - 127);
        if (!isfinite(value) || fabs(value) > 3.4028234663852886e38)
            return -3;
        out[c] = (float)value;
    }
    return 0;
}

int kdo_mxfp4_decode_rows(const uint8_t* blocks, const uint8_t* scales, size_t rows,
                          size_t cols, float* out) {
    if (!cols || cols % 32)
        return -1;
    for (size_t r = 0; r < rows; ++r) {
        const int rc = mxfp4_row(blocks + r * (cols / 2), scales + r * (cols / 32), cols,
                                 out + r * cols);
        if (rc)
            return rc;
    }
    return 0;
}

static int finite_to_float(double v, float* out) {
    if (!isfinite(v) || fabs(v) > 3.4028234663852886e38)
        return -3;
    *out = (float)v;
    return 0;
}

int kdo_mxfp4_matvec(const uint8_t* blocks, const uint8_t* scales, size_t rows, size_t cols,
                     const float* x, float* y) {
    if (!cols || cols % 32)
        return -1;
    for (size_t c = 0; c < cols; ++c)
        if (!isfinite(x[c]))
            return -4;
    float* row = (float*)malloc(cols * sizeof(float));
    if (!row)
        return -5;
    for (size_t r = 0; r < rows; ++r) {
        int rc = mxfp4_row(blocks + r * (cols / 2), scales + r * (cols / 32), cols, row);
        double sum = 0.0;
        for (size_t c = 0; !rc && c < cols; ++c)
            sum += (double)row[c] * (double)x[c];
        if (!rc)
            rc = finite_to_float(sum, &y[r]);
        if (rc) {
            free(row);
            return rc;
        }
    }
    free(row);
    return 0;
}

/* -------------------------------------------------------------------- MoE */

/* The reference orders the experts with std::partial_sort(order, order + k, order + E,
 * [&](a, b) { return p[a] > p[b]; }) over order = 0..E-1 (qwen_layers.cpp:409-416).
 * libstdc++ implements it as a heap selection followed by a heap sort of the first k
 * (std::__heap_select, std::__sort_heap, both over std::__adjust_heap); the functions
 * below restate that published binary-heap algorithm step for step, because its order
 * among equal probabilities (and among NaN ones, which compare false both ways) is the
 * reference's selection order.  Pinned against std::partial_sort itself (compiled
 * reference bindings) on random tie patterns. */
static int route_before(const float* p, int32_t a, int32_t b) {
    return p[a] > p[b];
}

/* The hole at `hole` moves down to a leaf along the child that is "larger" under the
 * comparator (the right child unless the left one compares before it), then `value` is
 * pushed back up towards `top`. */
static void heap_adjust(int32_t* h, size_t hole, size_t len, int32_t value, const float* p) {
    const size_t top = hole;
    size_t child = hole;
    while (child < (len - 1) / 2) {
        child = 2 * (child + 1);
        if (route_before(p, h[child], h[child - 1]))
            --child;
        h[hole] = h[child];
        hole = child;
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
        child = 2 * (child + 1);
        h[hole] = h[child - 1];
        hole = child - 1;
    }
    while (hole > top) {
        const size_t parent = (hole - 1) / 2;
        if (!route_before(p, h[parent], value))
            break;
        h[hole] = h[parent];
        hole = parent;
    }
    h[hole] = value;
}

/* order[0..k) = the first k of std::partial_sort over experts 0..E-1. */
static void route_partial_sort(const float* p, size_t experts, size_t k, int32_t* order) {
    for (size_t i = 0; i < k; ++i)
        order[i] = (int32_t)i;
    if (k >= 2) /* make_heap */
        for (size_t parent = (k - 2) / 2;; --parent) {
            heap_adjust(order, parent, k, order[parent], p);
            if (!parent)
                break;
        }
    /* heap select: position i still holds expert i when it is visited */
    for (size_t i = k; i < experts; ++i)
        if (route_before(p, (int32_t)i, order[0])) {
            heap_adjust(order, 0, k, (int32_t)i, p); /* pop_heap: old top goes to i */
        }
    for (size_t last = k; last > 1;) { /* sort_heap */
        --last;
        const int32_t value = order[last];
        order[last] = order[0];
        heap_adjust(order, 0, last, value, p);
    }
}

void kdo_moe_route(const float* logits, size_t tokens, size_t experts, size_t top_k,
                   int32_t* idx, float* w) {
    float* p = (float*)malloc(experts * sizeof(float));
    for (size_t t = 0; t < tokens; ++t) {
        const float* l = logits + t * experts;
        float maximum = l[0]; /* std::max_element: the first e with no l[e] < later */
        for (size_t e = 1; e < experts; ++e)
            maximum = maximum < l[e] ? l[e] : maximum;
        double total = 0.0;
        for (size_t e = 0; e < experts; ++e) {
            p[e] = expf(l[e] - maximum);
            total += (double)p[e];
        }
        for (size_t e = 0; e < experts; ++e)
            p[e] = (float)((double)p[e] / total);
        route_partial_sort(p, experts, top_k, idx + t * top_k);
        float sum = 0.0f;
        for (size_t i = 0; i < top_k; ++i) {
            w[t * top_k + i] = p[idx[t * top_k + i]];
            sum += w[t * top_k + i];
        }
        sum = sum > 6.103515625e-5f ? sum : 6.103515625e-5f;
        for (size_t i = 0; i < top_k; ++i)
            w[t * top_k + i] /= sum;
    }
    free(p);
}

void kdo_moe_permute(const int32_t* idx, size_t tokens, size_t top_k, size_t experts,
                     int32_t* offsets, int32_t* perm) {
    const size_t slots = tokens * top_k;
    memset(offsets, 0, (experts + 1) * sizeof(int32_t));
    for (size_t s = 0; s < slots; ++s)
        offsets[idx[s] + 1] += 1;
    for (size_t e = 0; e < experts; ++e)
        offsets[e + 1] += offsets[e];
    size_t position = 0;
    for (size_t e = 0; e < experts; ++e)
        for (size_t s = 0; s < slots; ++s)
            if ((size_t)idx[s] == e)
                perm[position++] = (int32_t)s;
}

static float silu(float v) {
    return v / (1.0f + expf(-v));
}

typedef struct {
    const uint16_t* x;
    size_t tokens, hidden, inter, experts, top_k;
    const uint8_t *gate_blocks, *gate_scales, *up_blocks, *up_scales, *down_blocks, *down_scales;
    const int32_t *offsets, *perm;
    const float* w;
    float* contribution; /* [slots * hidden] */
    atomic_size_t next;
    atomic_int error;
} moe_work;

static void* moe_worker(void* arg) {
    moe_work* m = (moe_work*)arg;
    const size_t H = m->hidden, I = m->inter;
    float* xrow = (float*)malloc(H * sizeof(float) * 1);
    float* wrow = (float*)malloc((H > I ? H : I) * sizeof(float));
    for (;;) {
        const size_t e = atomic_fetch_add(&m->next, 1);
        if (e >= m->experts || atomic_load(&m->error))
            break;
        const size_t first = (size_t)m->offsets[e], count = (size_t)m->offsets[e + 1] - first;
        if (!count)
            continue;
        float* xs = (float*)malloc(count * H * sizeof(float));
        float* g = (float*)malloc(count * I * sizeof(float));
        float* u = (float*)malloc(count * I * sizeof(float));
        for (size_t r = 0; r < count; ++r) {
            const size_t token = (size_t)m->perm[first + r] / m->top_k;
            for (size_t c = 0; c < H; ++c)
                xs[r * H + c] = kdo_bf16_to_float(m->x[token * H + c]);
        }
        int rc = 0;
        /* gate and up: [I rows x H cols] per expert */
        for (int which = 0; which < 2 && !rc; ++which) {
            const uint8_t* blocks = (which ? m->up_blocks : m->gate_blocks) + e * I * (H / 2);
            const uint8_t* scales = (which ? m->up_scales : m->gate_scales) + e * I * (H / 32);
            float* outp = which ? u : g;
            for (size_t n = 0; n < I && !rc; ++n) {
                rc = mxfp4_row(blocks + n * (H / 2), scales + n * (H / 32), H, wrow);
                for (size_t r = 0; r < count && !rc; ++r) {
                    double sum = 0.0;
                    for (size_t c = 0; c < H; ++c)
                        sum += (double)wrow[c] * (double)xs[r * H + c];
                    rc = finite_to_float(sum, &outp[r * I + n]);
                }
            }
        }
        /* h = silu(g) * u, in float */
        for (size_t i = 0; i < count * I && !rc; ++i)
            g[i] = silu(g[i]) * u[i];
        /* down: [H rows x I cols]; contribution = down * w[slot] */
        const uint8_t* blocks = m->down_blocks + e * H * (I / 2);
        const uint8_t* scales = m->down_scales + e * H * (I / 32);
        for (size_t d = 0; d < H && !rc; ++d) {
            rc = mxfp4_row(blocks + d * (I / 2), scales + d * (I / 32), I, wrow);
            for (size_t r = 0; r < count && !rc; ++r) {
                double sum = 0.0;
                for (size_t c = 0; c < I; ++c)
                    sum += (double)wrow[c] * (double)g[r * I + c];
                float down = 0.0f;
                rc = finite_to_float(sum, &down);
                const size_t slot = (size_t)m->perm[first + r];
                m->contribution[slot * H + d] = down * m->w[slot];
            }
        }
        free(xs), free(g), free(u);
        if (rc)
            atomic_store(&m->error, rc);
    }
    free(xrow);
    free(wrow);
    return NULL;
}

int kdo_moe_forward(const uint16_t* x, const float* logits, size_t tokens, size_t hidden,
                    size_t inter, size_t experts, size_t top_k,
                    const uint8_t* gate_blocks, const uint8_t* gate_scales,
                    const uint8_t* up_blocks, const uint8_t* up_scales,
                    const uint8_t* down_blocks, const uint8_t* down_scales,
                    float* y, int32_t* idx, float* w, int32_t* offsets, int32_t* perm,
                    int threads) {
    if (!hidden || !inter || hidden % 32 || inter % 32 || !top_k || top_k > experts || threads < 1)
        return -1;
    for (size_t i = 0; i < tokens * hidden; ++i)
        if (!isfinite(kdo_bf16_to_float(x[i])))
            return -4;
    kdo_moe_route(logits, tokens, experts, top_k, idx, w);
    kdo_moe_permute(idx, tokens, top_k, experts, offsets, perm);
    float* contribution = (float*)calloc(tokens * top_k * hidden + 1, sizeof(float));
    if (!contribution)
        return -5;
    moe_work work = {x, tokens, hidden, inter, experts, top_k, gate_blocks, gate_scales,
                     up_blocks, up_scales, down_blocks, down_scales, offsets, perm, w,
                     contribution, 0, 0};
    pthread_t* pool = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    int started = 0;
    for (int t = 1; t < threads && pool; ++t)
        if (pthread_create(&pool[started], NULL, moe_worker, &work) == 0)
            ++started;
    moe_worker(&work);
    for (int t = 0; t < started; ++t)
        pthread_join(pool[t], NULL);
    free(pool);
    const int rc = atomic_load(&work.error);
    if (!rc)
        for (size_t t = 0; t < tokens; ++t)
            for (size_t d = 0; d < hidden; ++d) {
                float sum = 0.0f;
                for (size_t i = 0; i < top_k; ++i)
                    sum += contribution[(t * top_k + i) * hidden + d];
                y[t * hidden + d] = sum;
            }
    free(contribution);
    return rc;
}

/* ------------------------------------------- MoE, fp32 products (CPU baseline) */

/* The same layer with every product accumulated in fp32 and vectorised with AVX2 FMA
 * (eight lanes, four accumulators, summed pairwise at the end): the fast CPU form that
 * sits beside the exact double-accumulation flow as a baseline.  It is timed only, not a
 * checker.  Work is split as the reference worker splits a projection, into units of 64
 * output rows (IW/src/models/text/gguf_weights.cpp:400-446) taken from a shared counter:
 * phase 1 the (expert, 64 gate/up rows) units, phase 2 the (expert, 64 down rows) units. */

typedef struct {
    const uint16_t* x;
    size_t hidden, inter, experts, top_k;
    const uint8_t *gate_blocks, *gate_scales, *up_blocks, *up_scales, *down_blocks, *down_scales;
    const int32_t *offsets, *perm;
    const float* w;
    float *xs, *g, *u, *contribution; /* xs, g, u: rows in permuted (expert-major) order */
    size_t units, phase;
    atomic_size_t next;
    atomic_int error;
} moe32_work;

/* One decoded MXFP4 row in fp32 (exact: an E2M1 value times a power of two). */
static int mxfp4_row_f32(const uint8_t* blocks, const uint8_t* scales, size_t cols, float* out) {
    static const float value[16] = {0.0f, 0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                                    -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};
    for (size_t b = 0; b < cols / 32; ++b) {
        if (scales[b] == 255)
            return -2;
        const float scale = ldexpf(1.0f, (int)scales[b] - 127);
        for (size_t i = 0; i < 16; ++i) {
            const uint8_t byte = blocks[16 * b + i];
            out[32 * b + 2 * i] = value[byte & 15u] * scale;
            out[32 * b + 2 * i + 1] = value[byte >> 4] * scale;
        }
    }
    for (size_t c = 0; c < cols; ++c)
        if (!isfinite(out[c]))
            return -3;
    return 0;
}

__attribute__((target("avx2,fma"))) static float dot_avx2(const float* a, const float* b,
                                                          size_t n) {
    __m256 s0 = _mm256_setzero_ps(), s1 = s0, s2 = s0, s3 = s0;
    size_t i = 0;
    for (; i + 32 <= n; i += 32) {
        s0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), s0);
        s1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), s1);
        s2 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 16), _mm256_loadu_ps(b + i + 16), s2);
        s3 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 24), _mm256_loadu_ps(b + i + 24), s3);
    }
    for (; i + 8 <= n; i += 8)
        s0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), s0);
    const __m256 s = _mm256_add_ps(_mm256_add_ps(s0, s1), _mm256_add_ps(s2, s3));
    float lanes[8];
    _mm256_storeu_ps(lanes, s);
    float total = ((lanes[0] + lanes[1]) + (lanes[2] + lanes[3])) +
                  ((lanes[4] + lanes[5]) + (lanes[6] + lanes[7]));
    for (; i < n; ++i)
        total += a[i] * b[i];
    return total;
}

static float dot_f32(const float* a, const float* b, size_t n) {
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma"))
        return dot_avx2(a, b, n);
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i)
        s += a[i] * b[i];
    return s;
}

static void* moe32_worker(void* arg) {
    moe32_work* m = (moe32_work*)arg;
    const size_t H = m->hidden, I = m->inter;
    const size_t in = m->phase == 1 ? H : I, out = m->phase == 1 ? I : H;
    const size_t blocks_per_expert = (out + 63) / 64;
    float* wrow = (float*)malloc(in * sizeof(float));
    for (;;) {
        const size_t unit = atomic_fetch_add(&m->next, 1);
        if (unit >= m->units || atomic_load(&m->error))
            break;
        const size_t e = unit / blocks_per_expert, r0 = unit % blocks_per_expert * 64;
        const size_t first = (size_t)m->offsets[e], count = (size_t)m->offsets[e + 1] - first;
        const size_t r1 = r0 + 64 < out ? r0 + 64 : out;
        int rc = 0;
        for (size_t n = r0; n < r1 && count && !rc; ++n) {
            if (m->phase == 1) {
                for (int which = 0; which < 2 && !rc; ++which) {
                    const uint8_t* b = (which ? m->up_blocks : m->gate_blocks) + (e * I + n) * (H / 2);
                    const uint8_t* sc = (which ? m->up_scales : m->gate_scales) + (e * I + n) * (H / 32);
                    float* o = which ? m->u : m->g;
                    rc = mxfp4_row_f32(b, sc, H, wrow);
                    for (size_t r = 0; r < count && !rc; ++r)
                        o[(first + r) * I + n] = dot_f32(wrow, m->xs + (first + r) * H, H);
                }
            } else {
                rc = mxfp4_row_f32(m->down_blocks + (e * H + n) * (I / 2),
                                   m->down_scales + (e * H + n) * (I / 32), I, wrow);
                for (size_t r = 0; r < count && !rc; ++r) {
                    const size_t slot = (size_t)m->perm[first + r];
                    m->contribution[slot * H + n] =
                        dot_f32(wrow, m->g + (first + r) * I, I) * m->w[slot];
                }
            }
        }
        if (rc)
            atomic_store(&m->error, rc);
    }
    free(wrow);
    return NULL;
}

static int moe32_phase(moe32_work* m, size_t phase, int threads) {
    const size_t out = phase == 1 ? m->inter : m->hidden;
    m->phase = phase;
    m->units = m->experts * ((out + 63) / 64);
    atomic_store(&m->next, 0);
    pthread_t* pool = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
    int started = 0;
    for (int t = 1; t < threads && pool; ++t)
        if (pthread_create(&pool[started], NULL, moe32_worker, m) == 0)
            ++started;
    moe32_worker(m);
    for (int t = 0; t < started; ++t)
        pthread_join(pool[t], NULL);
    free(pool);
    return atomic_load(&m->error);
}

int kdo_moe_forward_f32(const uint16_t* x, const float* logits, size_t tokens, size_t hidden,
                        size_t inter, size_t experts, size_t top_k,
                        const uint8_t* gate_blocks, const uint8_t* gate_scales,
                        const uint8_t* up_blocks, const uint8_t* up_scales,
                        const uint8_t* down_blocks, const uint8_t* down_scales, float* y,
                        int threads) {
    if (!hidden || !inter || hidden % 32 || inter % 32 || !top_k || top_k > experts ||
        threads < 1)
        return -1;
    const size_t slots = tokens * top_k;
    int32_t* idx = (int32_t*)malloc(slots * sizeof(int32_t));
    float* w = (float*)malloc(slots * sizeof(float));
    int32_t* offsets = (int32_t*)malloc((experts + 1) * sizeof(int32_t));
    int32_t* perm = (int32_t*)malloc((slots + 1) * sizeof(int32_t));
    float* xs = (float*)malloc((slots * hidden + 1) * sizeof(float));
    float* g = (float*)malloc((slots * inter + 1) * sizeof(float));
    float* u = (float*)malloc((slots * inter + 1) * sizeof(float));
    float* contribution = (float*)calloc(slots * hidden + 1, sizeof(float));
    int rc = (idx && w && offsets && perm && xs && g && u && contribution) ? 0 : -5;
    if (!rc) {
        kdo_moe_route(logits, tokens, experts, top_k, idx, w);
        kdo_moe_permute(idx, tokens, top_k, experts, offsets, perm);
        for (size_t p = 0; p < slots; ++p)
            for (size_t c = 0; c < hidden; ++c)
                xs[p * hidden + c] = kdo_bf16_to_float(x[(size_t)perm[p] / top_k * hidden + c]);
        moe32_work work = {x, hidden, inter, experts, top_k, gate_blocks, gate_scales,
                           up_blocks, up_scales, down_blocks, down_scales, offsets, perm, w,
                           xs, g, u, contribution, 0, 0, 0, 0};
        rc = moe32_phase(&work, 1, threads);
        for (size_t i = 0; !rc && i < slots * inter; ++i)
            g[i] = silu(g[i]) * u[i];
        if (!rc)
            rc = moe32_phase(&work, 2, threads);
        for (size_t t = 0; !rc && t < tokens; ++t)
            for (size_t d = 0; d < hidden; ++d) {
                float sum = 0.0f;
                for (size_t i = 0; i < top_k; ++i)
                    sum += contribution[(t * top_k + i) * hidden + d];
                y[t * hidden + d] = sum;
            }
    }
    free(idx), free(w), free(offsets), free(perm), free(xs), free(g), free(u);
    free(contribution);
    return rc;
}

/* ------------------------------------------------------------ GGUF MoE layer */

static float silu_f(float v) {
    return v / (1.0f + expf(-v));
}

static float sigmoid_f(float v) {
    return 1.0f / (1.0f + expf(-v));
}

static int product(const kdo_gguf_tensor* m, size_t expert, const float* x, size_t rows,
                   size_t in, size_t out, float* y) {
    return kdo_gemv(m->encoding, m->weights + expert * m->expert_bytes, m->row_bytes, x, rows,
                    in, out, y, out);
}

int kdo_moe_gguf_forward(const kdo_moe_gguf_layer* L, const float* x, size_t rows, float* y,
                         int32_t* idx, float* w) {
    if (!L || !x || !y || !idx || !w || !rows || !L->top_k || L->top_k > L->experts)
        return -1;
    const size_t H = L->hidden, E = L->experts, K = L->top_k, F = L->ff, S = L->shared_ff;
    float* logits = (float*)malloc(rows * E * sizeof(float));
    float* sg = (float*)malloc(rows * S * sizeof(float));
    float* su = (float*)malloc(rows * S * sizeof(float));
    float* shared_down = (float*)malloc(rows * H * sizeof(float));
    float* g = (float*)malloc(F * sizeof(float));
    float* u = (float*)malloc(F * sizeof(float));
    float* down = (float*)malloc(rows * K * H * sizeof(float));
    int rc = -2;
    if (!logits || !sg || !su || !shared_down || !g || !u || !down)
        goto done;
    rc = -1;
    /* router and the shared expert's gate / up (qwen_layers.cpp:383-396) */
    if (product(&L->router, 0, x, rows, H, E, logits) ||
        product(&L->gate_shexp, 0, x, rows, H, S, sg) ||
        product(&L->up_shexp, 0, x, rows, H, S, su))
        goto done;
    for (size_t i = 0; i < rows * S; ++i)
        sg[i] = silu_f(sg[i]) * su[i];
    kdo_moe_route(logits, rows, E, K, idx, w); /* :397-425 */
    /* each selection: gate / up, silu * up, down, times its weight (:427-468) */
    for (size_t s = 0; s < rows * K; ++s) {
        const size_t e = (size_t)idx[s];
        const float* xs = x + (s / K) * H;
        if (product(&L->gate_exps, e, xs, 1, H, F, g) || product(&L->up_exps, e, xs, 1, H, F, u))
            goto done;
        for (size_t j = 0; j < F; ++j)
            g[j] = silu_f(g[j]) * u[j];
        if (product(&L->down_exps, e, g, 1, F, H, down + s * H))
            goto done;
        for (size_t d = 0; d < H; ++d)
            down[s * H + d] = down[s * H + d] * w[s];
    }
    if (product(&L->down_shexp, 0, sg, rows, S, H, shared_down))
        goto done;
    /* :469-491: selection-order sum plus the gated shared expert */
    for (size_t t = 0; t < rows; ++t) {
        float gate = 0.0f;
        for (size_t c = 0; c < H; ++c)
            gate += L->shared_gate[c] * x[t * H + c];
        gate = sigmoid_f(gate);
        for (size_t d = 0; d < H; ++d) {
            float sum = 0.0f;
            for (size_t i = 0; i < K; ++i)
                sum += down[(t * K + i) * H + d];
            y[t * H + d] = sum + shared_down[t * H + d] * gate;
        }
    }
    rc = 0;
done:
    free(logits), free(sg), free(su), free(shared_down), free(g), free(u), free(down);
    return rc;
}
