// Prefill GEMM over the tile-packed GGUF bank copy for gfx950: Y[m, n] (fp32) =
// sum_k X[m, k] W[n, k] for the kadan encodings Q4_K, Q8_0 and Q6_K.
//
// The reference runs prefill chunks by decoding a packed tile to fp32 and calling
// cublasSgemm (IW/src/cuda/h3_compute.cu:2201-2218,2451, project<float> :1780-2530; IW =
// services/hikari/inference_worker), so its product is the fp32 product of exactly
// decoded weights (kadan::gguf::decode, IW/include/kadan/gguf_quantization.hpp:631-762).
// Here the weights stay packed in HBM and are dequantised in registers to fp16 MFMA
// operands; the activations are fp16 after an exact power-of-two scale per token (so
// no value overflows fp16 and none goes subnormal); products accumulate in fp32 on
// v_mfma_f32_32x32x16_f16 and the scale is undone in the epilogue.  Roundings: the
// activation once to fp16; the weight once (Q8_0: fp16(d * q); Q4_K: fp16(q * fp16(d *
// sc) - fp16(dmin * m)); Q6_K: fp16((q - 32) * fp16(d * sc))).
//
// Kernels:
//   stage_kernel<ENC>  one workgroup per token row: the row's power-of-two scale, and the
//                      row as fp16 in the order the weight lanes consume each 256-value
//                      group (the permutation depends on the format's packed lane image)
//   gemm_kernel<ENC, W> 128 tokens x 256 weight rows per workgroup, W = 4 wavefronts
//                      each owning two 32-row weight operands (W = 8: one) and all 128
//                      tokens; weights go from HBM straight into operand registers
//                      (16-byte loads of the packed lane images, issued one group
//                      ahead) and are dequantised there; activations are staged into
//                      swizzled LDS by global->LDS DMA; the fp32 output tile leaves
//                      through LDS as whole rows.
#include "kdq_common.hpp"

#include <algorithm>

namespace kdq {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int PM = 128;                      // tokens per workgroup tile (4 blocks of 32)
constexpr int NB = 2;                        // 32-row weight operands per wavefront
constexpr int kTiles = 8 * NB;               // 16-row packed tiles per workgroup
constexpr int kStageRow = 512;               // LDS bytes per token of one staged group
constexpr int kDmaRows = 1024 / kStageRow;   // token rows per 64-lane 16-byte DMA
constexpr int kOutPitch = kTiles * 16 * 4 + 16;  // fp32 output row in LDS (+16: banks)
// LDS of a workgroup with TM-token tiles: two activation stages, reused for the output
template <int TM> constexpr size_t gemm_lds =
    std::max(size_t(TM) * kOutPitch, 2 * size_t(TM) * kStageRow);
constexpr size_t kLds = gemm_lds<PM>;

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void global_void;

// ------------------------------------------------------------------ formats
//
// Lane (r, h) of a 32-row weight operand (MFMA lane r + 32h: weight row r, K values
// 8h..8h+7 of each 16-value sub-step) reads, for group chunk G = 2j + h (j = 0, 1), the
// packed lane position l = 16G + r % 16 of tile r / 16.  Sub-step s = 8j + 4p + u (p,
// u as each format names them) gives the lane 8 values of chunk G; value(s, h, e) is the
// group index (0..255) of operand element e, which the staging kernel uses to place the
// activations.  Packed units (kdq_gguf_pack): Q4_K 2304 B = code pieces 0, 1 (bytes
// 16p..16p+15 of sub-block pair G), 16-byte row headers at 2048 + 16 (r % 16); Q8_0 4352
// B = pieces 2c + hh (bytes 16hh..16hh+15 of block 2G + c), scale dwords at 4096 + 4l
// (d of blocks 2G, 2G+1); Q6_K 3360 B = ql pieces 0, 1 (bytes 32G + 16p..), the qh bit
// pairs in piece 2 (dword m: position 8m + i in the high nibble of byte i, 8m + 4 + i in
// its low nibble, block-0 bits | block-1 bits << 2), scale dwords at 3072 + 4l (the
// chunk's four int8 scales), row d at 3328 + 4 (slot / 2).
template <int ENC> struct GemmFormat;

template <> struct GemmFormat<KDQ_Q4_K> {
    static constexpr int unit = 2304, loads = 5;  // per operand and group
    struct Regs {
        u32x4 code[2][2];
        u32x4 head;
    };
    // operand element e of sub-step s: low nibbles of code bytes 16p + 4u + {0, 2, 1, 3}
    // (block 2G), then the high nibbles of the same bytes (block 2G + 1)
    __host__ __device__ static unsigned value(unsigned s, unsigned h, unsigned e) {
        const unsigned G = 2 * (s / 8) + h, p = (s / 4) % 2, u = s % 4;
        const unsigned ord[4] = {0, 2, 1, 3};
        return 64 * G + (e >= 4 ? 32 : 0) + 16 * p + 4 * u + ord[e % 4];
    }
};

template <> struct GemmFormat<KDQ_Q8_0> {
    static constexpr int unit = 4352, loads = 10;
    struct Regs {
        u32x4 code[2][4];
        unsigned scale[2];
    };
    // s = 8j + 4c + 2hh + v: bytes 16hh + 8v .. +7 of block 2G + c, in order
    __host__ __device__ static unsigned value(unsigned s, unsigned h, unsigned e) {
        const unsigned G = 2 * (s / 8) + h, c = (s / 4) % 2, hh = (s / 2) % 2, v = s % 2;
        return 64 * G + 32 * c + 16 * hh + 8 * v + e;
    }
};

template <> struct GemmFormat<KDQ_Q6_K> {
    static constexpr int unit = 3360, loads = 9;
    struct Regs {
        u32x4 code[2][2];
        u32x4 qh[2];
        unsigned scale[2];
        unsigned d;
    };
    // s = 8j + 4p + u: ql bytes 16p + 4u + {0..3} of chunk G; their low nibbles are
    // super-block positions 128(G/2) + 32(G%2) + t (t = 16p + 4u + i), the high nibbles
    // the same + 64
    __host__ __device__ static unsigned value(unsigned s, unsigned h, unsigned e) {
        const unsigned G = 2 * (s / 8) + h, p = (s / 4) % 2, u = s % 4;
        return 128 * (G / 2) + 32 * (G % 2) + (e >= 4 ? 64 : 0) + 16 * p + 4 * u + e % 4;
    }
};

__device__ __forceinline__ f16x2 pair(float v) {
    const _Float16 h = _Float16(v);
    return f16x2{h, h};
}

__device__ __forceinline__ f16x2 as_f16x2(unsigned v) {
    return __builtin_bit_cast(f16x2, v);
}

// fp16 value as fp32 (exact), of the low or high half of a dword
__device__ __forceinline__ float half_lo(unsigned v) {
    return float(__builtin_bit_cast(_Float16, uint16_t(v & 0xffffu)));
}
__device__ __forceinline__ float half_hi(unsigned v) {
    return float(__builtin_bit_cast(_Float16, uint16_t(v >> 16)));
}

// Per-group operand scales of one lane (computed once per group from its registers).
template <int ENC> struct Scales;

// Q4_K: for the lane's blocks 4j + 2h + b (b = 0, 1): fp16(d * sc) and fp16(-dmin * m)
template <> struct Scales<KDQ_Q4_K> {
    f16x2 dsc[2][2], ndm[2][2];
    __device__ __forceinline__ void prepare(const GemmFormat<KDQ_Q4_K>::Regs& g, unsigned h,
                                            unsigned& flags) {
        const float d = half_lo(g.head.x), dmin = half_hi(g.head.x);
        const unsigned s[3] = {g.head.y, g.head.z, g.head.w};  // scale bytes 0..11
        auto byte = [&](unsigned i) { return (s[i / 4] >> (8 * (i % 4))) & 255u; };
        if (!isfinite(d) || !isfinite(dmin))
            flags |= 1u;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const unsigned k = 4 * j + 2 * h + b;  // block of the super-block
                unsigned sc, m;
                if (k < 4) {
                    sc = byte(k) & 63u;
                    m = byte(k + 4) & 63u;
                } else {
                    sc = (byte(k + 4) & 15u) | ((byte(k - 4) >> 6) << 4);
                    m = (byte(k + 4) >> 4) | ((byte(k) >> 6) << 4);
                }
                const float a = d * float(sc), c = dmin * float(m);
                if (15.f * fabsf(a) + fabsf(c) > 65504.f)
                    flags |= 2u;  // a weight past the fp16 range
                dsc[j][b] = pair(a);
                ndm[j][b] = pair(-c);
            }
    }
};

// Q8_0: d of blocks 2G + c
template <> struct Scales<KDQ_Q8_0> {
    f16x2 d[2][2];
    __device__ __forceinline__ void prepare(const GemmFormat<KDQ_Q8_0>::Regs& g, unsigned,
                                            unsigned& flags) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const unsigned sc = g.scale[j];
            const float d0 = half_lo(sc), d1 = half_hi(sc);
            if (!isfinite(d0) || !isfinite(d1))
                flags |= 1u;
            if (128.f * fmaxf(fabsf(d0), fabsf(d1)) > 65504.f)
                flags |= 2u;
            d[j][0] = as_f16x2(__builtin_amdgcn_perm(sc, sc, 0x01000100u));
            d[j][1] = as_f16x2(__builtin_amdgcn_perm(sc, sc, 0x03020302u));
        }
    }
};

// Q6_K: fp16(d * sc) of the four 16-value scales the lane's chunk uses, per j
template <> struct Scales<KDQ_Q6_K> {
    f16x2 dsc[2][4];
    __device__ __forceinline__ void prepare(const GemmFormat<KDQ_Q6_K>::Regs& g, unsigned r,
                                            unsigned& flags) {
        const float d = (r % 2) ? half_hi(g.d) : half_lo(g.d);
        if (!isfinite(d))
            flags |= 1u;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float a = d * float(int8_t((g.scale[j] >> (8 * i)) & 255u));
                if (32.f * fabsf(a) > 65504.f)
                    flags |= 2u;
                dsc[j][i] = pair(a);
            }
    }
};

// The 8 fp16 weights of sub-step s (operand element order of GemmFormat::value).
template <int ENC>
__device__ __forceinline__ f16x8 dequant(const typename GemmFormat<ENC>::Regs& g,
                                         const Scales<ENC>& sc, int s, unsigned magic);

template <>
__device__ __forceinline__ f16x8 dequant<KDQ_Q4_K>(const GemmFormat<KDQ_Q4_K>::Regs& g,
                                                   const Scales<KDQ_Q4_K>& sc, int s,
                                                   unsigned magic) {
    const int j = s / 8, p = (s / 4) % 2, u = s % 4;
    const unsigned w = g.code[j][p][u], w8 = w >> 8;
    const f16x2 k1024 = as_f16x2(0x64006400u);      // 1024
    const f16x2 sixteenth = as_f16x2(0x2c002c00u);  // 1/16
    const f16x2 m64 = as_f16x2(0xd400d400u);        // -64
    // 1024 + q (low nibbles) or 1024 + 16 q (high), then exactly q
    const f16x2 q0 = as_f16x2((w & 0x000f000fu) | magic) - k1024;
    const f16x2 q1 = as_f16x2((w8 & 0x000f000fu) | magic) - k1024;
    const f16x2 q2 = __builtin_elementwise_fma(as_f16x2((w & 0x00f000f0u) | magic), sixteenth, m64);
    const f16x2 q3 = __builtin_elementwise_fma(as_f16x2((w8 & 0x00f000f0u) | magic), sixteenth, m64);
    const f16x2 r0 = __builtin_elementwise_fma(q0, sc.dsc[j][0], sc.ndm[j][0]);
    const f16x2 r1 = __builtin_elementwise_fma(q1, sc.dsc[j][0], sc.ndm[j][0]);
    const f16x2 r2 = __builtin_elementwise_fma(q2, sc.dsc[j][1], sc.ndm[j][1]);
    const f16x2 r3 = __builtin_elementwise_fma(q3, sc.dsc[j][1], sc.ndm[j][1]);
    return f16x8{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
}

template <>
__device__ __forceinline__ f16x8 dequant<KDQ_Q8_0>(const GemmFormat<KDQ_Q8_0>::Regs& g,
                                                   const Scales<KDQ_Q8_0>& sc, int s, unsigned) {
    const int j = s / 8, c = (s / 4) % 2, hh = (s / 2) % 2, v = s % 2;
    const u32x4 piece = g.code[j][2 * c + hh];
    const unsigned w0 = v ? piece.z : piece.x, w1 = v ? piece.w : piece.y;
    const f16x2 bias = as_f16x2(0x64806480u);  // 1152
    // (b ^ 0x80) in the mantissa of 1024: 1152 + q exactly, then q
    auto two = [&](unsigned w, unsigned sel) {
        return as_f16x2(__builtin_amdgcn_perm(0u, w, sel) ^ 0x64806480u) - bias;
    };
    const f16x2 d = sc.d[j][c];
    const f16x2 r0 = two(w0, 0x0c010c00u) * d, r1 = two(w0, 0x0c030c02u) * d;
    const f16x2 r2 = two(w1, 0x0c010c00u) * d, r3 = two(w1, 0x0c030c02u) * d;
    return f16x8{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
}

template <>
__device__ __forceinline__ f16x8 dequant<KDQ_Q6_K>(const GemmFormat<KDQ_Q6_K>::Regs& g,
                                                   const Scales<KDQ_Q6_K>& sc, int s,
                                                   unsigned magic) {
    const int j = s / 8, p = (s / 4) % 2, u = s % 4;
    const unsigned ql = g.code[j][p][u];
    const u32x4 qh = g.qh[j];
    const unsigned m = 2 * p + u / 2;
    const unsigned qd = m == 0 ? qh.x : m == 1 ? qh.y : m == 2 ? qh.z : qh.w;
    const unsigned qn = (u % 2 ? qd : qd >> 4) & 0x0f0f0f0fu;
    const unsigned lo = (ql & 0x0f0f0f0fu) | ((qn & 0x03030303u) << 4);  // block-0 codes
    const unsigned hi = ((ql >> 4) & 0x0f0f0f0fu) | ((qn & 0x0c0c0c0cu) << 2);
    const f16x2 k1056 = as_f16x2(0x64206420u);  // 1024 + 32
    auto two = [&](unsigned w, unsigned sel) {
        return as_f16x2(__builtin_amdgcn_perm(0u, w, sel) | magic) - k1056;  // q - 32
    };
    const f16x2 a = sc.dsc[j][p], b = sc.dsc[j][2 + p];
    const f16x2 r0 = two(lo, 0x0c010c00u) * a, r1 = two(lo, 0x0c030c02u) * a;
    const f16x2 r2 = two(hi, 0x0c010c00u) * b, r3 = two(hi, 0x0c030c02u) * b;
    return f16x8{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
}

// Weight load i (0 .. loads - 1) of one operand's group into its registers.  `base` is
// the operand's lane address in group 0 (tile, plus 16 * (16h + r % 16)).
template <int ENC>
__device__ __forceinline__ void load_item(const uint8_t* base, size_t off, unsigned h,
                                          unsigned r, typename GemmFormat<ENC>::Regs& g,
                                          int i) {
    const uint8_t* p = base + off;
    const unsigned lane_bytes = 16 * (16 * h + r % 16);  // already in `base`
    if constexpr (ENC == KDQ_Q4_K) {
        if (i < 4)
            g.code[i / 2][i % 2] = load16(p + 1024 * (i % 2) + 512 * (i / 2));
        else
            g.head = load16(p + 2048 + 16 * (r % 16) - lane_bytes);
    } else if constexpr (ENC == KDQ_Q8_0) {
        if (i < 8)
            g.code[i / 4][i % 4] = load16(p + 1024 * (i % 4) + 512 * (i / 4));
        else
            g.scale[i - 8] = load4(p + 4096 + 128 * (i - 8) + 4 * (16 * h + r % 16) - lane_bytes);
    } else {
        if (i < 4)
            g.code[i / 2][i % 2] = load16(p + 1024 * (i % 2) + 512 * (i / 2));
        else if (i < 6)
            g.qh[i - 4] = load16(p + 2048 + 512 * (i - 4));
        else if (i < 8)
            g.scale[i - 6] = load4(p + 3072 + 128 * (i - 6) + 4 * (16 * h + r % 16) - lane_bytes);
        else
            g.d = load4(p + 3328 + 4 * ((r % 16) / 2) - lane_bytes);
    }
}

// The GEMM's scale checks over a whole packed matrix, without the product: 32 threads
// per (16-row tile, 256-value group), lane (r = s, h) of the GEMM's operand lanes for row
// slot s, each loading that lane's registers as the GEMM does and running the same
// Scales::prepare, so a matrix this finds clean never raises a flag in the GEMM.
template <int ENC>
__global__ __launch_bounds__(256) void check_kernel(const uint8_t* __restrict__ w,
                                                    unsigned groups, size_t units,
                                                    unsigned* __restrict__ flags) {
    using F = GemmFormat<ENC>;
    const size_t id = size_t(blockIdx.x) * 256 + threadIdx.x;
    const size_t unit = id / 32;
    if (unit >= units)
        return;
    const unsigned s = threadIdx.x % 16, h = (threadIdx.x / 16) % 2;
    const uint8_t* base = w + unit * F::unit + 16 * (16 * h + s);
    typename F::Regs g;
#pragma unroll
    for (int i = 0; i < F::loads; ++i)
        load_item<ENC>(base, 0, h, s, g, i);
    unsigned f = 0;
    Scales<ENC> sc;
    sc.prepare(g, ENC == KDQ_Q6_K ? s : h, f);
    if (f)
        atomicOr(flags, f);
    (void)groups;
}

// ------------------------------------------------------------------ staging

// Row t of x (fp32, k values): its scale sigma = 2^e with max|x| / sigma in [2^14, 2^15)
// (1 for an all-zero row), and fp16(x / sigma) permuted per 256-value group: logical
// 16-byte chunk q = 16j + 8h + 4p + u of a group holds operand elements 0..7 of sub-step
// s = 8j + 4p + u for lane half h.  One 256-thread workgroup per row; the row passes
// through LDS.  Grouped (MoE) form: row t is x[slot_of[t] / topk] (a zero row when
// slot_of[t] < 0) and rows from *used on are not staged.
template <int ENC>
__global__ __launch_bounds__(256) void stage_kernel(const float* __restrict__ x, unsigned k,
                                                    uint16_t* __restrict__ xs,
                                                    float* __restrict__ sigma,
                                                    const int32_t* __restrict__ slot_of,
                                                    unsigned topk,
                                                    const unsigned* __restrict__ used) {
    extern __shared__ __align__(16) float row[];
    __shared__ float wave_max[4];
    const unsigned t = blockIdx.x;
    if (used && t >= *used)
        return;
    const int slot = slot_of ? slot_of[t] : 0;
    const bool zero = slot < 0;
    const float* src = x + (slot_of ? size_t(zero ? 0 : slot / int(topk)) : size_t(t)) * k;
    float amax = 0.f;
    for (unsigned i = threadIdx.x; i < k / 4; i += 256) {
        const float4 v = zero ? make_float4(0.f, 0.f, 0.f, 0.f)
                              : reinterpret_cast<const float4*>(src)[i];
        reinterpret_cast<float4*>(row)[i] = v;
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        if (!(isfinite(v.x) && isfinite(v.y) && isfinite(v.z) && isfinite(v.w)))
            amax = INFINITY;
    }
    amax = wave_max_nonneg(amax);
    if (threadIdx.x % 64 == 0)
        wave_max[threadIdx.x / 64] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(wave_max[0], wave_max[1]), fmaxf(wave_max[2], wave_max[3]));
    // exponent of amax (normal or subnormal), scale 2^(e - 14)
    int e = 0;
    float scale = 1.f, inv = 1.f;
    if (isfinite(amax) && amax >= 0x1p-100f) {  // (smaller rows: their fp16 values are 0)
        (void)frexpf(amax, &e);  // amax in [2^(e-1), 2^e)
        scale = ldexpf(1.f, e - 15);
        inv = ldexpf(1.f, 15 - e);
    } else if (!isfinite(amax)) {
        scale = __builtin_nanf("");  // a non-finite input poisons its row
    }
    if (threadIdx.x == 0)
        sigma[t] = scale;
    uint16_t* dst = xs + size_t(t) * k;
    for (unsigned c = threadIdx.x; c < k / 8; c += 256) {
        const unsigned g = c / 32, q = c % 32;
        const unsigned h = (q / 8) % 2, s = 8 * (q / 16) + 4 * ((q / 4) % 2) + q % 4;
        unsigned words[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = row[256 * g + GemmFormat<ENC>::value(s, h, 2 * i)] * inv;
            const float b = row[256 * g + GemmFormat<ENC>::value(s, h, 2 * i + 1)] * inv;
            words[i] = unsigned(__builtin_bit_cast(uint16_t, _Float16(a))) |
                       unsigned(__builtin_bit_cast(uint16_t, _Float16(b))) << 16;
        }
        *reinterpret_cast<uint4*>(dst + 8 * size_t(c)) =
            make_uint4(words[0], words[1], words[2], words[3]);
    }
}

// ------------------------------------------------------------------- GEMM

// Workgroup tile: 128 tokens x 256 weight rows (16 packed tiles); wavefront w owns tiles
// 4w .. 4w + 3 as two 32-row operands.  K runs over 256-value groups; each group's 128
// tokens x 512 bytes of permuted activations are staged into LDS by 16-byte DMA
// (double-buffered, one group ahead), chunk q of token t at t*512 + 16*(q ^ (t % 16)),
// and the next group's weight registers load during the current group's sub-steps.
// `xs` has rows up to the next multiple of 128 tokens (rows past m are computed, never
// stored).  *status |= 1 for a non-finite weight scale, |= 2 when a dequantised weight
// could pass the fp16 range (the caller then takes another path).
//
// K slices (narrow products, too few tiles for the compute units): workgroup slice `ks`
// runs groups [ks * per, (ks + 1) * per) and writes its fp32 tile to part[ks] (m x n);
// reduce_kernel then sums the slices in order.
//
// Grouped (MoE) form, `tile_expert` given: token tile t multiplies the weights of expert
// tile_expert[t] of a stack of packed experts `expert_bytes` apart; tiles whose entry is
// negative are skipped (the whole workgroup returns before any barrier).
//
// TM = 64 (the grouped form's token tiles: experts average a few dozen rows) halves the
// token tile: two token blocks per operand, two workgroups per compute unit (Q8_0: one;
// at two its registers spill).
//
// PAIR (grouped, four wavefronts): a workgroup takes 128 output rows of two matrices
// stored alike, `w` (gate) and `w2` (up); wavefront w's operand 0 is gate rows
// 32w .. 32w + 31 of the tile and operand 1 the same rows of up, and the epilogue writes
// silu(gate) * up (the reference's silu, on the scaled-back fp32 values) — one staging
// of x and no SwiGLU pass, the same bits as the two products and the pass.
template <int ENC, int W, int TM, bool PAIR = false>
__global__ __launch_bounds__(W * 64, TM == PM || ENC == KDQ_Q8_0 ? 1 : 2) void gemm_kernel(
    const uint16_t* __restrict__ xs, const float* __restrict__ sigma,
    const uint8_t* __restrict__ w, unsigned m, unsigned n, unsigned k, unsigned slices,
    unsigned per, float* __restrict__ y, float* __restrict__ part, unsigned* __restrict__ status,
    const int32_t* __restrict__ tile_expert, size_t expert_bytes,
    const uint8_t* __restrict__ w2 = nullptr) {
    using F = GemmFormat<ENC>;
    using Regs = typename F::Regs;
    extern __shared__ __align__(16) uint8_t lds[];
    // W wavefronts of NBW 32-row operands each (8 operands, 256 rows, per workgroup), TB
    // token blocks of 32
    constexpr int NBW = 8 / W, TB = TM / 32;
    constexpr int DMAS = TM / kDmaRows / W;  // DMA instructions per wavefront per group
    constexpr int SB = TM * kStageRow;       // bytes of one activation stage
    static_assert(!PAIR || NBW == 2, "a pair is two operands of one wavefront");
    constexpr int TILES = PAIR ? kTiles / 2 : kTiles;  // 16-row output tiles per workgroup

    const unsigned groups = k / 256, wtiles = (n + 15) / 16;
    const unsigned m_tiles = (m + TM - 1) / TM, n_tiles = (wtiles + TILES - 1) / TILES;
    // XCD-aware order: the M tiles of one weight tile (and K slice) run together on one
    // XCD (L2).
    const unsigned id = blockIdx.x, xcd = id % 8, local = id / 8;
    const unsigned per_xcd = (m_tiles * n_tiles * slices + 7) / 8;
    const unsigned linear = xcd * per_xcd + local;
    if (local >= per_xcd || linear >= m_tiles * n_tiles * slices)
        return;
    const unsigned n_tile = linear / (m_tiles * slices);
    const unsigned slice = (linear / m_tiles) % slices, m0 = (linear % m_tiles) * TM;
    if (tile_expert) {
        const int e = tile_expert[m0 / TM];
        if (e < 0)
            return;
        w += size_t(e) * expert_bytes;
        if constexpr (PAIR)
            w2 += size_t(e) * expert_bytes;
    }
    // slices = ceil(groups / per), so every slice has at least one group
    const unsigned g_begin = slice * per, g_end = min(groups, g_begin + per);
    float* __restrict__ dst_base = slices > 1 ? part + size_t(slice) * m * n : y;

    const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const unsigned lane = threadIdx.x % 64;
    const unsigned r = lane % 32, h = lane / 32;
    const size_t row_pitch = size_t(k) * 2;

    // operand c = tiles tile0 + 2c (rows 0-15) and tile0 + 2c + 1 (rows 16-31); tiles
    // past the end load the last tile, and their results are never stored
    const unsigned tile0 = n_tile * TILES + wave * 2 * (PAIR ? 1 : NBW);
    const uint8_t* base[NBW];
#pragma unroll
    for (int c = 0; c < NBW; ++c)
        base[c] = (PAIR && c == 1 ? w2 : w) +
                  size_t(min(tile0 + (PAIR ? 0 : 2 * c) + r / 16, wtiles - 1)) * groups *
                      F::unit +
                  16 * (16 * h + r % 16);
    auto load_weight = [&](unsigned g, Regs* rg, int i) {
        load_item<ENC>(base[i / F::loads], size_t(g) * F::unit, h, r, rg[i / F::loads],
                       i % F::loads);
    };

    // DMA: instruction J = wave * DMAS + j covers tokens 2J, 2J + 1 of the tile; lane L
    // fills LDS chunk L % 32 of token 2J + L / 32 from logical chunk (L % 32) ^ (token % 16)
    unsigned xlane[8];  // per J % 8 (the swizzle repeats every 16 tokens)
#pragma unroll
    for (int jm = 0; jm < 8; ++jm) {
        const unsigned tok = kDmaRows * jm + lane / 32;
        xlane[jm] = unsigned(tok * row_pitch) + 16 * ((lane % 32) ^ tok);
    }
    const uint8_t* xtile = reinterpret_cast<const uint8_t*>(xs) + size_t(m0) * row_pitch;
    auto stage_one = [&](unsigned g, unsigned buf, int j) {
        const unsigned J = wave * DMAS + j;
        __builtin_amdgcn_global_load_lds(
            (global_void*)(xtile + size_t(g) * 512 + (J / 8) * (16 * row_pitch) + xlane[J % 8]),
            (lds_void*)(lds + buf * SB + J * 1024), 16, 0, 0);
    };
    constexpr int kLoads = DMAS + F::loads * NBW, kPerStep = 4;
    static_assert(kLoads <= 16 * kPerStep, "the loads must fit the group's sub-steps");
    auto issue = [&](int s, unsigned g, unsigned buf, Regs* rg) {
#pragma unroll
        for (int i = kPerStep * s; i < kPerStep * (s + 1) && i < kLoads; ++i) {
            if (i < DMAS)
                stage_one(g, buf, i);
            else
                load_weight(g, rg, i - DMAS);
        }
    };
    auto issue_all = [&](unsigned g, unsigned buf, Regs* rg) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            if (i < DMAS)
                stage_one(g, buf, i);
            else
                load_weight(g, rg, i - DMAS);
        }
    };

    f32x16 acc[NBW][TB];
#pragma unroll
    for (int c = 0; c < NBW; ++c)
#pragma unroll
        for (int b = 0; b < TB; ++b)
            acc[c][b] = f32x16{};

    unsigned flags = 0;
    unsigned magic = 0x64006400u;  // kept in a VGPR: the mask-and-or takes one SGPR only
    asm volatile("" : "+v"(magic));
    // 16 sub-steps per group, software-pipelined by one sub-step: while the TB * NBW MFMAs
    // of sub-step s run, the activation operands of s + 1 are read from LDS and its
    // weights dequantised; one MFMA, then up to four VALU ops / one LDS read / one load.
    auto compute = [&](unsigned buf, const Regs* rg, unsigned next_g, unsigned next_buf,
                       Regs* next_rg) {
        const uint8_t* a = lds + buf * SB + r * kStageRow;
        auto read_x = [&](int s, f16x8* xf) {
            const unsigned q = 16 * (s / 8) + 8 * h + 4 * ((s / 4) % 2) + s % 4;
#pragma unroll
            for (int b = 0; b < TB; ++b)
                xf[b] = *reinterpret_cast<const f16x8*>(a + b * 32 * kStageRow +
                                                         16 * (q ^ (r % 16)));
        };
        Scales<ENC> sc[NBW];
#pragma unroll
        for (int c = 0; c < NBW; ++c)
            sc[c].prepare(rg[c], ENC == KDQ_Q6_K ? r : h, flags);
        f16x8 xf[2][TB], wf[2][NBW];
        read_x(0, xf[0]);
#pragma unroll
        for (int c = 0; c < NBW; ++c)
            wf[0][c] = dequant<ENC>(rg[c], sc[c], 0, magic);
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            __builtin_amdgcn_sched_barrier(0);
            issue(s, next_g, next_buf, next_rg);
            if (s + 1 < 16) {
                read_x(s + 1, xf[(s + 1) % 2]);
#pragma unroll
                for (int c = 0; c < NBW; ++c)
                    wf[(s + 1) % 2][c] = dequant<ENC>(rg[c], sc[c], s + 1, magic);
            }
#pragma unroll
            for (int c = 0; c < NBW; ++c)
#pragma unroll
                for (int b = 0; b < TB; ++b) {
                    acc[c][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[s % 2][c], xf[s % 2][b],
                                                                       acc[c][b], 0, 0, 0);
                    if constexpr (NBW == 1)  // the MFMAs stay in their sub-step (else the
                        asm volatile("" : "+v"(acc[c][b]));  // compiler sinks them all)
                }
#pragma unroll
            for (int q = 0; q < TB * NBW; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 32 / (TB * NBW), 0);  // VALU
                if (q < TB)
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
                if (q < kPerStep)
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one global load
            }
        }
    };

    // Ping-pong over group pairs: group g in buffer 0 / registers ra, g + 1 in buffer 1 /
    // rb; each compute issues the other buffer's loads.  After the last pair the prefetch
    // reloads the last group (consumed only when the group count is odd).
    Regs ra[NBW], rb[NBW];
    const unsigned last = g_end - 1;
    issue_all(g_begin, 0, ra);
    unsigned g = g_begin;
    for (; g + 1 < g_end; g += 2) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        compute(0, ra, g + 1, 1, rb);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        compute(1, rb, min(g + 2, last), 0, ra);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no DMA outlives the workgroup
    if (g < g_end) {  // odd group count: the last group sits in buffer 0 / ra
        __syncthreads();
        compute(0, ra, last, 1, rb);  // its prefetch reloads the last group (never used)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }

    // Output tile through LDS (free after the K loop): D of operand c, token block b holds
    // token 32b + r and weight rows 8(v / 4) + 4h + v % 4 of the operand's 32; scaled
    // back by the token's sigma, written as [token][row] fp32, then stored as whole rows.
    float sig[TB];
#pragma unroll
    for (int b = 0; b < TB; ++b) {
        const unsigned tok = m0 + 32 * b + r;
        sig[b] = tok < m ? sigma[tok] : 1.f;
    }
    __syncthreads();  // every wavefront is done reading the activation stages
    if constexpr (PAIR) {
#pragma unroll
        for (int b = 0; b < TB; ++b)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const unsigned row = wave * 32 + 8 * q + 4 * h;
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    v[i] = silu_of(acc[0][b][4 * q + i] * sig[b]) * (acc[1][b][4 * q + i] * sig[b]);
                *reinterpret_cast<float4*>(lds + (32 * b + r) * kOutPitch + 4 * row) =
                    make_float4(v[0], v[1], v[2], v[3]);
            }
    } else {
#pragma unroll
        for (int c = 0; c < NBW; ++c)
#pragma unroll
            for (int b = 0; b < TB; ++b)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const unsigned row = (wave * NBW + c) * 32 + 8 * q + 4 * h;
                    *reinterpret_cast<float4*>(lds + (32 * b + r) * kOutPitch + 4 * row) =
                        make_float4(acc[c][b][4 * q] * sig[b], acc[c][b][4 * q + 1] * sig[b],
                                    acc[c][b][4 * q + 2] * sig[b], acc[c][b][4 * q + 3] * sig[b]);
                }
    }
    __syncthreads();
    const unsigned f0 = n_tile * TILES * 16;       // first weight row of the tile
    constexpr int kChunks = TILES * 16 * 4 / 16;  // 16-byte chunks per token row
    for (unsigned e = threadIdx.x; e < TM * kChunks; e += W * 64) {
        const unsigned t = e / kChunks, ch = e % kChunks, tok = m0 + t, f = f0 + 4 * ch;
        if (tok >= m || f >= n)
            continue;
        const float4 v = *reinterpret_cast<const float4*>(lds + t * kOutPitch + 16 * ch);
        float* dst = dst_base + size_t(tok) * n + f;
        if (f + 3 < n && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
            *reinterpret_cast<float4*>(dst) = v;
        } else {
            const float vals[4] = {v.x, v.y, v.z, v.w};
            for (unsigned j = 0; j < 4 && f + j < n; ++j)
                dst[j] = vals[j];
        }
    }
    if (status) {
        unsigned all = flags;
        for (int o = 32; o > 0; o >>= 1)
            all |= __shfl_xor(all, o, 64);
        if (lane == 0 && all)
            atomicOr(status, all);
    }
}

// y[i] = sum of the K slices' partials part[s][i] in slice order (4 values per thread).
__global__ __launch_bounds__(256) void reduce_kernel(const float* __restrict__ part,
                                                     size_t count, unsigned slices,
                                                     float* __restrict__ y) {
    const size_t i = (size_t(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i >= count)
        return;
    if (i + 4 <= count && (count % 4) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0) {
        float4 acc = *reinterpret_cast<const float4*>(part + i);
        for (unsigned s = 1; s < slices; ++s) {
            const float4 v = *reinterpret_cast<const float4*>(part + size_t(s) * count + i);
            acc = make_float4(acc.x + v.x, acc.y + v.y, acc.z + v.z, acc.w + v.w);
        }
        *reinterpret_cast<float4*>(y + i) = acc;
    } else {
        for (size_t j = i; j < i + 4 && j < count; ++j) {
            float acc = part[j];
            for (unsigned s = 1; s < slices; ++s)
                acc += part[size_t(s) * count + j];
            y[j] = acc;
        }
    }
}

// K slices: enough workgroups for the compute units when the output tiles are few, each
// slice at least 2 groups (512 values) deep.
// Returns the groups per slice; the slice count is ceil(groups / per) (no empty slice).
unsigned gemm_slice_depth(size_t m, size_t n, size_t k) {
    const size_t groups = k / 256;
    const size_t tiles = ((m + PM - 1) / PM) * (((n + 15) / 16 + kTiles - 1) / kTiles);
    const size_t units = compute_units();
    if (tiles * 3 >= units * 2)
        return unsigned(groups);
    size_t ks = std::max<size_t>(1, units / tiles);
    ks = std::min(ks, std::max<size_t>(1, groups / 2));
    return unsigned((groups + ks - 1) / ks);
}

// Wavefronts per GEMM workgroup: 8 with one 32-row operand each where two operands per
// wavefront do not fit the registers (Q6_K spilled 240 bytes per lane: 4096->14336 at 512
// tokens 125 -> 83 us with 8), else 4 (Q4_K and Q8_0 measured 2-4 % slower with 8).
template <int ENC> constexpr int gemm_waves = ENC == KDQ_Q6_K ? 8 : 4;

// Token tile of the grouped (MoE) form: an expert's rows are padded to whole tiles, and
// experts average a few dozen rows in a prefill chunk, so its tiles are 64 tokens.
constexpr int kGroupTM = int(kGroupedTileRows);

template <int ENC>
int configure() {
    static bool configured = false;  // one attribute call per instantiation
    if (!configured) {
        KDQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&stage_kernel<ENC>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024));
        KDQ_HIP(hipFuncSetAttribute(
            reinterpret_cast<const void*>(&gemm_kernel<ENC, gemm_waves<ENC>, PM>),
            hipFuncAttributeMaxDynamicSharedMemorySize, int(kLds)));
        KDQ_HIP(hipFuncSetAttribute(
            reinterpret_cast<const void*>(&gemm_kernel<ENC, gemm_waves<ENC>, kGroupTM>),
            hipFuncAttributeMaxDynamicSharedMemorySize, int(gemm_lds<kGroupTM>)));
        if constexpr (gemm_waves<ENC> == 4)
            KDQ_HIP(hipFuncSetAttribute(
                reinterpret_cast<const void*>(&gemm_kernel<ENC, 4, kGroupTM, true>),
                hipFuncAttributeMaxDynamicSharedMemorySize, int(gemm_lds<kGroupTM>)));
        configured = true;
    }
    return KDQ_OK;
}

// Grouped form: x staged through the position -> slot map, then one GEMM launch over the
// token tiles; `up` given (four-wavefront encodings): the paired launch writing
// silu(gate x) * (up x).
template <int ENC>
int launch_grouped(const void* packed, const void* up, size_t expert_bytes,
                   const int32_t* tile_expert, size_t n, size_t k, const float* x,
                   const int32_t* inv, unsigned topk, const unsigned* used, size_t positions,
                   float* y, unsigned* status, uint16_t* xs, float* sigma, hipStream_t st) {
    int rc;
    if ((rc = configure<ENC>()))
        return rc;
    hipLaunchKernelGGL(stage_kernel<ENC>, dim3(unsigned(positions)), dim3(256), k * 4, st, x,
                       unsigned(k), xs, sigma, inv, topk, used);
    KDQ_HIP(hipGetLastError());
    const size_t wtiles = (n + 15) / 16;
    const auto* w = static_cast<const uint8_t*>(packed);
    if (up) {
        if constexpr (gemm_waves<ENC> == 4) {
            constexpr size_t pair_tiles = kTiles / 2;
            const size_t tiles = (positions / kGroupTM) * ((wtiles + pair_tiles - 1) / pair_tiles);
            hipLaunchKernelGGL((gemm_kernel<ENC, 4, kGroupTM, true>),
                               dim3(unsigned((tiles + 7) / 8 * 8)), dim3(4 * 64),
                               gemm_lds<kGroupTM>, st, xs, sigma, w, unsigned(positions),
                               unsigned(n), unsigned(k), 1u, unsigned(k / 256), y, nullptr,
                               status, tile_expert, expert_bytes,
                               static_cast<const uint8_t*>(up));
            KDQ_HIP(hipGetLastError());
            return KDQ_OK;
        }
        return KDQ_ERR_UNSUPPORTED;
    }
    const size_t tiles = (positions / kGroupTM) * ((wtiles + kTiles - 1) / kTiles);
    const unsigned grid = unsigned((tiles + 7) / 8 * 8);
    hipLaunchKernelGGL((gemm_kernel<ENC, gemm_waves<ENC>, kGroupTM>), dim3(grid),
                       dim3(gemm_waves<ENC> * 64), gemm_lds<kGroupTM>, st, xs, sigma, w,
                       unsigned(positions), unsigned(n), unsigned(k), 1u, unsigned(k / 256), y,
                       nullptr, status, tile_expert, expert_bytes, nullptr);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}

// Scratch of one dense GEMM call: x staged as fp16 rows padded to whole token tiles, the
// row scales, and the K slices' partials (none with one slice).
struct GemmScratch {
    size_t xs, sigma, part, total;
};

GemmScratch gemm_scratch(size_t m, size_t n, size_t k) {
    const size_t m_pad = (m + PM - 1) / PM * PM;
    const unsigned per = gemm_slice_depth(m, n, k);
    const unsigned slices = unsigned((k / 256 + per - 1) / per);
    GemmScratch g;
    g.xs = (m_pad * k * 2 + 255) & ~size_t(255);
    g.sigma = (m * 4 + 255) & ~size_t(255);
    g.part = slices > 1 ? (size_t(slices) * m * n * 4 + 255) & ~size_t(255) : 0;
    g.total = g.xs + g.sigma + g.part;
    return g;
}

template <int ENC>
int launch_gemm(const float* x, const uint8_t* packed, size_t m, size_t n, size_t k, float* y,
                unsigned* status, uint8_t* scratch, hipStream_t st) {
    int rc;
    const size_t m_pad = (m + PM - 1) / PM * PM;
    const unsigned per = gemm_slice_depth(m, n, k);
    const unsigned slices = unsigned((k / 256 + per - 1) / per);
    const GemmScratch g = gemm_scratch(m, n, k);
    auto* xs = reinterpret_cast<uint16_t*>(scratch);
    auto* sigma = reinterpret_cast<float*>(scratch + g.xs);
    auto* part = slices > 1 ? reinterpret_cast<float*>(scratch + g.xs + g.sigma) : nullptr;
    if ((rc = configure<ENC>()))
        return rc;
    hipLaunchKernelGGL(stage_kernel<ENC>, dim3(unsigned(m)), dim3(256), k * 4, st, x,
                       unsigned(k), xs, sigma, nullptr, 1u, nullptr);
    KDQ_HIP(hipGetLastError());
    const size_t wtiles = (n + 15) / 16;
    const size_t tiles = (m_pad / PM) * ((wtiles + kTiles - 1) / kTiles) * slices;
    const unsigned grid = unsigned((tiles + 7) / 8 * 8);
    hipLaunchKernelGGL((gemm_kernel<ENC, gemm_waves<ENC>, PM>), dim3(grid), dim3(gemm_waves<ENC> * 64), kLds, st, xs, sigma, packed,
                       unsigned(m), unsigned(n), unsigned(k), slices, per, y, part, status,
                       nullptr, size_t(0));
    KDQ_HIP(hipGetLastError());
    if (slices > 1) {
        const size_t count = m * n;
        hipLaunchKernelGGL(reduce_kernel, dim3(unsigned((count / 4 + 256) / 256)), dim3(256), 0,
                           st, part, count, slices, y);
        KDQ_HIP(hipGetLastError());
    }
    return KDQ_OK;
}

}  // namespace

int gemm_check(int encoding, const void* packed, size_t n, size_t k, unsigned* flags,
               hipStream_t st) {
    const size_t units = (n + 15) / 16 * (k / 256);
    const dim3 grid(unsigned((units * 32 + 255) / 256));
    auto* w = static_cast<const uint8_t*>(packed);
    switch (encoding) {
    case KDQ_Q4_K:
        hipLaunchKernelGGL(check_kernel<KDQ_Q4_K>, grid, dim3(256), 0, st, w, unsigned(k / 256),
                           units, flags);
        break;
    case KDQ_Q8_0:
        hipLaunchKernelGGL(check_kernel<KDQ_Q8_0>, grid, dim3(256), 0, st, w, unsigned(k / 256),
                           units, flags);
        break;
    case KDQ_Q6_K:
        hipLaunchKernelGGL(check_kernel<KDQ_Q6_K>, grid, dim3(256), 0, st, w, unsigned(k / 256),
                           units, flags);
        break;
    default:
        return KDQ_ERR_UNSUPPORTED;
    }
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}

size_t dense_gemm_scratch(size_t m, size_t n, size_t k) {
    return gemm_scratch(m, n, k).total;
}

int dense_gemm(int encoding, const void* packed, size_t n, size_t k, const float* x, size_t m,
               float* y, unsigned* status, void* scratch, hipStream_t st) {
    auto* w = static_cast<const uint8_t*>(packed);
    auto* sc = static_cast<uint8_t*>(scratch);
    switch (encoding) {
    case KDQ_Q4_K:
        return launch_gemm<KDQ_Q4_K>(x, w, m, n, k, y, status, sc, st);
    case KDQ_Q8_0:
        return launch_gemm<KDQ_Q8_0>(x, w, m, n, k, y, status, sc, st);
    case KDQ_Q6_K:
        return launch_gemm<KDQ_Q6_K>(x, w, m, n, k, y, status, sc, st);
    default:
        return KDQ_ERR_UNSUPPORTED;
    }
}

int dense_gemm_pair(int encoding, const void* gate, const void* up, size_t n, size_t k,
                    const float* x, size_t m, float* y, unsigned* status, void* scratch,
                    hipStream_t st) {
    if (!grouped_gemm_takes(encoding, k) || !grouped_gemm_pairs(encoding))
        return KDQ_ERR_UNSUPPORTED;
    auto* sc = static_cast<uint8_t*>(scratch);
    const GemmScratch g = gemm_scratch(m, n, k);  // covers m rounded up to 128 rows
    auto launch = [&](auto kernel, auto stage) -> int {
        int rc;
        if ((rc = encoding == KDQ_Q4_K ? configure<KDQ_Q4_K>() : configure<KDQ_Q8_0>()))
            return rc;
        auto* xs = reinterpret_cast<uint16_t*>(sc);
        auto* sigma = reinterpret_cast<float*>(sc + g.xs);
        hipLaunchKernelGGL(stage, dim3(unsigned(m)), dim3(256), k * 4, st, x, unsigned(k), xs,
                           sigma, nullptr, 1u, nullptr);
        KDQ_HIP(hipGetLastError());
        const size_t tiles = (m + kGroupTM - 1) / kGroupTM * (((n + 15) / 16 + 7) / 8);
        hipLaunchKernelGGL(kernel, dim3(unsigned((tiles + 7) / 8 * 8)), dim3(4 * 64),
                           gemm_lds<kGroupTM>, st, xs, sigma, static_cast<const uint8_t*>(gate),
                           unsigned(m), unsigned(n), unsigned(k), 1u, unsigned(k / 256), y,
                           nullptr, status, nullptr, size_t(0),
                           static_cast<const uint8_t*>(up));
        KDQ_HIP(hipGetLastError());
        return KDQ_OK;
    };
    return encoding == KDQ_Q4_K
               ? launch(gemm_kernel<KDQ_Q4_K, 4, kGroupTM, true>, stage_kernel<KDQ_Q4_K>)
               : launch(gemm_kernel<KDQ_Q8_0, 4, kGroupTM, true>, stage_kernel<KDQ_Q8_0>);
}

bool grouped_gemm_takes(int encoding, size_t k) {
    return (encoding == KDQ_Q4_K || encoding == KDQ_Q8_0 || encoding == KDQ_Q6_K) &&
           k % 256 == 0 && k <= 32768;
}

int grouped_gemm(int encoding, const void* packed, size_t expert_bytes,
                 const int32_t* tile_expert, size_t n, size_t k, const float* x,
                 const int32_t* inv, unsigned topk, const unsigned* used, size_t positions,
                 float* y, unsigned* status, uint16_t* xs, float* sigma, hipStream_t st,
                 const void* up) {
    if (!grouped_gemm_takes(encoding, k) || positions % kGroupTM ||
        (up && !grouped_gemm_pairs(encoding)))
        return KDQ_ERR_UNSUPPORTED;
    switch (encoding) {
    case KDQ_Q4_K:
        return launch_grouped<KDQ_Q4_K>(packed, up, expert_bytes, tile_expert, n, k, x, inv,
                                        topk, used, positions, y, status, xs, sigma, st);
    case KDQ_Q8_0:
        return launch_grouped<KDQ_Q8_0>(packed, up, expert_bytes, tile_expert, n, k, x, inv,
                                        topk, used, positions, y, status, xs, sigma, st);
    default:
        return launch_grouped<KDQ_Q6_K>(packed, up, expert_bytes, tile_expert, n, k, x, inv,
                                        topk, used, positions, y, status, xs, sigma, st);
    }
}

bool grouped_gemm_pairs(int encoding) {
    return encoding == KDQ_Q4_K || encoding == KDQ_Q8_0;
}

}  // namespace kdq

using namespace kdq;

extern "C" int kdq_gemm_packed(int encoding, const void* packed, size_t n, size_t k,
                               const float* x, size_t m, float* y, unsigned* status,
                               void* stream) {
    if (!packed || !x || !y || !m || !n || !k)
        return KDQ_ERR_ARGUMENT;
    if (encoding != KDQ_Q4_K && encoding != KDQ_Q8_0 && encoding != KDQ_Q6_K)
        return KDQ_ERR_UNSUPPORTED;
    if (k % 256 || k > 32768 || m > 0xffffffu || n > 0xffffffu)
        return KDQ_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(packed) % 16 ||
        reinterpret_cast<uintptr_t>(y) % 4)
        return KDQ_ERR_ALIGNMENT;
    const size_t packed_bytes = kdq_gguf_packed_bytes(encoding, k, n);
    if (overlaps(y, m * n * 4, x, m * k * 4) || overlaps(y, m * n * 4, packed, packed_bytes))
        return KDQ_ERR_ALIAS;
    int rc;
    void* scratch = workspace(dense_gemm_scratch(m, n, k), &rc);
    if (rc)
        return rc;
    return dense_gemm(encoding, packed, n, k, x, m, y, status, scratch,
                      static_cast<hipStream_t>(stream));
}

extern "C" int kdq_gguf_gemm_check(int encoding, const void* packed, size_t n, size_t k,
                                   unsigned* flags, void* stream) {
    if (!packed || !flags || !n || !k)
        return KDQ_ERR_ARGUMENT;
    if (encoding != KDQ_Q4_K && encoding != KDQ_Q8_0 && encoding != KDQ_Q6_K)
        return KDQ_ERR_UNSUPPORTED;
    if (k % 256 || k > 32768 || n > 0xffffffu)
        return KDQ_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(packed) % 16 || reinterpret_cast<uintptr_t>(flags) % 4)
        return KDQ_ERR_ALIGNMENT;
    return gemm_check(encoding, packed, n, k, flags, static_cast<hipStream_t>(stream));
}
