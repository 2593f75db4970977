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
//   packed_gemm_kernel  the same product over the tile-packed Q4_0 layout that the
//                    decode GEMV reads (kdq_gguf_pack): 128x256 output tile per
//                    workgroup; weights go from HBM straight into 32x32x16 MFMA operand
//                    registers (16-byte loads of the packed lane images) and are
//                    dequantised there; activations are staged into swizzled LDS by
//                    global->LDS DMA in the order the weight lanes consume them, so no
//                    LDS traffic is spent on weights.
#include "kdq_common.hpp"

namespace kdq {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// --------------------------------------------------------------- quantizer

// Thread t of the grid handles 8 consecutive values; 4 threads share one block.
// `q`/`d` (codes and scales) and `dequant` (fp16(code * d)) are each optional.  With
// PERMUTED the dequantised values of each 32-value block are stored in the order that
// packed_gemm_kernel's operand lanes take them from Q4_0 code dword u (values 4u..4u+3
// in its low nibbles, 16+4u..16+4u+3 in its high nibbles): positions 8u..8u+7 hold
// values 4u + {0, 2, 1, 3} and 16 + 4u + {0, 2, 1, 3}.
template <bool PERMUTED>
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
    if (q)
        *reinterpret_cast<uint2*>(q + e) = make_uint2(packed[0], packed[1]);
    if (dequant) {
        if constexpr (PERMUTED) {
            // this thread's quads of values are 2j and 2j+1 of its block (j = t % 4);
            // quad w (values 4w..4w+3) goes to positions 8(w % 4) + 4(w / 4) + {0, 2, 1, 3}
            uint16_t* block = dequant + (e & ~size_t(31));
            const unsigned j = unsigned(t % 4);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const unsigned w = 2 * j + h;
                const unsigned v01 = halves[2 * h], v23 = halves[2 * h + 1];
                *reinterpret_cast<uint2*>(block + 8 * (w % 4) + 4 * (w / 4)) =
                    make_uint2(__builtin_amdgcn_perm(v23, v01, 0x05040100u),   // v0, v2
                               __builtin_amdgcn_perm(v23, v01, 0x07060302u));  // v1, v3
            }
        } else {
            *reinterpret_cast<uint4*>(dequant + e) =
                make_uint4(halves[0], halves[1], halves[2], halves[3]);
        }
    }
    if (d && (t & 3) == 0)
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

// ------------------------------------------------- GEMM over tile-packed weights

// Tile-packed Q4_0 (kdq_gguf_pack): one 2304-byte unit per (16 weight rows, 256 values);
// packed lane position l = 16G + r holds bytes [16l, 16l+16) of piece p (codes of block
// 2G + p of row r, 1024 bytes per piece) and dword l of the scales (d of blocks 2G and
// 2G + 1).  The A operand of v_mfma_f32_32x32x16_f16 (32 weight rows x 16 K values,
// lane l = r + 32h holding 8 K values of row r) is built from two tiles: at sub-step
// (j, p, u) lane (r, h) takes code dword u of packed position 16(2j + h) + r % 16 of
// tile r / 16, i.e. values 4u..4u+3 and 16+4u..16+4u+3 of block 4j + 2h + p.  Those
// 16-byte loads cover whole 512-byte runs of each tile's pieces.
constexpr int kUnitBytes = 2304;
constexpr int PM = 128;                      // tokens per workgroup tile (4 blocks of 32)
constexpr int kStageRow = 512;               // LDS bytes per token of one staged group
constexpr int kStageBytes = PM * kStageRow;  // 64 KB
constexpr int kDmaRows = 1024 / kStageRow;   // token rows per 64-lane 16-byte DMA

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void global_void;

// One Q4_0 code dword (bytes b0..b3) -> the 8 fp16 operand values round((q - 8) * d)
// in operand order lo(b0), lo(b2), lo(b1), lo(b3), hi(b0), hi(b2), hi(b1), hi(b3): the
// pairs (b0, b2) and (b1, b3) sit 16 bits apart in the dword and its 8-bit shift, so
// each fp16 pair is one mask-and-or with the 0x6400 exponent (1024 + nibble, or
// 1024 + 16 * nibble for high nibbles), then an exact shift to q - 8 and one rounding.
__device__ __forceinline__ f16x8 dequant_dword(unsigned w, f16x2 d, unsigned magic) {
    const f16x2 lo_bias = __builtin_bit_cast(f16x2, 0x64086408u);  // 1032
    const f16x2 sixteenth = __builtin_bit_cast(f16x2, 0x2c002c00u);  // 1/16
    const f16x2 hi_bias = __builtin_bit_cast(f16x2, 0xd480d480u);   // -72
    const unsigned w8 = w >> 8;
    const f16x2 x0 = __builtin_bit_cast(f16x2, (w & 0x000f000fu) | magic);
    const f16x2 x1 = __builtin_bit_cast(f16x2, (w8 & 0x000f000fu) | magic);
    const f16x2 x2 = __builtin_bit_cast(f16x2, (w & 0x00f000f0u) | magic);
    const f16x2 x3 = __builtin_bit_cast(f16x2, (w8 & 0x00f000f0u) | magic);
    const f16x2 r0 = (x0 - lo_bias) * d;                                   // exact q - 8
    const f16x2 r1 = (x1 - lo_bias) * d;
    const f16x2 r2 = __builtin_elementwise_fma(x2, sixteenth, hi_bias) * d;  // exact q - 8
    const f16x2 r3 = __builtin_elementwise_fma(x3, sixteenth, hi_bias) * d;
    return f16x8{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
}

// One group of a 32-row weight operand in a lane's registers: code pieces [j][p] and the
// scale dwords [j] (d of blocks 4j + 2h and 4j + 2h + 1).
struct RowGroup {
    u32x4 code[2][2];
    unsigned scale[2];
};

// Workgroup tile: 128 tokens x 64*NB weight rows; each of the 4 wavefronts owns NB
// 32-row weight operands and all 128 tokens, so every weight byte is loaded and
// dequantised once per workgroup, straight into operand registers.  The K loop runs
// over 256-value groups: per group the workgroup stages its 128 tokens x 512 bytes of
// permuted activations into LDS with 16-byte DMA (double-buffered, one group ahead)
// and each wavefront loads its operands' next group into registers.  LDS chunk q (16
// bytes, 4 per block: q = 4 * block + u) of token t sits at t*512 + 16*(q ^ (t % 16)):
// the 16 tokens a quarter-wavefront reads fall in 16 distinct bank groups.  `xs` has
// rows up to the next multiple of 128 tokens (rows past m are computed, never stored).
template <int NB>
__global__ __launch_bounds__(256, 1) void packed_gemm_kernel(const uint16_t* __restrict__ xs,
                                                             const uint8_t* __restrict__ w,
                                                             unsigned m, unsigned n, unsigned k,
                                                             uint16_t* __restrict__ y) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int TILES = 8 * NB;               // 16-row weight tiles per workgroup
    constexpr int DMAS = PM / kDmaRows / 4;     // DMA instructions per wavefront per group

    const unsigned groups = k / 256, wtiles = (n + 15) / 16;
    const unsigned m_tiles = (m + PM - 1) / PM, n_tiles = (wtiles + TILES - 1) / TILES;
    // XCD-aware order: the M tiles of one weight tile run together on one XCD (L2).
    const unsigned id = blockIdx.x, xcd = id % 8, local = id / 8;
    const unsigned per_xcd = (m_tiles * n_tiles + 7) / 8;
    const unsigned linear = xcd * per_xcd + local;
    if (local >= per_xcd || linear >= m_tiles * n_tiles)
        return;
    const unsigned n_tile = linear / m_tiles, m0 = (linear % m_tiles) * PM;

    const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const unsigned lane = threadIdx.x % 64;
    const unsigned r = lane % 32, h = lane / 32;
    const size_t row_pitch = size_t(k) * 2;

    // weight operands of this wavefront: operand c is tiles tile0 + 2c (rows 0-15) and
    // tile0 + 2c + 1 (rows 16-31); tiles past the end load the last tile and their
    // results are never stored
    const unsigned tile0 = (n_tile * 4 + wave) * 2 * NB;
    const uint8_t* wrow[NB];
#pragma unroll
    for (int c = 0; c < NB; ++c)
        wrow[c] = w + size_t(min(tile0 + 2 * c + r / 16, wtiles - 1)) * groups * kUnitBytes +
                  16 * (16 * h + r % 16);
    // weight item i of a group (6 per operand: four code pieces, two scale dwords)
    auto load_weight = [&](unsigned g, RowGroup* rg, int i) {
        const size_t off = size_t(g) * kUnitBytes;
        const int c = i / 6, e = i % 6;
        if (e < 4) {
            const int j = e / 2, p = e % 2;
            rg[c].code[j][p] = load16(wrow[c] + off + 1024 * p + 512 * j);
        } else {
            // scale dword of packed position 16(2j + h) + r % 16
            const int j = e - 4;
            rg[c].scale[j] = load4(wrow[c] + off + 2048 + 128 * j - 12 * (16 * h + r % 16));
        }
    };
    auto load_weights = [&](unsigned g, RowGroup* rg) {
#pragma unroll
        for (int i = 0; i < 6 * NB; ++i)
            load_weight(g, rg, i);
    };

    // DMA: instruction J = wave * DMAS + j covers tokens 2J, 2J + 1 of the tile; lane L
    // fills LDS chunk L % 32 of token 2J + L / 32, i.e. logical chunk (L % 32) ^ (token % 16),
    // which is bytes [16q, 16q + 16) of the token's 512-byte permuted group.
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
            (lds_void*)(lds + buf * kStageBytes + J * 1024), 16, 0, 0);
    };
    auto stage = [&](unsigned g, unsigned buf) {
#pragma unroll
        for (int j = 0; j < DMAS; ++j)
            stage_one(g, buf, j);
    };
    // the next group's loads (DMAS activation DMAs, then 6 * NB weight loads), issued a
    // few per sub-step so that a burst of loads never blocks the MFMA issue
    constexpr int kLoads = DMAS + 6 * NB, kPerStep = 4;
    static_assert(kLoads <= 16 * kPerStep, "the loads must fit the group's sub-steps");
    auto issue = [&](int s, unsigned g, unsigned buf, RowGroup* rg) {
#pragma unroll
        for (int i = kPerStep * s; i < kPerStep * (s + 1) && i < kLoads; ++i) {
            if (i < DMAS)
                stage_one(g, buf, i);
            else
                load_weight(g, rg, i - DMAS);
        }
    };

    f32x16 acc[NB][4];
#pragma unroll
    for (int c = 0; c < NB; ++c)
#pragma unroll
        for (int b = 0; b < 4; ++b)
            acc[c][b] = f32x16{};

    unsigned magic = 0x64006400u;  // kept in a VGPR: the mask-and-or takes one SGPR only
    asm volatile("" : "+v"(magic));
    // 16 sub-steps per group, s = 8j + 4p + u.  Software-pipelined by one sub-step: while
    // the 4 * NB MFMAs of sub-step s run, the activation operands of s + 1 are read from
    // LDS and its weight operands dequantised, and the instruction order interleaves
    // them (one MFMA, then up to four VALU ops / one LDS read): with one wavefront per
    // SIMD nothing else fills the issue slots behind a run of back-to-back MFMAs.
    auto compute = [&](unsigned buf, const RowGroup* rg, unsigned next_g, unsigned next_buf,
                       RowGroup* next_rg) {
        const uint8_t* a = lds + buf * kStageBytes + r * kStageRow;
        auto read_x = [&](int s, f16x8* xf) {
            const unsigned q = 16 * (s / 8) + 8 * h + 4 * ((s / 4) % 2) + s % 4;
#pragma unroll
            for (int b = 0; b < 4; ++b)
                xf[b] = *reinterpret_cast<const f16x8*>(a + b * 32 * kStageRow +
                                                         16 * (q ^ (r % 16)));
        };
        // fp16 scale pairs (d, d) of the four blocks each operand lane touches this group
        f16x2 d[NB][2][2];
#pragma unroll
        for (int c = 0; c < NB; ++c)
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const unsigned sc = rg[c].scale[j];
                d[c][j][0] = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(sc, sc, 0x01000100u));
                d[c][j][1] = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(sc, sc, 0x03020302u));
            }
        auto weights = [&](int s, f16x8* wf) {
            const int j = s / 8, p = (s / 4) % 2, u = s % 4;
#pragma unroll
            for (int c = 0; c < NB; ++c)
                wf[c] = dequant_dword(rg[c].code[j][p][u], d[c][j][p], magic);
        };
        f16x8 xf[2][4], wf[2][NB];
        read_x(0, xf[0]);
        weights(0, wf[0]);
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            __builtin_amdgcn_sched_barrier(0);
            issue(s, next_g, next_buf, next_rg);
            if (s + 1 < 16) {
                read_x(s + 1, xf[(s + 1) % 2]);
                weights(s + 1, wf[(s + 1) % 2]);
            }
#pragma unroll
            for (int c = 0; c < NB; ++c)
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    acc[c][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(wf[s % 2][c], xf[s % 2][b],
                                                                       acc[c][b], 0, 0, 0);
#pragma unroll
            for (int q = 0; q < 4 * NB; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // up to four VALU
                if (q < 4)
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
                if (q < kPerStep)
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one global load
            }
        }
    };

    // Ping-pong over group pairs: group g in buffer 0 / registers ra, g + 1 in buffer 1 /
    // rb; each compute issues the other buffer's loads.  After the last pair the prefetch
    // reloads the last group (consumed only when the group count is odd); the
    // accumulators never change registers between paths.
    RowGroup ra[NB], rb[NB];
    const unsigned last = groups - 1;
    stage(0, 0);
    load_weights(0, ra);
    unsigned g = 0;
    for (; g + 1 < groups; g += 2) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        compute(0, ra, g + 1, 1, rb);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        compute(1, rb, min(g + 2, last), 0, ra);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no DMA outlives the workgroup
    if (g < groups) {  // odd group count: the last group sits in buffer 0 / ra
        __syncthreads();
        compute(0, ra, last, 1, rb);  // its prefetch reloads the last group (never used)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }

    // Output tile through LDS (free after the K loop): D of operand c, token block b holds
    // token 32b + r and weight rows 8(v / 4) + 4h + v % 4 of the operand's 32 in each lane;
    // each wavefront writes its 128 x 64NB fp16 slice as [token][row] (pitch kOutPitch), then
    // the workgroup stores whole token rows with 16-byte writes.
    constexpr int kOutPitch = TILES * 32 + 16;  // bytes; the 16 spreads tokens over banks
    __syncthreads();  // every wavefront is done reading the activation stages
#pragma unroll
    for (int c = 0; c < NB; ++c)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                unsigned hv[4];
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    hv[v] = __builtin_bit_cast(uint16_t, _Float16(acc[c][b][4 * q + v]));
                const unsigned row = (wave * NB + c) * 32 + 8 * q + 4 * h;
                *reinterpret_cast<uint2*>(lds + (32 * b + r) * kOutPitch + 2 * row) =
                    make_uint2(hv[0] | hv[1] << 16, hv[2] | hv[3] << 16);
            }
    __syncthreads();
    const unsigned f0 = n_tile * TILES * 16;              // first weight row of the tile
    constexpr int kChunks = TILES * 16 * 2 / 16;          // 16-byte chunks per token row
    for (unsigned e = threadIdx.x; e < PM * kChunks; e += 256) {
        const unsigned t = e / kChunks, ch = e % kChunks, tok = m0 + t, f = f0 + 8 * ch;
        if (tok >= m || f >= n)
            continue;
        const u32x4 v = *reinterpret_cast<const u32x4*>(lds + t * kOutPitch + 16 * ch);
        uint16_t* dst = y + size_t(tok) * n + f;
        if (f + 7 < n && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
            *reinterpret_cast<u32x4*>(dst) = v;
        } else {
            const unsigned words[4] = {v.x, v.y, v.z, v.w};
            for (unsigned j = 0; j < 8 && f + j < n; ++j)
                dst[j] = uint16_t(words[j / 2] >> (16 * (j % 2)));
        }
    }
}

template <int NB>
int launch_packed_gemm(const uint16_t* xs, const uint8_t* w, unsigned m, unsigned n,
                       unsigned k, uint16_t* y, hipStream_t stream) {
    const unsigned wtiles = (n + 15) / 16;
    const unsigned tiles = ((m + PM - 1) / PM) * ((wtiles + 8 * NB - 1) / (8 * NB));
    const unsigned grid = (tiles + 7) / 8 * 8;
    const size_t lds = 2 * kStageBytes;
    KDQ_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&packed_gemm_kernel<NB>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
    hipLaunchKernelGGL((packed_gemm_kernel<NB>), dim3(grid), dim3(256), lds, stream, xs, w, m, n,
                       k, y);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}

template <bool PERMUTED = false>
int launch_quantize(const uint16_t* x, size_t m, size_t k, int8_t* q, float* d,
                    uint16_t* dequant, hipStream_t stream) {
    const size_t threads = m * k / 8;
    hipLaunchKernelGGL(quantize_kernel<PERMUTED>, dim3(unsigned((threads + 255) / 256)),
                       dim3(256), 0, stream, x, m * k, q, d, dequant);
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

extern "C" int kdq_gemm_q4_0_packed(const void* packed, size_t n, size_t k, const uint16_t* x_f16,
                                    size_t m, uint16_t* y_f16, void* stream) {
    if (!packed || !x_f16 || !y_f16 || !m || !n || !k)
        return KDQ_ERR_ARGUMENT;
    if (k % 256 || m > 0xffffffu || n > 0xffffffu || k > 0xffffffu)
        return KDQ_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(x_f16) % 16 || reinterpret_cast<uintptr_t>(packed) % 16 ||
        reinterpret_cast<uintptr_t>(y_f16) % 2)
        return KDQ_ERR_ALIGNMENT;
    const size_t packed_bytes = kdq_gguf_packed_bytes(KDQ_Q4_0, k, n);
    if (overlaps(y_f16, m * n * 2, x_f16, m * k * 2) ||
        overlaps(y_f16, m * n * 2, packed, packed_bytes))
        return KDQ_ERR_ALIAS;
    // permuted activations, rows padded to the 128-token tile (padding never stored)
    int rc;
    const size_t m_pad = (m + PM - 1) / PM * PM;
    auto* xs = static_cast<uint16_t*>(workspace(m_pad * k * 2, &rc));
    if (rc)
        return rc;
    auto st = static_cast<hipStream_t>(stream);
    rc = launch_quantize<true>(x_f16, m, k, nullptr, nullptr, xs, st);
    if (rc)
        return rc;
    return launch_packed_gemm<2>(xs, static_cast<const uint8_t*>(packed), unsigned(m),
                                 unsigned(n), unsigned(k), y_f16, st);
}
