// MXFP4 mixture-of-experts layer for gfx950.  The reference has no device MoE: this
// composes MoeLayer::forward (IW/src/models/text/qwen_layers.cpp:378-492; IW =
// services/hikari/inference_worker) with the MXFP4 product semantics of
// IW/src/weights/quantization.cpp:79-99,207-247, behind include/kadan_amd.h.
//
//   route_kernel      one wavefront per token: softmax (float exp, double total),
//                     top-k by logit (equal logits keep the lower expert), renormalise
//   permute_kernel    one workgroup: stable counting sort of the slots by expert
//                     (expert-major, slot ascending) plus the list of work items
//                     (expert, first row) of at most kItemRows rows each
//   gate_up_kernel    grouped GEMM over work items: gathered bf16 token rows x FP4
//                     gate and up rows dequantized in registers to bf16
//                     (v_cvt_scalef32_pk_bf16_fp4, exact), v_mfma_f32_32x32x16_bf16 with
//                     fp32 accumulation, fused h = silu(g) * u stored as bf16 hi + lo
//   down_kernel       grouped GEMM h x FP4 down rows (hi and lo terms), scaled by the
//                     routing weight of the row's slot
//   combine_kernel    y[t] = sum_i contribution[t*k + i] in selection order (float)
#include "kdq_common.hpp"

#include <cmath>

namespace kdq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kMaxTopK = 8, kMaxExperts = 256;
constexpr int kTileRows = 32, kTiles = 4, kItemRows = kTileRows * kTiles;

// ------------------------------------------------------------------ routing

__device__ __forceinline__ double wave_sum_double(double v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1)
        v += __shfl_xor(v, offset, 64);
    return v;
}

__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits,
                                                    unsigned tokens, unsigned experts,
                                                    unsigned top_k, int32_t* __restrict__ idx,
                                                    float* __restrict__ weight) {
    const unsigned lane = threadIdx.x % 64;
    const unsigned t = blockIdx.x * 4 + threadIdx.x / 64;
    if (t >= tokens)
        return;
    const float* l = logits + size_t(t) * experts;
    float v[4], p[4];
    float maximum = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const unsigned e = lane + 64 * j;
        v[j] = e < experts ? l[e] : -INFINITY;
        maximum = fmaxf(maximum, v[j]);
    }
    maximum = wave_max(maximum);
    double total = 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const unsigned e = lane + 64 * j;
        p[j] = e < experts ? expf(v[j] - maximum) : 0.f;
        total += double(p[j]);
    }
    total = wave_sum_double(total);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        p[j] = float(double(p[j]) / total);

    unsigned taken = 0;
    float sum = 0.f, chosen_p = 0.f;
    int chosen_e = 0;
    for (unsigned i = 0; i < top_k; ++i) {
        float bv = -INFINITY;
        int be = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = int(lane + 64 * j);
            if (unsigned(e) < experts && !(taken & (1u << j)) && (v[j] > bv || (v[j] == bv && e < be))) {
                bv = v[j];
                be = e;
            }
        }
#pragma unroll
        for (int offset = 32; offset > 0; offset >>= 1) {
            const float ov = __shfl_xor(bv, offset, 64);
            const int oe = __shfl_xor(be, offset, 64);
            if (ov > bv || (ov == bv && oe < be)) {
                bv = ov;
                be = oe;
            }
        }
        const unsigned owner = unsigned(be) % 64, slot = unsigned(be) / 64;
        if (lane == owner)
            taken |= 1u << slot;
        float mine = p[0];
#pragma unroll
        for (int j = 1; j < 4; ++j)
            mine = slot == unsigned(j) ? p[j] : mine;
        const float pb = __shfl(mine, int(owner), 64);
        sum += pb;  // sequential, in selection order
        if (lane == i) {
            chosen_p = pb;
            chosen_e = be;
        }
    }
    sum = fmaxf(sum, 6.103515625e-5f);
    if (lane < top_k) {
        idx[size_t(t) * top_k + lane] = chosen_e;
        weight[size_t(t) * top_k + lane] = chosen_p / sum;
    }
}

// Stable counting sort of slots by expert, in one workgroup; also the work items.
__global__ __launch_bounds__(1024) void permute_kernel(const int32_t* __restrict__ idx,
                                                       unsigned slots, unsigned experts,
                                                       int32_t* __restrict__ offsets,
                                                       int32_t* __restrict__ perm,
                                                       int32_t* __restrict__ items,
                                                       int32_t* __restrict__ item_count) {
    __shared__ int counts[kMaxExperts], base[kMaxExperts];
    __shared__ int wave_counts[16][kMaxExperts];
    const unsigned tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    for (unsigned e = tid; e < experts; e += 1024)
        counts[e] = 0;
    __syncthreads();
    for (unsigned s = tid; s < slots; s += 1024)
        atomicAdd(&counts[idx[s]], 1);
    __syncthreads();
    if (tid == 0) {
        int acc = 0, n = 0;
        for (unsigned e = 0; e < experts; ++e) {
            offsets[e] = acc;
            base[e] = acc;
            for (int r = 0; r < counts[e]; r += kItemRows) {
                items[2 * n] = int(e);
                items[2 * n + 1] = r;
                ++n;
            }
            acc += counts[e];
        }
        offsets[experts] = acc;
        *item_count = n;
    }
    __syncthreads();
    const unsigned long long below = (1ull << lane) - 1ull;
    for (unsigned first = 0; first < slots; first += 1024) {
        for (unsigned i = tid; i < 16 * kMaxExperts; i += 1024)
            (&wave_counts[0][0])[i] = 0;
        __syncthreads();
        const unsigned s = first + tid;
        const bool valid = s < slots;
        const int e = valid ? idx[s] : 0;
        unsigned long long same = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const unsigned long long ones = __ballot(valid && ((e >> b) & 1));
            same &= ((e >> b) & 1) ? ones : ~ones;
        }
        const int rank = __popcll(same & below);
        const int group = __popcll(same);
        if (valid && rank == group - 1)
            wave_counts[wave][e] = group;
        __syncthreads();
        if (valid) {
            int r = base[e] + rank;
            for (unsigned w = 0; w < wave; ++w)
                r += wave_counts[w][e];
            perm[r] = int(s);
        }
        __syncthreads();
        for (unsigned x = tid; x < experts; x += 1024) {
            int add = 0;
            for (unsigned w = 0; w < 16; ++w)
                add += wave_counts[w][x];
            base[x] += add;
        }
        __syncthreads();
    }
}

// --------------------------------------------------------------- grouped GEMMs

__device__ __forceinline__ float e8m0(unsigned s) {
    return __uint_as_float(s << 23);  // exponent field only: the converter reads 2^(s-127)
}

// 32 FP4 values (16 bytes, low nibble first) times 2^(scale-127) -> 32 exact bf16,
// as four 8-value MFMA operands.
__device__ __forceinline__ void dequant32(const u32x4 codes, unsigned scale, bf16x8 out[4]) {
    const float s = e8m0(scale);
    const unsigned w[4] = {codes.x, codes.y, codes.z, codes.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[q], s, 0);
        const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[q], s, 1);
        const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[q], s, 2);
        const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[q], s, 3);
        out[q] = bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
    }
}

__device__ __forceinline__ bf16x8 load_bf16x8(const uint16_t* p) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(p);
    return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ float silu(float x) {
    return x / (1.0f + expf(-x));
}

__device__ __forceinline__ uint16_t bf16_rne(float x) {
    return __builtin_bit_cast(uint16_t, __bf16(x));
}

__device__ __forceinline__ float bf16_value(uint16_t b) {
    return __uint_as_float(unsigned(b) << 16);
}

struct Item {
    int expert, first, count, segment;
};

__device__ __forceinline__ Item load_item(const int32_t* items, const int32_t* offsets,
                                          unsigned item) {
    Item it;
    it.expert = items[2 * item];
    it.first = items[2 * item + 1];
    it.segment = offsets[it.expert];
    it.count = min(kItemRows, offsets[it.expert + 1] - it.segment - it.first);
    return it;
}

// Workgroup: `waves` wavefronts, wavefront w owns output features
// (blockIdx.x * waves + w) * 32 .. +31 of both gate and up; blockIdx.y is the item.
// The k axis runs in chunks of 64: lane group g (lane / 32) holds the 32 values
// 64c + 32g .. +31 of its row (one MXFP4 scale block), fed to four MFMAs of 16.
__global__ __launch_bounds__(256) void gate_up_kernel(
    const uint16_t* __restrict__ x, unsigned hidden, unsigned inter, unsigned top_k,
    const uint8_t* __restrict__ gate_blocks, const uint8_t* __restrict__ gate_scales,
    const uint8_t* __restrict__ up_blocks, const uint8_t* __restrict__ up_scales,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ items, const int32_t* __restrict__ item_count,
    uint16_t* __restrict__ h_hi, uint16_t* __restrict__ h_lo) {
    if (int(blockIdx.y) >= *item_count)
        return;
    const Item it = load_item(items, offsets, blockIdx.y);
    const unsigned waves = blockDim.x / 64, wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const unsigned i32 = lane % 32, g = lane / 32;
    const unsigned f = (blockIdx.x * waves + wave) * 32 + i32;
    const int tiles = (it.count + kTileRows - 1) / kTileRows;

    const uint16_t* xrow[kTiles];
#pragma unroll
    for (int m = 0; m < kTiles; ++m) {
        const int r = m * kTileRows + int(i32);
        xrow[m] = r < it.count ? x + size_t(perm[it.segment + it.first + r] / int(top_k)) * hidden
                               : nullptr;
    }
    const size_t wrow = (size_t(it.expert) * inter + f);
    const uint8_t* gb = gate_blocks + wrow * (hidden / 2);
    const uint8_t* ub = up_blocks + wrow * (hidden / 2);
    const uint8_t* gs = gate_scales + wrow * (hidden / 32);
    const uint8_t* us = up_scales + wrow * (hidden / 32);

    f32x16 acc_g[kTiles], acc_u[kTiles];
#pragma unroll
    for (int m = 0; m < kTiles; ++m)
        acc_g[m] = acc_u[m] = f32x16{};

    for (unsigned c = 0; c < hidden / 64; ++c) {
        const unsigned kb = 64 * c + 32 * g;
        bf16x8 bg[4], bu[4];
        dequant32(load16(gb + kb / 2), gs[kb / 32], bg);
        dequant32(load16(ub + kb / 2), us[kb / 32], bu);
#pragma unroll
        for (int m = 0; m < kTiles; ++m) {
            if (m >= tiles)
                break;
            bf16x8 a[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                a[j] = xrow[m] ? load_bf16x8(xrow[m] + kb + 8 * j) : bf16x8{};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc_g[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[j], bg[j], acc_g[m], 0, 0, 0);
                acc_u[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[j], bu[j], acc_u[m], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < kTiles; ++m) {
        if (m >= tiles)
            break;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int r = m * kTileRows + 8 * (v / 4) + 4 * int(g) + (v % 4);
            if (r < it.count) {
                const float h = silu(acc_g[m][v]) * acc_u[m][v];
                const uint16_t hi = bf16_rne(h);
                const uint16_t lo = bf16_rne(h - bf16_value(hi));
                const size_t at = size_t(it.segment + it.first + r) * inter + f;
                h_hi[at] = hi;
                h_lo[at] = lo;
            }
        }
    }
}

// contribution[slot, d] = w[slot] * sum_k (h_hi + h_lo)[p, k] * down[e, d, k]
__global__ __launch_bounds__(256) void down_kernel(
    const uint16_t* __restrict__ h_hi, const uint16_t* __restrict__ h_lo, unsigned hidden,
    unsigned inter, const uint8_t* __restrict__ down_blocks,
    const uint8_t* __restrict__ down_scales, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ perm, const float* __restrict__ weight,
    const int32_t* __restrict__ items, const int32_t* __restrict__ item_count,
    float* __restrict__ contribution) {
    if (int(blockIdx.y) >= *item_count)
        return;
    const Item it = load_item(items, offsets, blockIdx.y);
    const unsigned waves = blockDim.x / 64, wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const unsigned i32 = lane % 32, g = lane / 32;
    const unsigned d = (blockIdx.x * waves + wave) * 32 + i32;
    const int tiles = (it.count + kTileRows - 1) / kTileRows;

    const size_t wrow = size_t(it.expert) * hidden + d;
    const uint8_t* db = down_blocks + wrow * (inter / 2);
    const uint8_t* ds = down_scales + wrow * (inter / 32);

    size_t hrow[kTiles];
    bool valid[kTiles];
#pragma unroll
    for (int m = 0; m < kTiles; ++m) {
        const int r = m * kTileRows + int(i32);
        valid[m] = r < it.count;
        hrow[m] = size_t(it.segment + it.first + (valid[m] ? r : 0)) * inter;
    }
    f32x16 acc[kTiles];
#pragma unroll
    for (int m = 0; m < kTiles; ++m)
        acc[m] = f32x16{};

    for (unsigned c = 0; c < inter / 64; ++c) {
        const unsigned kb = 64 * c + 32 * g;
        bf16x8 b[4];
        dequant32(load16(db + kb / 2), ds[kb / 32], b);
#pragma unroll
        for (int m = 0; m < kTiles; ++m) {
            if (m >= tiles)
                break;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bf16x8 ah = valid[m] ? load_bf16x8(h_hi + hrow[m] + kb + 8 * j) : bf16x8{};
                const bf16x8 al = valid[m] ? load_bf16x8(h_lo + hrow[m] + kb + 8 * j) : bf16x8{};
                acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, b[j], acc[m], 0, 0, 0);
                acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, b[j], acc[m], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < kTiles; ++m) {
        if (m >= tiles)
            break;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int r = m * kTileRows + 8 * (v / 4) + 4 * int(g) + (v % 4);
            if (r < it.count) {
                const int slot = perm[it.segment + it.first + r];
                contribution[size_t(slot) * hidden + d] = acc[m][v] * weight[slot];
            }
        }
    }
}

__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ contribution,
                                                      unsigned tokens, unsigned hidden,
                                                      unsigned top_k, float* __restrict__ y) {
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= size_t(tokens) * hidden)
        return;
    const size_t t = i / hidden, d = i % hidden;
    float sum = 0.f;
    for (unsigned k = 0; k < top_k; ++k)
        sum += contribution[(t * top_k + k) * hidden + d];
    y[i] = sum;
}

__global__ __launch_bounds__(256) void mxfp4_dequant_kernel(const uint8_t* __restrict__ blocks,
                                                            const uint8_t* __restrict__ scales,
                                                            size_t rows, size_t cols,
                                                            float* __restrict__ out,
                                                            unsigned* status) {
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;  // one byte = 2 values
    unsigned bad = 0;
    if (i < rows * cols / 2) {
        const size_t r = i / (cols / 2), c = (i % (cols / 2)) * 2;
        const unsigned byte = blocks[i];
        const unsigned s = scales[r * (cols / 32) + c / 32];
        if (s == 255)
            bad |= 1u;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const unsigned code = (byte >> (4 * h)) & 15u;
            const float mag[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
            float v = 0.f;
#pragma unroll
            for (int q = 0; q < 8; ++q)
                v = (code & 7u) == unsigned(q) ? mag[q] : v;
            v = ldexpf(v, int(s) - 127);
            if (!isfinite(v))
                bad |= 2u;
            out[r * cols + c + h] = (code & 8u) ? -v : v;
        }
    }
    if (status && bad)
        atomicOr(status, bad);
}

// Workspace carve-up (device bytes, 256-aligned pieces).
struct MoeScratch {
    int32_t *idx, *offsets, *perm, *items, *item_count;
    float* weight;
    uint16_t *h_hi, *h_lo;
    float* contribution;
};

size_t align256(size_t n) {
    return (n + 255) & ~size_t(255);
}

size_t moe_scratch_bytes(size_t tokens, size_t hidden, size_t inter, size_t experts,
                         size_t top_k) {
    const size_t slots = tokens * top_k, items = slots / kItemRows + experts + 1;
    return align256(slots * 4) * 3 + align256((experts + 1) * 4) + align256(items * 8) +
           align256(4) + 2 * align256(slots * inter * 2) + align256(slots * hidden * 4);
}

MoeScratch carve(uint8_t* p, size_t tokens, size_t hidden, size_t inter, size_t experts,
                 size_t top_k) {
    const size_t slots = tokens * top_k, items = slots / kItemRows + experts + 1;
    MoeScratch s;
    auto take = [&](size_t n) {
        uint8_t* q = p;
        p += align256(n);
        return q;
    };
    s.idx = reinterpret_cast<int32_t*>(take(slots * 4));
    s.weight = reinterpret_cast<float*>(take(slots * 4));
    s.perm = reinterpret_cast<int32_t*>(take(slots * 4));
    s.offsets = reinterpret_cast<int32_t*>(take((experts + 1) * 4));
    s.items = reinterpret_cast<int32_t*>(take(items * 8));
    s.item_count = reinterpret_cast<int32_t*>(take(4));
    s.h_hi = reinterpret_cast<uint16_t*>(take(slots * inter * 2));
    s.h_lo = reinterpret_cast<uint16_t*>(take(slots * inter * 2));
    s.contribution = reinterpret_cast<float*>(take(slots * hidden * 4));
    return s;
}

int check_route(const float* logits, size_t tokens, size_t experts, size_t top_k) {
    if (!logits || !tokens || !experts || !top_k)
        return KDQ_ERR_ARGUMENT;
    if (experts > kMaxExperts || top_k > kMaxTopK || top_k > experts || tokens > (1u << 24) ||
        tokens * top_k > (size_t(1) << 26))
        return KDQ_ERR_SHAPE;
    return KDQ_OK;
}

// Waves per workgroup for an N dimension of n features (32 per wave): the largest of
// 4, 3, 2, 1 dividing n / 32.
unsigned waves_for(size_t n) {
    const size_t tiles = n / 32;
    for (unsigned w : {4u, 3u, 2u})
        if (tiles % w == 0)
            return w;
    return 1;
}

int launch_route(const float* logits, size_t tokens, size_t experts, size_t top_k,
                 int32_t* idx, float* w, int32_t* offsets, int32_t* perm, int32_t* items,
                 int32_t* item_count, hipStream_t stream) {
    hipLaunchKernelGGL(route_kernel, dim3(unsigned((tokens + 3) / 4)), dim3(256), 0, stream,
                       logits, unsigned(tokens), unsigned(experts), unsigned(top_k), idx, w);
    KDQ_HIP(hipGetLastError());
    hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(1024), 0, stream, idx,
                       unsigned(tokens * top_k), unsigned(experts), offsets, perm, items,
                       item_count);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}

}  // namespace
}  // namespace kdq

using namespace kdq;

extern "C" int kdq_moe_route(const float* logits, size_t tokens, size_t experts, size_t top_k,
                             int32_t* idx, float* w, int32_t* offsets, int32_t* perm,
                             void* stream) {
    int rc = check_route(logits, tokens, experts, top_k);
    if (rc)
        return rc;
    if (!idx || !w || !offsets || !perm)
        return KDQ_ERR_ARGUMENT;
    const size_t items = tokens * top_k / kItemRows + experts + 1;
    auto* scratch = static_cast<int32_t*>(workspace(items * 8 + 256, &rc));
    if (rc)
        return rc;
    return launch_route(logits, tokens, experts, top_k, idx, w, offsets, perm, scratch,
                        scratch + items * 2, static_cast<hipStream_t>(stream));
}

extern "C" int kdq_mxfp4_dequantize(const uint8_t* blocks, const uint8_t* scales, size_t rows,
                                    size_t cols, float* out, unsigned* status, void* stream) {
    if (!blocks || !scales || !out || !rows || !cols)
        return KDQ_ERR_ARGUMENT;
    if (cols % 32 || mul_overflows(rows, cols))
        return KDQ_ERR_SHAPE;
    const size_t threads = rows * cols / 2;
    hipLaunchKernelGGL(mxfp4_dequant_kernel, dim3(unsigned((threads + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), blocks, scales, rows, cols, out,
                       status);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}

extern "C" int kdq_moe_mxfp4(const uint16_t* x_bf16, const float* logits, size_t tokens,
                             size_t hidden, size_t inter, size_t experts, size_t top_k,
                             const uint8_t* gate_blocks, const uint8_t* gate_scales,
                             const uint8_t* up_blocks, const uint8_t* up_scales,
                             const uint8_t* down_blocks, const uint8_t* down_scales, float* y,
                             int32_t* idx, float* w, int32_t* offsets, int32_t* perm,
                             void* stream) {
    int rc = check_route(logits, tokens, experts, top_k);
    if (rc)
        return rc;
    if (!x_bf16 || !y || !gate_blocks || !gate_scales || !up_blocks || !up_scales ||
        !down_blocks || !down_scales || !hidden || !inter)
        return KDQ_ERR_ARGUMENT;
    if (hidden % 64 || inter % 64 || hidden > (1u << 20) || inter > (1u << 20))
        return KDQ_ERR_SHAPE;
    if (overlaps(y, tokens * hidden * 4, x_bf16, tokens * hidden * 2) ||
        overlaps(y, tokens * hidden * 4, logits, tokens * experts * 4))
        return KDQ_ERR_ALIAS;
    const size_t bytes = moe_scratch_bytes(tokens, hidden, inter, experts, top_k);
    auto* base = static_cast<uint8_t*>(workspace(bytes, &rc));
    if (rc)
        return rc;
    MoeScratch s = carve(base, tokens, hidden, inter, experts, top_k);
    if (idx)
        s.idx = idx;
    if (w)
        s.weight = w;
    if (offsets)
        s.offsets = offsets;
    if (perm)
        s.perm = perm;
    auto st = static_cast<hipStream_t>(stream);
    rc = launch_route(logits, tokens, experts, top_k, s.idx, s.weight, s.offsets, s.perm,
                      s.items, s.item_count, st);
    if (rc)
        return rc;
    const size_t slots = tokens * top_k;
    const unsigned max_items = unsigned(slots / kItemRows + experts + 1);
    const unsigned wg = waves_for(inter);
    hipLaunchKernelGGL(gate_up_kernel, dim3(unsigned(inter / 32 / wg), max_items), dim3(64 * wg),
                       0, st, x_bf16, unsigned(hidden), unsigned(inter), unsigned(top_k),
                       gate_blocks, gate_scales, up_blocks, up_scales, s.offsets, s.perm,
                       s.items, s.item_count, s.h_hi, s.h_lo);
    KDQ_HIP(hipGetLastError());
    const unsigned wd = waves_for(hidden);
    hipLaunchKernelGGL(down_kernel, dim3(unsigned(hidden / 32 / wd), max_items), dim3(64 * wd), 0,
                       st, s.h_hi, s.h_lo, unsigned(hidden), unsigned(inter), down_blocks,
                       down_scales, s.offsets, s.perm, s.weight, s.items, s.item_count,
                       s.contribution);
    KDQ_HIP(hipGetLastError());
    const size_t n = tokens * hidden;
    hipLaunchKernelGGL(combine_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st,
                       s.contribution, unsigned(tokens), unsigned(hidden), unsigned(top_k), y);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}
