// Shared device/host helpers for the gfx950 kernels of the quantized matmul path.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "kadan_amd.h"

namespace kdq {

// 16-byte load that only assumes 4-byte alignment (gfx950 global loads of four
// dwords need dword alignment only; the compiler emits global_load_dwordx4).
typedef unsigned u32x4 __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ u32x4 load16(const uint8_t* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ unsigned load4(const uint8_t* p) {
    return *reinterpret_cast<const unsigned*>(p);
}

// Loads at 2-byte alignment (Q6_K super-blocks are 210 bytes, so every other one starts
// two bytes past a dword): gfx950 global loads run in unaligned-access mode, and the
// compiler still emits one global_load_dwordx4 / dwordx2 / dword for each.
typedef unsigned u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));
typedef unsigned u32x2_a2 __attribute__((ext_vector_type(2), aligned(2)));
typedef unsigned u32_a2 __attribute__((aligned(2)));

__device__ __forceinline__ u32x4 load16_a2(const uint8_t* p) {
    const u32x4_a2 v = *reinterpret_cast<const u32x4_a2*>(p);
    return u32x4{v.x, v.y, v.z, v.w};
}

__device__ __forceinline__ uint2 load8_a2(const uint8_t* p) {
    const u32x2_a2 v = *reinterpret_cast<const u32x2_a2*>(p);
    return make_uint2(v.x, v.y);
}

__device__ __forceinline__ unsigned load4_a2(const uint8_t* p) {
    return *reinterpret_cast<const u32_a2*>(p);
}

// Non-temporal (streaming) variants for weight bytes read once per launch: the loads
// carry the nt cache policy so a weight stream larger than the caches does not evict
// what is reused (activations, outputs).  Same alignment rules as load16 / load4.
__device__ __forceinline__ u32x4 stream16(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

__device__ __forceinline__ unsigned stream4(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const unsigned*>(p));
}

// Exact IEEE binary16 -> binary32 by integer construction (keeps NaN payloads),
// IW/include/kadan/gguf_quantization.hpp:576-593 semantics.
__device__ __forceinline__ float half_exact(unsigned h) {
    const unsigned sign = (h & 0x8000u) << 16;
    const unsigned e = (h >> 10) & 31u;
    const unsigned m = h & 1023u;
    if (e == 31u)
        return __uint_as_float(sign | 0x7f800000u | (m << 13));
    if (e == 0u)  // zero / subnormal: m * 2^-24 is exact
        return __uint_as_float(sign | __float_as_uint(float(m) * 0x1p-24f));
    return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
}

// Hardware conversion (exact for every finite half; NaNs come out quiet).
__device__ __forceinline__ float half_hw(unsigned h) {
    return float(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h)));
}

// Separately rounded fp32 operations (the decode must never be contracted into an
// FMA: IW/include/kadan/gguf_quantization.hpp:595-621).
__device__ __forceinline__ float mul_rn(float a, float b) {
    return __fmul_rn(a, b);
}
__device__ __forceinline__ float sub_rn(float a, float b) {
    return __fsub_rn(a, b);
}

__device__ __forceinline__ int sdot4(unsigned a, unsigned b, int c) {
    return __builtin_amdgcn_sdot4(int(a), int(b), c, false);
}

// Sum across the 64 lanes of a wavefront (result valid in every lane).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1)
        v += __shfl_xor(v, offset, 64);
    return v;
}

// Lanes of the rows in ROW_MASK read lane-permuted `v` (DPP control CTRL); the other
// rows read 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_read(float v) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

// Sum over the 64 lanes with DPP row operations (no LDS traffic): pairs, quads, half
// rows and rows of 16 by permutation, then the row totals are chained into lane 63,
// whose value every lane returns.  Needs all 64 lanes active.
__device__ __forceinline__ float wave_total(float v) {
    v += dpp_read<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]
    v += dpp_read<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]
    v += dpp_read<0x141, 0xf>(v);  // row_half_mirror
    v += dpp_read<0x140, 0xf>(v);  // row_mirror: every lane holds its row's sum
    v += dpp_read<0x142, 0xa>(v);  // row_bcast:15 -> rows 1 and 3
    v += dpp_read<0x143, 0xc>(v);  // row_bcast:31 -> rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Butterfly partner within each group of four lanes (xor 1 / xor 2) by DPP quad
// permutation; all four lanes of a group must be active.
__device__ __forceinline__ float quad_xor1(float v) {
    return dpp_read<0xb1, 0xf>(v);
}
__device__ __forceinline__ float quad_xor2(float v) {
    return dpp_read<0x4e, 0xf>(v);
}
__device__ __forceinline__ int quad_xor1(int v) {
    return __builtin_amdgcn_update_dpp(0, v, 0xb1, 0xf, 0xf, false);
}
__device__ __forceinline__ int quad_xor2(int v) {
    return __builtin_amdgcn_update_dpp(0, v, 0x4e, 0xf, 0xf, false);
}

// Maximum over the 64 lanes by DPP (as wave_total), for values >= 0: lanes outside a
// broadcast's row mask read 0, and fmaxf skips NaN.  Every lane returns it.
__device__ __forceinline__ float wave_max_nonneg(float v) {
    v = fmaxf(v, dpp_read<0xb1, 0xf>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_read<0x4e, 0xf>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_read<0x141, 0xf>(v));  // row_half_mirror
    v = fmaxf(v, dpp_read<0x140, 0xf>(v));  // row_mirror
    v = fmaxf(v, dpp_read<0x142, 0xa>(v));  // row_bcast:15
    v = fmaxf(v, dpp_read<0x143, 0xc>(v));  // row_bcast:31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1)
        v = fmaxf(v, __shfl_xor(v, offset, 64));
    return v;
}

// Host helpers --------------------------------------------------------------

// A decode-time product whose weights start at job.weights + min(*index, index_limit - 1)
// * index_stride when `index` (a device pointer) is set: the expert slice a device-side
// routing chose.  Products of streamed encodings run fused on the MFMA kernel, the rest
// on the exact kernel.  The jobs must satisfy kdq_gemv's argument rules (unchecked).
// With `paired` set (MFMA kernel only: swiglu_pairable), the job multiplies x by two
// matrices of the same shape and encoding, job.weights (gate) and `paired` (up, at the
// same expert offset), and writes silu(gate x) * (up x).
struct IndexedJob {
    kdq_matvec_job job;
    const int32_t* index;
    size_t index_stride;
    unsigned index_limit;
    const void* paired;
};
int indexed_gemv_batch(const IndexedJob* jobs, size_t count, hipStream_t stream);
// `count` products in one launch, all as `first` except that job j reads
// x + (j / x_every) * x_step, writes y + j * y_step and takes its expert from index[j]
// (each job takes `first`'s rows, x rows at x + r * in and y rows at y + r * stride; the
// MFMA kernel takes up to its plan's batch of rows, the exact kernel any, without
// `paired`).  A job whose index[j] is negative is skipped.
int indexed_gemv_affine(const IndexedJob& first, unsigned count, size_t x_step, size_t y_step,
                        hipStream_t stream, unsigned x_every = 1);
// The same over tile-packed weights (kdq_gguf_pack; Q4_0 / Q8_0 / Q4_K / Q6_K, columns a
// multiple of 16): `first.job.weights` (and `paired`) are packed stacks whose experts lie
// `index_stride` bytes apart; KDQ_ERR_UNSUPPORTED where the MFMA kernel does not take it.
int indexed_gemv_affine_packed(const IndexedJob& first, unsigned count, size_t x_step,
                               size_t y_step, hipStream_t stream, unsigned x_every = 1);
// Whether `count` jobs like j (an affine launch when count > 1) run on the MFMA kernel
// with a paired matrix.
bool swiglu_pairable(const kdq_matvec_job& j, size_t count);

// One token's MoE layer in two launches (gguf_gemv.hip):
//   up:   the F32 router GEMV, whose last workgroup routes the token (route_select) and
//         publishes the selection; the experts' paired gate / up, each workgroup waiting
//         (bounded; status bit 3 past the bound) for the selection once its activation
//         loads are out; the shared expert's paired gate / up in the same launch;
//   down: the experts' and the shared expert's down rows, the last workgroup of each row
//         block combining it (selection order, plus shared * sigmoid(gate_vector . x)).
// experts_up: paired, x = the token, y = [top_k][ff], index = idx (which the up launch
// writes, with w); experts_down: x = experts_up's y, y = [top_k][hidden], index = idx;
// shared_up: paired, one job; shared_down: x = shared_up's y, y = [hidden].  counters:
// device scratch of counter_count unsigned (the up launch clears them); gate: one float
// of device scratch.  Returns
// KDQ_ERR_UNSUPPORTED, having launched nothing, when the shapes or encodings are not
// among those instantiated (Q4_K expert gate / up with Q8_0 or Q4_K shared gate / up,
// inputs of 1280..4096 values; Q6_K or Q4_K downs of at most 1024 inputs); with
// check_only it launches nothing either way.
// Tokens of one fused decode call (moe_decode_fused): more take the staged path.
constexpr unsigned kFusedDecodeTokens = 8;
struct DecodeMoe {
    kdq_matvec_job router;  // F32, x = the tokens, y = logits (device scratch)
    IndexedJob experts_up, shared_up, experts_down, shared_down;
    bool up_packed, down_packed;
    float* logits;
    unsigned experts, top_k, hidden, tokens;
    int32_t* idx;
    float* w;
    const float* gate_vector;
    const float* x;
    float* y;
    unsigned* status;
    unsigned* counters;
    unsigned counter_count;
    float* gate;  // device scratch: the shared gate's sigmoid per token, between the launches
};
int moe_decode_fused(const DecodeMoe& m, hipStream_t stream, bool check_only);

// silu and sigmoid as the reference defines them (IW/src/models/text/gguf_weights.cpp:627-633)
__device__ __forceinline__ float silu_of(float v) {
    return v / (1.0f + expf(-v));
}
__device__ __forceinline__ float sigmoid_of(float v) {
    return 1.0f / (1.0f + expf(-v));
}

// The MoE router of kdq_moe_route (softmax with a double total, top-k by probability,
// weights renormalised by max(sum, 2^-14)) without the expert permutation.
// Grouped prefill GEMM (gguf_gemm.hip): y[p, :] = W_{e(p)} x_p for positions p in token
// tiles of kGroupedTileRows (positions a multiple of it), tile t's weights expert tile_expert[t] of a
// stack of tile-packed experts expert_bytes apart (tiles with a negative entry skipped);
// x_p = x[inv[p] / topk] (zero rows where inv[p] < 0), rows from *used on unstaged.
// xs (positions * k * 2 bytes) and sigma (positions * 4) are the caller's scratch.
// Q4_K / Q8_0 / Q6_K, k % 256 == 0, k <= 32768.
constexpr unsigned kGroupedTileRows = 64;
bool grouped_gemm_takes(int encoding, size_t k);
// `up` (another stack stored alike; grouped_gemm_pairs(encoding)): one launch writing
// y = silu(W_gate x) * (W_up x) with the reference's silu, bit-identical to the two
// products followed by that SwiGLU.
int grouped_gemm(int encoding, const void* packed, size_t expert_bytes,
                 const int32_t* tile_expert, size_t n, size_t k, const float* x,
                 const int32_t* inv, unsigned topk, const unsigned* used, size_t positions,
                 float* y, unsigned* status, uint16_t* xs, float* sigma, hipStream_t st,
                 const void* up = nullptr);
bool grouped_gemm_pairs(int encoding);
int route_selection(const float* logits, size_t tokens, size_t experts, size_t top_k,
                    int32_t* idx, float* w, hipStream_t stream);
// Dense prefill GEMM over one tile-packed matrix (kdq_gemm_packed's product) with the
// caller's scratch of dense_gemm_scratch(m, n, k) bytes: y[m x n] = x[m x k] W^T.
size_t dense_gemm_scratch(size_t m, size_t n, size_t k);
// y[m x n] = silu(x Wg^T) * (x Wu^T) for two tile-packed matrices stored alike
// (grouped_gemm_pairs(encoding)), one launch on 64-token tiles, no K slices; the same
// scratch as dense_gemm.
int dense_gemm_pair(int encoding, const void* gate, const void* up, size_t n, size_t k,
                    const float* x, size_t m, float* y, unsigned* status, void* scratch,
                    hipStream_t st);
int dense_gemm(int encoding, const void* packed, size_t n, size_t k, const float* x, size_t m,
               float* y, unsigned* status, void* scratch, hipStream_t st);

inline size_t block_values(int encoding) {
    switch (encoding) {
    case KDQ_BF16:
    case KDQ_F32:
    case KDQ_F16:
        return 1;
    case KDQ_Q4_0:
    case KDQ_Q8_0:
    case KDQ_IQ4_NL:
        return 32;
    case KDQ_Q3_K:
    case KDQ_Q4_K:
    case KDQ_Q6_K:
    case KDQ_IQ4_XS:
    case KDQ_IQ3_XXS:
    case KDQ_IQ2_S:
    case KDQ_IQ3_S:
        return 256;
    default:
        return 0;
    }
}

inline size_t block_bytes(int encoding) {
    switch (encoding) {
    case KDQ_Q4_0:
    case KDQ_IQ4_NL:
        return 18;
    case KDQ_Q8_0:
        return 34;
    case KDQ_Q4_K:
        return 144;
    case KDQ_Q3_K:
    case KDQ_IQ3_S:
        return 110;
    case KDQ_IQ3_XXS:
        return 98;
    case KDQ_IQ2_S:
        return 82;
    case KDQ_Q6_K:
        return 210;
    case KDQ_IQ4_XS:
        return 136;
    case KDQ_BF16:
    case KDQ_F16:
        return 2;
    case KDQ_F32:
        return 4;
    default:
        return 0;
    }
}

// Records a HIP failure for kdq_last_hip_error() and returns KDQ_ERR_HIP.
int hip_failure(hipError_t error);

// Per-device cached workspace (grown on demand, released by kdq_release_scratch).
void* workspace(size_t bytes, int* status);

// Compute units of the current device (cached per device; 256 if the query fails).
unsigned compute_units();

inline bool overlaps(const void* a, size_t an, const void* b, size_t bn) {
    if (!a || !b || !an || !bn)
        return false;
    const auto x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x <= y ? y - x < an : x - y < bn;
}

inline bool misaligned(const void* p, size_t alignment) {
    return reinterpret_cast<uintptr_t>(p) % alignment != 0;
}

inline bool mul_overflows(size_t a, size_t b) {
    return b && a > SIZE_MAX / b;
}

}  // namespace kdq

#define KDQ_HIP(call)                                   \
    do {                                                \
        const hipError_t kdq_error_ = (call);           \
        if (kdq_error_ != hipSuccess)                   \
            return ::kdq::hip_failure(kdq_error_);      \
    } while (0)
