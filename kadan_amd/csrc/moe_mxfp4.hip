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
constexpr int kTileRows = 32, kTiles = 2, kItemRows = kTileRows * kTiles;
constexpr int kGemmWaves = 4;  // wavefronts per grouped-GEMM workgroup, 64 weight rows each
constexpr int kStepK = 64;     // K values per step: 16 FP4 bytes per lane

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
                                                       int32_t* __restrict__ item_count,
                                                       int32_t* __restrict__ position) {
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
            if (position)
                position[s] = r;  // inverse permutation
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

// ------------------------------------------------------------ packed weights
//
// The grouped GEMMs read expert weights in a packed layout, written once per weight set
// by kdq_moe_mxfp4_pack from the reference layout (blocks [E][R][C/2], scales
// [E][R][C/32]).  For each expert and each group of 32 rows (R % 32 == 0) and each step of
// 64 values (C % 64 == 0):
//   codes:  one 1 KB block, lane l = i + 32h holding bytes 32q + 16h .. +15 of row 32G + i
//           (values 64q + 32h .. +31): a wavefront's load of a step is 8 whole lines;
//   scales: per 4 steps one 256-byte block, byte j of lane l's dword = the E8M0 scale of
//           values 64(4p + j) + 32h .. +31 of row 32G + i (zero past the last step).
// Layout: codes [E][R/32][C/64][64][16 B], then scales [E][R/32][ceil(C/256)][64][4 B].

struct Packed {
    size_t groups, steps, scale_groups;  // per expert: row groups, steps, scale groups
    size_t code_bytes, scale_bytes;      // whole tensor
};

__host__ __device__ inline Packed packed_shape(size_t experts, size_t rows, size_t cols) {
    Packed p;
    p.groups = rows / 32;
    p.steps = cols / 64;
    p.scale_groups = (p.steps + 3) / 4;
    p.code_bytes = experts * rows * cols / 2;
    p.scale_bytes = experts * p.groups * p.scale_groups * 256;
    return p;
}

__global__ __launch_bounds__(256) void pack_codes_kernel(const uint8_t* __restrict__ blocks,
                                                         size_t units, size_t steps, size_t cols,
                                                         uint8_t* __restrict__ out) {
    const size_t u = size_t(blockIdx.x) * blockDim.x + threadIdx.x;  // one 16-byte unit
    if (u >= units)
        return;
    const unsigned l = unsigned(u % 64);
    const size_t q = (u / 64) % steps, eg = u / (64 * steps);  // eg = expert * groups + group
    const size_t row = eg * 32 + l % 32;
    *reinterpret_cast<u32x4*>(out + u * 16) =
        load16(blocks + row * (cols / 2) + q * 32 + 16 * (l / 32));
}

__global__ __launch_bounds__(256) void pack_scales_kernel(const uint8_t* __restrict__ scales,
                                                          size_t words, size_t scale_groups,
                                                          size_t steps, size_t cols,
                                                          unsigned* __restrict__ out) {
    const size_t u = size_t(blockIdx.x) * blockDim.x + threadIdx.x;  // one dword
    if (u >= words)
        return;
    const unsigned l = unsigned(u % 64);
    const size_t p = (u / 64) % scale_groups, eg = u / (64 * scale_groups);
    const uint8_t* row = scales + (eg * 32 + l % 32) * (cols / 32);
    unsigned word = 0;
#pragma unroll
    for (unsigned j = 0; j < 4; ++j) {
        const size_t q = 4 * p + j;
        if (q < steps)
            word |= unsigned(row[2 * q + l / 32]) << (8 * j);
    }
    out[u] = word;
}

// Grouped GEMMs on v_mfma_f32_32x32x16_bf16.  A workgroup of kGemmWaves wavefronts works
// on one work item (expert e, up to kItemRows consecutive rows of its segment: one or two
// MFMA row tiles of 32) and one K slice.  Every wavefront owns two 32-row weight groups
// (gate and up of the same 32 features, or two groups of down rows) and multiplies each
// staged activation fragment into both.  The weight operand B streams from the packed
// layout: per 64-value step, lane (f = lane % 32, h = lane / 32) holds 32 FP4 values of its
// row (16 bytes) and MFMA t takes values 32h + 8t .. +7 of them (the activation operand
// uses the same k order), dequantized with v_cvt_scalef32_pk_bf16_fp4, which is exact.
// The activation operand A (the item's occupied row tiles) is staged per chunk of steps
// into LDS by the whole workgroup, double-buffered.  Each lane issues chunk c + 2's
// activation loads, then chunk c + 1's weight loads, while chunk c is multiplied and chunk
// c + 1 is stored to LDS; all loads are unconditional (indices past the end are clamped
// to valid data), so each wait counts exactly the loads the next step needs.

// Staged rows: PLANES planes of CHUNK steps of 64 bf16 values per row, 16 bytes of pad.
template <int CHUNK, int PLANES> struct Stage {
    static constexpr int pitch = CHUNK * PLANES * kStepK * 2 + 16;
    static constexpr int buffer = kItemRows * pitch;
    static constexpr int pieces = CHUNK * PLANES * 8;  // 16-byte pieces per row
};

// This thread's share of a staged chunk of ROWS rows: pieces i = 0..per_thread-1 are row
// (tid / pieces + i * rows_step) at the same offset (tid % pieces) for every chunk.
template <int CHUNK, int PLANES, int ROWS> struct StageThread {
    using S = Stage<CHUNK, PLANES>;
    static constexpr int threads = kGemmWaves * 64;
    static_assert(ROWS * S::pieces % threads == 0, "pieces cover the threads exactly");
    static constexpr int per_thread = ROWS * S::pieces / threads;
    static constexpr int rows_step = threads / S::pieces;
    const uint16_t* src[per_thread];  // row start in its plane (always a valid row)
    bool valid[per_thread];           // the row exists (else it is stored as zeros)
    unsigned step, plane, sub;
};

// Plane p of the staged operand starts at base + p * plane_stride (one base pointer keeps
// the loads global: a per-thread choice between pointers would make them flat);
// `row_offset(r)` is the element offset of row r within a plane, or -1 past the item.
template <int CHUNK, int PLANES, int ROWS, class RowOffset>
__device__ __forceinline__ StageThread<CHUNK, PLANES, ROWS> stage_thread(const uint16_t* base,
                                                                         size_t plane_stride,
                                                                         RowOffset row_offset) {
    using T = StageThread<CHUNK, PLANES, ROWS>;
    using S = Stage<CHUNK, PLANES>;
    T t;
    const unsigned within = threadIdx.x % S::pieces;
    t.step = within / (8 * PLANES);
    t.plane = (within / 8) % PLANES;
    t.sub = within % 8;
#pragma unroll
    for (int i = 0; i < T::per_thread; ++i) {
        const unsigned row = threadIdx.x / S::pieces + i * T::rows_step;
        const long long at = row_offset(row);
        t.valid[i] = at >= 0;
        t.src[i] = base + t.plane * plane_stride + (at >= 0 ? at : row_offset(0));
    }
    return t;
}

template <int CHUNK, int PLANES, int ROWS> struct StagePieces {
    u32x4 v[StageThread<CHUNK, PLANES, ROWS>::per_thread];
};

// Loads the pieces of the chunk starting at step q (steps past `last` re-read `last`).
template <int CHUNK, int PLANES, int ROWS>
__device__ __forceinline__ void stage_load(const StageThread<CHUNK, PLANES, ROWS>& t, unsigned q,
                                           unsigned last, StagePieces<CHUNK, PLANES, ROWS>& P) {
    const unsigned step = min(q + t.step, last);
#pragma unroll
    for (int i = 0; i < StageThread<CHUNK, PLANES, ROWS>::per_thread; ++i)
        P.v[i] = *reinterpret_cast<const u32x4*>(t.src[i] + size_t(step) * kStepK + t.sub * 8);
}

// Stores a loaded chunk to LDS: every piece, also those of steps past the end of the K
// range (they land in buffer space no MFMA reads), without branches, so no path leaves
// a load outstanding.
template <int CHUNK, int PLANES, int ROWS>
__device__ __forceinline__ void stage_store(const StageThread<CHUNK, PLANES, ROWS>& t,
                                            const StagePieces<CHUNK, PLANES, ROWS>& P,
                                            uint8_t* buf) {
    using T = StageThread<CHUNK, PLANES, ROWS>;
    using S = Stage<CHUNK, PLANES>;
#pragma unroll
    for (int i = 0; i < T::per_thread; ++i) {
        const unsigned row = threadIdx.x / S::pieces + i * T::rows_step;
        *reinterpret_cast<u32x4*>(buf + row * S::pitch + (t.step * PLANES + t.plane) * 128 +
                                  t.sub * 16) = t.valid[i] ? P.v[i] : u32x4{0, 0, 0, 0};
    }
}

// 8 exact bf16 values from one dword of a lane's 16 FP4 bytes.
__device__ __forceinline__ bf16x8 dequant8(unsigned word, float scale) {
    const bf16x2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 0);
    const bf16x2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 1);
    const bf16x2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 2);
    const bf16x2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 3);
    return bf16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

__device__ __forceinline__ bf16x8 lds_bf16x8(const uint8_t* p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(p));
}

// One wavefront's two packed weight groups (codes at + step * 1 KB, scales at + group * 64
// dwords, both already offset by the lane).
struct WavePair {
    const uint8_t* codes[2];
    const unsigned* scales[2];
};

__device__ __forceinline__ WavePair wave_pair(const uint8_t* packed, const Packed& shape,
                                              size_t group0, size_t group1, unsigned lane) {
    WavePair w;
    const size_t g[2] = {group0, group1};
#pragma unroll
    for (int m = 0; m < 2; ++m) {
        w.codes[m] = packed + g[m] * shape.steps * 1024 + lane * 16;
        w.scales[m] = reinterpret_cast<const unsigned*>(packed + shape.code_bytes +
                                                        g[m] * shape.scale_groups * 256) +
                      lane;
    }
    return w;
}

// K slice `slice` of `slices`: [begin, end) in steps, begin a multiple of 8 (two scale
// groups).
__device__ __forceinline__ void slice_steps(unsigned steps, unsigned slices, unsigned slice,
                                            unsigned& begin, unsigned& end) {
    const unsigned per = ((steps + slices - 1) / slices + 7) / 8 * 8;
    begin = min(steps, slice * per);
    end = min(steps, begin + per);
}

__device__ __forceinline__ void issue_fence() {
    asm volatile("" ::: "memory");  // keeps the load issue order (activation pointers are
    __builtin_amdgcn_sched_barrier(0);  // not restrict)
}

// acc[m][t] += A(rows of tile t, steps [q0, q1)) * B(group m of the pair), q0 % 8 == 0.
// Activations are loaded two chunks ahead of their MFMAs (stored to LDS one chunk ahead),
// weights one chunk ahead, scale dwords with the first chunk of their 4 steps.  The loop
// runs whole periods of 8 steps (two scale groups) unrolled, so every ring slot stays in
// fixed registers (a rotating copy would wait for the loads just issued) and no early exit
// reaches the loop head with loads outstanding; chunks past the end multiply nothing.
template <int CHUNK, int PLANES, int TILES>
__device__ __forceinline__ void gemm_pair(const StageThread<CHUNK, PLANES, TILES * kTileRows>& st,
                                          const WavePair& w, unsigned q0, unsigned q1,
                                          bool active, unsigned i32, unsigned h,
                                          uint8_t (&stage)[2][Stage<CHUNK, PLANES>::buffer],
                                          f32x16 (&acc)[2][TILES]) {
    static_assert(CHUNK == 1 || CHUNK == 2 || CHUNK == 4, "chunks tile the scale groups");
    using S = Stage<CHUNK, PLANES>;
    constexpr int ROWS = TILES * kTileRows, PERIOD = 8 / CHUNK;
    auto load_codes = [&](unsigned q, u32x4(&c)[CHUNK][2]) {
#pragma unroll
        for (int s = 0; s < CHUNK; ++s)
#pragma unroll
            for (int m = 0; m < 2; ++m)
                c[s][m] = load16(w.codes[m] + size_t(min(q + s, q1 - 1)) * 1024);
    };
    auto load_scales = [&](unsigned q, unsigned(&sc)[2]) {
#pragma unroll
        for (int m = 0; m < 2; ++m)
            sc[m] = w.scales[m][size_t(min(q, q1 - 1) / 4) * 64];
    };
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int t = 0; t < TILES; ++t)
            acc[m][t] = f32x16{};
    StagePieces<CHUNK, PLANES, ROWS> xr[2];
    u32x4 wc[2][CHUNK][2];
    unsigned sc[2][2];
    stage_load(st, q0, q1 - 1, xr[0]);
    issue_fence();
    load_codes(q0, wc[0]);
    load_scales(q0, sc[0]);
    issue_fence();
    stage_load(st, q0 + CHUNK, q1 - 1, xr[1]);
    issue_fence();
    stage_store(st, xr[0], stage[0]);
    __syncthreads();
    const unsigned chunks = (q1 - q0 + CHUNK - 1) / CHUNK;
    const unsigned periods = (chunks + PERIOD - 1) / PERIOD;
    for (unsigned p = 0; p < periods; ++p) {
#pragma unroll
        for (int u = 0; u < PERIOD; ++u) {
            const unsigned q = q0 + (p * PERIOD + u) * CHUNK;
            stage_load(st, q + 2 * CHUNK, q1 - 1, xr[u % 2]);
            issue_fence();
            load_codes(q + CHUNK, wc[(u + 1) % 2]);
            if ((u + 1) * CHUNK % 4 == 0)
                load_scales(q + CHUNK, sc[((u + 1) * CHUNK / 4) % 2]);
            issue_fence();
            if (active) {
                const unsigned steps = q < q1 ? min(unsigned(CHUNK), q1 - q) : 0u;
#pragma unroll
                for (int s = 0; s < CHUNK; ++s) {
                    if (unsigned(s) >= steps)
                        continue;
                    const int qs = u * CHUNK + s;  // step within the period
                    float scale[2];
#pragma unroll
                    for (int m = 0; m < 2; ++m)
                        scale[m] = e8m0((sc[(qs / 4) % 2][m] >> (8 * (qs % 4))) & 0xffu);
                    const uint8_t* buf = stage[u % 2];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const bf16x8 b0 = dequant8(wc[u % 2][s][0][k], scale[0]);
                        const bf16x8 b1 = dequant8(wc[u % 2][s][1][k], scale[1]);
#pragma unroll
                        for (int t = 0; t < TILES; ++t) {
                            const uint8_t* rowp = buf + (t * kTileRows + i32) * S::pitch +
                                                  s * PLANES * 128 + (32 * h + 8 * k) * 2;
#pragma unroll
                            for (int pl = 0; pl < PLANES; ++pl) {
                                const bf16x8 a = lds_bf16x8(rowp + pl * 128);
                                acc[0][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                                    a, b0, acc[0][t], 0, 0, 0);
                                acc[1][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                                    a, b1, acc[1][t], 0, 0, 0);
                            }
                        }
                    }
                }
            }
            stage_store(st, xr[(u + 1) % 2], stage[(u + 1) % 2]);  // also past the end
            __syncthreads();
        }
    }
}

// Output row of accumulator element v in lane half h of tile t (32x32 MFMA layout).
__device__ __forceinline__ int acc_row(int t, int v, unsigned h) {
    return t * kTileRows + 8 * (v / 4) + 4 * int(h) + (v % 4);
}

// gate/up: grid (groups of 4 feature groups of 32, items, K slices).  Wavefront w
// multiplies gate and up rows of features 32 (4 x + w) .. +31.  One slice: h = silu(g) * u
// as bf16 hi + lo; more: fp32 partials of g and u (summed by finalize_kernel).
__global__ __launch_bounds__(kGemmWaves * 64) void gate_up_kernel(
    const uint16_t* x, unsigned hidden, unsigned inter, unsigned experts, unsigned top_k,
    const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ items, const int32_t* __restrict__ item_count,
    uint16_t* __restrict__ h_hi, uint16_t* __restrict__ h_lo, float* __restrict__ part_g,
    float* __restrict__ part_u, size_t part_stride) {
    constexpr int CHUNK = 2;
    __shared__ __align__(16) uint8_t stage[2][Stage<CHUNK, 1>::buffer];
    __shared__ long long src[kItemRows];
    if (int(blockIdx.y) >= *item_count)
        return;
    const Item it = load_item(items, offsets, blockIdx.y);
    const unsigned wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const unsigned i32 = lane % 32, h = lane / 32;
    const Packed shape = packed_shape(1, inter, hidden);  // per expert
    const unsigned fg = blockIdx.x * kGemmWaves + wave;   // feature group of 32
    const bool active = fg < shape.groups;                // uniform per wavefront
    const unsigned f = (active ? fg : 0) * 32 + i32;
    unsigned q0, q1;
    slice_steps(unsigned(shape.steps), gridDim.z, blockIdx.z, q0, q1);
    if (q0 >= q1)
        return;
    if (threadIdx.x < kItemRows) {
        const int r = int(threadIdx.x);
        src[r] = r < it.count ? (long long)(perm[it.segment + it.first + r] / int(top_k)) * hidden
                              : -1;
    }
    __syncthreads();
    const Packed whole = packed_shape(experts, inter, hidden);
    const size_t group = size_t(it.expert) * shape.groups + (active ? fg : 0);
    WavePair wg = wave_pair(gate, whole, group, group, lane);
    const WavePair wu = wave_pair(up, whole, group, group, lane);
    wg.codes[1] = wu.codes[0];
    wg.scales[1] = wu.scales[0];

    // straight-line code per tile count: no accumulator moves between control paths
    auto run = [&]<int TILES>() {
        const auto st = stage_thread<CHUNK, 1, TILES * kTileRows>(
            x, 0, [&](unsigned r) { return src[r]; });
        f32x16 acc[2][TILES];
        gemm_pair<CHUNK, 1, TILES>(st, wg, q0, q1, active, i32, h, stage, acc);
        if (!active)
            return;
        if (gridDim.z > 1) {
#pragma unroll
            for (int t = 0; t < TILES; ++t)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int r = acc_row(t, v, h);
                    if (r < it.count) {
                        const size_t at = blockIdx.z * part_stride +
                                          size_t(it.segment + it.first + r) * inter + f;
                        part_g[at] = acc[0][t][v];
                        part_u[at] = acc[1][t][v];
                    }
                }
            return;
        }
#pragma unroll
        for (int t = 0; t < TILES; ++t)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = acc_row(t, v, h);
                if (r < it.count) {
                    const float hv = silu(acc[0][t][v]) * acc[1][t][v];
                    const uint16_t hi = bf16_rne(hv);
                    const size_t at = size_t(it.segment + it.first + r) * inter + f;
                    h_hi[at] = hi;
                    h_lo[at] = bf16_rne(hv - bf16_value(hi));
                }
            }
    };
    if (it.count <= kTileRows)
        run.template operator()<1>();
    else
        run.template operator()<2>();
}

// h = silu(sum_s g_s) * (sum_s u_s), slices summed in order, as bf16 hi + lo.
__global__ __launch_bounds__(256) void finalize_kernel(const float* __restrict__ part_g,
                                                       const float* __restrict__ part_u,
                                                       size_t count, unsigned slices,
                                                       uint16_t* __restrict__ h_hi,
                                                       uint16_t* __restrict__ h_lo) {
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= count)
        return;
    float gs = 0.f, us = 0.f;
    for (unsigned s = 0; s < slices; ++s) {
        gs += part_g[s * count + i];
        us += part_u[s * count + i];
    }
    const float hv = silu(gs) * us;
    const uint16_t hi = bf16_rne(hv);
    h_hi[i] = hi;
    h_lo[i] = bf16_rne(hv - bf16_value(hi));
}

// down: grid (groups of 4 row pairs of 64, items, K slices); wavefront w multiplies the
// down rows 64 (4 x + w) .. +63 (two groups of 32).  fp32 partial sums of h x down (hi
// plane at h, lo plane at h + plane_stride) per slice, indexed by the slot's position in
// the permutation.
__global__ __launch_bounds__(kGemmWaves * 64) void down_kernel(
    const uint16_t* hp, size_t plane_stride, unsigned hidden, unsigned inter, unsigned experts,
    const uint8_t* __restrict__ down, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ items, const int32_t* __restrict__ item_count,
    float* __restrict__ part_d, size_t part_stride) {
    constexpr int CHUNK = 1;
    __shared__ __align__(16) uint8_t stage[2][Stage<CHUNK, 2>::buffer];
    if (int(blockIdx.y) >= *item_count)
        return;
    const Item it = load_item(items, offsets, blockIdx.y);
    const unsigned wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const unsigned i32 = lane % 32, h = lane / 32;
    const Packed shape = packed_shape(1, hidden, inter);  // per expert
    const unsigned pair = blockIdx.x * kGemmWaves + wave;
    const bool active = pair < shape.groups / 2;
    const unsigned g0 = (active ? pair : 0) * 2;
    unsigned q0, q1;
    slice_steps(unsigned(shape.steps), gridDim.z, blockIdx.z, q0, q1);
    if (q0 >= q1)
        return;
    const Packed whole = packed_shape(experts, hidden, inter);
    const size_t base = size_t(it.expert) * shape.groups + g0;
    const WavePair w = wave_pair(down, whole, base, base + 1, lane);
    auto row_offset = [&](unsigned r) {
        return r < unsigned(it.count) ? (long long)(it.segment + it.first + r) * inter : -1ll;
    };
    auto run = [&]<int TILES>() {
        const auto st = stage_thread<CHUNK, 2, TILES * kTileRows>(hp, plane_stride, row_offset);
        f32x16 acc[2][TILES];
        gemm_pair<CHUNK, 2, TILES>(st, w, q0, q1, active, i32, h, stage, acc);
        if (!active)
            return;
#pragma unroll
        for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int t = 0; t < TILES; ++t)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int r = acc_row(t, v, h);
                    if (r < it.count)
                        part_d[blockIdx.z * part_stride +
                               size_t(it.segment + it.first + r) * hidden + (g0 + m) * 32 + i32] =
                            acc[m][t][v];
                }
    };
    if (it.count <= kTileRows)
        run.template operator()<1>();
    else
        run.template operator()<2>();
}

// y[t, d] = sum_i w[t k + i] * (sum_s part_d[s, position(t k + i), d]), in selection order;
// one thread per 4 consecutive d.  Every load is issued before the sums (slot indices past
// top_k are clamped and their terms dropped), so the partials arrive together.
template <int SLICES>
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ part_d,
                                                      size_t part_stride, unsigned slices,
                                                      const int32_t* __restrict__ position,
                                                      const float* __restrict__ weight,
                                                      unsigned tokens, unsigned hidden,
                                                      unsigned top_k, float* __restrict__ y) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    const unsigned quads = hidden / 4;
    if (i >= size_t(tokens) * quads)
        return;
    const size_t t = i / quads, d = (i % quads) * 4;
    int pos[kMaxTopK];
    float wk[kMaxTopK];
#pragma unroll
    for (unsigned k = 0; k < kMaxTopK; ++k) {
        const size_t slot = t * top_k + min(k, top_k - 1);
        pos[k] = position[slot];
        wk[k] = weight[slot];
    }
    const unsigned ns = SLICES ? unsigned(SLICES) : slices;
    f32x4 down[kMaxTopK];
#pragma unroll
    for (unsigned k = 0; k < kMaxTopK; ++k)
        down[k] = *reinterpret_cast<const f32x4*>(part_d + size_t(pos[k]) * hidden + d);
    for (unsigned s = 1; s < ns; ++s)
#pragma unroll
        for (unsigned k = 0; k < kMaxTopK; ++k)
            down[k] += *reinterpret_cast<const f32x4*>(part_d + s * part_stride +
                                                       size_t(pos[k]) * hidden + d);
    f32x4 sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (unsigned k = 0; k < kMaxTopK; ++k)
        if (k < top_k)
            sum += down[k] * wk[k];
    *reinterpret_cast<f32x4*>(y + t * hidden + d) = sum;
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
    int32_t *idx, *offsets, *perm, *position, *items, *item_count;
    float* weight;
    uint16_t *h_hi, *h_lo;
    float *part_g, *part_u, *part_d;
};

// Grid columns of the grouped GEMMs: kGemmWaves feature groups of 32 (gate/up) or row
// pairs of 64 (down) per workgroup.
unsigned gate_up_columns(size_t inter) {
    return unsigned((inter / 32 + kGemmWaves - 1) / kGemmWaves);
}

unsigned down_columns(size_t hidden) {
    return unsigned((hidden / 64 + kGemmWaves - 1) / kGemmWaves);
}

// K slices of the grouped GEMMs: enough workgroups for about two per compute unit (two
// fit at once) when the items are few (decode), one slice otherwise; slices are whole
// multiples of 8 steps and none is empty.
struct MoeSlices {
    unsigned gate_up, down;
};

MoeSlices moe_slices(size_t tokens, size_t hidden, size_t inter, size_t experts,
                     size_t top_k) {
    const size_t items = std::min(tokens * top_k, experts);  // at least this many
    const size_t target = 2 * size_t(compute_units());
    auto slices = [&](size_t columns, size_t steps) {
        size_t ks = std::max<size_t>(1, (target + columns * items - 1) / (columns * items));
        ks = std::min(ks, steps);
        const size_t per = ((steps + ks - 1) / ks + 7) / 8 * 8;
        return unsigned((steps + per - 1) / per);
    };
    return MoeSlices{slices(gate_up_columns(inter), hidden / kStepK),
                     slices(down_columns(hidden), inter / kStepK)};
}

size_t align256(size_t n) {
    return (n + 255) & ~size_t(255);
}

size_t moe_scratch_bytes(size_t tokens, size_t hidden, size_t inter, size_t experts,
                         size_t top_k, MoeSlices ks) {
    const size_t slots = tokens * top_k, items = slots / kItemRows + experts + 1;
    const size_t partial_gu = ks.gate_up > 1 ? 2 * align256(ks.gate_up * slots * inter * 4) : 0;
    return align256(slots * 4) * 4 + align256((experts + 1) * 4) + align256(items * 8) +
           align256(4) + 2 * align256(slots * inter * 2) + partial_gu +
           align256(ks.down * slots * hidden * 4);
}

MoeScratch carve(uint8_t* p, size_t tokens, size_t hidden, size_t inter, size_t experts,
                 size_t top_k, MoeSlices ks) {
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
    s.position = reinterpret_cast<int32_t*>(take(slots * 4));
    s.offsets = reinterpret_cast<int32_t*>(take((experts + 1) * 4));
    s.items = reinterpret_cast<int32_t*>(take(items * 8));
    s.item_count = reinterpret_cast<int32_t*>(take(4));
    s.h_hi = reinterpret_cast<uint16_t*>(take(slots * inter * 2));
    s.h_lo = reinterpret_cast<uint16_t*>(take(slots * inter * 2));
    s.part_g = s.part_u = nullptr;
    if (ks.gate_up > 1) {
        s.part_g = reinterpret_cast<float*>(take(ks.gate_up * slots * inter * 4));
        s.part_u = reinterpret_cast<float*>(take(ks.gate_up * slots * inter * 4));
    }
    s.part_d = reinterpret_cast<float*>(take(ks.down * slots * hidden * 4));
    return s;
}

size_t packed_bytes(size_t experts, size_t rows, size_t cols) {
    const Packed p = packed_shape(experts, rows, cols);
    return p.code_bytes + p.scale_bytes;
}

int launch_pack(const uint8_t* blocks, const uint8_t* scales, size_t experts, size_t rows,
                size_t cols, uint8_t* packed, hipStream_t stream) {
    const Packed p = packed_shape(experts, rows, cols);
    const size_t units = p.code_bytes / 16, words = p.scale_bytes / 4;
    hipLaunchKernelGGL(pack_codes_kernel, dim3(unsigned((units + 255) / 256)), dim3(256), 0,
                       stream, blocks, units, p.steps, cols, packed);
    KDQ_HIP(hipGetLastError());
    hipLaunchKernelGGL(pack_scales_kernel, dim3(unsigned((words + 255) / 256)), dim3(256), 0,
                       stream, scales, words, p.scale_groups, p.steps, cols,
                       reinterpret_cast<unsigned*>(packed + p.code_bytes));
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}

int check_pack(const uint8_t* blocks, const uint8_t* scales, size_t experts, size_t rows,
               size_t cols, const uint8_t* packed) {
    if (!blocks || !scales || !packed || !experts || !rows || !cols)
        return KDQ_ERR_ARGUMENT;
    if (rows % 32 || cols % 64 || experts > kMaxExperts || rows > (1u << 20) ||
        cols > (1u << 20))
        return KDQ_ERR_SHAPE;
    if (misaligned(blocks, 16) || misaligned(packed, 256))
        return KDQ_ERR_ALIGNMENT;
    const size_t bytes = packed_bytes(experts, rows, cols);
    if (overlaps(packed, bytes, blocks, experts * rows * cols / 2) ||
        overlaps(packed, bytes, scales, experts * rows * cols / 32))
        return KDQ_ERR_ALIAS;
    return KDQ_OK;
}

int check_route(const float* logits, size_t tokens, size_t experts, size_t top_k) {
    if (!logits || !tokens || !experts || !top_k)
        return KDQ_ERR_ARGUMENT;
    if (experts > kMaxExperts || top_k > kMaxTopK || top_k > experts || tokens > (1u << 24) ||
        tokens * top_k > (size_t(1) << 26))
        return KDQ_ERR_SHAPE;
    return KDQ_OK;
}

int launch_route(const float* logits, size_t tokens, size_t experts, size_t top_k,
                 int32_t* idx, float* w, int32_t* offsets, int32_t* perm, int32_t* items,
                 int32_t* item_count, int32_t* position, hipStream_t stream) {
    hipLaunchKernelGGL(route_kernel, dim3(unsigned((tokens + 3) / 4)), dim3(256), 0, stream,
                       logits, unsigned(tokens), unsigned(experts), unsigned(top_k), idx, w);
    KDQ_HIP(hipGetLastError());
    hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(1024), 0, stream, idx,
                       unsigned(tokens * top_k), unsigned(experts), offsets, perm, items,
                       item_count, position);
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
                        scratch + items * 2, nullptr, static_cast<hipStream_t>(stream));
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

namespace kdq {
namespace {

int check_layer(const uint16_t* x_bf16, const float* logits, size_t tokens, size_t hidden,
                size_t inter, size_t experts, size_t top_k, float* y) {
    int rc = check_route(logits, tokens, experts, top_k);
    if (rc)
        return rc;
    if (!x_bf16 || !y || !hidden || !inter)
        return KDQ_ERR_ARGUMENT;
    if (hidden % 64 || inter % 64 || hidden > (1u << 20) || inter > (1u << 20))
        return KDQ_ERR_SHAPE;
    if (misaligned(x_bf16, 16) || misaligned(y, 16))
        return KDQ_ERR_ALIGNMENT;
    if (overlaps(y, tokens * hidden * 4, x_bf16, tokens * hidden * 2) ||
        overlaps(y, tokens * hidden * 4, logits, tokens * experts * 4))
        return KDQ_ERR_ALIAS;
    return KDQ_OK;
}

// The layer over packed weights; `scratch` holds moe_scratch_bytes(...).
int launch_layer(const uint16_t* x_bf16, const float* logits, size_t tokens, size_t hidden,
                 size_t inter, size_t experts, size_t top_k, const uint8_t* gate,
                 const uint8_t* up, const uint8_t* down, float* y, int32_t* idx, float* w,
                 int32_t* offsets, int32_t* perm, uint8_t* scratch, MoeSlices ks,
                 hipStream_t st) {
    MoeScratch s = carve(scratch, tokens, hidden, inter, experts, top_k, ks);
    if (idx)
        s.idx = idx;
    if (w)
        s.weight = w;
    if (offsets)
        s.offsets = offsets;
    if (perm)
        s.perm = perm;
    int rc = launch_route(logits, tokens, experts, top_k, s.idx, s.weight, s.offsets, s.perm,
                          s.items, s.item_count, s.position, st);
    if (rc)
        return rc;
    const size_t slots = tokens * top_k;
    const unsigned max_items = unsigned(std::min(slots, slots / kItemRows + experts + 1));
    hipLaunchKernelGGL(gate_up_kernel, dim3(gate_up_columns(inter), max_items, ks.gate_up),
                       dim3(kGemmWaves * 64), 0, st, x_bf16, unsigned(hidden), unsigned(inter),
                       unsigned(experts), unsigned(top_k), gate, up, s.offsets, s.perm, s.items, s.item_count,
                       s.h_hi, s.h_lo, s.part_g, s.part_u, slots * inter);
    KDQ_HIP(hipGetLastError());
    if (ks.gate_up > 1) {
        const size_t n = slots * inter;
        hipLaunchKernelGGL(finalize_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st,
                           s.part_g, s.part_u, n, ks.gate_up, s.h_hi, s.h_lo);
        KDQ_HIP(hipGetLastError());
    }
    hipLaunchKernelGGL(down_kernel, dim3(down_columns(hidden), max_items, ks.down),
                       dim3(kGemmWaves * 64), 0, st, s.h_hi, size_t(s.h_lo - s.h_hi),
                       unsigned(hidden), unsigned(inter), unsigned(experts), down, s.offsets,
                       s.items, s.item_count, s.part_d, slots * hidden);
    KDQ_HIP(hipGetLastError());
    const size_t n = tokens * hidden / 4;
    const dim3 grid(unsigned((n + 255) / 256));
    const size_t stride = slots * hidden;
    if (ks.down == 1)
        hipLaunchKernelGGL(combine_kernel<1>, grid, dim3(256), 0, st, s.part_d, stride, 1u,
                           s.position, s.weight, unsigned(tokens), unsigned(hidden),
                           unsigned(top_k), y);
    else if (ks.down == 2)
        hipLaunchKernelGGL(combine_kernel<2>, grid, dim3(256), 0, st, s.part_d, stride, 2u,
                           s.position, s.weight, unsigned(tokens), unsigned(hidden),
                           unsigned(top_k), y);
    else
        hipLaunchKernelGGL(combine_kernel<0>, grid, dim3(256), 0, st, s.part_d, stride, ks.down,
                           s.position, s.weight, unsigned(tokens), unsigned(hidden),
                           unsigned(top_k), y);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}

}  // namespace
}  // namespace kdq

extern "C" size_t kdq_moe_mxfp4_packed_bytes(size_t experts, size_t rows, size_t cols) {
    if (!experts || !rows || !cols || rows % 32 || cols % 64)
        return 0;
    return packed_bytes(experts, rows, cols);
}

extern "C" int kdq_moe_mxfp4_pack(const uint8_t* blocks, const uint8_t* scales, size_t experts,
                                  size_t rows, size_t cols, uint8_t* packed, void* stream) {
    const int rc = check_pack(blocks, scales, experts, rows, cols, packed);
    if (rc)
        return rc;
    return launch_pack(blocks, scales, experts, rows, cols, packed,
                       static_cast<hipStream_t>(stream));
}

extern "C" int kdq_moe_mxfp4_packed(const uint16_t* x_bf16, const float* logits, size_t tokens,
                                    size_t hidden, size_t inter, size_t experts, size_t top_k,
                                    const uint8_t* gate, const uint8_t* up, const uint8_t* down,
                                    float* y, int32_t* idx, float* w, int32_t* offsets,
                                    int32_t* perm, void* stream) {
    int rc = check_layer(x_bf16, logits, tokens, hidden, inter, experts, top_k, y);
    if (rc)
        return rc;
    if (!gate || !up || !down)
        return KDQ_ERR_ARGUMENT;
    if (misaligned(gate, 256) || misaligned(up, 256) || misaligned(down, 256))
        return KDQ_ERR_ALIGNMENT;
    const MoeSlices ks = moe_slices(tokens, hidden, inter, experts, top_k);
    auto* scratch = static_cast<uint8_t*>(
        workspace(moe_scratch_bytes(tokens, hidden, inter, experts, top_k, ks), &rc));
    if (rc)
        return rc;
    return launch_layer(x_bf16, logits, tokens, hidden, inter, experts, top_k, gate, up, down,
                        y, idx, w, offsets, perm, scratch, ks, static_cast<hipStream_t>(stream));
}

// Reference-layout weights: packed into the workspace on every call, then the layer.
extern "C" int kdq_moe_mxfp4(const uint16_t* x_bf16, const float* logits, size_t tokens,
                             size_t hidden, size_t inter, size_t experts, size_t top_k,
                             const uint8_t* gate_blocks, const uint8_t* gate_scales,
                             const uint8_t* up_blocks, const uint8_t* up_scales,
                             const uint8_t* down_blocks, const uint8_t* down_scales, float* y,
                             int32_t* idx, float* w, int32_t* offsets, int32_t* perm,
                             void* stream) {
    int rc = check_layer(x_bf16, logits, tokens, hidden, inter, experts, top_k, y);
    if (rc)
        return rc;
    if (!gate_blocks || !gate_scales || !up_blocks || !up_scales || !down_blocks ||
        !down_scales)
        return KDQ_ERR_ARGUMENT;
    if (misaligned(gate_blocks, 16) || misaligned(up_blocks, 16) || misaligned(down_blocks, 16))
        return KDQ_ERR_ALIGNMENT;
    const size_t gu = align256(packed_bytes(experts, inter, hidden));
    const size_t dn = align256(packed_bytes(experts, hidden, inter));
    const MoeSlices ks = moe_slices(tokens, hidden, inter, experts, top_k);
    auto* base = static_cast<uint8_t*>(
        workspace(2 * gu + dn + moe_scratch_bytes(tokens, hidden, inter, experts, top_k, ks), &rc));
    if (rc)
        return rc;
    auto st = static_cast<hipStream_t>(stream);
    uint8_t *gate = base, *up = base + gu, *down = base + 2 * gu;
    if ((rc = launch_pack(gate_blocks, gate_scales, experts, inter, hidden, gate, st)) ||
        (rc = launch_pack(up_blocks, up_scales, experts, inter, hidden, up, st)) ||
        (rc = launch_pack(down_blocks, down_scales, experts, hidden, inter, down, st)))
        return rc;
    return launch_layer(x_bf16, logits, tokens, hidden, inter, experts, top_k, gate, up, down,
                        y, idx, w, offsets, perm, base + 2 * gu + dn, ks, st);
}
