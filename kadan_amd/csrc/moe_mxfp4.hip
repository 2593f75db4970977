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
constexpr int kGemmWaves = 8;  // wavefronts per grouped-GEMM workgroup, 32 weight rows each
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

// Grouped GEMMs on v_mfma_f32_32x32x16_bf16.  A workgroup of kGemmWaves wavefronts works
// on one work item (expert e, up to kItemRows consecutive rows of its segment: one or two
// MFMA row tiles of 32) and one K slice; every wavefront owns 32 weight rows.  The weight
// operand B streams from HBM: lane (f = lane % 32, g = lane / 32) loads per 64-value step
// the 16 bytes (32 FP4 values) k = 64q + 32g .. +31 of its row and their E8M0 scale, and
// MFMA t takes values 32g + 8t .. +7 of them (the activation operand uses the same k
// order), dequantized with v_cvt_scalef32_pk_bf16_fp4, which is exact.  The activation
// operand A (the item's occupied row tiles) is staged per chunk of steps into LDS by the
// whole workgroup, double-buffered; one staged chunk serves all 8 wavefronts (256 weight
// rows).  Every lane issues chunk c + 2's activation loads, then its weight loads, while
// chunk c is multiplied and chunk c + 1 is stored to LDS; all loads are unconditional
// (indices past the end are clamped to valid data), so each wait counts exactly the loads
// the next step needs and the weight loads stay in flight across the chunk barrier.

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
    static constexpr int per_thread = (ROWS * S::pieces + threads - 1) / threads;
    static constexpr int rows_step = threads / S::pieces;
    const uint16_t* src[per_thread];  // row start in its plane (always a valid row)
    bool valid[per_thread];           // the row exists (else it is stored as zeros)
    bool stores[per_thread];          // the piece lies inside the ROWS staged rows
    unsigned step, plane, sub;
};

// `row_offset(p, r)` is the element offset of row r in plane p, or -1 past the item.
template <int CHUNK, int PLANES, int ROWS, class RowOffset>
__device__ __forceinline__ StageThread<CHUNK, PLANES, ROWS> stage_thread(
    const uint16_t* const (&planes)[PLANES], RowOffset row_offset) {
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
        const long long at = row < unsigned(ROWS) ? row_offset(t.plane, row) : -1;
        t.stores[i] = row < unsigned(ROWS);
        t.valid[i] = at >= 0;
        t.src[i] = planes[t.plane] + (at >= 0 ? at : row_offset(t.plane, 0));
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

template <int CHUNK, int PLANES, int ROWS>
__device__ __forceinline__ void stage_store(const StageThread<CHUNK, PLANES, ROWS>& t,
                                            const StagePieces<CHUNK, PLANES, ROWS>& P,
                                            unsigned steps, uint8_t* buf) {
    using T = StageThread<CHUNK, PLANES, ROWS>;
    using S = Stage<CHUNK, PLANES>;
    if (t.step >= steps)
        return;
#pragma unroll
    for (int i = 0; i < T::per_thread; ++i) {
        const unsigned row = threadIdx.x / S::pieces + i * T::rows_step;
        if (t.stores[i])
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

// Packed weights of one lane for one step (16 FP4 bytes and their scale).
struct WStep {
    u32x4 codes;
    unsigned scale;
};

__device__ __forceinline__ WStep load_wstep(const uint8_t* row, const uint8_t* srow, unsigned q,
                                            unsigned g) {
    WStep w;
    w.codes = load16(row + size_t(q) * 32 + 16 * g);
    w.scale = srow[size_t(q) * 2 + g];
    return w;
}

// Steps of K slice `slice` of `steps` total: [begin, end).
__device__ __forceinline__ void slice_steps(unsigned steps, unsigned slices, unsigned slice,
                                            unsigned& begin, unsigned& end) {
    const unsigned per = (steps + slices - 1) / slices;
    begin = min(steps, slice * per);
    end = min(steps, begin + per);
}

// One step of MFMAs for one weight matrix: acc[m] += A(tile m, step s) * B(step).
template <int PLANES, int TILES>
__device__ __forceinline__ void step_mfma(const WStep& w, const uint8_t* buf, int pitch, int s,
                                          unsigned i32, unsigned g, f32x16 (&acc)[TILES]) {
    const float scale = e8m0(w.scale);
    const unsigned c[4] = {w.codes.x, w.codes.y, w.codes.z, w.codes.w};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const bf16x8 b = dequant8(c[t], scale);
#pragma unroll
        for (int m = 0; m < TILES; ++m) {
            const uint8_t* rowp = buf + (m * kTileRows + i32) * pitch + s * PLANES * 128 +
                                  (32 * g + 8 * t) * 2;
#pragma unroll
            for (int p = 0; p < PLANES; ++p)
                acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lds_bf16x8(rowp + p * 128), b,
                                                                 acc[m], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);  // one MFMA group's operands live at a time
    }
}

__device__ __forceinline__ void issue_fence() {
    asm volatile("" ::: "memory");  // keeps the load issue order (activation pointers are
    __builtin_amdgcn_sched_barrier(0);  // not restrict)
}

// The K loop shared by both GEMMs: acc += A(rows, [q0, q1)) * B(rows w of one matrix).
// Activations run two chunks ahead of the MFMAs, weights WDEPTH - 1 chunks ahead; a
// chunk's weight loads for one lane are consecutive 16-byte pieces of its row, issued
// back to back so each 128-byte line is requested once.
template <int CHUNK, int PLANES, int TILES, int WDEPTH>
__device__ __forceinline__ void gemm_loop(const StageThread<CHUNK, PLANES, TILES * kTileRows>& st,
                                          const uint8_t* wb, const uint8_t* ws, unsigned q0,
                                          unsigned q1, bool active, unsigned i32, unsigned g,
                                          uint8_t (&stage)[2][Stage<CHUNK, PLANES>::buffer],
                                          f32x16 (&acc)[TILES]) {
    static_assert(WDEPTH == 2 || WDEPTH == 3, "weight ring");
    using S = Stage<CHUNK, PLANES>;
    constexpr int ROWS = TILES * kTileRows;
    auto load_w = [&](unsigned q, WStep(&w)[CHUNK]) {
#pragma unroll
        for (int s = 0; s < CHUNK; ++s)
            w[s] = load_wstep(wb, ws, min(q + s, q1 - 1), g);
    };
#pragma unroll
    for (int m = 0; m < TILES; ++m)
        acc[m] = f32x16{};
    StagePieces<CHUNK, PLANES, ROWS> pa, pb;
    WStep wa[CHUNK], wm[CHUNK], wn[CHUNK];
    stage_load(st, q0, q1 - 1, pa);
    issue_fence();
    load_w(q0, wa);
    issue_fence();
    stage_load(st, q0 + CHUNK, q1 - 1, pb);
    issue_fence();
    if constexpr (WDEPTH == 3) {
        load_w(q0 + CHUNK, wm);
        issue_fence();
    }
    stage_store(st, pa, min(unsigned(CHUNK), q1 - q0), stage[0]);
    __syncthreads();
    pa = pb;
    unsigned buf = 0;
    for (unsigned q = q0; q < q1; q += CHUNK, buf ^= 1) {
        const unsigned steps = min(unsigned(CHUNK), q1 - q), qn = q + CHUNK;
        stage_load(st, qn + CHUNK, q1 - 1, pb);
        issue_fence();
        if constexpr (WDEPTH == 3)
            load_w(qn + CHUNK, wn);
        else
            load_w(qn, wm);
        issue_fence();
        if (active) {
#pragma unroll
            for (int s = 0; s < CHUNK; ++s)
                if (unsigned(s) < steps)
                    step_mfma<PLANES, TILES>(wa[s], stage[buf], S::pitch, s, i32, g, acc);
        }
        if (qn < q1)
            stage_store(st, pa, min(unsigned(CHUNK), q1 - qn), stage[buf ^ 1]);
        __syncthreads();
#pragma unroll
        for (int s = 0; s < CHUNK; ++s) {
            wa[s] = wm[s];
            if constexpr (WDEPTH == 3)
                wm[s] = wn[s];
        }
        pa = pb;
    }
}

// gate/up: grid (feature groups of 128, items, K slices).  Wavefront w multiplies the gate
// (w even) or up (w odd) rows of features n0 + 32 (w / 2) .. +31.  One slice: h =
// silu(g) * u as bf16 hi + lo (g passes through LDS); more: fp32 partials of g and u
// (summed by finalize_kernel).
__global__ __launch_bounds__(kGemmWaves * 64) void gate_up_kernel(
    const uint16_t* x, unsigned hidden, unsigned inter, unsigned top_k,
    const uint8_t* __restrict__ gate_blocks, const uint8_t* __restrict__ gate_scales,
    const uint8_t* __restrict__ up_blocks, const uint8_t* __restrict__ up_scales,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ perm,
    const int32_t* __restrict__ items, const int32_t* __restrict__ item_count,
    uint16_t* __restrict__ h_hi, uint16_t* __restrict__ h_lo, float* __restrict__ part_g,
    float* __restrict__ part_u, size_t part_stride) {
    constexpr int CHUNK = 2;
    using S = Stage<CHUNK, 1>;
    static_assert(2 * S::buffer >= (kGemmWaves / 2) * kTiles * 16 * 64 * 4, "gate exchange");
    __shared__ __align__(16) uint8_t stage[2][S::buffer];
    __shared__ long long src[kItemRows];
    if (int(blockIdx.y) >= *item_count)
        return;
    const Item it = load_item(items, offsets, blockIdx.y);
    const unsigned wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const unsigned i32 = lane % 32, g = lane / 32;
    const unsigned mat = wave % 2, tile = wave / 2;
    const unsigned f0 = blockIdx.x * (kGemmWaves / 2) * 32 + tile * 32;
    const bool active = f0 < inter;  // uniform per wavefront
    const unsigned f = active ? f0 + i32 : i32;
    unsigned q0, q1;
    slice_steps(hidden / kStepK, gridDim.z, blockIdx.z, q0, q1);
    if (q0 >= q1)
        return;
    if (threadIdx.x < kItemRows) {
        const int r = int(threadIdx.x);
        src[r] = r < it.count ? (long long)(perm[it.segment + it.first + r] / int(top_k)) * hidden
                              : -1;
    }
    __syncthreads();
    const size_t wrow = size_t(it.expert) * inter + f;
    const uint8_t* wb = (mat ? up_blocks : gate_blocks) + wrow * (hidden / 2);
    const uint8_t* ws = (mat ? up_scales : gate_scales) + wrow * (hidden / 32);
    const uint16_t* planes[1] = {x};

    // straight-line code per tile count: no accumulator moves between control paths
    auto run = [&]<int TILES>() {
        const auto st = stage_thread<CHUNK, 1, TILES * kTileRows>(
            planes, [&](unsigned, unsigned r) { return src[r]; });
        f32x16 acc[TILES];
        gemm_loop<CHUNK, 1, TILES, 3>(st, wb, ws, q0, q1, active, i32, g, stage, acc);
        if (gridDim.z > 1) {
            if (!active)
                return;
            float* part = (mat ? part_u : part_g) + blockIdx.z * part_stride;
#pragma unroll
            for (int m = 0; m < TILES; ++m)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int r = m * kTileRows + 8 * (v / 4) + 4 * int(g) + (v % 4);
                    if (r < it.count)
                        part[size_t(it.segment + it.first + r) * inter + f] = acc[m][v];
                }
            return;
        }
        // the gate values of feature tile `tile` pass to its up wavefront through LDS (the
        // stage buffers are free after the last barrier): xg[tile][m][v][lane]
        float* xg = reinterpret_cast<float*>(&stage[0][0]);
        if (mat == 0 && active)
#pragma unroll
            for (int m = 0; m < TILES; ++m)
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    xg[((tile * kTiles + m) * 16 + v) * 64 + lane] = acc[m][v];
        __syncthreads();
        if (mat == 0 || !active)
            return;
#pragma unroll
        for (int m = 0; m < TILES; ++m)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = m * kTileRows + 8 * (v / 4) + 4 * int(g) + (v % 4);
                if (r < it.count) {
                    const float gv = xg[((tile * kTiles + m) * 16 + v) * 64 + lane];
                    const float h = silu(gv) * acc[m][v];
                    const uint16_t hi = bf16_rne(h);
                    const size_t at = size_t(it.segment + it.first + r) * inter + f;
                    h_hi[at] = hi;
                    h_lo[at] = bf16_rne(h - bf16_value(hi));
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
    const float h = silu(gs) * us;
    const uint16_t hi = bf16_rne(h);
    h_hi[i] = hi;
    h_lo[i] = bf16_rne(h - bf16_value(hi));
}

// down: grid (feature groups of 256, items, K slices); fp32 partial sums of h x down
// (hi and lo planes) per slice, indexed by the slot's position in the permutation.
__global__ __launch_bounds__(kGemmWaves * 64) void down_kernel(
    const uint16_t* h_hi, const uint16_t* h_lo, unsigned hidden, unsigned inter,
    const uint8_t* __restrict__ down_blocks, const uint8_t* __restrict__ down_scales,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ items,
    const int32_t* __restrict__ item_count, float* __restrict__ part_d, size_t part_stride) {
    constexpr int CHUNK = 1;
    __shared__ __align__(16) uint8_t stage[2][Stage<CHUNK, 2>::buffer];
    if (int(blockIdx.y) >= *item_count)
        return;
    const Item it = load_item(items, offsets, blockIdx.y);
    const unsigned wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const unsigned i32 = lane % 32, g = lane / 32;
    const unsigned d0 = (blockIdx.x * kGemmWaves + wave) * 32;
    const bool active = d0 < hidden;
    const unsigned d = active ? d0 + i32 : i32;
    unsigned q0, q1;
    slice_steps(inter / kStepK, gridDim.z, blockIdx.z, q0, q1);
    if (q0 >= q1)
        return;
    const size_t wrow = size_t(it.expert) * hidden + d;
    const uint8_t* db = down_blocks + wrow * (inter / 2);
    const uint8_t* ds = down_scales + wrow * (inter / 32);
    const uint16_t* planes[2] = {h_hi, h_lo};
    auto row_offset = [&](unsigned, unsigned r) {
        return r < unsigned(it.count) ? (long long)(it.segment + it.first + r) * inter : -1ll;
    };
    auto run = [&]<int TILES>() {
        const auto st = stage_thread<CHUNK, 2, TILES * kTileRows>(planes, row_offset);
        f32x16 acc[TILES];
        gemm_loop<CHUNK, 2, TILES, 3>(st, db, ds, q0, q1, active, i32, g, stage, acc);
        if (!active)
            return;
#pragma unroll
        for (int m = 0; m < TILES; ++m)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = m * kTileRows + 8 * (v / 4) + 4 * int(g) + (v % 4);
                if (r < it.count)
                    part_d[blockIdx.z * part_stride +
                           size_t(it.segment + it.first + r) * hidden + d] = acc[m][v];
            }
    };
    if (it.count <= kTileRows)
        run.template operator()<1>();
    else
        run.template operator()<2>();
}

// y[t, d] = sum_i w[t k + i] * (sum_s part_d[s, position(t k + i), d]), in selection order.
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ part_d,
                                                      size_t part_stride, unsigned slices,
                                                      const int32_t* __restrict__ position,
                                                      const float* __restrict__ weight,
                                                      unsigned tokens, unsigned hidden,
                                                      unsigned top_k, float* __restrict__ y) {
    const size_t i = size_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= size_t(tokens) * hidden)
        return;
    const size_t t = i / hidden, d = i % hidden;
    float sum = 0.f;
    for (unsigned k = 0; k < top_k; ++k) {
        const size_t slot = t * top_k + k;
        const size_t at = size_t(position[slot]) * hidden + d;
        float down = 0.f;
        for (unsigned s = 0; s < slices; ++s)
            down += part_d[s * part_stride + at];
        sum += down * weight[slot];
    }
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
    int32_t *idx, *offsets, *perm, *position, *items, *item_count;
    float* weight;
    uint16_t *h_hi, *h_lo;
    float *part_g, *part_u, *part_d;
};

// K slices of the grouped GEMMs: enough workgroups for about two per compute unit when
// the items are few (decode), one slice otherwise; no slice is empty.
struct MoeSlices {
    unsigned gate_up, down;
};

MoeSlices moe_slices(size_t tokens, size_t hidden, size_t inter, size_t experts,
                     size_t top_k) {
    const size_t items = std::min(tokens * top_k, experts);  // at least this many
    const size_t target = 2 * size_t(compute_units());
    auto slices = [&](size_t groups, size_t steps) {
        size_t ks = std::max<size_t>(1, (target + groups * items - 1) / (groups * items));
        ks = std::min(ks, steps);
        const size_t per = (steps + ks - 1) / ks;
        return unsigned((steps + per - 1) / per);
    };
    return MoeSlices{slices((inter / 32 + kGemmWaves / 2 - 1) / (kGemmWaves / 2), hidden / kStepK),
                     slices((hidden / 32 + kGemmWaves - 1) / kGemmWaves, inter / kStepK)};
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
    const MoeSlices ks = moe_slices(tokens, hidden, inter, experts, top_k);
    const size_t bytes = moe_scratch_bytes(tokens, hidden, inter, experts, top_k, ks);
    auto* base = static_cast<uint8_t*>(workspace(bytes, &rc));
    if (rc)
        return rc;
    MoeScratch s = carve(base, tokens, hidden, inter, experts, top_k, ks);
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
                      s.items, s.item_count, s.position, st);
    if (rc)
        return rc;
    const size_t slots = tokens * top_k;
    const unsigned max_items = unsigned(std::min(slots, slots / kItemRows + experts + 1));
    const unsigned groups_gu = unsigned((inter / 32 + kGemmWaves / 2 - 1) / (kGemmWaves / 2));
    const unsigned groups_d = unsigned((hidden / 32 + kGemmWaves - 1) / kGemmWaves);
    hipLaunchKernelGGL(gate_up_kernel, dim3(groups_gu, max_items, ks.gate_up),
                       dim3(kGemmWaves * 64), 0, st, x_bf16, unsigned(hidden), unsigned(inter),
                       unsigned(top_k), gate_blocks, gate_scales, up_blocks, up_scales,
                       s.offsets, s.perm, s.items, s.item_count, s.h_hi, s.h_lo, s.part_g,
                       s.part_u, slots * inter);
    KDQ_HIP(hipGetLastError());
    if (ks.gate_up > 1) {
        const size_t n = slots * inter;
        hipLaunchKernelGGL(finalize_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st,
                           s.part_g, s.part_u, n, ks.gate_up, s.h_hi, s.h_lo);
        KDQ_HIP(hipGetLastError());
    }
    hipLaunchKernelGGL(down_kernel, dim3(groups_d, max_items, ks.down), dim3(kGemmWaves * 64),
                       0, st, s.h_hi, s.h_lo, unsigned(hidden), unsigned(inter), down_blocks,
                       down_scales, s.offsets, s.items, s.item_count, s.part_d,
                       slots * hidden);
    KDQ_HIP(hipGetLastError());
    const size_t n = tokens * hidden;
    hipLaunchKernelGGL(combine_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, st,
                       s.part_d, slots * hidden, ks.down, s.position, s.weight,
                       unsigned(tokens), unsigned(hidden), unsigned(top_k), y);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}
