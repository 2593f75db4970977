// MXFP4 mixture-of-experts layer for gfx950.  The reference has no device MoE: this
// composes MoeLayer::forward (IW/src/models/text/qwen_layers.cpp:378-492; IW =
// services/hikari/inference_worker) with the MXFP4 product semantics of
// IW/src/weights/quantization.cpp:79-99,207-247, behind include/kadan_amd.h.
//
//   route_kernel      one wavefront per token: softmax (float exp, double total),
//                     top-k in std::partial_sort's order, renormalise;
//                     the token's activations as FP8 terms with E8M0 block scales
//   route_wg_kernel   the same selection, one workgroup per token (few tokens)
//   permute_kernel    one workgroup: stable counting sort of the slots by expert
//                     (expert-major, slot ascending) plus the list of work items
//                     (expert, first row) of at most kItemRows rows each
//   chunk_count_kernel, chunk_place_kernel  the same sort for more slots, one workgroup
//                     per 1024 slots: ranks and counts per chunk, then the placement
//   gate_up_kernel    grouped GEMM over work items on the scaled MFMA
//                     (v_mfma_scale_f32_32x32x64_f8f6f4): FP8 activation terms x the packed
//                     FP4 gate and up rows with their E8M0 scales, fp32 accumulation, fused
//                     h = silu(g) * u stored as FP8 terms for the down product
//   gather_kernel     x gathered by the permutation into per-item activation tiles as FP8
//                     terms (the grouped GEMMs' A operand, 1 KB contiguous per load)
//   prologue_kernel   small layers: route + permute + gather in one workgroup
//   finalize_kernel   (K-sliced layers only) slices summed in order, then h as FP8 terms
//   down_kernel       grouped GEMM h x FP4 down rows, fp32 partial rows per slot
//   combine_kernel    y[t] = sum_i w[t*k + i] * down[t*k + i] in selection order (float)
#include "kdq_common.hpp"

#include <cmath>
#include <mutex>
#include <utility>

namespace kdq {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kMaxTopK = 8, kMaxExperts = 256;
constexpr int kTileRows = 32, kTiles = 2, kItemRows = kTileRows * kTiles;
constexpr int kGemmWaves = 4;  // wavefronts per gate/up workgroup, 64 weight rows each
constexpr int kDownWaves = 8;  // wavefronts per down workgroup (two per SIMD share a staging)
constexpr int kStepK = 64;     // K values per step: 16 FP4 bytes per lane
constexpr int kPrologueSlots = 64;  // layers of at most this many slots use prologue_kernel
}  // namespace
// Bytes of kdq_moe_mxfp4_packed_noalloc's static scratch (64 MiB: C4 geometry up to 128
// tokens, 128 experts up to 16 tokens).
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
namespace {

// ------------------------------------------------------------------ routing

#include "kdq_route.hpp"

// Token t by one whole wavefront: its selection stored to idx / weight (and lds_idx).
__device__ __forceinline__ void route_token(const float* __restrict__ logits, unsigned t,
                                            unsigned experts, unsigned top_k,
                                            int32_t* __restrict__ idx, float* __restrict__ weight,
                                            unsigned lane, int* lds_idx = nullptr) {
    int e;
    float we;
    route_select(logits, t, experts, top_k, lane, e, we);
    if (lane < top_k) {
        idx[size_t(t) * top_k + lane] = e;
        weight[size_t(t) * top_k + lane] = we;
        if (lds_idx)
            lds_idx[t * top_k + lane] = e;
    }
}

__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits,
                                                    unsigned tokens, unsigned experts,
                                                    unsigned top_k, int32_t* __restrict__ idx,
                                                    float* __restrict__ weight) {
    const unsigned t = blockIdx.x * 4 + threadIdx.x / 64;
    if (t < tokens)
        route_token(logits, t, experts, top_k, idx, weight, threadIdx.x % 64);
}

// Token blockIdx.x by a whole workgroup of 256 threads (route_select_wg): the same
// selection as route_kernel's in a fraction of its latency, for a few tokens.
__global__ __launch_bounds__(256) void route_wg_kernel(const float* __restrict__ logits,
                                                       unsigned experts, unsigned top_k,
                                                       int32_t* __restrict__ idx,
                                                       float* __restrict__ weight) {
    __shared__ __align__(16) RouteScratch scratch;
    const unsigned t = blockIdx.x;
    int e = 0;
    float we = 0.f;
    route_select_wg<4, kMaxTopK, false>(logits + size_t(t) * experts, experts, top_k, scratch,
                                        e, we);
    if (threadIdx.x < top_k) {
        idx[size_t(t) * top_k + threadIdx.x] = e;
        weight[size_t(t) * top_k + threadIdx.x] = we;
    }
}

// Up to this many tokens one workgroup routes each token (route_wg_kernel), past it one
// wavefront (route_kernel).
constexpr size_t kRouteWgTokens = 64;

void launch_route_selection(const float* logits, size_t tokens, size_t experts,
                            size_t top_k, int32_t* idx, float* w, hipStream_t stream) {
    if (tokens <= kRouteWgTokens)
        hipLaunchKernelGGL(route_wg_kernel, dim3(unsigned(tokens)), dim3(256), 0, stream,
                           logits, unsigned(experts), unsigned(top_k), idx, w);
    else
        hipLaunchKernelGGL(route_kernel, dim3(unsigned((tokens + 3) / 4)), dim3(256), 0,
                           stream, logits, unsigned(tokens), unsigned(experts),
                           unsigned(top_k), idx, w);
}

// The experts' layout for a permutation, in LDS: per expert its slot count, its first
// position (segment), and the first numbers of its heavy and light work items.
struct ExpertLayout {
    int counts[kMaxExperts], segment[kMaxExperts], heavy_base[kMaxExperts],
        light_base[kMaxExperts];
    int heavy_total;
};

// Wavefront 0, counts filled: exclusive prefix sums over the experts of their slots and
// of their heavy and light work items (ceil(count / kItemRows) items, the last one light
// when it has at most kTileRows rows); lane l takes experts 4l .. 4l + 3.  offsets
// [experts + 1] and *item_count are written when given.
__device__ __forceinline__ void expert_layout(ExpertLayout& L, unsigned experts,
                                              bool heavy_first, unsigned lane,
                                              int32_t* __restrict__ offsets,
                                              int32_t* __restrict__ item_count) {
    int c[4], hv[4], lt[4], slot_sum = 0, heavy_sum = 0, light_sum = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const unsigned e = 4 * lane + j;
        c[j] = e < experts ? L.counts[e] : 0;
        const int n = (c[j] + kItemRows - 1) / kItemRows;
        lt[j] = heavy_first && n > 0 && c[j] - (n - 1) * kItemRows <= kTileRows ? 1 : 0;
        hv[j] = n - lt[j];
        slot_sum += c[j];
        heavy_sum += hv[j];
        light_sum += lt[j];
    }
    int slot_scan = slot_sum, heavy_scan = heavy_sum, light_scan = light_sum;
#pragma unroll
    for (int d = 1; d < 64; d *= 2) {  // inclusive over the lanes
        const int a = __shfl_up(slot_scan, d, 64), b = __shfl_up(heavy_scan, d, 64),
                  l = __shfl_up(light_scan, d, 64);
        if (lane >= unsigned(d)) {
            slot_scan += a;
            heavy_scan += b;
            light_scan += l;
        }
    }
    int acc = slot_scan - slot_sum, hb = heavy_scan - heavy_sum, lb = light_scan - light_sum;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const unsigned e = 4 * lane + j;
        if (e < experts) {
            if (offsets)
                offsets[e] = acc;
            L.segment[e] = acc;
            L.heavy_base[e] = hb;
            L.light_base[e] = lb;
        }
        acc += c[j];
        hb += hv[j];
        lb += lt[j];
    }
    if (lane == 63) {
        if (offsets)
            offsets[experts] = slot_scan;
        if (item_count)
            *item_count = heavy_scan + light_scan;
        L.heavy_total = heavy_scan;
    }
}

// Item of chunk k (rows 64k ..) of expert e: its heavy items in order, then its light one.
__device__ __forceinline__ int item_of(const ExpertLayout& L, bool heavy_first, unsigned e,
                                       int k) {
    const int n = (L.counts[e] + kItemRows - 1) / kItemRows;  // chunks of expert e
    const int heavy =
        n - (heavy_first && n > 0 && L.counts[e] - (n - 1) * kItemRows <= kTileRows ? 1 : 0);
    return k < heavy ? L.heavy_base[e] + k : L.heavy_total + L.light_base[e];
}

// Every expert's work items (expert, first row), by all threads of the workgroup.
__device__ __forceinline__ void write_items(const ExpertLayout& L, bool heavy_first,
                                            unsigned experts, int32_t* __restrict__ items) {
    for (unsigned e = threadIdx.x; e < experts; e += blockDim.x)
        for (int r = 0, k = 0; r < L.counts[e]; r += kItemRows, ++k) {
            const int n = item_of(L, heavy_first, e, k);
            items[2 * n] = int(e);
            items[2 * n + 1] = r;
        }
}

// Within a wavefront: the rank of this lane's slot among the lanes below it with the same
// expert, and how many lanes have that expert (experts below 256).
__device__ __forceinline__ void wave_match(bool valid, int e, unsigned lane, int& rank,
                                           int& group) {
    unsigned long long same = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const unsigned long long ones = __ballot(valid && ((e >> b) & 1));
        same &= ((e >> b) & 1) ? ones : ~ones;
    }
    rank = __popcll(same & ((1ull << lane) - 1ull));
    group = __popcll(same);
}

// Slot at position r: perm[r], position[s] (when given) and slot_row[r] = item *
// kItemRows + row (the K-sliced finalize runs over occupied rows only).
__device__ __forceinline__ void place_slot(const ExpertLayout& L, bool heavy_first, unsigned s,
                                           int e, int r, int32_t* __restrict__ perm,
                                           int32_t* __restrict__ position,
                                           int32_t* __restrict__ slot_row) {
    perm[r] = int(s);
    if (position)
        position[s] = r;  // inverse permutation
    const int within = r - L.segment[e];
    slot_row[r] = item_of(L, heavy_first, unsigned(e), within / kItemRows) * kItemRows +
                  within % kItemRows;
}

// Stable counting sort of slots by expert (expert-major, slot ascending) by one workgroup
// of 1024 threads (every thread calls it), 1024 slots at a time; also the work items.
// With heavy_first, work items are numbered heavy first: every item of more than
// kTileRows rows (two activation tiles, twice the MFMAs of a one-tile item), by expert,
// then the one-tile items.  The grouped GEMMs' workgroups are dispatched in item order,
// so the two-tile ones start first and spread over the compute units instead of landing
// together (C4 T=256, every workgroup resident at once: 149 -> 144 us).  Otherwise
// items follow the experts (C5, several rounds of workgroups: 689 against 704 us).
__device__ __forceinline__ void permute_slots(const int32_t* __restrict__ idx, unsigned slots,
                                              bool heavy_first,
                                              unsigned experts, int32_t* __restrict__ offsets,
                                              int32_t* __restrict__ perm,
                                              int32_t* __restrict__ items,
                                              int32_t* __restrict__ item_count,
                                              int32_t* __restrict__ position,
                                              int32_t* __restrict__ slot_row) {
    __shared__ ExpertLayout L;
    __shared__ int base[kMaxExperts];
    __shared__ int wave_counts[16][kMaxExperts];
    const unsigned tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    for (unsigned e = tid; e < experts; e += 1024)
        L.counts[e] = 0;
    __syncthreads();
    for (unsigned s = tid; s < slots; s += 1024)
        atomicAdd(&L.counts[idx[s]], 1);
    __syncthreads();
    if (wave == 0)
        expert_layout(L, experts, heavy_first, lane, offsets, item_count);
    __syncthreads();
    for (unsigned e = tid; e < experts; e += 1024)
        base[e] = L.segment[e];
    write_items(L, heavy_first, experts, items);
    for (unsigned first = 0; first < slots; first += 1024) {
        for (unsigned i = tid; i < 16 * kMaxExperts; i += 1024)
            (&wave_counts[0][0])[i] = 0;
        __syncthreads();
        const unsigned s = first + tid;
        const bool valid = s < slots;
        const int e = valid ? idx[s] : 0;
        int rank, group;
        wave_match(valid, e, lane, rank, group);
        if (valid && rank == group - 1)
            wave_counts[wave][e] = group;
        __syncthreads();
        if (valid) {
            int r = base[e] + rank;
            for (unsigned w = 0; w < wave; ++w)
                r += wave_counts[w][e];
            place_slot(L, heavy_first, s, e, r, perm, position, slot_row);
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

// The same sort over many chunks of 1024 slots, one workgroup a chunk, in two launches
// (the one-workgroup form spends ~1.9 us a chunk on one compute unit).
// chunk_count_kernel: each slot's rank among the earlier slots of its chunk with the same
// expert (chunk_rank[s]) and each chunk's count of every expert (chunk_counts[c][e]).
__global__ __launch_bounds__(1024) void chunk_count_kernel(const int32_t* __restrict__ idx,
                                                           unsigned slots, unsigned experts,
                                                           int32_t* __restrict__ chunk_counts,
                                                           int32_t* __restrict__ chunk_rank) {
    __shared__ int wave_counts[16][kMaxExperts];
    const unsigned tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    for (unsigned i = tid; i < 16 * kMaxExperts; i += 1024)
        (&wave_counts[0][0])[i] = 0;
    const unsigned s = blockIdx.x * 1024 + tid;
    const bool valid = s < slots;
    const int e = valid ? idx[s] : 0;
    __syncthreads();
    int rank, group;
    wave_match(valid, e, lane, rank, group);
    if (valid && rank == group - 1)
        wave_counts[wave][e] = group;
    __syncthreads();
    if (valid) {
        int r = rank;
        for (unsigned w = 0; w < wave; ++w)
            r += wave_counts[w][e];
        chunk_rank[s] = r;
    }
    for (unsigned x = tid; x < experts; x += 1024) {
        int total = 0;
        for (unsigned w = 0; w < 16; ++w)
            total += wave_counts[w][x];
        chunk_counts[size_t(blockIdx.x) * experts + x] = total;
    }
}

// chunk_place_kernel: every workgroup sums the chunks' counts (the experts' totals and, for
// its own chunk, the slots of each expert in earlier chunks) and places its chunk's slots;
// workgroup 0 also writes offsets, the work items and their count.
__global__ __launch_bounds__(1024) void chunk_place_kernel(
    const int32_t* __restrict__ idx, unsigned slots, unsigned experts, unsigned heavy_first,
    const int32_t* __restrict__ chunk_counts, const int32_t* __restrict__ chunk_rank,
    int32_t* __restrict__ offsets, int32_t* __restrict__ perm, int32_t* __restrict__ items,
    int32_t* __restrict__ item_count, int32_t* __restrict__ position,
    int32_t* __restrict__ slot_row) {
    __shared__ ExpertLayout L;
    __shared__ int before[kMaxExperts];
    const unsigned tid = threadIdx.x, wave = tid / 64, lane = tid % 64, c = blockIdx.x;
    const unsigned s = c * 1024 + tid;
    const bool valid = s < slots;
    const int e = valid ? idx[s] : 0;
    const int r_chunk = valid ? chunk_rank[s] : 0;
    for (unsigned x = tid; x < experts; x += 1024) {
        int total = 0, earlier = 0;
        for (unsigned k0 = 0; k0 < gridDim.x; k0 += 8) {  // eight loads in flight at once
            int v[8];
#pragma unroll
            for (unsigned j = 0; j < 8; ++j)
                v[j] = chunk_counts[size_t(min(k0 + j, gridDim.x - 1)) * experts + x];
#pragma unroll
            for (unsigned j = 0; j < 8; ++j) {
                const unsigned k = k0 + j;
                total += k < gridDim.x ? v[j] : 0;
                earlier += k < c ? v[j] : 0;
            }
        }
        L.counts[x] = total;
        before[x] = earlier;
    }
    __syncthreads();
    if (wave == 0)
        expert_layout(L, experts, heavy_first != 0, lane, c == 0 ? offsets : nullptr,
                      c == 0 ? item_count : nullptr);
    __syncthreads();
    if (c == 0)
        write_items(L, heavy_first != 0, experts, items);
    if (valid)
        place_slot(L, heavy_first != 0, s, e, L.segment[e] + before[e] + r_chunk, perm, position,
                   slot_row);
}

__global__ __launch_bounds__(1024) void permute_kernel(const int32_t* __restrict__ idx,
                                                       unsigned slots, unsigned experts,
                                                       int32_t* __restrict__ offsets,
                                                       int32_t* __restrict__ perm,
                                                       int32_t* __restrict__ items,
                                                       int32_t* __restrict__ item_count,
                                                       int32_t* __restrict__ position,
                                                       int32_t* __restrict__ slot_row,
                                                       unsigned heavy_first) {
    permute_slots(idx, slots, heavy_first != 0, experts, offsets, perm, items, item_count,
                  position, slot_row);
}

// --------------------------------------------------------------- grouped GEMMs

// silu(x) = x / (1 + e^-x) from the hardware exponential and reciprocal (each within an
// ulp or two): h leaves as FP8 terms good to about 12 bits, so the epilogue's cost, not
// the last bits of silu, is what matters; infinities and NaN come out as in the
// reference's x / (1 + expf(-x)).
__device__ __forceinline__ float silu(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504088896341f));
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

// ------------------------------------------------------------- FP8 activation tiles
//
// The grouped GEMMs run on v_mfma_scale_f32_32x32x64_f8f6f4: FP8 (E4M3) activations times
// the FP4 (E2M1) weights, each operand with an E8M0 scale per 32 K values.  An activation
// value is carried as a sum of FP8 terms sharing one block scale 2^e per 32 values (e such
// that the block's largest magnitude lands in [128, 256)): term 1 is the value rounded to
// E4M3 (round to nearest even), term 2 the remainder rounded, and so on.  Two terms hold
// every bf16 value exactly (8 significant bits: 4 + 4; values under 2^-2 of the scale
// keep an absolute error below 2^-10 of it); three terms carry h = silu(g) * u to about
// 12 significant bits.  A block with a non-finite value gets the E8M0 NaN scale (255) and
// FP8 NaN codes, so every product that touches it is NaN, as in fp32.
//
// Activations reach the MFMAs as tiles: tile tau = 2 * item + t holds rows 32t .. 32t+31
// of work item `item` (its slots in permutation order), gathered once so that every
// wavefront load of an A operand is 1 KB contiguous, as the packed weights are.  For
// step q (64 K values) of tile tau, with TERMS terms:
//   codes  tile_codes(tau) + (q * TERMS + k) * 2048 + piece * 1024 + 16 * lane, 16 bytes:
//          lane r + 32h holds row r's values 16h + i (piece 0) and 32 + 16h + i (piece 1)
//          of the step, i = 0..15 (the lane's half of the MFMA A operand), term k
//   scales tile_scales(tau) + (q / 4) * 256 + 4 * lane + q % 4: the E8M0 scale of row r's
//          values 64q + 32h .. +31 (lane r + 32h supplies the scale of K block h)
// codes of all tiles first (steps * TERMS * 2 KB each), then their scales
// (ceil(steps / 4) * 256 bytes each).

typedef int v8i32 __attribute__((ext_vector_type(8)));
typedef int v4i32 __attribute__((ext_vector_type(4)));

constexpr int kXTerms = 2, kHTerms = 3;

struct Tiles {
    uint8_t* codes;   // tile 0's codes
    uint8_t* scales;  // tile 0's scales
    size_t code_stride, scale_stride;  // bytes per tile
};

__host__ __device__ inline Tiles tile_layout(uint8_t* base, size_t tiles, size_t steps, int terms) {
    Tiles l;
    l.code_stride = steps * size_t(terms) * 2048;
    l.scale_stride = (steps + 3) / 4 * 256;
    l.codes = base;
    l.scales = base + tiles * l.code_stride;
    return l;
}

__host__ __device__ inline size_t tile_bytes(size_t tiles, size_t steps, int terms) {
    return tiles * (steps * size_t(terms) * 2048 + (steps + 3) / 4 * 256);
}

// e with 2^-e * amax in [128, 256) for a finite amax > 0, within the E8M0 range.
__device__ __forceinline__ int block_exponent(float amax) {
    const int ex = int((__float_as_uint(amax) >> 23) & 255u) - 127;
    return max(-127, min(127, ex - 7));
}

// TERMS FP8 terms of 16 values already multiplied by 2^-e, four bytes per dword in value
// order; v is consumed.
template <int TERMS>
__device__ __forceinline__ void fp8_terms16(float (&v)[16], u32x4 (&out)[TERMS]) {
#pragma unroll
    for (int t = 0; t < TERMS; ++t) {
        unsigned w[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * d], v[4 * d + 1], 0, false);
            const int both = __builtin_amdgcn_cvt_pk_fp8_f32(v[4 * d + 2], v[4 * d + 3], lo, true);
            w[d] = unsigned(both);
            if (t + 1 < TERMS) {  // the remainder is exact in fp32 (Sterbenz)
                v[4 * d] -= __builtin_amdgcn_cvt_f32_fp8(both, 0);
                v[4 * d + 1] -= __builtin_amdgcn_cvt_f32_fp8(both, 1);
                v[4 * d + 2] -= __builtin_amdgcn_cvt_f32_fp8(both, 2);
                v[4 * d + 3] -= __builtin_amdgcn_cvt_f32_fp8(both, 3);
            }
        }
        out[t] = u32x4{w[0], w[1], w[2], w[3]};
    }
}

// Row r's 32-value block b of one tile (codes/scales of that tile): block b = 2q + hb of
// step q; its values 0..15 belong to lane r (piece hb), 16..31 to lane r + 32 (piece hb).
// A 32-value block as TERMS FP8 terms: values 0..15 into tl, 16..31 into th; returns the
// block's E8M0 scale byte.
template <int TERMS>
__device__ __forceinline__ uint8_t block_terms(float (&v)[32], bool finite, u32x4 (&tl)[TERMS],
                                               u32x4 (&th)[TERMS]) {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i)
        amax = fmaxf(amax, fabsf(v[i]));
    const int e = block_exponent(amax);
    float lo[16], hi[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        lo[i] = finite ? __builtin_amdgcn_ldexpf(v[i], -e) : 0.f;
        hi[i] = finite ? __builtin_amdgcn_ldexpf(v[16 + i], -e) : 0.f;
    }
    fp8_terms16<TERMS>(lo, tl);
    fp8_terms16<TERMS>(hi, th);
    if (!finite) {  // FP8 NaN codes as well as the NaN scale: NaN however it is read
#pragma unroll
        for (int k = 0; k < TERMS; ++k)
            tl[k] = th[k] = u32x4{0x7f7f7f7fu, 0x7f7f7f7fu, 0x7f7f7f7fu, 0x7f7f7f7fu};
    }
    return finite ? uint8_t(e + 127) : uint8_t(255);
}

template <int TERMS>
__device__ __forceinline__ void store_tile_block(float (&v)[32], bool finite, uint8_t* codes,
                                                 uint8_t* scales, unsigned r, unsigned b) {
    u32x4 tl[TERMS], th[TERMS];
    const uint8_t scale = block_terms<TERMS>(v, finite, tl, th);
    const unsigned q = b / 2, hb = b % 2;
    uint8_t* at = codes + size_t(q) * TERMS * 2048 + hb * 1024;
#pragma unroll
    for (int k = 0; k < TERMS; ++k) {
        *reinterpret_cast<u32x4*>(at + k * 2048 + 16 * r) = tl[k];
        *reinterpret_cast<u32x4*>(at + k * 2048 + 16 * (r + 32)) = th[k];
    }
    scales[(q / 4) * 256 + 4 * (r + 32 * hb) + q % 4] = scale;
}

// Row r (of 32) of activation tile tau from token row `token` of x (bf16 [tokens][hidden]),
// 32-value block b: its kXTerms FP8 terms and scale in the tile layout.
// 32 bf16 values from src as fp32 (exact); returns whether all are finite.
__device__ __forceinline__ bool load_bf16_block(const uint16_t* src16, float (&v)[32]) {
    const uint8_t* src = reinterpret_cast<const uint8_t*>(src16);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const u32x4 w = load16(src + 16 * c);
        const unsigned ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // bf16 -> fp32 is exact
            v[8 * c + 2 * i] = __uint_as_float(ws[i] << 16);
            v[8 * c + 2 * i + 1] = __uint_as_float(ws[i] & 0xffff0000u);
        }
    }
    bool finite = true;
#pragma unroll
    for (int i = 0; i < 32; ++i)
        finite = finite && isfinite(v[i]);
    return finite;
}

__device__ __forceinline__ void gather_block(const uint16_t* __restrict__ x, unsigned hidden,
                                             size_t token, uint8_t* __restrict__ xa,
                                             size_t tiles, size_t tau, unsigned r, unsigned b) {
    float v[32];
    const bool finite = load_bf16_block(x + token * hidden + 32 * b, v);
    const Tiles l = tile_layout(xa, tiles, hidden / 64, kXTerms);
    store_tile_block<kXTerms>(v, finite, l.codes + tau * l.code_stride,
                              l.scales + tau * l.scale_stride, r, b);
}

// x gathered by the permutation into gate/up's activation tiles as kXTerms FP8 terms:
// grid (row-blocks / 256, tiles); thread `id` of tile tau takes tile row id % 32,
// 32-value block id / 32.  Rows past an item's count and absent tiles are not written:
// a row of an MFMA's A operand only reaches the same row of its result, which is not stored.
__global__ __launch_bounds__(256) void gather_kernel(const uint16_t* __restrict__ x,
                                                     unsigned hidden, unsigned top_k,
                                                     const int32_t* __restrict__ offsets,
                                                     const int32_t* __restrict__ perm,
                                                     const int32_t* __restrict__ items,
                                                     const int32_t* __restrict__ item_count,
                                                     uint8_t* __restrict__ xa, size_t tiles) {
    const unsigned blocks = hidden / 32, id = blockIdx.x * 256 + threadIdx.x;
    const unsigned tau = blockIdx.y, item = tau / 2, t = tau % 2;
    if (id >= 32 * blocks || int(item) >= *item_count)
        return;
    const Item it = load_item(items, offsets, item);
    // rows fastest: a wavefront's lanes take 32 rows of two blocks, so each term's stores
    // fill 512 contiguous bytes of the tile layout (lane r + 32h holds row r)
    const int row = int(32 * t + id % 32);
    if (row >= it.count)
        return;
    const size_t token = size_t(perm[it.segment + it.first + row] / int(top_k));
    gather_block(x, hidden, token, xa, tiles, tau, id % 32, id / 32);
}

// Small layers (decode, at most kPrologueSlots slots): routing, permutation and gather in
// one workgroup of 1024 threads, one launch instead of three, with every intermediate in
// LDS: the routed experts, the permutation (one wavefront: a slot's position is the number
// of slots of a lower expert plus those of its own expert before it, the same stable order
// as permute_slots; with at most kItemRows slots per expert each expert is one item) and,
// when they fit, the token rows of x, which the waves that do not route copy into LDS
// while routing runs.  The global outputs are those of route_kernel + permute_kernel.
constexpr unsigned kPrologueXBytes = 48 * 1024;

__global__ __launch_bounds__(1024) void prologue_kernel(
    const float* __restrict__ logits, unsigned tokens, unsigned experts, unsigned top_k,
    int32_t* __restrict__ idx, float* __restrict__ weight, int32_t* __restrict__ offsets,
    int32_t* __restrict__ perm, int32_t* __restrict__ items, int32_t* __restrict__ item_count,
    int32_t* __restrict__ position, int32_t* __restrict__ slot_row,
    const uint16_t* __restrict__ x, unsigned hidden, uint8_t* __restrict__ xa, size_t tiles) {
    extern __shared__ __align__(16) uint8_t x_rows[];  // tokens * hidden bf16, if they fit
    __shared__ int s_idx[kPrologueSlots], s_perm[kPrologueSlots], s_row[kPrologueSlots];
    const unsigned wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const unsigned slots = tokens * top_k;
    const size_t x_bytes = size_t(tokens) * hidden * 2;
    const bool x_in_lds = x_bytes <= kPrologueXBytes;
    const unsigned routers = min(tokens, 16u);
    for (unsigned t = wave; t < tokens; t += 16)
        route_token(logits, t, experts, top_k, idx, weight, lane, s_idx);
    if (x_in_lds && wave >= routers) {  // x rows into LDS meanwhile (16-byte units)
        const unsigned helpers = (16 - routers) * 64, me = threadIdx.x - routers * 64;
        for (size_t u = me; u < x_bytes / 16; u += helpers)
            *reinterpret_cast<u32x4*>(x_rows + 16 * u) =
                load16(reinterpret_cast<const uint8_t*>(x) + 16 * u);
    }
    __syncthreads();
    if (x_in_lds && routers == 16) {  // every wave routed: copy now
        for (size_t u = threadIdx.x; u < x_bytes / 16; u += 1024)
            *reinterpret_cast<u32x4*>(x_rows + 16 * u) =
                load16(reinterpret_cast<const uint8_t*>(x) + 16 * u);
    }
    if (wave == 0) {
        const bool valid = lane < slots;
        const int e = valid ? s_idx[lane] : 0x7fffffff;
        int lower = 0, before = 0;
        for (unsigned j = 0; j < slots; ++j) {
            const int ej = s_idx[j];
            lower += ej < e;
            before += (ej == e) & (j < lane);
        }
        // the expert's first slots, one per used expert
        const unsigned long long leads = __ballot(valid && before == 0);
        if (valid) {
            perm[lower + before] = int(lane);
            position[lane] = lower + before;
            s_perm[lower + before] = int(lane);
        }
        // offsets[e] = slots routed to experts below e
        for (unsigned x_e = lane; x_e <= experts; x_e += 64) {
            int below = 0;
            for (unsigned j = 0; j < slots; ++j)
                below += s_idx[j] < int(x_e);
            offsets[x_e] = below;
        }
        // item of each used expert: the number of used experts below it
        int item = 0;
        for (unsigned j = 0; j < slots; ++j)
            item += ((leads >> j) & 1ull) && s_idx[j] < e;
        if (valid) {
            slot_row[lower + before] = item * kItemRows + before;
            s_row[lower + before] = item * kItemRows + before;
            if (before == 0) {
                items[2 * item] = e;
                items[2 * item + 1] = 0;
            }
        }
        if (lane == 0)
            *item_count = int(__popcll(leads));
    }
    __syncthreads();
    // every occupied row: position g, 32-value block b
    const unsigned blocks = hidden / 32;
    const uint16_t* rows = x_in_lds ? reinterpret_cast<const uint16_t*>(x_rows) : x;
    for (unsigned u = threadIdx.x; u < slots * blocks; u += 1024) {
        const unsigned g = u / blocks;
        const unsigned item = unsigned(s_row[g]) / kItemRows, row = unsigned(s_row[g]) % kItemRows;
        const size_t token = size_t(s_perm[g] / int(top_k));
        gather_block(rows, hidden, token, xa, tiles, 2 * size_t(item) + row / 32, row % 32,
                     u % blocks);
    }
}

// ------------------------------------------------------------- grouped GEMMs
//
// A workgroup of kGemmWaves wavefronts takes one work item (expert e, up to kItemRows
// consecutive rows of its segment: one or two activation tiles of 32 rows) and one K
// slice; every wavefront owns two 32-row weight groups (gate and up of the same 32
// features, or two groups of down rows) and multiplies the item's tiles into both.  Per
// 64-value step a lane loads its 16 FP4 bytes of each group (the packed layout is the
// MFMA's B operand as it lies; 1 KB contiguous per wavefront) and, per 4 steps, one scale
// dword per group and per tile, whose byte the MFMA's op_sel picks.  The loop runs whole
// periods of four steps unrolled, so every register slot stays fixed, every load is
// unconditional (steps past the end re-read the last one) and each wait counts exactly
// the loads the next step needs.

// A operand from a lane's two 16-byte pieces; B operand from its 16 FP4 bytes (the MFMA
// reads four registers of an FP4 operand; the other four are left undefined).
__device__ __forceinline__ v8i32 a_operand(const u32x4& lo, const u32x4& hi) {
    return v8i32{int(lo.x), int(lo.y), int(lo.z), int(lo.w),
                 int(hi.x), int(hi.y), int(hi.z), int(hi.w)};
}

__device__ __forceinline__ v8i32 b_operand(const u32x4& c) {
    const v4i32 v{int(c.x), int(c.y), int(c.z), int(c.w)};
    return __builtin_shufflevector(v, v, 0, 1, 2, 3, -1, -1, -1, -1);
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

// K slice `slice` of `slices`: [begin, end) in steps, begin a multiple of 8.
__device__ __forceinline__ void slice_steps(unsigned steps, unsigned slices, unsigned slice,
                                            unsigned& begin, unsigned& end) {
    const unsigned per = ((steps + slices - 1) / slices + 7) / 8 * 8;
    begin = min(steps, slice * per);
    end = min(steps, begin + per);
}

__device__ __forceinline__ void issue_order() {
    asm volatile("" ::: "memory");  // keeps the load issue order (activation pointers are
    __builtin_amdgcn_sched_barrier(0);  // not restrict)
}

// The item's activation tiles pass through LDS: per chunk of kChunk steps the workgroup
// copies the chunk of every tile it multiplies (contiguous in the tile layout: kChunk *
// TERMS * 2 KB per tile) into one of two LDS buffers, 16 bytes per thread per piece, and
// every wavefront reads its MFMA A operands from there at lane * 16 (conflict free): one
// activation load per thread and piece instead of one per wavefront.  A chunk is loaded
// while the one before it is multiplied and stored behind it, with one workgroup barrier
// per chunk; weights stream per wavefront BRING - 1 steps ahead.  (Measured at T = 256,
// 32 experts: activations loaded by every wavefront from L2 kept the address unit 60 %
// busy and the MFMAs 18 %; staging two chunks ahead or weights seven steps ahead were
// slower; so was a register cap for three workgroups per compute unit, which spills.)
constexpr int kChunk = 2;

template <int TERMS, int TILES, int WAVES = kGemmWaves> struct StageCopy {
    static constexpr int chunk_bytes = TILES * kChunk * TERMS * 2048;  // one LDS buffer
    static constexpr int threads = WAVES * 64;
    // per thread; when the chunk's 16-byte pieces are not a multiple of the threads, the
    // last piece of the threads past the end is clamped on load and not stored
    static constexpr int pieces = (chunk_bytes / 16 + threads - 1) / threads;
    static constexpr bool ragged = chunk_bytes / 16 % threads != 0;
    const uint8_t* src[pieces];  // piece j of this thread at step 0 (tile base + offset)
    unsigned step[pieces];       // step of the piece within the chunk
};

template <int TERMS, int TILES, int WAVES>
__device__ __forceinline__ StageCopy<TERMS, TILES, WAVES> stage_copy(const Tiles& l,
                                                                     unsigned item) {
    using C = StageCopy<TERMS, TILES, WAVES>;
    C c;
    constexpr int per_tile = kChunk * TERMS * 2048;
#pragma unroll
    for (int j = 0; j < C::pieces; ++j) {
        const unsigned o = min(unsigned(threadIdx.x + j * WAVES * 64) * 16,
                               unsigned(C::chunk_bytes - 16));  // byte in the chunk
        const unsigned t = o / per_tile, within = o % per_tile;
        c.step[j] = within / (TERMS * 2048);
        c.src[j] = l.codes + (2 * size_t(item) + t) * l.code_stride + within % (TERMS * 2048);
    }
    return c;
}


// acc[m][t] += A(tile t, steps [q0, q1)) * B(group m), q0 % 8 == 0; A through LDS, weights
// BRING - 1 steps ahead (BRING = 4 or 8 steps: whole scale groups and LDS buffer pairs),
// with the non-temporal policy when NT (weights read once per layer call).
template <int TERMS, int TILES, bool NT, int BRING = 4, int WAVES = kGemmWaves>
__device__ __forceinline__ void staged_pair(const Tiles& l, unsigned item, unsigned lane,
                                            const WavePair& w, unsigned q0, unsigned q1,
                                            bool active, uint8_t* stage,
                                            f32x16 (&acc)[2][TILES]) {
    using C = StageCopy<TERMS, TILES, WAVES>;
    const C cp = stage_copy<TERMS, TILES, WAVES>(l, item);
    const unsigned* ascale[TILES];
#pragma unroll
    for (int t = 0; t < TILES; ++t)
        ascale[t] = reinterpret_cast<const unsigned*>(l.scales + (2 * size_t(item) + t) * l.scale_stride) +
                    lane;
    struct BSlot {
        u32x4 c[2];
        unsigned s[2];
        unsigned as[TILES];
    };
    auto load_b = [&](unsigned q, BSlot& B) {
        q = min(q, q1 - 1);
#pragma unroll
        for (int m = 0; m < 2; ++m)
            B.c[m] = NT ? stream16(w.codes[m] + size_t(q) * 1024)
                        : load16(w.codes[m] + size_t(q) * 1024);
#pragma unroll
        for (int m = 0; m < 2; ++m)
            B.s[m] = w.scales[m][size_t(q / 4) * 64];
#pragma unroll
        for (int t = 0; t < TILES; ++t)
            B.as[t] = ascale[t][size_t(q / 4) * 64];
    };
    struct Pieces {
        u32x4 v[C::pieces];
    };
    auto stage_load = [&](unsigned qc, Pieces& P) {  // chunk starting at step qc
#pragma unroll
        for (int j = 0; j < C::pieces; ++j)
            P.v[j] = load16(cp.src[j] + size_t(min(qc + cp.step[j], q1 - 1)) * TERMS * 2048);
    };
    auto stage_store = [&](const Pieces& P, int buffer) {
#pragma unroll
        for (int j = 0; j < C::pieces; ++j) {
            const unsigned o = (threadIdx.x + j * WAVES * 64) * 16;
            if (!C::ragged || j + 1 < C::pieces || o < unsigned(C::chunk_bytes))
                *reinterpret_cast<u32x4*>(stage + buffer * C::chunk_bytes + o) = P.v[j];
        }
    };
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int t = 0; t < TILES; ++t)
            acc[m][t] = f32x16{};
    BSlot bs[BRING];
    Pieces xr;
    stage_load(q0, xr);
    issue_order();
#pragma unroll
    for (int d = 0; d + 1 < BRING; ++d)
        load_b(q0 + d, bs[d]);
    issue_order();
    stage_store(xr, 0);
    __syncthreads();
    // one chunk (kChunk = 2 steps) per call; CI = chunk index within the BRING-step period
    auto chunk = [&]<int CI>(unsigned qc) {
        constexpr int C2 = CI % 2;  // LDS buffer
        stage_load(qc + kChunk, xr);
        issue_order();
        auto step = [&]<int S>() {
            constexpr int U = CI * kChunk + S;  // step within the period
            const unsigned q = qc + S;
            load_b(q + BRING - 1, bs[(U + BRING - 1) % BRING]);
            if (active && q < q1) {
                const BSlot& B = bs[U];
                const uint8_t* buf = stage + C2 * C::chunk_bytes + 16 * lane;
#pragma unroll
                for (int t = 0; t < TILES; ++t)
#pragma unroll
                    for (int k = 0; k < TERMS; ++k) {
                        const uint8_t* p = buf + ((t * kChunk + S) * TERMS + k) * 2048;
                        const v8i32 av = a_operand(*reinterpret_cast<const u32x4*>(p),
                                                   *reinterpret_cast<const u32x4*>(p + 1024));
#pragma unroll
                        for (int m = 0; m < 2; ++m)
                            acc[m][t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                                av, b_operand(B.c[m]), acc[m][t], 0 /* A: fp8 e4m3 */,
                                4 /* B: fp4 e2m1 */, U % 4, int(B.as[t]), U % 4, int(B.s[m]));
                    }
            }
        };
        step.template operator()<0>();
        step.template operator()<1>();
        stage_store(xr, (C2 + 1) % 2);  // also past the end (never read)
        __syncthreads();
    };
    const unsigned periods = (q1 - q0 + BRING - 1) / BRING;
    for (unsigned p = 0; p < periods; ++p) {
        const unsigned qc = q0 + p * BRING;
        chunk.template operator()<0>(qc);
        chunk.template operator()<1>(qc + kChunk);
        if constexpr (BRING == 8) {
            chunk.template operator()<2>(qc + 2 * kChunk);
            chunk.template operator()<3>(qc + 3 * kChunk);
        }
    }
}

// Output row of accumulator element v in lane half h of tile t (32x32 MFMA layout).
__device__ __forceinline__ int acc_row(int t, int v, unsigned h) {
    return t * kTileRows + 8 * (v / 4) + 4 * int(h) + (v % 4);
}

// Maximum over the 32 lanes of this lane's half of the wavefront (all 64 lanes active):
// the row of 16 by DPP, then rows 0/1 and 2/3 by gfx950's row swap (v_permlane16_swap:
// each lane ends with its own row's value and its partner row's, in some order).
__device__ __forceinline__ float half_max(float v) {
    v = fmaxf(v, dpp_read<0xb1, 0xf>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_read<0x4e, 0xf>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_read<0x141, 0xf>(v));  // row_half_mirror
    v = fmaxf(v, dpp_read<0x140, 0xf>(v));  // row_mirror: the row of 16's maximum
    const auto pair = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                       false, false);
    return fmaxf(__uint_as_float(pair[0]), __uint_as_float(pair[1]));
}

// h for row r (0..31) of an activation tile of the down product, feature f, held with the
// other 31 features of its 32-value block by the 32 lanes of this half of the wavefront
// (one row per register).  The block scale comes from the half; each lane writes its
// value's terms as single bytes (codes/scales of that tile).
__device__ __forceinline__ void store_h(float hv, unsigned r, unsigned f, uint8_t* codes,
                                        uint8_t* scales, bool store) {
    const bool finite = half_max(isfinite(hv) ? 0.f : 1.f) == 0.f;
    const int e = block_exponent(half_max(fabsf(hv)));
    float v = finite ? __builtin_amdgcn_ldexpf(hv, -e) : 0.f;
    if (!store)
        return;
    const unsigned q = f / 64, k = f % 64;
    // value k of step q: lane r + 32 ((k / 16) % 2), piece k / 32, byte k % 16
    uint8_t* at = codes + size_t(q) * kHTerms * 2048 + (k / 32) * 1024 +
                  16 * (r + 32 * ((k / 16) % 2)) + k % 16;
#pragma unroll
    for (int t = 0; t < kHTerms; ++t) {
        const int c = __builtin_amdgcn_cvt_pk_fp8_f32(v, 0.f, 0, false);
        at[t * 2048] = finite ? uint8_t(c & 0xff) : uint8_t(0x7f);  // 0x7f: FP8 NaN
        v -= __builtin_amdgcn_cvt_f32_fp8(c, 0);
    }
    if (f % 32 == 0)
        scales[(q / 4) * 256 + 4 * (r + 32 * ((f / 32) % 2)) + q % 4] =
            finite ? uint8_t(e + 127) : uint8_t(255);
}

// h = silu(g) * u of the wavefront's 32 features (feature group fg; lanes i and i + 32
// hold feature i) for every row of the item's tiles, into the down product's activation
// tiles: kHTerms FP8 terms and one E8M0 scale per row's 32-value block (the half-wavefront
// maximum).  The features fill one 1 KB piece of each (tile, step, term) block, so the term
// bytes are assembled in the wavefront's 1 KB of LDS and leave as one 16-byte store per
// lane; every row is written (rows past the item's count only reach result rows that are
// never stored).
template <int TILES>
__device__ __forceinline__ void store_h_tiles(const f32x16 (&acc)[2][TILES], unsigned fg,
                                              unsigned lane, size_t item, const Tiles& hl,
                                              uint8_t* lds) {
    const unsigned i32 = lane % 32, h = lane / 32;
    const unsigned q = fg / 2, piece = fg % 2;
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
        const size_t tau = 2 * item + t;
        uint8_t* codes = hl.codes + tau * hl.code_stride + size_t(q) * kHTerms * 2048 + piece * 1024;
        uint8_t* scales = hl.scales + tau * hl.scale_stride + (q / 4) * 256 + q % 4;
        uint8_t term[kHTerms][16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const unsigned r = 8 * (v / 4) + 4 * h + v % 4;
            const float hv = silu(acc[0][t][v]) * acc[1][t][v];
            // one maximum for the block scale and its finiteness: a non-finite value
            // counts as +inf
            const float m = half_max(isfinite(hv) ? fabsf(hv) : INFINITY);
            const bool finite = m != INFINITY;
            const int e = block_exponent(m);
            float val = finite ? __builtin_amdgcn_ldexpf(hv, -e) : 0.f;
#pragma unroll
            for (int k = 0; k < kHTerms; ++k) {
                const int c = __builtin_amdgcn_cvt_pk_fp8_f32(val, 0.f, 0, false);
                term[k][v] = finite ? uint8_t(c & 0xff) : uint8_t(0x7f);  // 0x7f: FP8 NaN
                val -= __builtin_amdgcn_cvt_f32_fp8(c, 0);
            }
            if (i32 == 0)
                scales[4 * (r + 32 * piece)] = finite ? uint8_t(e + 127) : uint8_t(255);
        }
#pragma unroll
        for (int k = 0; k < kHTerms; ++k) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const unsigned r = 8 * (v / 4) + 4 * h + v % 4;
                lds[(r + 32 * (i32 / 16)) * 16 + i32 % 16] = term[k][v];
            }
            *reinterpret_cast<u32x4*>(codes + k * 2048 + 16 * lane) =
                *reinterpret_cast<const u32x4*>(lds + 16 * lane);
        }
    }
}

// The (column, item) cell of a grouped GEMM workgroup.  The grid's x dimension holds
// cols x items_pad cells (items_pad a multiple of 8): workgroup L runs on XCD L % 8, and
// XCD k takes items k, k + 8, ..., each with all its column workgroups in a row, so one
// XCD's L2 serves an item's activation tiles to every column that multiplies them.
struct ItemCell {
    unsigned col, item;
};
__device__ __forceinline__ ItemCell item_cell(unsigned cols) {
    const unsigned xcd = blockIdx.x % 8, j = blockIdx.x / 8;
    return ItemCell{j % cols, (j / cols) * 8 + xcd};
}

// gate/up: grid (cells of item_cell: groups of kGemmWaves feature groups of 32 x items,
// K slices).  Wavefront w multiplies gate and up rows of features 32 (kGemmWaves col + w)
// .. +31.  One slice:
// h = silu(g) * u into the down product's activation tiles; more: fp32 partials of g and u
// per (tile row, feature) (finalize_kernel).
// Three workgroups per compute unit (168 registers, no spill): measured 187 -> 174 us at
// T = 256 and 0.79 -> 0.75 ms at C5.  (down_kernel would spill at that cap.)
template <bool NT>
__global__ __launch_bounds__(kGemmWaves * 64, 3) void gate_up_kernel(
    const uint8_t* __restrict__ xa, unsigned hidden, unsigned inter, unsigned experts,
    size_t tiles, const uint8_t* __restrict__ gate, const uint8_t* __restrict__ up,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ items,
    const int32_t* __restrict__ item_count, uint8_t* __restrict__ ha,
    float* __restrict__ part_g, float* __restrict__ part_u, size_t part_stride,
    unsigned cols) {
    __shared__ __align__(16) uint8_t stage[2 * StageCopy<kXTerms, 2>::chunk_bytes];
    const ItemCell cell = item_cell(cols);
    if (int(cell.item) >= *item_count)
        return;
    const Item it = load_item(items, offsets, cell.item);
    const unsigned wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const unsigned i32 = lane % 32, h = lane / 32;
    const Packed shape = packed_shape(1, inter, hidden);  // per expert
    const unsigned fg = cell.col * kGemmWaves + wave;     // feature group of 32
    const bool active = fg < shape.groups;                // uniform per wavefront
    const unsigned f = (active ? fg : 0) * 32 + i32;
    unsigned q0, q1;
    slice_steps(unsigned(shape.steps), gridDim.z, blockIdx.z, q0, q1);
    if (q0 >= q1)
        return;
    const Packed whole = packed_shape(experts, inter, hidden);
    const size_t group = size_t(it.expert) * shape.groups + (active ? fg : 0);
    WavePair wp = wave_pair(gate, whole, group, group, lane);
    const WavePair wu = wave_pair(up, whole, group, group, lane);
    wp.codes[1] = wu.codes[0];
    wp.scales[1] = wu.scales[0];
    const Tiles xl = tile_layout(const_cast<uint8_t*>(xa), tiles, hidden / 64, kXTerms);
    const Tiles hl = tile_layout(ha, tiles, inter / 64, kHTerms);

    auto run = [&]<int TILES>() {
        f32x16 acc[2][TILES];
        staged_pair<kXTerms, TILES, NT>(xl, cell.item, lane, wp, q0, q1, active, stage, acc);
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
                                          (size_t(cell.item) * kItemRows + r) * inter + f;
                        part_g[at] = acc[0][t][v];
                        part_u[at] = acc[1][t][v];
                    }
                }
            return;
        }
        // the LDS stage is free once staged_pair has returned (it ends on a barrier
        // after the last MFMA read); each wavefront takes its own 1 KB of it
        store_h_tiles<TILES>(acc, fg, lane, cell.item, hl, stage + wave * 1024);
    };
    if (it.count <= kTileRows)
        run.template operator()<1>();
    else
        run.template operator()<2>();
}

// h = silu(sum_s g_s) * (sum_s u_s), slices summed in order, into the down product's
// activation tiles: grid (inter / 256, slots): one thread per (occupied row, feature),
// the row slot_row[position] = item * kItemRows + row; each half wavefront one 32-feature
// block (inter % 64 == 0).
__global__ __launch_bounds__(256) void finalize_kernel(const float* __restrict__ part_g,
                                                       const float* __restrict__ part_u,
                                                       size_t part_stride, unsigned inter,
                                                       unsigned slices,
                                                       const int32_t* __restrict__ slot_row,
                                                       uint8_t* __restrict__ ha, size_t tiles) {
    const unsigned at_row = unsigned(slot_row[blockIdx.y]);
    const unsigned item = at_row / kItemRows, row = at_row % kItemRows;
    const unsigned f = blockIdx.x * 256 + threadIdx.x;
    const bool live = f < inter;
    const size_t at = size_t(at_row) * inter + (live ? f : 0);
    float gs = 0.f, us = 0.f;
    for (unsigned s = 0; s < slices; ++s) {
        gs += part_g[s * part_stride + at];
        us += part_u[s * part_stride + at];
    }
    const Tiles hl = tile_layout(ha, tiles, inter / 64, kHTerms);
    const size_t tau = 2 * size_t(item) + row / kTileRows;
    store_h(silu(gs) * us, row % kTileRows, live ? f : 0, hl.codes + tau * hl.code_stride,
            hl.scales + tau * hl.scale_stride, live);
}

// down: grid (cells of item_cell: groups of row pairs of 64 x items, K slices); wavefront w
// multiplies the down rows 64 (kDownWaves col + w) .. +63 (two groups of 32).  fp32 partial
// sums of h x down per slice, indexed by the slot's position in the permutation.
template <bool NT>
__global__ __launch_bounds__(kDownWaves * 64) void down_kernel(
    const uint8_t* __restrict__ ha, size_t tiles, unsigned hidden, unsigned inter,
    unsigned experts, const uint8_t* __restrict__ down, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ items, const int32_t* __restrict__ item_count,
    float* __restrict__ part_d, size_t part_stride, unsigned cols) {
    __shared__ __align__(16) uint8_t stage[2 * StageCopy<kHTerms, 2, kDownWaves>::chunk_bytes];
    const ItemCell cell = item_cell(cols);
    if (int(cell.item) >= *item_count)
        return;
    const Item it = load_item(items, offsets, cell.item);
    const unsigned wave = threadIdx.x / 64, lane = threadIdx.x % 64;
    const unsigned i32 = lane % 32, h = lane / 32;
    const Packed shape = packed_shape(1, hidden, inter);  // per expert
    const unsigned pair = cell.col * kDownWaves + wave;
    const bool active = pair < shape.groups / 2;
    const unsigned g0 = (active ? pair : 0) * 2;
    unsigned q0, q1;
    slice_steps(unsigned(shape.steps), gridDim.z, blockIdx.z, q0, q1);
    if (q0 >= q1)
        return;
    const Packed whole = packed_shape(experts, hidden, inter);
    const size_t base = size_t(it.expert) * shape.groups + g0;
    const WavePair w = wave_pair(down, whole, base, base + 1, lane);
    const Tiles hl = tile_layout(const_cast<uint8_t*>(ha), tiles, inter / 64, kHTerms);
    auto run = [&]<int TILES>() {
        f32x16 acc[2][TILES];
        staged_pair<kHTerms, TILES, NT, 4, kDownWaves>(hl, cell.item, lane, w, q0, q1, active,
                                                       stage, acc);
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


// ------------------------------------------------------------ single-token decode
//
// One token routes to top_k distinct experts, so every slot is a one-row product of its
// own expert.  Two launches replace the five of the general path:
//
//   decode_gate_up_kernel  grid (inter / 32 feature groups, top_k slots), 2 * runs waves:
//     waves 0 .. runs-1 multiply the gate rows and waves runs .. 2 runs-1 the up rows of
//     the slot's expert for the group's 32 features, each over its own run of whole quads
//     (4 steps of 64 K values) of the hidden dimension.  Wavefront 0 routes the token
//     (route_select over its logits) while the others write x into LDS as kXTerms FP8
//     terms with 32-value block scales, in the term-row layout below; then every
//     wavefront issues all weight loads of a batch of quads at once.  The runs' results
//     meet in LDS and are summed in run order; h = silu(g) * u is stored as kHTerms FP8
//     terms in the term-row layout for the down product.  Workgroup (0, 0) also writes
//     the routing outputs.
//   decode_down_kernel  grid (hidden / 32 row groups, 2 halves of the slots), half_slots *
//     runs waves: wave (i, p) multiplies slot i's h by its expert's down rows over run p
//     of the inter dimension; per slot the runs are summed in order, then sum_i w_i *
//     down_i over the half's slots in selection order; the two halves' sums meet by
//     atomic addition onto y, which the gate/up kernel zeroed (two addends onto zero: the
//     result does not depend on their order).
//
// Term rows: the token's activation is a sum of FP8 terms (kXTerms for x, kHTerms for h)
// sharing one E8M0 scale per 32-value block, and row k of the MFMA's A operand carries
// term k (rows past the terms are zero), so one MFMA per step multiplies every term by
// the weights and the token's product is the sum of result rows 0 .. terms-1 (accumulator
// elements 0 .. terms-1 of lanes 0..31).  Per step q of a row vector and per term k, 64
// bytes: bytes 32h .. 32h+15 hold term k of values 64q + 16h .. +15 and bytes
// 32h+16 .. 32h+31 of values 64q + 32 + 16h .. +15 (what lane k + 32h of the A operand
// holds); the block scales are shared by the rows (lane r + 32b supplies block b's).

constexpr int kDecodeWaves = 16;
constexpr unsigned kDecodeMaxSteps = 256;  // hidden / 64 of the single-token path (x in LDS)

template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    [&]<int... I>(std::integer_sequence<int, I...>) {
        (f.template operator()<I>(), ...);
    }(std::make_integer_sequence<int, N>{});
}

// One packed 32-row group of an expert as buffer resources (wave-uniform): its codes
// (steps KB) and its scale dwords (per 4 steps, 256 bytes).  Loads address a lane's bytes
// by a per-lane offset and the step by a uniform one, so a batch of loads costs one
// address register.
struct DecodeGroup {
    __amdgpu_buffer_rsrc_t codes, scales;
};

__device__ __forceinline__ DecodeGroup decode_group(const uint8_t* packed, const Packed& whole,
                                                    const Packed& one, size_t eg) {
    constexpr int kRawWord3 = 0x00020000;  // raw (untyped) buffer, 32-bit data
    DecodeGroup g;
    g.codes = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(packed + eg * one.steps * 1024), 0, int(one.steps * 1024),
        kRawWord3);
    g.scales = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(packed + whole.code_bytes + eg * one.scale_groups * 256), 0,
        int(one.scale_groups * 256), kRawWord3);
    return g;
}

// The streamed weights of quads [qb, qb + NQ) of one group: all 4 NQ code loads and NQ
// scale loads in flight at once (non-temporal), loads past the last step clamped to it.
template <int NQ> struct DecodeB {
    u32x4 c[4 * NQ];
    unsigned s[NQ];
};

template <int NQ>
__device__ __forceinline__ void decode_load_b(const DecodeGroup& g, unsigned lane, unsigned qb,
                                              unsigned steps, DecodeB<NQ>& b) {
    typedef unsigned u4 __attribute__((ext_vector_type(4)));
    constexpr int kNonTemporal = 2;
    const unsigned quads = (steps + 3) / 4;
#pragma unroll
    for (int j = 0; j < 4 * NQ; ++j) {
        const u4 v = __builtin_amdgcn_raw_buffer_load_b128(
            g.codes, int(lane * 16), int(min(4 * qb + j, steps - 1) * 1024), kNonTemporal);
        b.c[j] = u32x4{v.x, v.y, v.z, v.w};
    }
#pragma unroll
    for (int j = 0; j < NQ; ++j)
        b.s[j] = __builtin_amdgcn_raw_buffer_load_b32(
            g.scales, int(lane * 4), int(min(qb + j, quads - 1) * 256), kNonTemporal);
}

// acc += A x B over the steps of quads [qb, qb + NQ) below `end` (the end of the
// wavefront's run, or of the dimension): the lane's A operand of step q (its term row)
// from a_of(q, lo, hi) (LDS) and its scale byte from as_of(q).
template <int NQ, class AOf, class SOf>
__device__ __forceinline__ void decode_mma(const DecodeB<NQ>& b, unsigned qb, unsigned end,
                                           AOf a_of, SOf as_of, f32x16& acc) {
    static_for<4 * NQ>([&]<int J>() {
        const unsigned q = 4 * qb + J;
        if (q < end) {
            u32x4 lo, hi;
            a_of(q, lo, hi);
            acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
                a_operand(lo, hi), b_operand(b.c[J]), acc, 0 /* A: fp8 e4m3 */,
                4 /* B: fp4 e2m1 */, 0, int(as_of(q)), J % 4, int(b.s[J / 4]));
        }
    });
}

// The token's product: the sum of the term rows (accumulator elements 0 .. TERMS-1 of
// lanes 0..31), in term order.
template <int TERMS>
__device__ __forceinline__ float term_sum(const f32x16& acc) {
    float v = acc[0];
#pragma unroll
    for (int k = 1; k < TERMS; ++k)
        v += acc[k];
    return v;
}

// h of feature 32 * group + i (i = lane % 32; both halves of the wavefront hold the same
// 32 values): block scale from the half's maximum, kHTerms FP8 terms into the term-row
// layout of the slot (codes: the slot's steps, scales: its blocks); lanes < 32 store.
__device__ __forceinline__ void store_decode_h(float hv, unsigned group, unsigned lane,
                                               uint8_t* codes, uint8_t* scales) {
    const bool finite = half_max(isfinite(hv) ? 0.f : 1.f) == 0.f;
    const int e = block_exponent(half_max(fabsf(hv)));
    float v = finite ? __builtin_amdgcn_ldexpf(hv, -e) : 0.f;
    if (lane >= 32)
        return;
    const unsigned q = group / 2, b = group % 2;
    uint8_t* at = codes + size_t(q) * kHTerms * 64 + (lane / 16) * 32 + b * 16 + lane % 16;
#pragma unroll
    for (int t = 0; t < kHTerms; ++t) {
        const int c = __builtin_amdgcn_cvt_pk_fp8_f32(v, 0.f, 0, false);
        at[t * 64] = finite ? uint8_t(c & 0xff) : uint8_t(0x7f);  // 0x7f: FP8 NaN
        v -= __builtin_amdgcn_cvt_f32_fp8(c, 0);
    }
    if (lane == 0)
        scales[group] = finite ? uint8_t(e + 127) : uint8_t(255);
}

// Quarter u (values 8u .. 8u+7) of x into the term-row layout: the four lanes of a DPP
// quad hold one 32-value block (u = 4b + j, lane % 4 = j) and share its maximum and its
// finiteness, so every lane converts 8 values; lanes with `live` false take part in the
// quad reductions only.  Bit-identical to converting the block in one lane.
__device__ __forceinline__ void stage_x_quarter(const uint16_t* __restrict__ x, unsigned u,
                                                bool live, uint8_t* xq, uint8_t* xs) {
    const u32x4 w = live ? load16(reinterpret_cast<const uint8_t*>(x + 8 * u))
                         : u32x4{0u, 0u, 0u, 0u};
    const unsigned ws[4] = {w.x, w.y, w.z, w.w};
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // bf16 -> fp32 is exact
        v[2 * i] = __uint_as_float(ws[i] << 16);
        v[2 * i + 1] = __uint_as_float(ws[i] & 0xffff0000u);
    }
    float amax = 0.f, bad = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        amax = fmaxf(amax, fabsf(v[i]));
        bad = isfinite(v[i]) ? bad : 1.f;
    }
    amax = fmaxf(amax, quad_xor1(amax));
    amax = fmaxf(amax, quad_xor2(amax));
    bad = fmaxf(bad, quad_xor1(bad));
    bad = fmaxf(bad, quad_xor2(bad));
    if (!live)
        return;
    const bool finite = bad == 0.f;
    const int e = block_exponent(amax);
    unsigned t[kXTerms][2];
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        float q[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            q[i] = finite ? __builtin_amdgcn_ldexpf(v[4 * d + i], -e) : 0.f;
#pragma unroll
        for (int k = 0; k < kXTerms; ++k) {
            const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
            const int both = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], lo, true);
            t[k][d] = finite ? unsigned(both) : 0x7f7f7f7fu;
            if (k + 1 < kXTerms) {  // the remainder is exact in fp32 (Sterbenz)
                q[0] -= __builtin_amdgcn_cvt_f32_fp8(both, 0);
                q[1] -= __builtin_amdgcn_cvt_f32_fp8(both, 1);
                q[2] -= __builtin_amdgcn_cvt_f32_fp8(both, 2);
                q[3] -= __builtin_amdgcn_cvt_f32_fp8(both, 3);
            }
        }
    }
    const unsigned b = u / 4, j = u % 4;
    uint8_t* at = xq + (b / 2) * kXTerms * 64 + (j / 2) * 32 + (b % 2) * 16 + (j % 2) * 8;
#pragma unroll
    for (int k = 0; k < kXTerms; ++k)
        *reinterpret_cast<uint2*>(at + k * 64) = make_uint2(t[k][0], t[k][1]);
    if (j == 0)
        xs[b] = finite ? uint8_t(e + 127) : uint8_t(255);
}

template <int NQ, int R>
__global__ __launch_bounds__(kDecodeWaves * 64) void decode_gate_up_kernel(
    const uint16_t* __restrict__ x, const float* __restrict__ logits, unsigned hidden,
    unsigned inter, unsigned experts, unsigned top_k, const uint8_t* __restrict__ gate,
    const uint8_t* __restrict__ up, unsigned runs, unsigned run_quads,
    int32_t* __restrict__ idx, float* __restrict__ weight, int32_t* __restrict__ offsets,
    int32_t* __restrict__ perm, uint8_t* __restrict__ hq, uint8_t* __restrict__ hs,
    float* __restrict__ y_zero) {
    // x in the term-row layout (every step), its block scales, 32 zero bytes
    __shared__ __align__(16) uint8_t xq[kDecodeMaxSteps * kXTerms * 64 + 32];
    __shared__ uint8_t xs[kDecodeMaxSteps * 2];
    __shared__ int s_expert;
    __shared__ float red[kDecodeWaves][32];
    // the wavefront index as a uniform value (the weight loads' offsets and resources are
    // per wavefront)
    const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
    const unsigned steps = hidden / 64, quads = (steps + 3) / 4;
    const unsigned slot = blockIdx.y, group = blockIdx.x;
    uint8_t* zero = xq + steps * kXTerms * 64;
    if (y_zero) {  // the output the down kernel's two halves add into
        const unsigned wg = blockIdx.y * gridDim.x + blockIdx.x, wgs = gridDim.x * gridDim.y;
        for (unsigned i = wg * blockDim.x + threadIdx.x; i < hidden; i += wgs * blockDim.x)
            y_zero[i] = 0.f;
    }
    if (wave == 0) {
        // wavefront 0 routes the token (a few hundred bytes of logits) ...
        int selected;
        float selected_weight;
        route_select_r<R>(logits, 0, experts, top_k, lane, selected, selected_weight);
        if (lane == 0)
            s_expert = __builtin_amdgcn_readlane(selected, slot);
        if (blockIdx.x == 0 && blockIdx.y == 0) {
            // routing outputs; the experts of one token are distinct, so a slot's position
            // in the permutation is the number of selected experts below its own
            int lower = 0;
            for (unsigned j = 0; j < top_k; ++j)
                lower += __builtin_amdgcn_readlane(selected, j) < selected;
            if (lane < top_k) {
                idx[lane] = selected;
                weight[lane] = selected_weight;
                perm[lower] = int(lane);
            }
            for (unsigned b = lane; b <= experts; b += 64) {
                int below = 0;
                for (unsigned j = 0; j < top_k; ++j)
                    below += __builtin_amdgcn_readlane(selected, j) < int(b);
                offsets[b] = below;
            }
        }
    } else {
        // ... while the others write x as FP8 terms into LDS, one lane per 8 values
        if (threadIdx.x - 64 < 8)
            reinterpret_cast<unsigned*>(zero)[threadIdx.x - 64] = 0u;
        for (unsigned first = 0; first < 8 * steps; first += blockDim.x - 64) {
            const unsigned u = first + threadIdx.x - 64;
            if (__ballot(u < 8 * steps))  // whole wavefronts (the quads reduce by DPP)
                stage_x_quarter(x, u, u < 8 * steps, xq, xs);
        }
    }
    __syncthreads();
    const unsigned m = wave / runs, run = wave % runs;  // m = 0: gate rows, 1: up rows
    const unsigned qa = run * run_quads, qe = min(quads, qa + run_quads);
    const Packed whole = packed_shape(experts, inter, hidden), one = packed_shape(1, inter, hidden);
    const int expert = __builtin_amdgcn_readfirstlane(s_expert);
    const DecodeGroup wg =
        decode_group(m ? up : gate, whole, one, size_t(expert) * one.groups + group);
    // lane k + 32h reads term k's half h (rows past the terms read the zero bytes)
    const unsigned row = lane % 32;
    const uint8_t* xa = row < kXTerms ? xq + row * 64 + (lane / 32) * 32 : zero;
    const unsigned xstep = row < kXTerms ? kXTerms * 64 : 0;
    auto a_of = [&](unsigned q, u32x4& lo, u32x4& hi) {
        lo = *reinterpret_cast<const u32x4*>(xa + q * xstep);
        hi = *reinterpret_cast<const u32x4*>(xa + q * xstep + 16);
    };
    auto as_of = [&](unsigned q) { return unsigned(xs[2 * q + lane / 32]); };
    f32x16 acc = {};
    for (unsigned qb = qa; qb < qe; qb += NQ) {
        DecodeB<NQ> b;
        decode_load_b<NQ>(wg, lane, qb, steps, b);
        decode_mma<NQ>(b, qb, min(4 * qe, steps), a_of, as_of, acc);
    }
    if (lane < 32)
        red[wave][lane] = term_sum<kXTerms>(acc);
    __syncthreads();
    if (wave == 0) {
        const unsigned i = lane % 32;
        float g = 0.f, u = 0.f;
        for (unsigned r = 0; r < runs; ++r)
            g += red[r][i];
        for (unsigned r = 0; r < runs; ++r)
            u += red[runs + r][i];
        store_decode_h(silu(g) * u, group, lane, hq + size_t(slot) * (inter / 64) * kHTerms * 64,
                       hs + size_t(slot) * (inter / 32));
    }
}

// Per wavefront of decode_down_kernel, one batch of h in LDS: 4 NQ steps of kHTerms * 64
// code bytes, copied as whole 16-byte pieces per lane (the copy rounded up to 64 pieces),
// then their 8 NQ block scales.
template <int NQ> constexpr unsigned decode_stage_pieces() {
    return (4 * NQ * kHTerms * 64 / 16 + 63) / 64;  // per lane
}
template <int NQ> constexpr unsigned decode_stage_bytes() {
    return decode_stage_pieces<NQ>() * 64 * 16 + 8 * NQ;
}

template <int NQ>
__global__ __launch_bounds__(kDecodeWaves * 64) void decode_down_kernel(
    const uint8_t* __restrict__ hq, const uint8_t* __restrict__ hs, unsigned hidden,
    unsigned inter, unsigned experts, unsigned top_k, const uint8_t* __restrict__ down,
    const int32_t* __restrict__ idx, const float* __restrict__ weight, unsigned runs,
    unsigned run_quads, unsigned half_slots, float* __restrict__ y) {
    constexpr unsigned kStage = decode_stage_bytes<NQ>();
    constexpr unsigned kPieces = decode_stage_pieces<NQ>();  // per lane
    constexpr unsigned kScalesAt = kPieces * 64 * 16;
    __shared__ __align__(16) uint8_t stage[kDecodeWaves][kStage];
    __shared__ float red[kDecodeWaves][32];
    __shared__ __align__(16) uint8_t zero32[32];
    // the wavefront index as a uniform value (the weight loads' offsets and resources are
    // per wavefront)
    const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
    // this workgroup's half of the slots: [first_slot, last_slot)
    const unsigned first_slot = blockIdx.y * half_slots;
    const unsigned last_slot = min(top_k, first_slot + half_slots);
    const unsigned slot = first_slot + wave / runs, run = wave % runs;
    if (threadIdx.x < 8)
        reinterpret_cast<unsigned*>(zero32)[threadIdx.x] = 0u;
    __syncthreads();
    const unsigned steps = inter / 64, quads = (steps + 3) / 4;
    const unsigned group = blockIdx.x;
    f32x16 acc = {};
    if (slot < last_slot) {
        const Packed whole = packed_shape(experts, hidden, inter),
                     one = packed_shape(1, hidden, inter);
        const int expert = __builtin_amdgcn_readfirstlane(idx[slot]);
        const DecodeGroup wg = decode_group(down, whole, one, size_t(expert) * one.groups + group);
        const uint8_t* h_codes = hq + size_t(slot) * steps * kHTerms * 64;  // the slot's h
        const uint8_t* h_scales = hs + size_t(slot) * (inter / 32);
        uint8_t* mine = stage[wave];
        unsigned base = 0;  // the batch's first step
        // lane k + 32h reads term k's half h (rows past the terms read the zero block)
        const unsigned row = lane % 32;
        const uint8_t* ha = row < kHTerms ? mine + row * 64 + (lane / 32) * 32 : zero32;
        const unsigned hstep = row < kHTerms ? kHTerms * 64 : 0;
        auto a_of = [&](unsigned q, u32x4& lo, u32x4& hi) {
            const uint8_t* p = ha + (q - base) * hstep;
            lo = *reinterpret_cast<const u32x4*>(p);
            hi = *reinterpret_cast<const u32x4*>(p + 16);
        };
        auto as_of = [&](unsigned q) {
            return unsigned(mine[kScalesAt + 2 * (q - base) + lane / 32]);
        };
        const unsigned qe = min(quads, (run + 1) * run_quads);
        for (unsigned qb = run * run_quads; qb < qe; qb += NQ) {
            base = 4 * qb;
            // this batch's h (the steps of quads qb .., contiguous in the slot's h) first:
            // cache hits that arrive before the weights; then every weight load of the batch
            const size_t first = size_t(4 * qb) * kHTerms * 64, end = size_t(steps) * kHTerms * 64;
            u32x4 piece[kPieces];
#pragma unroll
            for (unsigned j = 0; j < kPieces; ++j) {
                const size_t at = first + 16 * size_t(lane + 64 * j);
                piece[j] = load16(h_codes + min(at, end - 16));
            }
            const unsigned scale_at = min(8 * qb + lane, inter / 32 - 1);
            const uint8_t scale = h_scales[scale_at];
            DecodeB<NQ> b;
            decode_load_b<NQ>(wg, lane, qb, steps, b);
#pragma unroll
            for (unsigned j = 0; j < kPieces; ++j)
                *reinterpret_cast<u32x4*>(mine + 16 * (lane + 64 * j)) = piece[j];
            if (lane < 8 * NQ)
                mine[kScalesAt + lane] = scale;
            decode_mma<NQ>(b, qb, min(4 * qe, steps), a_of, as_of, acc);
        }
    }
    if (lane < 32)
        red[wave][lane] = term_sum<kHTerms>(acc);
    __syncthreads();
    if (wave == 0 && lane < 32) {
        float sum = 0.f;
        for (unsigned i = first_slot; i < last_slot; ++i) {
            float d = 0.f;
            for (unsigned r = 0; r < runs; ++r)
                d += red[(i - first_slot) * runs + r][lane];
            sum += d * weight[i];
        }
        // two halves meet by atomic addition onto the zeroed output: 0 + a + b is the same
        // float whichever half arrives first
        if (gridDim.y == 1)
            y[size_t(group) * 32 + lane] = sum;
        else if (first_slot < last_slot)
            atomicAdd(y + size_t(group) * 32 + lane, sum);
    }
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
    int32_t *idx, *offsets, *perm, *position, *slot_row, *items, *item_count;
    float* weight;
    uint8_t *xa, *ha;  // activation tiles of gate/up (x) and of down (h)
    float *part_g, *part_u, *part_d;
};

// Grid columns of the grouped GEMMs: kGemmWaves feature groups of 32 (gate/up) or row
// pairs of 64 (down) per workgroup.
unsigned gate_up_columns(size_t inter) {
    return unsigned((inter / 32 + kGemmWaves - 1) / kGemmWaves);
}

unsigned down_columns(size_t hidden) {
    return unsigned((hidden / 64 + kDownWaves - 1) / kDownWaves);
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
    // workgroups for about two gate/up (four waves) or one down (eight waves) per compute
    // unit
    auto slices = [&](size_t columns, size_t steps, size_t per_cu, bool round_up) {
        const size_t target = per_cu * size_t(compute_units());
        size_t ks = round_up ? (target + columns * items - 1) / (columns * items)
                             : target / (columns * items);
        ks = std::min(std::max<size_t>(ks, 1), steps);
        const size_t per = ((steps + ks - 1) / ks + 7) / 8 * 8;
        return unsigned((steps + per - 1) / per);
    };
    // down rounds down: its workgroups (one per compute unit at its register count) then
    // run in one round rather than one and a part (C4 T=256: 1 slice, 192 workgroups)
    return MoeSlices{slices(gate_up_columns(inter), hidden / kStepK, 2, true),
                     slices(down_columns(hidden), inter / kStepK, 1, false)};
}

size_t align256(size_t n) {
    return (n + 255) & ~size_t(255);
}

// Work items of a layer (upper bound) and activation tiles (two per item).
size_t max_items(size_t slots, size_t experts) {
    return std::min(slots, slots / kItemRows + experts + 1);
}


size_t moe_scratch_bytes(size_t tokens, size_t hidden, size_t inter, size_t experts,
                         size_t top_k, MoeSlices ks) {
    const size_t slots = tokens * top_k, items = slots / kItemRows + experts + 1;
    const size_t tiles = 2 * max_items(slots, experts);
    const size_t partial_gu =
        ks.gate_up > 1 ? 2 * align256(ks.gate_up * tiles * kTileRows * inter * 4) : 0;
    return align256(slots * 4) * 5 + align256((experts + 1) * 4) + align256(items * 8) +
           align256(4) + align256(tile_bytes(tiles, hidden / 64, kXTerms)) +
           align256(tile_bytes(tiles, inter / 64, kHTerms)) + partial_gu +
           align256(ks.down * slots * hidden * 4);
}

MoeScratch carve(uint8_t* p, size_t tokens, size_t hidden, size_t inter, size_t experts,
                 size_t top_k, MoeSlices ks) {
    const size_t slots = tokens * top_k, items = slots / kItemRows + experts + 1;
    const size_t tiles = 2 * max_items(slots, experts);
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
    s.slot_row = reinterpret_cast<int32_t*>(take(slots * 4));
    s.offsets = reinterpret_cast<int32_t*>(take((experts + 1) * 4));
    s.items = reinterpret_cast<int32_t*>(take(items * 8));
    s.item_count = reinterpret_cast<int32_t*>(take(4));
    s.xa = take(tile_bytes(tiles, hidden / 64, kXTerms));
    s.ha = take(tile_bytes(tiles, inter / 64, kHTerms));
    s.part_g = s.part_u = nullptr;
    if (ks.gate_up > 1) {
        s.part_g = reinterpret_cast<float*>(take(ks.gate_up * tiles * kTileRows * inter * 4));
        s.part_u = reinterpret_cast<float*>(take(ks.gate_up * tiles * kTileRows * inter * 4));
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

// Scratch words of the chunked permutation (slot ranks, then per chunk a count per expert).
size_t chunk_scratch_words(size_t slots, size_t experts) {
    return slots + (slots + 1023) / 1024 * experts;
}

// `chunk_scratch` (chunk_scratch_words int32, or null): with more than kOneWgSlots slots
// the permutation runs chunked in two launches there.
constexpr size_t kOneWgSlots = 4096;

int launch_route(const float* logits, size_t tokens, size_t experts, size_t top_k,
                 int32_t* idx, float* w, int32_t* offsets, int32_t* perm, int32_t* items,
                 int32_t* item_count, int32_t* position, int32_t* slot_row,
                 int32_t* chunk_scratch, hipStream_t stream) {
    launch_route_selection(logits, tokens, experts, top_k, idx, w, stream);
    KDQ_HIP(hipGetLastError());
    // heavy items first when an average expert's rows fit one work item (the grouped
    // GEMMs' workgroups then all fit the compute units at once)
    const size_t slots = tokens * top_k;
    const unsigned heavy_first = slots <= experts * (kItemRows / 2) ? 1u : 0u;
    if (chunk_scratch && slots > kOneWgSlots) {
        const unsigned chunks = unsigned((slots + 1023) / 1024);
        int32_t* rank = chunk_scratch;
        int32_t* counts = chunk_scratch + slots;
        hipLaunchKernelGGL(chunk_count_kernel, dim3(chunks), dim3(1024), 0, stream, idx,
                           unsigned(slots), unsigned(experts), counts, rank);
        KDQ_HIP(hipGetLastError());
        hipLaunchKernelGGL(chunk_place_kernel, dim3(chunks), dim3(1024), 0, stream, idx,
                           unsigned(slots), unsigned(experts), heavy_first, counts, rank, offsets,
                           perm, items, item_count, position, slot_row);
    } else {
        hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(1024), 0, stream, idx, unsigned(slots),
                           unsigned(experts), offsets, perm, items, item_count, position,
                           slot_row, heavy_first);
    }
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}

}  // namespace
}  // namespace kdq

using namespace kdq;

namespace kdq {

int route_selection(const float* logits, size_t tokens, size_t experts, size_t top_k,
                    int32_t* idx, float* w, hipStream_t stream) {
    const int rc = check_route(logits, tokens, experts, top_k);
    if (rc)
        return rc;
    launch_route_selection(logits, tokens, experts, top_k, idx, w, stream);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}

}  // namespace kdq

extern "C" int kdq_moe_route(const float* logits, size_t tokens, size_t experts, size_t top_k,
                             int32_t* idx, float* w, int32_t* offsets, int32_t* perm,
                             void* stream) {
    int rc = check_route(logits, tokens, experts, top_k);
    if (rc)
        return rc;
    if (!idx || !w || !offsets || !perm)
        return KDQ_ERR_ARGUMENT;
    const size_t items = tokens * top_k / kItemRows + experts + 1, slots = tokens * top_k;
    auto* scratch = static_cast<int32_t*>(
        workspace(items * 8 + 256 + slots * 4 + chunk_scratch_words(slots, experts) * 4, &rc));
    if (rc)
        return rc;
    return launch_route(logits, tokens, experts, top_k, idx, w, offsets, perm, scratch,
                        scratch + items * 2, nullptr, scratch + items * 2 + 64,
                        scratch + items * 2 + 64 + slots, static_cast<hipStream_t>(stream));
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

// The single-token path (decode_gate_up_kernel + decode_down_kernel) takes one token
// whose x steps fit the gate/up kernel's LDS.
bool single_token_path(size_t tokens, size_t hidden) {
    return tokens == 1 && hidden / kStepK <= kDecodeMaxSteps;
}

// Runs of whole quads per wavefront: gate/up up to 8 runs per matrix, down up to
// 16 / ceil(top_k / 2) runs per slot (a down workgroup takes half the slots); `quads` per
// run.
struct DecodePlan {
    unsigned gu_runs, gu_quads, dn_runs, dn_quads;
};

DecodePlan decode_plan(size_t hidden, size_t inter, size_t top_k) {
    const unsigned qh = unsigned((hidden / kStepK + 3) / 4), qi = unsigned((inter / kStepK + 3) / 4);
    const unsigned gq = (qh + 7) / 8, gr = (qh + gq - 1) / gq;
    const unsigned half = unsigned((top_k + 1) / 2);  // slots per down workgroup
    const unsigned dmax = std::max(1u, unsigned(kDecodeWaves / half));
    const unsigned dq = (qi + dmax - 1) / dmax, dr = (qi + dq - 1) / dq;
    return DecodePlan{gr, gq, dr, dq};
}

// The single-token layer: h in the term-row layout at the start of the scratch's h
// tiles (top_k * inter / 64 steps of kHTerms * 64 bytes, then top_k * inter / 32 scale
// bytes; the tiles hold far more).
int launch_decode(const uint16_t* x_bf16, const float* logits, size_t hidden, size_t inter,
                  size_t experts, size_t top_k, const uint8_t* gate, const uint8_t* up,
                  const uint8_t* down, float* y, const MoeScratch& s, hipStream_t st) {
    const DecodePlan p = decode_plan(hidden, inter, top_k);
    const unsigned half = unsigned((top_k + 1) / 2), halves = top_k > 1 ? 2u : 1u;
    uint8_t* hq = s.ha;
    uint8_t* hs = s.ha + align256(top_k * (inter / kStepK) * kHTerms * 64);
    const dim3 gu_grid(unsigned(inter / 32), unsigned(top_k));
    const dim3 gu_block(2 * p.gu_runs * 64);
    auto gate_up = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, gu_grid, gu_block, 0, st, x_bf16, logits, unsigned(hidden),
                           unsigned(inter), unsigned(experts), unsigned(top_k), gate, up,
                           p.gu_runs, p.gu_quads, s.idx, s.weight, s.offsets, s.perm, hq, hs,
                           halves > 1 ? y : nullptr);
    };
    const bool few = experts <= 64;  // one routing probability per lane
    if (p.gu_quads == 1)
        few ? gate_up(decode_gate_up_kernel<1, 1>) : gate_up(decode_gate_up_kernel<1, 4>);
    else
        few ? gate_up(decode_gate_up_kernel<2, 1>) : gate_up(decode_gate_up_kernel<2, 4>);
    KDQ_HIP(hipGetLastError());
    const dim3 dn_grid(unsigned(hidden / 32), halves), dn_block(half * p.dn_runs * 64);
    auto down_launch = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dn_grid, dn_block, 0, st, hq, hs, unsigned(hidden),
                           unsigned(inter), unsigned(experts), unsigned(top_k), down, s.idx,
                           s.weight, p.dn_runs, p.dn_quads, half, y);
    };
    if (p.dn_quads == 1)
        down_launch(decode_down_kernel<1>);
    else if (p.dn_quads == 2)
        down_launch(decode_down_kernel<2>);
    else
        down_launch(decode_down_kernel<3>);
    KDQ_HIP(hipGetLastError());
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
    const size_t slots = tokens * top_k;
    const unsigned items = unsigned(max_items(slots, experts));
    const size_t tiles = 2 * size_t(items);
    if (single_token_path(tokens, hidden))
        return launch_decode(x_bf16, logits, hidden, inter, experts, top_k, gate, up, down, y, s,
                             st);
    const bool small = slots <= size_t(kPrologueSlots);
    if (small) {
        const size_t x_bytes = tokens * hidden * 2;
        hipLaunchKernelGGL(prologue_kernel, dim3(1), dim3(1024),
                           x_bytes <= kPrologueXBytes ? x_bytes : 0, st, logits,
                           unsigned(tokens), unsigned(experts), unsigned(top_k), s.idx, s.weight,
                           s.offsets, s.perm, s.items, s.item_count, s.position, s.slot_row,
                           x_bf16, unsigned(hidden), s.xa, tiles);
        KDQ_HIP(hipGetLastError());
    } else {
        // the activation tiles are written after the permutation: their space holds its
        // chunked form's scratch meanwhile
        const bool room = chunk_scratch_words(slots, experts) * 4 <=
                          tile_bytes(tiles, hidden / 64, kXTerms);
        int rc = launch_route(logits, tokens, experts, top_k, s.idx, s.weight, s.offsets, s.perm,
                              s.items, s.item_count, s.position, s.slot_row,
                              room ? reinterpret_cast<int32_t*>(s.xa) : nullptr, st);
        if (rc)
            return rc;
        hipLaunchKernelGGL(gather_kernel,
                           dim3(unsigned((32 * (hidden / 32) + 255) / 256), unsigned(tiles)),
                           dim3(256), 0, st, x_bf16, unsigned(hidden), unsigned(top_k),
                           s.offsets, s.perm, s.items, s.item_count, s.xa, tiles);
        KDQ_HIP(hipGetLastError());
    }
    // Weights stream with the non-temporal policy when an average expert's rows fit one
    // work item (each weight byte is then read once per call); with more rows, items of
    // one expert re-read its weights and the caches help (C4 T=256: 174 -> 169 us with
    // it; C5: 0.75 -> 0.77 ms).
    const bool nt = slots <= experts * (kItemRows / 2);
    const size_t part_gu = tiles * kTileRows * inter;
    // (column, item) cells in one grid dimension, items padded to a multiple of 8
    // (item_cell: an item's columns on one XCD)
    const unsigned items8 = (items + 7) / 8 * 8;
    const unsigned gu_cols = gate_up_columns(inter), d_cols = down_columns(hidden);
    const dim3 gu_grid(gu_cols * items8, 1, ks.gate_up);
    if (nt)
        hipLaunchKernelGGL(gate_up_kernel<true>, gu_grid, dim3(kGemmWaves * 64), 0, st, s.xa,
                           unsigned(hidden), unsigned(inter), unsigned(experts), tiles, gate, up,
                           s.offsets, s.items, s.item_count, s.ha, s.part_g, s.part_u, part_gu,
                           gu_cols);
    else
        hipLaunchKernelGGL(gate_up_kernel<false>, gu_grid, dim3(kGemmWaves * 64), 0, st, s.xa,
                           unsigned(hidden), unsigned(inter), unsigned(experts), tiles, gate, up,
                           s.offsets, s.items, s.item_count, s.ha, s.part_g, s.part_u, part_gu,
                           gu_cols);
    KDQ_HIP(hipGetLastError());
    if (ks.gate_up > 1) {
        hipLaunchKernelGGL(finalize_kernel, dim3(unsigned((inter + 255) / 256), unsigned(slots)),
                           dim3(256), 0, st, s.part_g, s.part_u, part_gu, unsigned(inter),
                           ks.gate_up, s.slot_row, s.ha, tiles);
        KDQ_HIP(hipGetLastError());
    }
    const size_t stride = slots * hidden;
    const dim3 d_grid(d_cols * items8, 1, ks.down);
    if (nt)
        hipLaunchKernelGGL(down_kernel<true>, d_grid, dim3(kDownWaves * 64), 0, st, s.ha, tiles,
                           unsigned(hidden), unsigned(inter), unsigned(experts), down, s.offsets,
                           s.items, s.item_count, s.part_d, stride, d_cols);
    else
        hipLaunchKernelGGL(down_kernel<false>, d_grid, dim3(kDownWaves * 64), 0, st, s.ha, tiles,
                           unsigned(hidden), unsigned(inter), unsigned(experts), down, s.offsets,
                           s.items, s.item_count, s.part_d, stride, d_cols);
    KDQ_HIP(hipGetLastError());
    const size_t n = tokens * hidden / 4;
    const dim3 grid(unsigned((n + 255) / 256));
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

// Scratch of kdq_moe_mxfp4_packed_noalloc: a file-scope device array, so that entry point
// never allocates.  Every device the library runs on holds its own copy until the process
// ends, and every call on a device shares that copy (calls that overlap on one device
// race).  The layer's kernels write every scratch byte they later read, so nothing needs
// clearing between calls.
static __device__ __align__(256) uint8_t scratch[kdq::kNoAllocScratchBytes];

namespace kdq {
namespace {
constexpr int kMaxDevices = 64;
std::mutex noalloc_mutex;
uint8_t* noalloc_address[kMaxDevices];  // the device address of `scratch`, per device

// The current device's address of `scratch`, looked up once per device with that device
// current (the host-side name of the array is not a device address).
int noalloc_scratch(uint8_t** out) {
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess)
        return hip_failure(e);
    if (device < 0 || device >= kMaxDevices)
        return KDQ_ERR_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(noalloc_mutex);
    if (!noalloc_address[device]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess)
            return hip_failure(e);
        noalloc_address[device] = static_cast<uint8_t*>(p);
    }
    *out = noalloc_address[device];
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
    auto* work = static_cast<uint8_t*>(
        workspace(moe_scratch_bytes(tokens, hidden, inter, experts, top_k, ks), &rc));
    if (rc)
        return rc;
    return launch_layer(x_bf16, logits, tokens, hidden, inter, experts, top_k, gate, up, down,
                        y, idx, w, offsets, perm, work, ks, static_cast<hipStream_t>(stream));
}

// The allocation-free variant of kdq_moe_mxfp4_packed: the same kernels, with the layer's
// scratch in the file-scope device array below instead of the per-device workspace.
extern "C" int kdq_moe_mxfp4_packed_noalloc(const uint16_t* x_bf16, const float* logits,
                                            size_t tokens, size_t hidden, size_t inter,
                                            size_t experts, size_t top_k, const uint8_t* gate,
                                            const uint8_t* up, const uint8_t* down, float* y,
                                            int32_t* idx, float* w, int32_t* offsets,
                                            int32_t* perm, void* stream) {
    int rc = check_layer(x_bf16, logits, tokens, hidden, inter, experts, top_k, y);
    if (rc)
        return rc;
    if (!gate || !up || !down)
        return KDQ_ERR_ARGUMENT;
    if (misaligned(gate, 256) || misaligned(up, 256) || misaligned(down, 256))
        return KDQ_ERR_ALIGNMENT;
    const MoeSlices ks = moe_slices(tokens, hidden, inter, experts, top_k);
    if (moe_scratch_bytes(tokens, hidden, inter, experts, top_k, ks) > kdq::kNoAllocScratchBytes)
        return KDQ_ERR_SCRATCH;  // the layer's scratch does not fit the static array
    uint8_t* work = nullptr;
    if ((rc = kdq::noalloc_scratch(&work)))
        return rc;
    return launch_layer(x_bf16, logits, tokens, hidden, inter, experts, top_k, gate, up, down,
                        y, idx, w, offsets, perm, work, ks, static_cast<hipStream_t>(stream));
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
