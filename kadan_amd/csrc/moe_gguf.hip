// GGUF mixture-of-experts layer on the device: the Qwen MoE layer of
// IW/src/models/text/qwen_layers.cpp:378-492 (MoeLayer::forward; IW =
// services/hikari/inference_worker) as one stream-ordered submission, with no host round
// trip between its stages (the reference returns to the host three times per layer).
//
// Stages, all on `stream`:
//   1. one GEMV batch over x: router logits and the shared expert's gate and up rows, as
//      one paired MFMA job that writes silu(gate) * up when the kernel takes the pair
//      (gate and up stored alike)
//   2. routing (route_selection: the kdq_moe_route kernel; softmax with a double total,
//      top-k by probability, weights renormalised by max(sum, 2^-14))
//   3. swiglu_kernel on the shared rows, unless paired in 1
//   4. one launch of every slot's expert gate / up GEMV (slot s reads token s / top_k's
//      row), each job's weights starting at the expert slice the routing wrote on the
//      device; paired with the swiglu like 1, else gate and up launches and swiglu_kernel
//   5. one launch of every slot's expert down GEMV, plus the shared expert's down
//   6. combine_kernel: y = sum over the selections, in selection order, of down * weight,
//      plus shared_down * sigmoid(ffn_gate_inp_shexp . x); the scalar is taken inside the
//      combine (a dot product of H values per workgroup), not by a launch of its own
// GEMVs of Q4_0 / Q8_0 / Q4_K / Q3_K / Q6_K / IQ4_XS / IQ4_NL run on the MFMA kernel
// (fused per shape), every other encoding on the exact kernel.
//
// Batches of more than kSlotRows rows (prefill chunks; the reference runs MoeLayer::forward
// on them with per-expert batch jobs of gathered rows, IW/include/kadan/dense_compute.hpp:
// 197-201) take stages 4-6 grouped by expert instead of per slot, so each expert's
// weights are read once per 8 of its rows rather than once per slot:
//   4'. group_kernel: a counting sort of the slots by expert into segments padded to whole
//       items of kItemRows rows (slot -> position, position -> slot, the expert of every
//       item, -1 past the used ones); gather_kernel: x rows into position order (padding
//       rows zero)
//   4''. one launch over the items of expert gate / up (8 rows each, weights at the
//       item's expert), paired with the swiglu like 4
//   5'. one launch over the items of expert down, plus the shared down
//   6'. combine_kernel as 6, each slot's down row read at its position
#include "kdq_common.hpp"

#include <algorithm>
#include <vector>

namespace kdq {
namespace {

// gate[i] = silu(gate[i]) * up[i] for i < n; grouped layers: only rows below *used of
// `width` values that hold a slot (padding rows of zero x keep gate = up = 0, which is
// already silu(0) * 0)
__global__ __launch_bounds__(256) void swiglu_kernel(float* gate, const float* up, size_t n,
                                                     const unsigned* used, unsigned width,
                                                     const int32_t* slot_of) {
    const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n)
        return;
    if (used && (i / width >= *used || slot_of[i / width] < 0))
        return;
    gate[i] = silu_of(gate[i]) * up[i];
}

// y[t, d] = (sum_{i < k} down[row(t, i), d] * w[t*k + i]) + shared[t, d] * sigmoid(s_t),
// row(t, i) = t*k + i (slot order) or pos[t*k + i] (grouped layers), in selection order;
// s_t = ffn_gate_inp_shexp . x[t], which every workgroup of token t takes itself in one
// fixed order (thread j: its float4 columns j, j + 256, ... with the four products of each
// fused in turn; the wavefront: an xor butterfly, which leaves the same float in every
// lane; the four wavefronts: (0 + 1) + (2 + 3)), so all of them use the same value.
// A non-finite value of ffn_gate_inp_shexp sets bit 1 of `status` (when given), as every
// other weight of the layer does; workgroup (0, 0) reports it, having read every value.
// Grid (ceil(hidden / 1024), tokens), 256 threads of 4 consecutive d each.
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ down,
                                                      const int32_t* __restrict__ pos,
                                                      const float* __restrict__ w,
                                                      const float* __restrict__ shared,
                                                      const float* __restrict__ gate_vector,
                                                      const float* __restrict__ x, unsigned k,
                                                      unsigned hidden, float* __restrict__ y,
                                                      unsigned* __restrict__ status) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    __shared__ float wave_sum[4];
    __shared__ int wave_bad[4];
    const size_t t = blockIdx.y;
    const unsigned quads = hidden / 4;
    const f32x4* xr = reinterpret_cast<const f32x4*>(x + t * hidden);
    const f32x4* vr = reinterpret_cast<const f32x4*>(gate_vector);
    float s = 0.f;
    bool finite = true;
    for (unsigned q = threadIdx.x; q < quads; q += 256) {
        const f32x4 a = xr[q], b = vr[q];
        finite = finite && isfinite(b.x) && isfinite(b.y) && isfinite(b.z) && isfinite(b.w);
        s = fmaf(a.x, b.x, s);
        s = fmaf(a.y, b.y, s);
        s = fmaf(a.z, b.z, s);
        s = fmaf(a.w, b.w, s);
    }
    for (int m = 32; m >= 1; m /= 2)
        s += __shfl_xor(s, m, 64);
    const bool bad = __any(!finite);
    if (threadIdx.x % 64 == 0) {
        wave_sum[threadIdx.x / 64] = s;
        wave_bad[threadIdx.x / 64] = bad;
    }
    __syncthreads();
    if (status && threadIdx.x == 0 && blockIdx.x == 0 && blockIdx.y == 0 &&
        (wave_bad[0] | wave_bad[1] | wave_bad[2] | wave_bad[3]))
        atomicOr(status, 1u);
    const float gate = sigmoid_of((wave_sum[0] + wave_sum[1]) + (wave_sum[2] + wave_sum[3]));
    const unsigned q = blockIdx.x * 256 + threadIdx.x;
    if (q >= quads)
        return;
    f32x4 sum = {0.f, 0.f, 0.f, 0.f};
    for (unsigned i = 0; i < k; ++i) {
        const size_t slot = t * k + i;
        const size_t row = pos ? size_t(pos[slot]) : slot;
        sum += *reinterpret_cast<const f32x4*>(down + row * hidden + 4 * size_t(q)) * w[slot];
    }
    const size_t at = t * hidden + 4 * size_t(q);
    *reinterpret_cast<f32x4*>(y + at) = sum + *reinterpret_cast<const f32x4*>(shared + at) * gate;
}

constexpr size_t kSlotRows = 8;          // batches up to this many rows run per slot
constexpr unsigned kItemRows = 8;        // rows of a grouped item (the MFMA GEMV's batch)
constexpr unsigned kTileRows = kGroupedTileRows;  // rows of a grouped GEMM token tile
constexpr size_t kMaxGroupedSlots = 8192;
// Batches from this many rows run the shared expert on the prefill GEMM (its launches
// cost more than the 8-row items below that: measured at 64 rows 33 us slower, at 512
// rows 65 us faster)
constexpr size_t kSharedGemmRows = 256;
constexpr size_t kDecodeCounters = 1024;  // row blocks of the fused decode's down launch

// Slots by expert into segments padded to multiples of `pad` (kItemRows, or kTileRows when
// a projection runs on the grouped GEMM): pos[s] (slot -> position), inv[p] (position ->
// slot, -1 for padding), item_expert[i] for the kItemRows-row items (-1 for items of
// padding only and past the used ones), tile_expert[j] for the kTileRows-row tiles when
// pad == kTileRows (-1 past the used ones), *used = positions in use, *gemm_status = 0.
// Positions within an expert follow the order of an LDS atomic (each slot's result depends
// only on its own row, so the layer's output does not).  One workgroup of 1024 threads;
// experts <= 256.
__global__ __launch_bounds__(1024) void group_kernel(const int32_t* __restrict__ idx,
                                                     unsigned slots, unsigned experts,
                                                     unsigned pad, unsigned max_items,
                                                     int32_t* __restrict__ pos,
                                                     int32_t* __restrict__ inv,
                                                     int32_t* __restrict__ item_expert,
                                                     int32_t* __restrict__ tile_expert,
                                                     unsigned* __restrict__ used,
                                                     unsigned* __restrict__ gemm_status) {
    __shared__ unsigned count[256], start[256], fill[256];
    __shared__ unsigned total;
    const unsigned t = threadIdx.x;
    if (t < 256) {
        count[t] = 0;
        fill[t] = 0;
    }
    __syncthreads();
    for (unsigned s = t; s < slots; s += 1024)
        atomicAdd(&count[min(unsigned(idx[s]), experts - 1)], 1u);
    __syncthreads();
    if (t < 64) {  // exclusive scan of the padded counts, four experts per lane
        unsigned padded[4], sum = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const unsigned e = 4 * t + k;
            padded[k] = e < experts ? (count[e] + pad - 1) / pad * pad : 0;
            sum += padded[k];
        }
        unsigned incl = sum;
        for (int off = 1; off < 64; off <<= 1) {
            const unsigned v = __shfl_up(incl, off);
            if (int(t) >= off)
                incl += v;
        }
        unsigned at = incl - sum;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            start[4 * t + k] = at;
            at += padded[k];
        }
        if (t == 63)
            total = incl;
    }
    __syncthreads();
    for (unsigned s = t; s < slots; s += 1024) {
        const unsigned e = min(unsigned(idx[s]), experts - 1);
        const unsigned p = start[e] + atomicAdd(&fill[e], 1u);
        pos[s] = int32_t(p);
        inv[p] = int32_t(s);
    }
    if (t < experts) {  // padding rows, the expert's items and tiles
        const unsigned first = start[t], n = count[t];
        const unsigned end = first + (n + pad - 1) / pad * pad;
        const unsigned live = first + (n + kItemRows - 1) / kItemRows * kItemRows;
        for (unsigned p = first + n; p < end; ++p)
            inv[p] = -1;
        for (unsigned i = first / kItemRows; i < end / kItemRows; ++i)
            item_expert[i] = i < live / kItemRows ? int32_t(t) : -1;
        if (pad == kTileRows)
            for (unsigned j = first / kTileRows; j < end / kTileRows; ++j)
                tile_expert[j] = int32_t(t);
    }
    for (unsigned i = total / kItemRows + t; i < max_items; i += 1024)
        item_expert[i] = -1;
    if (pad == kTileRows)
        for (unsigned j = total / kTileRows + t; j < max_items * kItemRows / kTileRows;
             j += 1024)
            tile_expert[j] = -1;
    if (t == 0) {
        *used = total;
        *gemm_status = 0;
    }
}

// xp[p] = x[inv[p] / k] (zero for padding rows), positions below *used; 4 values a thread.
__global__ __launch_bounds__(256) void gather_kernel(const float* __restrict__ x,
                                                     const int32_t* __restrict__ inv,
                                                     const unsigned* __restrict__ used,
                                                     unsigned k, unsigned hidden,
                                                     size_t positions, float* __restrict__ xp) {
    const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
    const unsigned quads = hidden / 4;
    const size_t p = i / quads;
    if (p >= positions || p >= *used)
        return;
    const size_t d = (i % quads) * 4;
    const int s = inv[p];
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (s >= 0)
        v = *reinterpret_cast<const float4*>(x + size_t(s / int(k)) * hidden + d);
    *reinterpret_cast<float4*>(xp + p * hidden + d) = v;
}

bool tensor_ok(const kdq_gguf_tensor& m, size_t rows, size_t in, bool expert) {
    const size_t values = block_values(m.encoding);
    return m.weights && values && in % values == 0 && in % 8 == 0 &&
           m.row_bytes >= in / values * block_bytes(m.encoding) &&
           (!expert || (m.expert_bytes >= rows * m.row_bytes && m.expert_bytes % 16 == 0));
}

kdq_matvec_job job(const kdq_gguf_tensor& m, const float* x, size_t rows, size_t in,
                   size_t out, float* y, unsigned* status) {
    kdq_matvec_job j{};
    j.weights = m.weights;
    j.input = x;
    j.output = y;
    j.status = status;
    j.row_bytes = m.row_bytes;
    j.stride = out;
    j.in = uint32_t(in);
    j.columns = uint32_t(out);
    j.rows = uint32_t(rows);
    j.encoding = m.encoding;
    return j;
}

// Gate and up stored alike (so one launch can read both at the same expert offset).
bool same_layout(const kdq_gguf_tensor& a, const kdq_gguf_tensor& b) {
    return a.encoding == b.encoding && a.row_bytes == b.row_bytes &&
           a.expert_bytes == b.expert_bytes;
}

size_t align256(size_t n) {
    return (n + 255) & ~size_t(255);
}

// A product over more than kItemRows rows as one launch of kItemRows-row jobs (x and y
// stepping by kItemRows rows; the MFMA kernel when the format takes it, with `paired`),
// then the remaining rows; up to kItemRows rows as one job.
int run_rows(const IndexedJob& ij, hipStream_t st) {
    const kdq_matvec_job& j = ij.job;
    if (j.rows <= kItemRows)
        return indexed_gemv_batch(&ij, 1, st);
    IndexedJob a = ij;
    a.job.rows = kItemRows;
    const size_t full = j.rows / kItemRows;
    int rc = indexed_gemv_affine(a, unsigned(full), size_t(kItemRows) * j.in,
                                 size_t(kItemRows) * j.stride, st);
    if (rc || j.rows % kItemRows == 0)
        return rc;
    IndexedJob rest = ij;
    rest.job.rows = j.rows % kItemRows;
    rest.job.input = j.input + full * kItemRows * j.in;
    rest.job.output = j.output + full * kItemRows * j.stride;
    return indexed_gemv_batch(&rest, 1, st);
}

// Whether an expert stack can run on the grouped GEMM: an encoding it takes, whole 16-row
// tiles per expert and experts stored back to back (one pack covers the stack).
bool gemm_stack(const kdq_gguf_tensor& m, size_t rows, size_t in) {
    return grouped_gemm_takes(m.encoding, in) && rows % 16 == 0 &&
           m.expert_bytes == rows * m.row_bytes && kdq_gguf_packed_bytes(m.encoding, in, rows);
}

__global__ void or_status_kernel(unsigned* status, const unsigned* from, unsigned mask) {
    if (threadIdx.x == 0 && (*from & mask))
        atomicOr(status, *from & mask);
}

// Whether a shared matrix (out x in) can run on the dense prefill GEMM.
bool gemm_matrix(const kdq_gguf_tensor& m, size_t out, size_t in) {
    return grouped_gemm_takes(m.encoding, in) && kdq_gguf_packed_bytes(m.encoding, in, out);
}

// Whether a gate job of `rows` rows can run paired with its up matrix through run_rows.
bool rows_pairable(const kdq_matvec_job& gate) {
    if (gate.rows <= kItemRows)
        return swiglu_pairable(gate, 1);
    kdq_matvec_job a = gate;
    a.rows = kItemRows;
    return gate.rows % kItemRows == 0 && swiglu_pairable(a, gate.rows / kItemRows);
}

int moe_gguf(const kdq_moe_gguf_layer* layer, const kdq_moe_gguf_packed_stacks* packed,
             const float* x, size_t rows, float* y, int32_t* selected, float* weights,
             unsigned* status, void* stream) {
    if (!layer || !x || !y || !rows)
        return KDQ_ERR_ARGUMENT;
    const kdq_moe_gguf_layer& L = *layer;
    const size_t H = L.hidden, E = L.experts, K = L.top_k, F = L.ff, S = L.shared_ff;
    if (!H || !E || !K || !F || !S || !L.shared_gate)
        return KDQ_ERR_ARGUMENT;
    const size_t slots = rows * K;
    const bool grouped = rows > kSlotRows;
    if (E > 256 || K > 8 || K > E || rows > 4096 || slots > kMaxGroupedSlots ||
        H > 0xffffffu || F > 0xffffffu || S > 0xffffffu)
        return KDQ_ERR_SHAPE;
    if (!tensor_ok(L.router, E, H, false) || !tensor_ok(L.gate_exps, F, H, true) ||
        !tensor_ok(L.up_exps, F, H, true) || !tensor_ok(L.down_exps, H, F, true) ||
        !tensor_ok(L.gate_shexp, S, H, false) || !tensor_ok(L.up_shexp, S, H, false) ||
        !tensor_ok(L.down_shexp, H, S, false))
        return KDQ_ERR_SHAPE;
    if (misaligned(x, 16) || misaligned(y, 16) || misaligned(L.shared_gate, 16))
        return KDQ_ERR_ALIGNMENT;
    if (packed)
        for (const void* p : {packed->gate_exps, packed->up_exps, packed->down_exps,
                              packed->gate_shexp, packed->up_shexp, packed->down_shexp})
            if (misaligned(p, 16))
                return KDQ_ERR_ALIGNMENT;
    if (overlaps(y, rows * H * 4, x, rows * H * 4))
        return KDQ_ERR_ALIAS;
    // workspace: logits, shared gate/up rows, an empty part (index 3), routing (unless the
    // caller takes it), expert gate/up rows, expert downs, shared down; grouped: per position
    // (slots padded per expert to whole items), plus x in position order, the slot and
    // position maps, the items' experts and the count of positions in use
    // (grouped on the GEMM: token tiles of kTileRows, the packed expert stacks, fp16 x)
    // the grouped GEMM pads every expert's rows to 64-row token tiles; it pays once the
    // experts average 4 rows or more (a 64-token top-8 chunk over 128 experts: 559 us
    // against 564 on 8-row GEMV items per call, 315 against 597 over checked resident
    // copies); sparser batches run as 8-row GEMV items, which read each expert's weights
    // about once
    const bool dense = slots >= 4 * E;
    const bool gemm_gu = grouped && dense && gemm_stack(L.gate_exps, F, H) &&
                         gemm_stack(L.up_exps, F, H);
    const bool gemm_dn = grouped && dense && gemm_stack(L.down_exps, H, F);
    const kdq_moe_gguf_packed_stacks none{};
    const kdq_moe_gguf_packed_stacks& pk = packed ? *packed : none;
    // Matrices the caller keeps packed and has checked (kdq_gguf_gemm_check) cannot raise
    // the GEMM's fp16-range flag; any other matrix on a GEMM makes the call wait once on
    // the host for that flag (below).
    const bool sh_checked = pk.checked && pk.gate_shexp && pk.up_shexp && pk.down_shexp;
    // the shared expert (every row) on the dense prefill GEMM from kSharedGemmRows rows,
    // when the call does not wait for the flag because of it alone (the wait costs more
    // than the shared products at these sizes)
    const bool gemm_sh = grouped && rows >= kSharedGemmRows && gemm_matrix(L.gate_shexp, S, H) &&
                         gemm_matrix(L.up_shexp, S, H) && gemm_matrix(L.down_shexp, H, S) &&
                         (gemm_gu || gemm_dn || sh_checked);
    const bool wait = (gemm_gu && !(pk.checked && pk.gate_exps && pk.up_exps)) ||
                      (gemm_dn && !(pk.checked && pk.down_exps)) || (gemm_sh && !sh_checked);
    const size_t pad = gemm_gu || gemm_dn ? kTileRows : kItemRows;
    const size_t positions = grouped ? (slots + (pad - 1) * E + pad - 1) / pad * pad : slots;
    const size_t items = positions / kItemRows;
    const size_t gu_bytes = gemm_gu ? kdq_gguf_packed_bytes(L.gate_exps.encoding, H, F) : 0;
    const size_t up_bytes = gemm_gu ? kdq_gguf_packed_bytes(L.up_exps.encoding, H, F) : 0;
    const size_t dn_bytes = gemm_dn ? kdq_gguf_packed_bytes(L.down_exps.encoding, F, H) : 0;
    const size_t xs_bytes = gemm_gu || gemm_dn ? positions * std::max(H, F) * 2 : 0;
    // the shared GEMMs: packed copies unless the caller keeps them, one GEMM scratch
    auto sh_pack = [&](const kdq_gguf_tensor& m, const void* given, size_t out, size_t in) {
        return gemm_sh && !given ? kdq_gguf_packed_bytes(m.encoding, in, out) : 0;
    };
    const size_t shg_bytes = sh_pack(L.gate_shexp, pk.gate_shexp, S, H);
    const size_t shu_bytes = sh_pack(L.up_shexp, pk.up_shexp, S, H);
    const size_t shd_bytes = sh_pack(L.down_shexp, pk.down_shexp, H, S);
    const size_t sh_scratch =
        gemm_sh ? std::max(dense_gemm_scratch(rows, S, H), dense_gemm_scratch(rows, H, S)) : 0;
    const size_t sizes[] = {rows * E * 4,      rows * S * 4,      rows * S * 4,
                            size_t(0),         slots * 4,         slots * 4,
                            positions * F * 4, positions * F * 4, positions * H * 4,
                            rows * H * 4,      grouped ? positions * H * 4 : 0,
                            grouped ? slots * 4 : 0, grouped ? positions * 4 : 0,
                            grouped ? items * 4 : 0, size_t(grouped ? 8 : 0),
                            grouped ? positions / kTileRows * 4 + 4 : 0,
                            pk.gate_exps ? 0 : gu_bytes * E, pk.up_exps ? 0 : up_bytes * E,
                            pk.down_exps ? 0 : dn_bytes * E, xs_bytes,
                            gemm_gu || gemm_dn ? positions * 4 : 0, shg_bytes, shu_bytes,
                            shd_bytes, sh_scratch,
                            rows <= kFusedDecodeTokens ? kDecodeCounters * 4 : 0};
    constexpr size_t kParts = sizeof(sizes) / sizeof(sizes[0]);
    size_t total = 0;
    for (size_t b : sizes)
        total += align256(b);
    int rc;
    auto* base = static_cast<uint8_t*>(workspace(total, &rc));
    if (rc)
        return rc;
    void* part[kParts];
    for (size_t i = 0, at = 0; i < kParts; at += align256(sizes[i]), ++i)
        part[i] = base + at;
    auto* logits = static_cast<float*>(part[0]);
    auto* sg = static_cast<float*>(part[1]);
    auto* su = static_cast<float*>(part[2]);
    // part[3] is empty: the shared-gate scalars are taken inside the combine
    auto* idx = selected ? selected : static_cast<int32_t*>(part[4]);
    auto* w = weights ? weights : static_cast<float*>(part[5]);
    auto* g = static_cast<float*>(part[6]);
    auto* u = static_cast<float*>(part[7]);
    auto* d = static_cast<float*>(part[8]);
    auto* ds = static_cast<float*>(part[9]);
    auto* xp = static_cast<float*>(part[10]);
    auto* pos = static_cast<int32_t*>(part[11]);
    auto* inv = static_cast<int32_t*>(part[12]);
    auto* item_expert = static_cast<int32_t*>(part[13]);
    auto* used = static_cast<unsigned*>(part[14]);
    auto* gemm_status = used + 1;
    auto* tile_expert = static_cast<int32_t*>(part[15]);
    auto* packed_gate = pk.gate_exps ? const_cast<void*>(pk.gate_exps) : part[16];
    auto* packed_up = pk.up_exps ? const_cast<void*>(pk.up_exps) : part[17];
    auto* packed_down = pk.down_exps ? const_cast<void*>(pk.down_exps) : part[18];
    auto* xs = static_cast<uint16_t*>(part[19]);
    auto* sigma = static_cast<float*>(part[20]);
    const void* sh_gate = pk.gate_shexp ? pk.gate_shexp : part[21];
    const void* sh_up = pk.up_shexp ? pk.up_shexp : part[22];
    const void* sh_down = pk.down_shexp ? pk.down_shexp : part[23];
    void* sh_work = part[24];
    auto* counters = static_cast<unsigned*>(part[25]);
    auto st = static_cast<hipStream_t>(stream);

    // up to kFusedDecodeTokens tokens: two fused launches (moe_decode_fused) where the
    // encodings and shapes are among those it instantiates
    if (rows <= kFusedDecodeTokens && same_layout(L.gate_exps, L.up_exps) &&
        same_layout(L.gate_shexp, L.up_shexp)) {
        const bool up_packed = pk.gate_exps && pk.up_exps;
        const bool down_packed = pk.down_exps != nullptr;
        DecodeMoe m{};
        m.router = job(L.router, x, rows, H, E, logits, status);
        m.experts_up = IndexedJob{job(L.gate_exps, x, 1, H, F, g, status), idx,
                                  up_packed ? kdq_gguf_packed_bytes(L.gate_exps.encoding, H, F)
                                            : L.gate_exps.expert_bytes,
                                  unsigned(E), up_packed ? pk.up_exps : L.up_exps.weights};
        if (up_packed)
            m.experts_up.job.weights = pk.gate_exps;
        m.shared_up = IndexedJob{job(L.gate_shexp, x, 1, H, S, sg, status), nullptr, 0, 1,
                                 L.up_shexp.weights};
        m.experts_down = IndexedJob{job(L.down_exps, g, 1, F, H, d, status), idx,
                                    down_packed ? kdq_gguf_packed_bytes(L.down_exps.encoding, F, H)
                                                : L.down_exps.expert_bytes,
                                    unsigned(E), nullptr};
        if (down_packed)
            m.experts_down.job.weights = pk.down_exps;
        m.shared_down = IndexedJob{job(L.down_shexp, sg, 1, S, H, ds, status), nullptr, 0, 1,
                                   nullptr};
        m.up_packed = up_packed;
        m.down_packed = down_packed;
        m.logits = logits;
        m.experts = unsigned(E);
        m.top_k = unsigned(K);
        m.hidden = unsigned(H);
        m.tokens = unsigned(rows);
        m.idx = idx;
        m.w = w;
        m.gate_vector = L.shared_gate;
        m.x = x;
        m.y = y;
        m.status = status;
        m.counters = counters;
        // row-block counts, then a gate scalar per token
        m.counter_count = unsigned(kDecodeCounters - kFusedDecodeTokens);
        m.gate = reinterpret_cast<float*>(counters + (kDecodeCounters - kFusedDecodeTokens));
        if (moe_decode_fused(m, st, true) == KDQ_OK)
            return moe_decode_fused(m, st, false);
    }

    // 1. router, shared gate / up (with the swiglu in the same launch when the MFMA kernel
    //    takes the pair); the shared-gate scalar is taken by the combine
    const kdq_matvec_job shared_gate = job(L.gate_shexp, x, rows, H, S, sg, status);
    const bool pair_shared =
        same_layout(L.gate_shexp, L.up_shexp) && rows_pairable(shared_gate);
    IndexedJob first[3] = {{job(L.router, x, rows, H, E, logits, status), nullptr, 0, 1, nullptr},
                           {shared_gate, nullptr, 0, 1, pair_shared ? L.up_shexp.weights : nullptr},
                           {job(L.up_shexp, x, rows, H, S, su, status), nullptr, 0, 1, nullptr}};
    // the shared gate / up on the row path (stage 1, or the GEMM path's exact fallback)
    auto shared_rows = [&]() -> int {
        int r;
        for (int i = 1; i < (pair_shared ? 2 : 3); ++i)
            if ((r = run_rows(first[i], st)))
                return r;
        if (!pair_shared) {
            hipLaunchKernelGGL(swiglu_kernel, dim3(unsigned((rows * S + 255) / 256)), dim3(256),
                               0, st, sg, su, rows * S, nullptr, 1u, nullptr);
            KDQ_HIP(hipGetLastError());
        }
        return KDQ_OK;
    };
    if (!grouped) {
        if ((rc = indexed_gemv_batch(first, pair_shared ? 2 : 3, st)))
            return rc;
    } else {
        if ((rc = run_rows(first[0], st)))
            return rc;
        if (!gemm_sh && (rc = shared_rows()))
            return rc;
    }
    // 2. routing, straight into the caller's buffers when given
    if ((rc = route_selection(logits, rows, E, K, idx, w, st)))
        return rc;
    // 3. shared swiglu, unless paired above (grouped batches: done with the shared rows)
    if (!grouped && !pair_shared) {
        hipLaunchKernelGGL(swiglu_kernel, dim3(unsigned((rows * S + 255) / 256)), dim3(256), 0,
                           st, sg, su, rows * S, nullptr, 1u, nullptr);
        KDQ_HIP(hipGetLastError());
    }
    if (grouped) {
        // 4'. slots grouped by expert into padded segments (8-row items, 64-row tiles)
        hipLaunchKernelGGL(group_kernel, dim3(1), dim3(1024), 0, st, idx, unsigned(slots),
                           unsigned(E), unsigned(pad), unsigned(items), pos, inv, item_expert,
                           tile_expert, used, gemm_status);
        KDQ_HIP(hipGetLastError());
        // the shared gate / up on the dense GEMM (after group_kernel, which clears the
        // GEMM flags), packed here unless the caller keeps them packed
        if (gemm_sh) {
            if ((!pk.gate_shexp &&
                 (rc = kdq_gguf_pack(L.gate_shexp.encoding, L.gate_shexp.weights,
                                     L.gate_shexp.row_bytes, H, S, part[21], st))) ||
                (!pk.up_shexp &&
                 (rc = kdq_gguf_pack(L.up_shexp.encoding, L.up_shexp.weights,
                                     L.up_shexp.row_bytes, H, S, part[22], st))) ||
                (!pk.down_shexp &&
                 (rc = kdq_gguf_pack(L.down_shexp.encoding, L.down_shexp.weights,
                                     L.down_shexp.row_bytes, S, H, part[23], st))))
                return rc;
            if (same_layout(L.gate_shexp, L.up_shexp) &&
                grouped_gemm_pairs(L.gate_shexp.encoding)) {
                // one paired launch writing silu(gate) * up
                if ((rc = dense_gemm_pair(L.gate_shexp.encoding, sh_gate, sh_up, S, H, x, rows,
                                          sg, gemm_status, sh_work, st)))
                    return rc;
            } else {
                if ((rc = dense_gemm(L.gate_shexp.encoding, sh_gate, S, H, x, rows, sg,
                                     gemm_status, sh_work, st)) ||
                    (rc = dense_gemm(L.up_shexp.encoding, sh_up, S, H, x, rows, su, gemm_status,
                                     sh_work, st)))
                    return rc;
                hipLaunchKernelGGL(swiglu_kernel, dim3(unsigned((rows * S + 255) / 256)),
                                   dim3(256), 0, st, sg, su, rows * S, nullptr, 1u, nullptr);
                KDQ_HIP(hipGetLastError());
            }
        }
        const size_t xs8 = kItemRows * H, fs8 = kItemRows * F;
        // the expert products on the GEMV items (every encoding; the fallback of the GEMM)
        auto items_gate_up = [&]() -> int {
            hipLaunchKernelGGL(gather_kernel, dim3(unsigned((positions * (H / 4) + 255) / 256)),
                               dim3(256), 0, st, x, inv, used, unsigned(K), unsigned(H),
                               positions, xp);
            KDQ_HIP(hipGetLastError());
            const IndexedJob gj{job(L.gate_exps, xp, kItemRows, H, F, g, status), item_expert,
                                L.gate_exps.expert_bytes, unsigned(E), nullptr};
            if (same_layout(L.gate_exps, L.up_exps) && swiglu_pairable(gj.job, items)) {
                IndexedJob pj = gj;
                pj.paired = L.up_exps.weights;
                return indexed_gemv_affine(pj, unsigned(items), xs8, fs8, st);
            }
            const IndexedJob uj{job(L.up_exps, xp, kItemRows, H, F, u, status), item_expert,
                                L.up_exps.expert_bytes, unsigned(E), nullptr};
            int r;
            if ((r = indexed_gemv_affine(gj, unsigned(items), xs8, fs8, st)) ||
                (r = indexed_gemv_affine(uj, unsigned(items), xs8, fs8, st)))
                return r;
            hipLaunchKernelGGL(swiglu_kernel, dim3(unsigned((positions * F + 255) / 256)),
                               dim3(256), 0, st, g, u, positions * F, used, unsigned(F), inv);
            KDQ_HIP(hipGetLastError());
            return KDQ_OK;
        };
        auto items_down = [&]() -> int {
            const IndexedJob dj{job(L.down_exps, g, kItemRows, F, H, d, status), item_expert,
                                L.down_exps.expert_bytes, unsigned(E), nullptr};
            return indexed_gemv_affine(dj, unsigned(items), fs8, xs8, st);
        };
        // 4''. expert gate / up
        if (gemm_gu) {  // both stacks packed (this call or the caller's), one grouped GEMM
                        // each, swiglu
            if ((!pk.gate_exps &&
                 (rc = kdq_gguf_pack(L.gate_exps.encoding, L.gate_exps.weights,
                                     L.gate_exps.row_bytes, H, E * F, packed_gate, st))) ||
                (!pk.up_exps &&
                 (rc = kdq_gguf_pack(L.up_exps.encoding, L.up_exps.weights, L.up_exps.row_bytes,
                                     H, E * F, packed_up, st))))
                return rc;
            if (same_layout(L.gate_exps, L.up_exps) &&
                grouped_gemm_pairs(L.gate_exps.encoding)) {
                // one paired launch: x staged once, h = silu(gate) * up in its epilogue
                if ((rc = grouped_gemm(L.gate_exps.encoding, packed_gate, gu_bytes, tile_expert,
                                       F, H, x, inv, unsigned(K), used, positions, g,
                                       gemm_status, xs, sigma, st, packed_up)))
                    return rc;
            } else {
                if ((rc = grouped_gemm(L.gate_exps.encoding, packed_gate, gu_bytes, tile_expert,
                                       F, H, x, inv, unsigned(K), used, positions, g,
                                       gemm_status, xs, sigma, st)) ||
                    (rc = grouped_gemm(L.up_exps.encoding, packed_up, up_bytes, tile_expert, F,
                                       H, x, inv, unsigned(K), used, positions, u, gemm_status,
                                       xs, sigma, st)))
                    return rc;
                hipLaunchKernelGGL(swiglu_kernel, dim3(unsigned((positions * F + 255) / 256)),
                                   dim3(256), 0, st, g, u, positions * F, used, unsigned(F),
                                   inv);
                KDQ_HIP(hipGetLastError());
            }
        } else if ((rc = items_gate_up())) {
            return rc;
        }
        // 5'. expert downs, the shared down
        if (gemm_dn) {
            if ((!pk.down_exps &&
                 (rc = kdq_gguf_pack(L.down_exps.encoding, L.down_exps.weights,
                                     L.down_exps.row_bytes, F, E * H, packed_down, st))) ||
                (rc = grouped_gemm(L.down_exps.encoding, packed_down, dn_bytes, tile_expert, H,
                                   F, g, nullptr, 1u, used, positions, d, gemm_status, xs,
                                   sigma, st)))
                return rc;
        } else if ((rc = items_down())) {
            return rc;
        }
        const IndexedJob sj{job(L.down_shexp, sg, rows, S, H, ds, status), nullptr, 0, 1,
                            nullptr};
        if (gemm_sh ? (rc = dense_gemm(L.down_shexp.encoding, sh_down, H, S, sg, rows, ds,
                                       gemm_status, sh_work, st))
                    : (rc = run_rows(sj, st)))
            return rc;
        auto combine = [&]() -> int {
            hipLaunchKernelGGL(combine_kernel, dim3(unsigned((H / 4 + 255) / 256), unsigned(rows)),
                               dim3(256), 0, st, d, pos, w, ds, L.shared_gate, x, unsigned(K),
                               unsigned(H), y, status);
            KDQ_HIP(hipGetLastError());
            return KDQ_OK;
        };
        // 6'. combine in selection order, each slot's down at its position
        if ((rc = combine()))
            return rc;
        if ((gemm_gu || gemm_dn || gemm_sh) && !wait) {
            // checked matrices: only the non-finite bit can be set; it goes to the
            // caller's status on the device
            if (status) {
                hipLaunchKernelGGL(or_status_kernel, dim3(1), dim3(64), 0, st, status,
                                   gemm_status, 1u);
                KDQ_HIP(hipGetLastError());
            }
        } else if (gemm_gu || gemm_dn || gemm_sh) {
            // the GEMM's flags: a non-finite scale is the caller's status bit 1; a scale
            // that could take a dequantised weight past the fp16 range (never in real
            // checkpoints) makes this call redo its expert products on the GEMV items,
            // which decode exactly (one host wait, only on this path)
            unsigned flags = 0;
            KDQ_HIP(hipMemcpyAsync(&flags, gemm_status, sizeof flags, hipMemcpyDeviceToHost,
                                   st));
            KDQ_HIP(hipStreamSynchronize(st));
            if (flags & 2u) {
                if ((gemm_sh && ((rc = shared_rows()) || (rc = run_rows(sj, st)))) ||
                    (rc = items_gate_up()) || (rc = items_down()) || (rc = combine()))
                    return rc;
            } else if ((flags & 1u) && status) {
                hipLaunchKernelGGL(or_status_kernel, dim3(1), dim3(64), 0, st, status,
                                   gemm_status, 1u);
                KDQ_HIP(hipGetLastError());
            }
        }
        return KDQ_OK;
    }
    // 4. expert gate / up at the routed slices, every slot in one launch (slot s reads
    //    token s / K's row and writes row s), as a pair with the swiglu when the MFMA
    //    kernel takes it, else two launches and the swiglu
    const IndexedJob gj{job(L.gate_exps, x, 1, H, F, g, status), idx, L.gate_exps.expert_bytes,
                        unsigned(E), nullptr};
    // resident packed stacks (kdq_moe_gguf_packed): the paired launch over them when the
    // MFMA kernel takes the packed form, else the row-major tensors
    rc = KDQ_ERR_UNSUPPORTED;
    if (pk.gate_exps && pk.up_exps && same_layout(L.gate_exps, L.up_exps)) {
        IndexedJob pj{job(L.gate_exps, x, 1, H, F, g, status), idx,
                      kdq_gguf_packed_bytes(L.gate_exps.encoding, H, F), unsigned(E),
                      pk.up_exps};
        pj.job.weights = pk.gate_exps;
        rc = indexed_gemv_affine_packed(pj, unsigned(slots), H, F, st, unsigned(K));
        if (rc && rc != KDQ_ERR_UNSUPPORTED)
            return rc;
    }
    if (rc == KDQ_OK) {
        // gate / up done on the packed stacks
    } else if (same_layout(L.gate_exps, L.up_exps) && swiglu_pairable(gj.job, slots)) {
        IndexedJob pj = gj;
        pj.paired = L.up_exps.weights;
        if ((rc = indexed_gemv_affine(pj, unsigned(slots), H, F, st, unsigned(K))))
            return rc;
    } else {
        const IndexedJob uj{job(L.up_exps, x, 1, H, F, u, status), idx, L.up_exps.expert_bytes,
                            unsigned(E), nullptr};
        if ((rc = indexed_gemv_affine(gj, unsigned(slots), H, F, st, unsigned(K))) ||
            (rc = indexed_gemv_affine(uj, unsigned(slots), H, F, st, unsigned(K))))
            return rc;
        hipLaunchKernelGGL(swiglu_kernel, dim3(unsigned((slots * F + 255) / 256)), dim3(256), 0,
                           st, g, u, slots * F, nullptr, 1u, nullptr);
        KDQ_HIP(hipGetLastError());
    }
    // 5. expert downs (one launch over every slot) and the shared down
    const IndexedJob dj{job(L.down_exps, g, 1, F, H, d, status), idx, L.down_exps.expert_bytes,
                        unsigned(E), nullptr};
    rc = KDQ_ERR_UNSUPPORTED;
    if (pk.down_exps) {
        IndexedJob pj = dj;
        pj.job.weights = pk.down_exps;
        pj.index_stride = kdq_gguf_packed_bytes(L.down_exps.encoding, F, H);
        rc = indexed_gemv_affine_packed(pj, unsigned(slots), F, H, st);
        if (rc && rc != KDQ_ERR_UNSUPPORTED)
            return rc;
    }
    if (rc != KDQ_OK && (rc = indexed_gemv_affine(dj, unsigned(slots), F, H, st)))
        return rc;
    const IndexedJob sj{job(L.down_shexp, sg, rows, S, H, ds, status), nullptr, 0, 1, nullptr};
    if ((rc = indexed_gemv_batch(&sj, 1, st)))
        return rc;
    // 6. combine
    hipLaunchKernelGGL(combine_kernel, dim3(unsigned((H / 4 + 255) / 256), unsigned(rows)),
                       dim3(256), 0, st, d, static_cast<const int32_t*>(nullptr), w, ds,
                       L.shared_gate, x, unsigned(K), unsigned(H), y, status);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}

}  // namespace
}  // namespace kdq

using namespace kdq;

extern "C" int kdq_moe_gguf(const kdq_moe_gguf_layer* layer, const float* x, size_t rows,
                            float* y, int32_t* selected, float* weights, unsigned* status,
                            void* stream) {
    return moe_gguf(layer, nullptr, x, rows, y, selected, weights, status, stream);
}

extern "C" int kdq_moe_gguf_packed(const kdq_moe_gguf_layer* layer,
                                   const kdq_moe_gguf_packed_stacks* packed, const float* x,
                                   size_t rows, float* y, int32_t* selected, float* weights,
                                   unsigned* status, void* stream) {
    return moe_gguf(layer, packed, x, rows, y, selected, weights, status, stream);
}
