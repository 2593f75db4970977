// GGUF mixture-of-experts layer on the device: the Qwen MoE layer of
// IW/src/models/text/qwen_layers.cpp:378-492 (MoeLayer::forward; IW =
// services/hikari/inference_worker) as one stream-ordered submission, with no host round
// trip between its stages (the reference returns to the host three times per layer).
//
// Stages, all on `stream`:
//   1. one GEMV batch over x: router logits, the shared-expert gate scalar
//      ffn_gate_inp_shexp . x (as a one-row fp32 matrix), and the shared expert's gate and
//      up rows, as one paired MFMA job that writes silu(gate) * up when the kernel takes
//      the pair (gate and up stored alike)
//   2. routing (route_selection: the kdq_moe_route kernel; softmax with a double total,
//      top-k by probability, weights renormalised by max(sum, 2^-14))
//   3. swiglu_kernel on the shared rows, unless paired in 1
//   4. one launch of every slot's expert gate / up GEMV (slot s reads token s / top_k's
//      row), each job's weights starting at the expert slice the routing wrote on the
//      device; paired with the swiglu like 1, else gate and up launches and swiglu_kernel
//   5. one launch of every slot's expert down GEMV, plus the shared expert's down
//   6. combine_kernel: y = sum over the selections, in selection order, of down * weight,
//      plus shared_down * sigmoid(gate scalar)
// GEMVs of Q4_0 / Q8_0 / Q4_K / Q3_K / Q6_K / IQ4_XS / IQ4_NL run on the MFMA kernel
// (fused per shape), every other encoding on the exact kernel.
#include "kdq_common.hpp"

#include <vector>

namespace kdq {
namespace {

__global__ __launch_bounds__(256) void swiglu_kernel(float* gate, const float* up, size_t n) {
    const size_t i = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (i < n)
        gate[i] = silu_of(gate[i]) * up[i];
}

// y[t, d] = (sum_{i < k} down[t*k + i, d] * w[t*k + i]) + shared[t, d] * sigmoid(gate[t])
__global__ __launch_bounds__(256) void combine_kernel(const float* down, const float* w,
                                                      const float* shared, const float* gate,
                                                      unsigned k, unsigned hidden,
                                                      size_t tokens, float* y) {
    const size_t e = size_t(blockIdx.x) * 256 + threadIdx.x;
    if (e >= tokens * hidden)
        return;
    const size_t t = e / hidden, d = e % hidden;
    float sum = 0.f;
    for (unsigned i = 0; i < k; ++i)
        sum += down[(t * k + i) * hidden + d] * w[t * k + i];
    y[e] = sum + shared[e] * sigmoid_of(gate[t]);
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

}  // namespace
}  // namespace kdq

using namespace kdq;

extern "C" int kdq_moe_gguf(const kdq_moe_gguf_layer* layer, const float* x, size_t rows,
                            float* y, int32_t* selected, float* weights, unsigned* status,
                            void* stream) {
    if (!layer || !x || !y || !rows)
        return KDQ_ERR_ARGUMENT;
    const kdq_moe_gguf_layer& L = *layer;
    const size_t H = L.hidden, E = L.experts, K = L.top_k, F = L.ff, S = L.shared_ff;
    if (!H || !E || !K || !F || !S || !L.shared_gate)
        return KDQ_ERR_ARGUMENT;
    const size_t slots = rows * K;
    if (E > 256 || K > 8 || K > E || slots > 512 || H > 0xffffffu || F > 0xffffffu ||
        S > 0xffffffu)
        return KDQ_ERR_SHAPE;
    if (!tensor_ok(L.router, E, H, false) || !tensor_ok(L.gate_exps, F, H, true) ||
        !tensor_ok(L.up_exps, F, H, true) || !tensor_ok(L.down_exps, H, F, true) ||
        !tensor_ok(L.gate_shexp, S, H, false) || !tensor_ok(L.up_shexp, S, H, false) ||
        !tensor_ok(L.down_shexp, H, S, false))
        return KDQ_ERR_SHAPE;
    if (misaligned(x, 16) || misaligned(y, 16) || misaligned(L.shared_gate, 16))
        return KDQ_ERR_ALIGNMENT;
    if (overlaps(y, rows * H * 4, x, rows * H * 4))
        return KDQ_ERR_ALIAS;
    // workspace: logits, shared gate/up rows, gate scalars, routing (unless the caller
    // takes it), expert gate/up rows, expert downs, shared down
    const size_t sizes[] = {rows * E * 4, rows * S * 4, rows * S * 4, rows * 4, slots * 4,
                            slots * 4, slots * F * 4, slots * F * 4, slots * H * 4, rows * H * 4};
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
    auto* gate = static_cast<float*>(part[3]);
    auto* idx = selected ? selected : static_cast<int32_t*>(part[4]);
    auto* w = weights ? weights : static_cast<float*>(part[5]);
    auto* g = static_cast<float*>(part[6]);
    auto* u = static_cast<float*>(part[7]);
    auto* d = static_cast<float*>(part[8]);
    auto* ds = static_cast<float*>(part[9]);
    auto st = static_cast<hipStream_t>(stream);

    // 1. router, shared-gate scalar, shared gate / up (with the swiglu in the same launch
    //    when the MFMA kernel takes the pair)
    const kdq_gguf_tensor gate_vector{L.shared_gate, H * 4, 0, KDQ_F32};
    const kdq_matvec_job shared_gate = job(L.gate_shexp, x, rows, H, S, sg, status);
    const bool pair_shared =
        same_layout(L.gate_shexp, L.up_shexp) && swiglu_pairable(shared_gate, 1);
    IndexedJob first[4] = {{job(L.router, x, rows, H, E, logits, status), nullptr, 0, 1, nullptr},
                           {job(gate_vector, x, rows, H, 1, gate, status), nullptr, 0, 1, nullptr},
                           {shared_gate, nullptr, 0, 1, pair_shared ? L.up_shexp.weights : nullptr},
                           {job(L.up_shexp, x, rows, H, S, su, status), nullptr, 0, 1, nullptr}};
    if ((rc = indexed_gemv_batch(first, pair_shared ? 3 : 4, st)))
        return rc;
    // 2. routing, straight into the caller's buffers when given
    if ((rc = route_selection(logits, rows, E, K, idx, w, st)))
        return rc;
    // 3. shared swiglu, unless paired above
    if (!pair_shared) {
        hipLaunchKernelGGL(swiglu_kernel, dim3(unsigned((rows * S + 255) / 256)), dim3(256), 0,
                           st, sg, su, rows * S);
        KDQ_HIP(hipGetLastError());
    }
    // 4. expert gate / up at the routed slices, every slot in one launch (slot s reads
    //    token s / K's row and writes row s), as a pair with the swiglu when the MFMA
    //    kernel takes it, else two launches and the swiglu
    const IndexedJob gj{job(L.gate_exps, x, 1, H, F, g, status), idx, L.gate_exps.expert_bytes,
                        unsigned(E), nullptr};
    if (same_layout(L.gate_exps, L.up_exps) && swiglu_pairable(gj.job, slots)) {
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
                           st, g, u, slots * F);
        KDQ_HIP(hipGetLastError());
    }
    // 5. expert downs (one launch over every slot) and the shared down
    const IndexedJob dj{job(L.down_exps, g, 1, F, H, d, status), idx, L.down_exps.expert_bytes,
                        unsigned(E), nullptr};
    if ((rc = indexed_gemv_affine(dj, unsigned(slots), F, H, st)))
        return rc;
    const IndexedJob sj{job(L.down_shexp, sg, rows, S, H, ds, status), nullptr, 0, 1, nullptr};
    if ((rc = indexed_gemv_batch(&sj, 1, st)))
        return rc;
    // 6. combine
    hipLaunchKernelGGL(combine_kernel, dim3(unsigned((rows * H + 255) / 256)), dim3(256), 0, st,
                       d, w, ds, gate, unsigned(K), unsigned(H), rows, y);
    KDQ_HIP(hipGetLastError());
    return KDQ_OK;
}
