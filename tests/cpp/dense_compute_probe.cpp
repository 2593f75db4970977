// Test shim: a C surface over kadan_amd::HipDenseCompute so the Python tests can drive
// the C++ host layer with host arrays and compare its results with the oracle.  Every
// entry returns 0 on success, or -1 with the exception text copied into `err`.
#include <cstring>
#include <exception>
#include <vector>

#include "kadan_amd_dense_compute.hpp"

using kadan_amd::HipDenseCompute;
using kadan_amd::ProjectionResult;
using kadan_amd::WeightIdentity;

namespace {

struct Probe {
    HipDenseCompute compute;
    std::size_t source_reads = 0;  // rows handed out by every weight source so far
    explicit Probe(int device) : compute(device) {}
};

WeightIdentity identity(unsigned long long id) {
    WeightIdentity w;
    w.inode = id;
    w.payload_end = id;
    return w;
}

int fail(const std::exception& e, char* err, std::size_t len) {
    if (err && len) {
        std::strncpy(err, e.what(), len - 1);
        err[len - 1] = 0;
    }
    return -1;
}

int encode(ProjectionResult r) {
    return r == ProjectionResult::unsupported ? 0 : r == ProjectionResult::unvalidated ? 1 : 2;
}

HipDenseCompute::GgufWeightSource source_for(Probe* p, const unsigned char* weights,
                                             std::size_t row_bytes) {
    return [p, weights, row_bytes](std::size_t first, std::span<std::byte> dst) {
        std::memcpy(dst.data(), weights + first * row_bytes, dst.size());
        p->source_reads += dst.size() / row_bytes;
    };
}

}  // namespace

extern "C" {

void* kdc_create(int device, char* err, std::size_t len) {
    try {
        return new Probe(device);
    } catch (const std::exception& e) {
        fail(e, err, len);
        return nullptr;
    }
}

void kdc_destroy(void* p) {
    delete static_cast<Probe*>(p);
}

std::size_t kdc_source_reads(void* p) {
    return static_cast<Probe*>(p)->source_reads;
}

std::size_t kdc_retained(void* p) {
    return static_cast<Probe*>(p)->compute.retained_weight_bytes();
}

std::size_t kdc_release(void* p, unsigned long long id) {
    const WeightIdentity w = identity(id);
    return static_cast<Probe*>(p)->compute.release_weights(std::span<const WeightIdentity>(&w, 1));
}

int kdc_release_scratch(void* p, char* err, std::size_t len) {
    try {
        static_cast<Probe*>(p)->compute.release_scratch();
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

// ggml_type: GGML type id (2, 8, 12, or any other id, which is unsupported here).
int kdc_dense_gguf(void* handle, unsigned long long id, unsigned ggml_type,
                   const unsigned char* weights, std::size_t row_bytes, const float* bias,
                   const float* x, std::size_t rows, std::size_t in, std::size_t out, float* y,
                   int retain, int cancel, int* result, char* err, std::size_t len) {
    try {
        auto* p = static_cast<Probe*>(handle);
        const auto enc = kadan_amd::gguf::encoding(ggml_type);
        if (!enc) {
            *result = 0;
            return 0;
        }
        const std::atomic_bool stop{cancel != 0};
        auto src = source_for(p, weights, row_bytes);
        *result = encode(p->compute.dense_gguf_source(
            identity(id), *enc, src, std::span<const float>(bias, bias ? out : 0),
            std::span<const float>(x, rows * in), in, out, std::span<float>(y, rows * out), stop,
            false, retain != 0));
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

// Parallel arrays, one entry per job; inputs[i] may repeat a pointer to share an input.
int kdc_dense_gguf_batch(void* handle, std::size_t count, const unsigned long long* ids,
                         const unsigned* ggml_types, const unsigned char* const* weights,
                         const std::size_t* row_bytes, const float* const* inputs,
                         const std::size_t* rows, const std::size_t* ins,
                         const std::size_t* outs, float* const* outputs, int* result, char* err,
                         std::size_t len) {
    try {
        auto* p = static_cast<Probe*>(handle);
        std::vector<WeightIdentity> idents(count);
        std::vector<HipDenseCompute::GgufWeightSource> sources(count);
        std::vector<HipDenseCompute::GgufBatchJob> jobs(count);
        for (std::size_t i = 0; i < count; ++i) {
            idents[i] = identity(ids[i]);
            sources[i] = source_for(p, weights[i], row_bytes[i]);
            jobs[i] = HipDenseCompute::GgufBatchJob{
                &idents[i], kadan_amd::gguf::encoding(ggml_types[i]), &sources[i],
                std::span<const float>(inputs[i], rows[i] * ins[i]), ins[i], outs[i],
                std::span<float>(outputs[i], rows[i] * outs[i]), true};
        }
        const std::atomic_bool stop{false};
        *result = encode(p->compute.dense_gguf_batch(jobs, stop));
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

int kdc_dense_gguf_q8(void* handle, unsigned long long id, const unsigned char* weights,
                      std::size_t row_bytes, const unsigned short* x, std::size_t rows,
                      std::size_t in, std::size_t out, unsigned short* y, int* result,
                      char* err, std::size_t len) {
    try {
        auto* p = static_cast<Probe*>(handle);
        const std::atomic_bool stop{false};
        auto src = source_for(p, weights, row_bytes);
        *result = encode(p->compute.dense_gguf_q8_source(
            identity(id), kadan_amd::gguf::Encoding::q4_0, src,
            std::span<const std::uint16_t>(x, rows * in), in, out,
            std::span<std::uint16_t>(y, rows * out), stop));
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

int kdc_moe_mxfp4(void* handle, unsigned long long id, std::size_t experts, std::size_t hidden,
                  std::size_t inter, const unsigned char* gate_blocks,
                  const unsigned char* gate_scales, const unsigned char* up_blocks,
                  const unsigned char* up_scales, const unsigned char* down_blocks,
                  const unsigned char* down_scales, const unsigned short* x, const float* logits,
                  std::size_t tokens, std::size_t top_k, float* y, int* selected, float* weights,
                  int* result, char* err, std::size_t len) {
    try {
        auto* p = static_cast<Probe*>(handle);
        const WeightIdentity ident = identity(id);
        const std::size_t fused = experts * inter * hidden;
        HipDenseCompute::Mxfp4Experts e{&ident,
                                        experts,
                                        hidden,
                                        inter,
                                        {gate_blocks, fused / 2},
                                        {gate_scales, fused / 32},
                                        {up_blocks, fused / 2},
                                        {up_scales, fused / 32},
                                        {down_blocks, fused / 2},
                                        {down_scales, fused / 32}};
        const std::atomic_bool stop{false};
        *result = encode(p->compute.moe_mxfp4(
            e, std::span<const std::uint16_t>(x, tokens * hidden),
            std::span<const float>(logits, tokens * experts), tokens, top_k,
            std::span<float>(y, tokens * hidden),
            std::span<std::int32_t>(selected, selected ? tokens * top_k : 0),
            std::span<float>(weights, weights ? tokens * top_k : 0), stop));
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

}  // extern "C"
