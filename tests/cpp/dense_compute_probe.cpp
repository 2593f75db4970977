// Test shim: a C surface over kadan_amd::HipDenseCompute and the checkpoint readers
// (kadan_amd::checkpoint) so the Python tests can drive the C++ host layer with host
// arrays and files and compare its results with the oracle.  Every entry returns 0 on
// success, or -1 with the exception text copied into `err`.
#include <atomic>
#include <cstring>
#include <exception>
#include <vector>

#include "kadan_amd_checkpoint.hpp"
#include "kadan_amd_dense_compute.hpp"

using kadan_amd::HipDenseCompute;
using kadan_amd::ProjectionResult;
using kadan_amd::WeightIdentity;

namespace {

struct Probe {
    HipDenseCompute compute;
    // rows handed out by every weight source so far (the read team calls sources from
    // several threads at once)
    std::atomic<std::size_t> source_reads{0};
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

void kdc_set_weight_limit(void* p, std::size_t bytes) {
    static_cast<Probe*>(p)->compute.set_weight_limit(bytes);
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
                   int retain, int cancel, int precise, int* result, char* err,
                   std::size_t len) {
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
            precise != 0, retain != 0));
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

// Parallel arrays, one entry per job; inputs[i] may repeat a pointer to share an input;
// ggml type 0 is an F32 job.
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
            // type 0: F32 rows (no encoding); another type without a kadan encoding is
            // refused here, before any read, as the integration adapter refuses it
            const auto enc = kadan_amd::gguf::encoding(ggml_types[i]);
            if (ggml_types[i] && !enc) {
                *result = 0;
                return 0;
            }
            idents[i] = identity(ids[i]);
            sources[i] = source_for(p, weights[i], row_bytes[i]);
            jobs[i] = HipDenseCompute::GgufBatchJob{
                &idents[i], enc, &sources[i],
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

// HipDenseCompute::batch_supported over jobs described as in kdc_dense_gguf_batch (ggml type
// 0: an F32 job, no encoding); no device, no weights.  1 eligible, 0 refused, -1 a type
// with no kadan encoding.
int kdc_batch_supported(std::size_t count, const unsigned* ggml_types, const std::size_t* rows,
                        const std::size_t* ins, const std::size_t* outs) {
    std::vector<WeightIdentity> idents(count);
    const HipDenseCompute::GgufWeightSource none = [](std::size_t, std::span<std::byte>) {};
    std::vector<std::vector<float>> inputs(count), outputs(count);
    std::vector<HipDenseCompute::GgufBatchJob> jobs(count);
    for (std::size_t i = 0; i < count; ++i) {
        const auto enc = kadan_amd::gguf::encoding(ggml_types[i]);
        if (ggml_types[i] && !enc)
            return -1;
        inputs[i].resize(rows[i] * ins[i]);
        outputs[i].resize(rows[i] * outs[i]);
        jobs[i] = HipDenseCompute::GgufBatchJob{&idents[i], enc, &none, inputs[i], ins[i], outs[i],
                                                outputs[i], true};
    }
    return HipDenseCompute::batch_supported(jobs) ? 1 : 0;
}

// HipDenseCompute::dense_source with F32 weights [out x in] from a FloatWeightSource.
int kdc_dense_source(void* handle, unsigned long long id, const float* weights,
                     const float* bias, const float* x, std::size_t rows, std::size_t in,
                     std::size_t out, float* y, int* result, char* err, std::size_t len) {
    try {
        auto* p = static_cast<Probe*>(handle);
        const HipDenseCompute::FloatWeightSource src = [p, weights, in](std::size_t first,
                                                                        std::span<float> dst) {
            std::memcpy(dst.data(), weights + first, dst.size_bytes());
            p->source_reads += dst.size() / in;
        };
        const std::atomic_bool stop{false};
        *result = encode(p->compute.dense_source(
            identity(id), src, std::span<const float>(bias, bias ? out : 0),
            std::span<const float>(x, rows * in), in, out, std::span<float>(y, rows * out),
            stop));
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

// ------------------------------------------------------------- checkpoints

using kadan_amd::checkpoint::GgufFiles;
using kadan_amd::checkpoint::SafetensorsFile;

void* kcp_gguf_open(const char* root, int cancelled, char* err, std::size_t len) {
    try {
        const std::atomic_bool cancel{cancelled != 0};
        return new GgufFiles(root, cancel);
    } catch (const std::exception& e) {
        fail(e, err, len);
        return nullptr;
    }
}

void kcp_gguf_close(void* c) {
    delete static_cast<GgufFiles*>(c);
}

std::size_t kcp_gguf_tensor_count(void* c) {
    return static_cast<GgufFiles*>(c)->size();
}

// shape in GGUF order (columns, rows, experts), the listed rank, GGML type, payload bytes
int kcp_gguf_tensor(void* c, const char* name, unsigned long long* shape, std::size_t* rank,
                    unsigned* type, unsigned long long* bytes, char* err, std::size_t len) {
    try {
        const auto& t = static_cast<GgufFiles*>(c)->info(std::string_view(name));
        shape[0] = t.columns;
        shape[1] = t.rows;
        shape[2] = t.experts;
        *rank = t.rank;
        *type = t.ggml_type;
        *bytes = t.bytes;
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

static void put_identity(const WeightIdentity& w, unsigned long long* out) {
    const std::uint64_t v[9] = {w.device, w.inode, w.file_size, w.modified_seconds,
                                w.modified_nanoseconds, w.changed_seconds,
                                w.changed_nanoseconds, w.payload_begin, w.payload_end};
    for (int i = 0; i < 9; ++i)
        out[i] = v[i];
}

int kcp_gguf_identity(void* c, const char* name, std::size_t expert, unsigned long long* out,
                      char* err, std::size_t len) {
    try {
        put_identity(static_cast<GgufFiles*>(c)->slice_identity(name, expert), out);
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

int kcp_gguf_check_unchanged(void* c, char* err, std::size_t len) {
    try {
        static_cast<GgufFiles*>(c)->verify_unchanged();
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

int kcp_gguf_read_packed(void* c, const char* name, std::size_t expert, std::size_t first,
                         void* out, std::size_t bytes, int cancelled, char* err,
                         std::size_t len) {
    try {
        const std::atomic_bool cancel{cancelled != 0};
        static_cast<GgufFiles*>(c)->copy_rows(
            name, expert, first, std::span<std::byte>(static_cast<std::byte*>(out), bytes),
            cancel);
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

int kcp_gguf_read_vector(void* c, const char* name, float* out, std::size_t n, char* err,
                         std::size_t len) {
    try {
        const std::atomic_bool cancel{false};
        static_cast<GgufFiles*>(c)->copy_vector(name, std::span<float>(out, n), cancel);
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

// kind: 0 text, 1 count, 2 real, 3 flag, 4 texts (joined by 0x1f), 5 integers, 6 reals,
// 7 flags, 8 has.  Arrays write up to *count values and set *count.
int kcp_gguf_meta(void* c, const char* key, int kind, char* text, std::size_t text_len,
                  long long* ints, double* nums, std::size_t* count, char* err,
                  std::size_t len) {
    try {
        const auto* g = static_cast<GgufFiles*>(c);
        auto put_text = [&](const std::string& s) {
            std::strncpy(text, s.c_str(), text_len - 1);
            text[text_len - 1] = 0;
        };
        if (kind == 8) {
            ints[0] = g->has(key);
            return 0;
        }
        const auto& v = g->value(key);
        switch (kind) {
        case 0: put_text(v.text()); break;
        case 1: ints[0] = (long long)v.count(); break;
        case 2: nums[0] = v.real(); break;
        case 3: ints[0] = v.flag(); break;
        case 4: {
            std::string joined;
            for (const auto& s : v.texts())
                joined += s + "\x1f";
            put_text(joined);
            break;
        }
        case 5: {
            const auto a = v.integers();
            for (std::size_t i = 0; i < a.size() && i < *count; ++i)
                ints[i] = a[i];
            *count = a.size();
            break;
        }
        case 6: {
            const auto a = v.reals();
            for (std::size_t i = 0; i < a.size() && i < *count; ++i)
                nums[i] = a[i];
            *count = a.size();
            break;
        }
        default: {
            const auto a = v.flags();
            for (std::size_t i = 0; i < a.size() && i < *count; ++i)
                ints[i] = a[i];
            *count = a.size();
            break;
        }
        }
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

// Decoded rows through the device of a dense probe (GgufFiles::decode_rows).
int kcp_gguf_read_rows(void* c, void* probe, const char* name, std::size_t expert,
                       std::size_t first, float* out, std::size_t n, char* err,
                       std::size_t len) {
    try {
        const std::atomic_bool cancel{false};
        static_cast<GgufFiles*>(c)->decode_rows(name, expert, first, std::span<float>(out, n),
                                                cancel, static_cast<Probe*>(probe)->compute);
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

// dense_gguf_source with the file set's own identity and row source: x [rows x in] ->
// y [rows x out] (in, out from the tensor's shape).
int kcp_gguf_dense_source(void* c, void* probe, const char* name, std::size_t expert,
                          const float* x, std::size_t rows, float* y, int* result,
                          char* err, std::size_t len) {
    try {
        auto* g = static_cast<GgufFiles*>(c);
        auto* p = static_cast<Probe*>(probe);
        const auto& t = g->info(std::string_view(name));
        const auto enc = kadan_amd::gguf::encoding(t.ggml_type);
        if (!enc) {
            *result = 0;
            return 0;
        }
        const std::atomic_bool cancel{false};
        const auto source = g->row_source(name, expert, cancel);
        const std::size_t in = t.columns, out = t.rows;
        *result = encode(p->compute.dense_gguf_source(
            g->slice_identity(name, expert), *enc, source, {},
            std::span<const float>(x, rows * in), in, out, std::span<float>(y, rows * out),
            cancel));
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

void* kcp_st_open(const char* path, char* err, std::size_t len) {
    try {
        return new SafetensorsFile(path);
    } catch (const std::exception& e) {
        fail(e, err, len);
        return nullptr;
    }
}

void kcp_st_close(void* s) {
    delete static_cast<SafetensorsFile*>(s);
}

int kcp_st_identity(void* s, const char* name, unsigned long long* out, char* err,
                    std::size_t len) {
    try {
        put_identity(static_cast<SafetensorsFile*>(s)->identity(name), out);
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

int kcp_st_metadata(void* s, const char* key, char* text, std::size_t text_len, char* err,
                    std::size_t len) {
    try {
        const auto v = static_cast<SafetensorsFile*>(s)->metadata(key);
        std::strncpy(text, v.c_str(), text_len - 1);
        text[text_len - 1] = 0;
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

int kcp_st_load_rows(void* s, const char* prefix, std::size_t expert, std::size_t first,
                     std::size_t count, std::size_t budget, unsigned char* blocks,
                     std::size_t blocks_n, unsigned char* scales, std::size_t scales_n,
                     std::size_t* columns, char* err, std::size_t len) {
    try {
        const auto r = static_cast<SafetensorsFile*>(s)->mxfp4_rows(prefix, expert, first, count,
                                                                    budget);
        *columns = r.columns;
        std::memcpy(blocks, r.blocks.data(), std::min(blocks_n, r.blocks.size()));
        std::memcpy(scales, r.scales.data(), std::min(scales_n, r.scales.size()));
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

// The MXFP4 MoE layer over a file's expert tensors: the <gate>, <up> and <down> prefixes'
// _blocks / _scales, loaded by mxfp4_experts; the set's bank identity is the gate blocks
// tensor's.
int kcp_st_moe(void* s, void* probe, const char* gate, const char* up, const char* down,
               const std::uint16_t* x, const float* logits, std::size_t tokens,
               std::size_t top_k, float* y, int* selected, float* weights, int* result,
               char* err, std::size_t len) {
    try {
        auto* file = static_cast<SafetensorsFile*>(s);
        std::size_t eg = 0, eu = 0, ed = 0;
        const std::size_t budget = std::size_t(1) << 34;
        const auto g = file->mxfp4_experts(gate, eg, budget);
        const auto u = file->mxfp4_experts(up, eu, budget);
        const auto d = file->mxfp4_experts(down, ed, budget);
        if (eg != eu || eg != ed || g.rows != u.rows || g.columns != d.rows ||
            d.columns != g.rows)
            throw std::invalid_argument("mxfp4_expert_shape");
        const WeightIdentity ident = file->identity(std::string(gate) + "_blocks");
        HipDenseCompute::Mxfp4Experts e{&ident, eg, g.columns, g.rows,
                                        g.blocks, g.scales, u.blocks, u.scales,
                                        d.blocks, d.scales};
        const std::atomic_bool stop{false};
        const std::size_t experts = eg, hidden = g.columns;
        *result = encode(static_cast<Probe*>(probe)->compute.moe_mxfp4(
            e, std::span<const std::uint16_t>(x, tokens * hidden),
            std::span<const float>(logits, tokens * experts), tokens, top_k,
            std::span<float>(y, tokens * hidden), std::span<std::int32_t>(selected, tokens * top_k),
            std::span<float>(weights, tokens * top_k), stop));
        return 0;
    } catch (const std::exception& e) {
        return fail(e, err, len);
    }
}

}  // extern "C"
