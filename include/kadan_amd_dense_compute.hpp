// kadan_amd host C++ layer: the GGUF / MXFP4 part of the reference worker's projection
// interface kadan::DenseCompute (IW/include/kadan/dense_compute.hpp:60-342, IW =
// services/hikari/inference_worker), implemented over the C ABI of kadan_amd.h.
//
// The types below restate the reference's (same names, members and meaning) so the
// model code that calls DenseCompute needs no change: a kadan::DenseCompute subclass
// forwards its GGUF virtuals to HipDenseCompute (a thin adapter, one call each).
// Contract, as the reference states it (dense_compute.hpp:58-59,174-179,215-218):
//   * host spans are borrowed: owned by the caller until return, never retained;
//   * every call is synchronous: all device work and source callbacks finish first;
//   * `unsupported` is returned before any source read or output write;
//   * execution failures throw std::runtime_error and are never retried.
#pragma once

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <thread>
#include <optional>
#include <span>
#include <tuple>
#include <vector>

namespace kadan_amd {

// IW/include/kadan/dense_compute.hpp:44-56
enum class ProjectionResult { unsupported, unvalidated, finite };

// IW/include/kadan/projection_math.hpp:16-19.  image_feed_forward lets the reference use
// TF32 products for image workloads; every product here is fp32 (or finer), so both
// policies run the same kernels.
enum class ProjectionPolicy { standard, image_feed_forward };

// IW/include/kadan/weight_identity.hpp:7-19
struct WeightIdentity {
    std::uint64_t device = 0;
    std::uint64_t inode = 0;
    std::uint64_t file_size = 0;
    std::uint64_t modified_seconds = 0;
    std::uint64_t modified_nanoseconds = 0;
    std::uint64_t changed_seconds = 0;
    std::uint64_t changed_nanoseconds = 0;
    std::uint64_t payload_begin = 0;
    std::uint64_t payload_end = 0;

    auto operator<=>(const WeightIdentity&) const = default;
};

namespace gguf {
// IW/include/kadan/gguf_quantization.hpp:16-27, plus q4_0 (GGML type 2), which the
// reference has no encoding for.  Every encoding runs on this implementation.
enum class Encoding { q3_k, q4_k, q8_0, q6_k, iq3_xxs, iq4_nl, iq4_xs, iq2_s, iq3_s, bf16, q4_0 };

// GGML type id -> encoding (IW/include/kadan/gguf_quantization.hpp:30-55, plus type 2).
std::optional<Encoding> encoding(std::uint32_t ggml_type);
bool supported(Encoding);                 // runs on this implementation
std::size_t block_values(Encoding);      // gguf_quantization.hpp:65-69 (+ q4_0: 32)
std::size_t block_bytes(Encoding);       // gguf_quantization.hpp:71-95 (+ q4_0: 18)
}  // namespace gguf

class HipDenseCompute {
public:
    // IW/include/kadan/dense_compute.hpp:170-172: whole packed rows; first is a row.
    using GgufWeightSource = std::function<void(std::size_t, std::span<std::byte>)>;
    // IW/include/kadan/dense_compute.hpp:223: F32 weights; first is an element offset, a
    // whole number of rows (first_row * in), as IW/src/cuda/h3_compute.cu:2113-2115 calls it.
    using FloatWeightSource = std::function<void(std::size_t, std::span<float>)>;

    // IW/include/kadan/dense_compute.hpp:197,201
    static constexpr std::size_t gguf_batch_rows = 8;
    static constexpr std::size_t gguf_batch_max_rows = 4096;

    // IW/include/kadan/dense_compute.hpp:205-213.  No encoding means F32 rows: the source
    // then delivers in * 4 bytes per row (IW/src/models/text/gguf_weights.cpp:460-461).
    struct GgufBatchJob {
        const WeightIdentity* identity;
        std::optional<gguf::Encoding> encoding;
        const GgufWeightSource* source;
        std::span<const float> input;
        std::size_t in, out;
        std::span<float> output;
        bool retain_misses;
    };

    // One MXFP4 expert tensor set in the GPT-OSS layout (IW/include/kadan/checkpoint.hpp:
    // 151-163): gate/up [experts, inter, hidden/2] + scales [experts, inter, hidden/32],
    // down [experts, hidden, inter/2] + scales [experts, hidden, inter/32].
    struct Mxfp4Experts {
        const WeightIdentity* identity;  // bank key of the whole set
        std::size_t experts, hidden, inter;
        std::span<const std::uint8_t> gate_blocks, gate_scales, up_blocks, up_scales,
            down_blocks, down_scales;
    };

    explicit HipDenseCompute(int device = 0);
    ~HipDenseCompute();
    HipDenseCompute(const HipDenseCompute&) = delete;
    HipDenseCompute& operator=(const HipDenseCompute&) = delete;

    // IW/include/kadan/dense_compute.hpp:180-194.  Rows <= gguf_batch_rows run the
    // decode-time product (fp32 decode, fp32 accumulation); more rows run the prefill GEMM
    // (kdq_gemm_packed: fp16 MFMA operands, weights dequantised to fp16 and x after a
    // per-row power-of-two scale, fp32 accumulation) over packed Q4_K / Q8_0 / Q6_K
    // weights, else the decode-time product per group.  `precise` keeps fp32 operands for
    // every row count: the exact-decode product (kdq_gemv_exact) over a row-major resident
    // copy of its own.  Bias is added to every output row.
    ProjectionResult dense_gguf_source(const WeightIdentity&, gguf::Encoding,
                                       const GgufWeightSource&, std::span<const float> bias,
                                       std::span<const float> input, std::size_t in,
                                       std::size_t out, std::span<float> output,
                                       const std::atomic_bool& cancel, bool precise = false,
                                       bool retain_misses = true);

    // IW/include/kadan/dense_compute.hpp:332-341 (the interface's one pure virtual): plain
    // F32 projection, weights [out x in] row-major, output [rows x out] = input . W^T +
    // bias.  Runs the exact-product kernel over F32 rows; nothing is retained.
    void dense(std::span<const float> weights, std::span<const float> bias,
               std::span<const float> input, std::size_t in, std::size_t out,
               std::span<float> output, const std::atomic_bool& cancel, bool precise = false);

    // IW/include/kadan/dense_compute.hpp:215-221: every job in one synchronous
    // submission; jobs sharing an input span upload it once.  Returns unvalidated (the
    // caller checks finiteness, IW/src/models/text/gguf_weights.cpp:478-484).  F32 jobs
    // (no encoding) follow the eligibility of IW/include/kadan/gguf_batch_partition.hpp:
    // 15-37 (in % 8 == 0, a row of at most 16 MiB) and run the exact fp32 product
    // (IW/src/cuda/h3_compute.cu:4076-4082).
    ProjectionResult dense_gguf_batch(std::span<const GgufBatchJob>, const std::atomic_bool&);
    // The eligibility rule dense_gguf_batch applies before any source read
    // (IW/include/kadan/gguf_batch_partition.hpp:15-37 gguf_batch_supported, restricted to
    // the encodings this implementation runs); needs no device.
    static bool batch_supported(std::span<const GgufBatchJob>);

    // IW/include/kadan/dense_compute.hpp:239-249: F32 projection whose weights [out x in]
    // come from `source`, kept in the weight bank under `identity` (the same entry an F32
    // batch job of that identity uses).  output [rows x out] = input . W^T + bias by the
    // exact fp32 product; any `in` (rows are zero-padded to a multiple of 8 on the
    // device).  Non-finite weights throw kdq_nonfinite_weight; returns finite when every
    // output is finite, else unvalidated.  `precise` and `policy` select nothing: the
    // product is fp32 either way (the reference's TF32 applies to image workloads only).
    ProjectionResult dense_source(const WeightIdentity&, const FloatWeightSource&,
                                  std::span<const float> bias, std::span<const float> input,
                                  std::size_t in, std::size_t out, std::span<float> output,
                                  const std::atomic_bool& cancel, bool precise = false,
                                  ProjectionPolicy policy = ProjectionPolicy::standard);

    // Prefill with quantized activations (no reference device counterpart: the reference's
    // CPU path, IW/src/models/text/cpu_matvec.cpp:28-66, quantizes activations the same
    // way).  Q4_0 weights only; fp16 inputs [rows x in] -> fp16 outputs [rows x out].
    ProjectionResult dense_gguf_q8_source(const WeightIdentity&, gguf::Encoding,
                                          const GgufWeightSource&,
                                          std::span<const std::uint16_t> input_f16,
                                          std::size_t in, std::size_t out,
                                          std::span<std::uint16_t> output_f16,
                                          const std::atomic_bool& cancel);

    // The MXFP4 MoE layer (MoeLayer::forward semantics, IW/src/models/text/qwen_layers.cpp:
    // 378-492, no shared expert).  x: bf16 [tokens x hidden]; logits fp32 [tokens x experts];
    // output fp32 [tokens x hidden]; selected/weights [tokens x top_k] are optional.
    ProjectionResult moe_mxfp4(const Mxfp4Experts&, std::span<const std::uint16_t> x_bf16,
                               std::span<const float> logits, std::size_t tokens,
                               std::size_t top_k, std::span<float> output,
                               std::span<std::int32_t> selected, std::span<float> weights,
                               const std::atomic_bool& cancel);

    // Whole packed rows of `in` values decoded on the device exactly as kadan::gguf::decode
    // (kdq_dequantize), output [rows x in]; throws "kdq_nonfinite_weight" when a decoded
    // value is not finite (the reference's gguf_nonfinite_weight check of read_rows,
    // IW/src/weights/gguf_checkpoint.cpp:628-636).
    void dequantize_rows(gguf::Encoding, std::span<const std::byte> packed, std::size_t in,
                         std::span<float> output);

    // The weight bank's device byte limit (0: none), the DeviceWeights envelope of the
    // reference (IW/include/kadan/device_weights.hpp:35-60,203-206).  A miss that would
    // pass it is not admitted and evicts nothing: dense_gguf_source streams it (existing
    // hits stay resident), a batch job holds it for the call only.  MoE expert sets count
    // against the limit but are always admitted.
    void set_weight_limit(std::size_t bytes);

    // IW/include/kadan/dense_compute.hpp:72-80: retire these identities from the bank.
    std::size_t release_weights(std::span<const WeightIdentity>);
    // Device bytes held by the weight bank.
    std::size_t retained_weight_bytes() const;
    // IW/include/kadan/dense_compute.hpp:63-66: release scratch (workspace) memory.
    void release_scratch();

private:
    struct Resident;
    struct ReadTeam;
    using BankKey = std::tuple<WeightIdentity, int, std::size_t, std::size_t>;

    // The resident weights of one projection, uploaded through the pinned staging on a
    // miss.  `type`: the GGML type of the rows (KDQ_F32 for F32 rows, stored with each
    // row zero-padded to a multiple of 8 values).  `product`: for the decode GEMV or the
    // prefill GEMM (tile-packed where the packed GEMV takes the shape, one copy for both),
    // else row-major rows.  Returns nullptr when `stream_miss` is set and the weights are
    // not in the bank, or would not fit its limit (the caller then streams them,
    // stream_product).
    const Resident* weights_for(const WeightIdentity&, int type, std::size_t in,
                                std::size_t out, const GgufWeightSource&, bool retain,
                                const std::atomic_bool& cancel,
                                std::unique_ptr<Resident>& transient, bool product,
                                bool stream_miss = false);
    // Reads rows [first, first + n) of `source` into pinned staging buffer `b` with the read
    // team, after the device has finished with that buffer's previous chunk.
    std::byte* stage_rows(unsigned b, const GgufWeightSource&, std::size_t first, std::size_t n,
                          std::size_t row_bytes);
    void staged(unsigned b);  // the device's reads of staging buffer b are enqueued
    // y[rows x out] = x . W^T with W streamed chunk by chunk through the staging buffers
    // (reads of one chunk overlap the upload, packing and product of the previous).
    void stream_product(gguf::Encoding, std::size_t in, std::size_t out, std::size_t rows,
                        const GgufWeightSource&, const float* dx, float* dy, unsigned* dstatus,
                        const std::atomic_bool& cancel, bool gemm);
    void* device_buffer(std::size_t slot, std::size_t bytes);
    void synchronize();

    int device_;
    void* stream_ = nullptr;
    mutable std::mutex mutex_;
    std::map<BankKey, std::unique_ptr<Resident>> bank_;
    std::vector<std::pair<void*, std::size_t>> buffers_;  // reusable device scratch
    void* pinned_[2] = {nullptr, nullptr};  // double-buffered host staging
    std::size_t pinned_bytes_ = 0;
    void* staged_[2] = {nullptr, nullptr};  // hipEvent_t: the device is done with pinned_[b]
    bool staged_pending_[2] = {false, false};
    std::unique_ptr<ReadTeam> team_;
    std::size_t weight_limit_ = 0;
};

}  // namespace kadan_amd
