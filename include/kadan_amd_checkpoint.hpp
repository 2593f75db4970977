// kadan_amd on-disk weight formats: the readers that bring checkpoint bytes to the
// quantized-weight matmul path, restating the reference worker's contracts
// (IW = services/hikari/inference_worker):
//   * GgufCheckpoint: GGUF v3, one file or a numbered split set
//     (IW/include/kadan/gguf_checkpoint.hpp:55-102, IW/src/weights/gguf_checkpoint.cpp:
//     438-720): bounded metadata parsing, per-tensor / per-expert WeightIdentity
//     (file stat tuple + payload byte range), check_unchanged, whole packed rows by pread;
//     source() adapts read_packed_rows to HipDenseCompute's GgufWeightSource.
//   * SafetensorsShard: one .safetensors file with the GPT-OSS MXFP4 expert tensors
//     (IW/include/kadan/checkpoint.hpp:151-163, IW/src/weights/checkpoint.cpp:669-730):
//     <prefix>_blocks U8 [experts, rows, groups, 16] and <prefix>_scales U8 [experts,
//     rows, groups], loaded still packed.
// Errors are std::invalid_argument / std::runtime_error with the reference's codes
// ("gguf_row_range", "gguf_checkpoint_changed", "mxfp4_expert_shape", ...).  Host only:
// nothing here touches a device.
#pragma once

#include <array>
#include <atomic>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <span>
#include <string>
#include <string_view>
#include <vector>

#include "kadan_amd_dense_compute.hpp"

namespace kadan_amd::checkpoint {

// IW/include/kadan/gguf_checkpoint.hpp:16-23
struct GgufTensor {
    std::string name;
    // GGML order: columns, rows, experts; omitted dimensions are one.
    std::array<std::uint64_t, 3> shape{1, 1, 1};
    std::size_t rank = 0;
    std::uint32_t type = 0;  // GGML type id
    std::uint64_t bytes = 0;
};

class GgufCheckpoint {
public:
    // `root`: a directory holding one .gguf file or a split set <p>-NNNNN-of-NNNNN.gguf.
    // Reads bounded metadata only.  F32, F16 and every encoding this library runs.
    GgufCheckpoint(const std::string& root, const std::atomic_bool& cancel);
    ~GgufCheckpoint();
    GgufCheckpoint(const GgufCheckpoint&) = delete;
    GgufCheckpoint& operator=(const GgufCheckpoint&) = delete;

    std::size_t tensor_count() const;
    const GgufTensor& tensor(std::string_view name) const;
    const GgufTensor& tensor_at(std::size_t index) const;
    // The file's stat tuple and the byte range of expert `expert`'s slice of the tensor.
    WeightIdentity identity(std::string_view name, std::size_t expert = 0) const;
    // Throws "gguf_checkpoint_changed" when any file's size or times changed.
    void check_unchanged() const;
    // Whole packed rows of expert `expert`, from `first_row`; output.size() is a whole
    // number of rows.  No decoding, no validation (the consumer validates).
    void read_packed_rows(std::string_view name, std::size_t expert, std::size_t first_row,
                          std::span<std::byte> output, const std::atomic_bool& cancel) const;
    // A whole F32 tensor, checked finite.
    void read_vector(std::string_view name, std::span<float> output,
                     const std::atomic_bool& cancel) const;
    // Decoded rows (fp32, exactly as kadan::gguf::decode): packed rows read here, decoded
    // on the device of `compute` (kdq_dequantize) and checked finite.
    void read_rows(std::string_view name, std::size_t expert, std::size_t first_row,
                   std::span<float> output, const std::atomic_bool& cancel,
                   HipDenseCompute& compute) const;
    // read_packed_rows of one expert as a HipDenseCompute::GgufWeightSource.
    HipDenseCompute::GgufWeightSource source(std::string_view name, std::size_t expert,
                                             const std::atomic_bool& cancel) const;

    // Metadata of the first file (IW/include/kadan/gguf_checkpoint.hpp:38-46).
    bool has(std::string_view key) const;
    std::string string(std::string_view key) const;
    std::uint64_t integer(std::string_view key) const;
    double number(std::string_view key) const;
    bool boolean(std::string_view key) const;
    std::vector<bool> booleans(std::string_view key) const;
    std::vector<std::string> strings(std::string_view key) const;
    std::vector<std::int64_t> integers(std::string_view key) const;
    std::vector<double> numbers(std::string_view key) const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

// Safetensors element types of the shard reader.
enum class Dtype { u8, i8, f16, bf16, f32, other };

struct SafetensorsTensor {
    std::string name;
    Dtype dtype = Dtype::other;
    std::vector<std::uint64_t> shape;
    std::uint64_t begin = 0, end = 0;  // byte range in the file
};

// One MXFP4 expert projection loaded packed: `rows` x `columns` values, blocks
// [rows, columns / 2] (element 2i the low nibble of byte i), scales [rows, columns / 32]
// (E8M0; 255 is refused).
struct Mxfp4Rows {
    std::size_t rows = 0, columns = 0;
    std::vector<std::uint8_t> blocks, scales;
};

class SafetensorsShard {
public:
    explicit SafetensorsShard(const std::string& path);
    ~SafetensorsShard();
    SafetensorsShard(const SafetensorsShard&) = delete;
    SafetensorsShard& operator=(const SafetensorsShard&) = delete;

    std::size_t tensor_count() const;
    const SafetensorsTensor& tensor(std::string_view name) const;
    WeightIdentity identity(std::string_view name) const;
    void check_unchanged() const;
    std::string metadata(std::string_view key) const;  // "__metadata__" strings
    // IW/src/weights/checkpoint.cpp:669-730 (load_mxfp4_expert_rows): rows [first, first +
    // count) of expert `expert` of <prefix>_blocks / <prefix>_scales; the byte total
    // must fit payload_budget ("payload_budget"); scales are validated.
    Mxfp4Rows load_mxfp4_expert_rows(std::string_view prefix, std::size_t expert,
                                     std::size_t first, std::size_t count,
                                     std::size_t payload_budget) const;
    // The whole expert set of one projection, in the GPT-OSS layout the MoE layer takes
    // (blocks [experts, rows, columns / 2], scales [experts, rows, columns / 32]).
    Mxfp4Rows load_mxfp4_experts(std::string_view prefix, std::size_t& experts,
                                 std::size_t payload_budget) const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
};

}  // namespace kadan_amd::checkpoint
