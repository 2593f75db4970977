// kadan_amd checkpoint readers: the two on-disk forms whose bytes feed the quantized-weight
// matmul path, read on the host and handed to the device layer still packed.
//
//   * GgufFiles: a directory holding one GGUF v3 file or a split set named
//     <stem>-NNNNN-of-NNNNN.gguf.  Tensor payloads are located, bounds-checked and read
//     as whole packed rows; each tensor (and each expert slice of a 3-D tensor) carries a
//     WeightIdentity, the key HipDenseCompute's weight bank uses.  The role matches the
//     reference worker's GGUF reader (IW/include/kadan/gguf_checkpoint.hpp:55-102; IW =
//     services/hikari/inference_worker); the error codes are the reference's, so a
//     caller's handling carries over.
//   * SafetensorsFile: one .safetensors file; the GPT-OSS MXFP4 expert tensors
//     <prefix>_blocks U8 [experts, rows, groups, 16] and <prefix>_scales U8 [experts,
//     rows, groups] (IW/include/kadan/checkpoint.hpp:151-163) load still packed, in the
//     layout HipDenseCompute::moe_mxfp4 takes.
//
// Every failure throws CheckpointError whose what() is a short code ("gguf_row_range",
// "gguf_checkpoint_changed", "mxfp4_expert_shape", ...).  Nothing here touches a device
// except GgufFiles::decode_rows, which runs through HipDenseCompute.
#pragma once

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <span>
#include <stdexcept>
#include <string>
#include <string_view>
#include <variant>
#include <vector>

#include "kadan_amd_dense_compute.hpp"

namespace kadan_amd::checkpoint {

struct CheckpointError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// One tensor of a GGUF file set, as the matmul path consumes it.  GGUF lists dimensions
// fastest first: ne0 values per row (`columns`), ne1 rows, ne2 experts; a dimension the
// file does not list is 1.
struct GgufTensorInfo {
    std::string name;
    std::uint32_t ggml_type = 0;
    std::size_t rank = 0;  // dimensions the file lists, 1..3
    std::uint64_t columns = 1, rows = 1, experts = 1;
    std::uint64_t row_bytes = 0;    // one packed row
    std::uint64_t slice_bytes = 0;  // one expert: rows * row_bytes
    std::uint64_t bytes = 0;        // the whole payload
    std::size_t file = 0;           // which file of the set holds it
    std::uint64_t offset = 0;       // payload start, from the beginning of that file
};

// One metadata value: a scalar, or an array of scalars of one GGUF value type.
class GgufValue {
public:
    using Scalar = std::variant<std::int64_t, std::uint64_t, double, bool, std::string>;

    GgufValue() = default;
    GgufValue(std::uint32_t type, bool array, std::vector<Scalar> items)
        : type_(type), array_(array), items_(std::move(items)) {}

    std::uint32_t gguf_type() const { return type_; }  // the scalar's or elements' type
    bool is_array() const { return array_; }

    // Scalars.  Each throws its own code when the value has another shape or type:
    std::string text() const;     // string                                gguf_metadata_string
    std::uint64_t count() const;  // integer >= 0 of any width             gguf_metadata_integer
    double real() const;          // float32 / float64                     gguf_metadata_number
    bool flag() const;            // bool                                  gguf_metadata_boolean
    // Arrays:
    std::vector<std::string> texts() const;    //                          gguf_metadata_strings
    std::vector<std::int64_t> integers() const;  // integers within int64  gguf_metadata_integers
    std::vector<double> reals() const;          //                         gguf_metadata_numbers
    std::vector<bool> flags() const;            //                         gguf_metadata_booleans

private:
    std::uint32_t type_ = 0;
    bool array_ = false;
    std::vector<Scalar> items_;
};

class GgufFiles {
public:
    // Opens `directory` (one .gguf file, or every file of one split set) and decodes each
    // file's header.  Payload bytes are not read.  Accepts F32, F16 and the GGUF
    // encodings the matmul path runs (kdq_block_values(type) != 0).
    GgufFiles(const std::string& directory, const std::atomic_bool& cancel);
    ~GgufFiles();
    GgufFiles(const GgufFiles&) = delete;
    GgufFiles& operator=(const GgufFiles&) = delete;

    std::size_t size() const;                             // tensors in the set
    const GgufTensorInfo& info(std::size_t index) const;  // file order; gguf_tensor_index
    const GgufTensorInfo& info(std::string_view name) const;  // gguf_missing_tensor

    // The holding file's stat tuple and the byte range of expert `expert`'s slice (the
    // whole payload for a tensor of rank < 3).  gguf_expert_range past the last expert.
    WeightIdentity slice_identity(std::string_view name, std::size_t expert = 0) const;
    // gguf_checkpoint_changed when any file's device, inode, size or times moved since
    // the set was opened.  Every payload read checks this first.
    void verify_unchanged() const;

    // Whole packed rows [first_row, first_row + out.size() / row_bytes) of one expert,
    // byte for byte.  gguf_row_range unless the tensor has rows (rank >= 2), `out` is a
    // whole number of rows and they all exist.
    void copy_rows(std::string_view name, std::size_t expert, std::size_t first_row,
                   std::span<std::byte> out, const std::atomic_bool& cancel) const;
    // A rank-1 F32 tensor, every value finite (gguf_vector_shape, gguf_nonfinite_weight).
    void copy_vector(std::string_view name, std::span<float> out,
                     const std::atomic_bool& cancel) const;
    // Rows decoded to fp32 on `compute`'s device exactly as kadan::gguf::decode does
    // (HipDenseCompute::dequantize_rows); F32 rows are copied.  Non-finite values throw.
    void decode_rows(std::string_view name, std::size_t expert, std::size_t first_row,
                     std::span<float> out, const std::atomic_bool& cancel,
                     HipDenseCompute& compute) const;
    // copy_rows of one expert as the weight source HipDenseCompute reads.  The source
    // keeps `cancel` and this object by reference.
    HipDenseCompute::GgufWeightSource row_source(std::string_view name, std::size_t expert,
                                                 const std::atomic_bool& cancel) const;

    // Metadata of the set's first file.  value(): gguf_missing_metadata when absent.
    bool has(std::string_view key) const;
    const GgufValue& value(std::string_view key) const;

private:
    struct State;
    std::unique_ptr<State> state_;
};

// Element types a safetensors header may name.
enum class Dtype { boolean, u8, i8, u16, i16, f16, bf16, u32, i32, f32, u64, i64, f64, f8_e4m3, f8_e5m2 };

struct SafetensorsInfo {
    std::string name;
    Dtype dtype = Dtype::u8;
    std::vector<std::uint64_t> shape;
    std::uint64_t begin = 0, end = 0;  // byte range, from the beginning of the file
};

// An MXFP4 projection loaded packed: `rows` x `columns` values; blocks [rows, columns / 2]
// (value 2i in the low nibble of byte i), E8M0 scales [rows, columns / 32], none 255.
struct Mxfp4Rows {
    std::size_t rows = 0, columns = 0;
    std::vector<std::uint8_t> blocks, scales;
};

class SafetensorsFile {
public:
    // Reads and checks the JSON header: every tensor's dtype, shape and data_offsets, the
    // offsets tiling the payload exactly, names and keys ASCII and unique.
    explicit SafetensorsFile(const std::string& path);
    ~SafetensorsFile();
    SafetensorsFile(const SafetensorsFile&) = delete;
    SafetensorsFile& operator=(const SafetensorsFile&) = delete;

    std::size_t size() const;
    const SafetensorsInfo& info(std::string_view name) const;  // missing_tensor
    WeightIdentity identity(std::string_view name) const;
    void verify_unchanged() const;                      // checkpoint_changed
    std::string metadata(std::string_view key) const;  // safetensors_missing_metadata

    // Rows [first, first + count) of expert `expert` of <prefix>_blocks / _scales, at most
    // `payload_budget` bytes together; every scale byte checked (invalid_block_scale).
    // Refusals: projection_range_or_name (empty prefix, no rows), missing_tensor,
    // mxfp4_dtype, mxfp4_expert_shape, payload_budget.
    Mxfp4Rows mxfp4_rows(std::string_view prefix, std::size_t expert, std::size_t first,
                         std::size_t count, std::size_t payload_budget) const;
    // Every expert of one projection: blocks [experts, rows, columns / 2], scales
    // [experts, rows, columns / 32]; the expert count in `experts`.
    Mxfp4Rows mxfp4_experts(std::string_view prefix, std::size_t& experts,
                            std::size_t payload_budget) const;

private:
    struct State;
    std::unique_ptr<State> state_;
};

}  // namespace kadan_amd::checkpoint
