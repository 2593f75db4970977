// On-disk readers of the quantized-weight matmul path: GGUF v3 (one file or a numbered
// split set) and safetensors shards with GPT-OSS MXFP4 experts.  Contracts restated from
// IW/src/weights/gguf_checkpoint.cpp:438-720 and IW/src/weights/checkpoint.cpp:669-730
// (IW = services/hikari/inference_worker): bounded metadata, immutable descriptors
// checked unchanged around every payload read, pread of whole rows, identities keyed by
// the file's stat tuple and the payload byte range.  The parsers are this library's own
// (the reference parses GGUF through ggml's gguf.cpp; safetensors through its own JSON
// reader).
#include "kadan_amd_checkpoint.hpp"

#include <algorithm>
#include <bit>
#include <cerrno>
#include <cmath>
#include <cstring>
#include <fcntl.h>
#include <filesystem>
#include <limits>
#include <regex>
#include <stdexcept>
#include <sys/stat.h>
#include <unistd.h>
#include <unordered_set>
#include <utility>
#include <variant>

#include "kadan_amd.h"

namespace kadan_amd::checkpoint {
namespace {

void require(bool ok, const char* what) {
    if (!ok)
        throw std::invalid_argument(what);
}

void stop(const std::atomic_bool& cancel, const char* what = "gguf_cancelled") {
    if (cancel.load())
        throw std::runtime_error(what);
}

std::uint64_t add(std::uint64_t a, std::uint64_t b, const char* what = "gguf_size_overflow") {
    require(b <= UINT64_MAX - a, what);
    return a + b;
}

std::uint64_t mul(std::uint64_t a, std::uint64_t b, const char* what = "gguf_size_overflow") {
    require(!b || a <= UINT64_MAX / b, what);
    return a * b;
}

// An open regular file and the stat it was opened with; every payload read is bracketed
// by unchanged() (size, mtime and ctime as at open).
struct File {
    int fd = -1;
    struct stat initial {};
    const char* changed_code = "gguf_checkpoint_changed";

    File(int descriptor, const char* changed, std::uint64_t minimum, bool directory = false)
        : fd(descriptor), changed_code(changed) {
        if (fd < 0)
            throw std::runtime_error(directory ? "checkpoint_open_failed" : "gguf_open_failed");
        if (::fstat(fd, &initial) ||
            (directory ? !S_ISDIR(initial.st_mode)
                       : (!S_ISREG(initial.st_mode) ||
                          std::uint64_t(initial.st_size) < minimum))) {
            ::close(fd);
            fd = -1;
            throw std::invalid_argument("gguf_not_regular_file");
        }
    }
    File(File&& o) noexcept
        : fd(std::exchange(o.fd, -1)), initial(o.initial), changed_code(o.changed_code) {}
    File(const File&) = delete;
    ~File() {
        if (fd >= 0)
            ::close(fd);
    }

    std::uint64_t size() const { return std::uint64_t(initial.st_size); }

    void unchanged() const {
        struct stat now {};
        if (::fstat(fd, &now) || now.st_size != initial.st_size ||
            now.st_mtim.tv_sec != initial.st_mtim.tv_sec ||
            now.st_mtim.tv_nsec != initial.st_mtim.tv_nsec ||
            now.st_ctim.tv_sec != initial.st_ctim.tv_sec ||
            now.st_ctim.tv_nsec != initial.st_ctim.tv_nsec)
            throw std::invalid_argument(changed_code);
    }

    WeightIdentity identity(std::uint64_t begin, std::uint64_t end) const {
        const auto& s = initial;
        return {std::uint64_t(s.st_dev), std::uint64_t(s.st_ino), std::uint64_t(s.st_size),
                std::uint64_t(s.st_mtim.tv_sec), std::uint64_t(s.st_mtim.tv_nsec),
                std::uint64_t(s.st_ctim.tv_sec), std::uint64_t(s.st_ctim.tv_nsec), begin, end};
    }

    void read(std::uint64_t at, std::span<std::uint8_t> out, const std::atomic_bool* cancel,
              const char* bounds = "gguf_read_bounds") const {
        require(at <= size() && out.size() <= size() - at, bounds);
        while (!out.empty()) {
            if (cancel)
                stop(*cancel);
            const auto n = ::pread(fd, out.data(), out.size(), off_t(at));
            if (n < 0 && errno == EINTR)
                continue;
            if (n <= 0)
                throw std::runtime_error("gguf_read_failed");
            at += std::uint64_t(n);
            out = out.subspan(std::size_t(n));
        }
    }
};

// ------------------------------------------------------------------- GGUF

// GGUF value types (the GGUF v3 specification).
enum : std::uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
    kString = 8, kArray = 9, kU64 = 10, kI64 = 11, kF64 = 12
};
constexpr std::uint64_t kMetadataLimit = 32 * 1024 * 1024;

std::size_t scalar_width(std::uint32_t type) {
    switch (type) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: throw std::invalid_argument("gguf_metadata_type");
    }
}

// One scalar kept as its type and raw little-endian bits.
struct Scalar {
    std::uint32_t type = kU8;
    std::uint64_t bits = 0;
};
struct Array {
    std::uint32_t element = kU8;
    std::vector<Scalar> values;
    std::vector<std::string> texts;
};
using Value = std::variant<Scalar, std::string, Array>;

bool is_integer(std::uint32_t t) {
    return t == kU8 || t == kI8 || t == kU16 || t == kI16 || t == kU32 || t == kI32 ||
           t == kU64 || t == kI64;
}

std::int64_t signed_of(const Scalar& s) {
    switch (s.type) {
    case kI8: return std::int8_t(s.bits);
    case kI16: return std::int16_t(s.bits);
    case kI32: return std::int32_t(s.bits);
    case kI64: return std::int64_t(s.bits);
    default: return std::int64_t(s.bits);
    }
}

double number_of(const Scalar& s) {
    if (s.type == kF32)
        return double(std::bit_cast<float>(std::uint32_t(s.bits)));
    if (s.type == kF64)
        return std::bit_cast<double>(s.bits);
    if (is_integer(s.type))
        return (s.type == kI8 || s.type == kI16 || s.type == kI32 || s.type == kI64)
                   ? double(signed_of(s))
                   : double(s.bits);
    throw std::invalid_argument("gguf_metadata_number");
}

// Values and bytes per block of the GGML types this reader accepts (F32 and the
// encodings of include/kadan_amd.h that kadan loads, plus Q4_0).
bool block_geometry(std::uint32_t type, std::uint64_t& values, std::uint64_t& bytes) {
    if (type == KDQ_F32) {
        values = 1, bytes = 4;
        return true;
    }
    if (type == KDQ_F16 || !kdq_block_values(int(type)))
        return false;
    values = kdq_block_values(int(type));
    bytes = kdq_block_bytes(int(type));
    return true;
}

// The GGUF header of one file, parsed with bounded reads through a 64 KiB window that
// never reaches past the metadata limit or the file.
class HeaderParser {
public:
    HeaderParser(const File& f, const std::atomic_bool& cancel) : file_(f), cancel_(cancel) {}

    std::uint64_t at = 0;

    void bytes(std::span<std::uint8_t> out) {
        stop(cancel_);
        require(at <= kMetadataLimit && out.size() <= kMetadataLimit - at, "gguf_metadata_limit");
        require(at <= file_.size() && out.size() <= file_.size() - at, "gguf_read_bounds");
        while (!out.empty()) {
            if (at < begin_ || at - begin_ >= size_) {
                begin_ = at;
                size_ = std::size_t(std::min<std::uint64_t>(
                    window_.size(), std::min(file_.size(), kMetadataLimit) - at));
                file_.read(at, std::span(window_).first(size_), &cancel_);
            }
            const std::size_t offset = std::size_t(at - begin_);
            const std::size_t n = std::min(out.size(), size_ - offset);
            std::memcpy(out.data(), window_.data() + offset, n);
            at += n;
            out = out.subspan(n);
        }
    }

    std::uint64_t u64() {
        std::array<std::uint8_t, 8> b{};
        bytes(b);
        std::uint64_t v = 0;
        for (int i = 0; i < 8; ++i)
            v |= std::uint64_t(b[i]) << (8 * i);
        return v;
    }
    std::uint32_t u32() {
        std::array<std::uint8_t, 4> b{};
        bytes(b);
        return std::uint32_t(b[0]) | std::uint32_t(b[1]) << 8 | std::uint32_t(b[2]) << 16 |
               std::uint32_t(b[3]) << 24;
    }
    std::string text(std::uint64_t limit) {
        const auto n = u64();
        require(n <= limit, "gguf_string_limit");
        std::string s(std::size_t(n), '\0');
        bytes({reinterpret_cast<std::uint8_t*>(s.data()), s.size()});
        require(s.find('\0') == std::string::npos, "gguf_string_nul");
        return s;
    }
    Scalar scalar(std::uint32_t type) {
        const std::size_t w = scalar_width(type);
        std::array<std::uint8_t, 8> b{};
        bytes(std::span(b).first(w));
        Scalar s{type, 0};
        for (std::size_t i = 0; i < w; ++i)
            s.bits |= std::uint64_t(b[i]) << (8 * i);
        return s;
    }
    Value value(std::uint32_t type) {
        if (type == kString)
            return text(1024 * 1024);
        if (type == kArray) {
            Array a;
            a.element = u32();
            const auto count = u64();
            require(count <= 524288 && a.element != kArray, "gguf_array_limit");
            if (a.element == kString) {
                for (std::uint64_t i = 0; i < count; ++i)
                    a.texts.push_back(text(1024 * 1024));
            } else {
                (void)scalar_width(a.element);
                for (std::uint64_t i = 0; i < count; ++i)
                    a.values.push_back(scalar(a.element));
            }
            return a;
        }
        return scalar(type);
    }

private:
    const File& file_;
    const std::atomic_bool& cancel_;
    std::array<std::uint8_t, 64 * 1024> window_{};
    std::uint64_t begin_ = 0;
    std::size_t size_ = 0;
};

struct ParsedFile {
    std::map<std::string, Value, std::less<>> metadata;
    std::vector<GgufTensor> tensors;
    std::vector<std::uint64_t> offsets;  // relative to the data section
    std::uint64_t data_begin = 0;
};

ParsedFile parse_gguf(const File& file, const std::atomic_bool& cancel) {
    HeaderParser p(file, cancel);
    ParsedFile out;
    require(p.u32() == 0x46554747u, "gguf_version");  // "GGUF"
    require(p.u32() == 3, "gguf_version");
    const auto tensor_count = p.u64(), kv_count = p.u64();
    require(tensor_count <= 200000 && kv_count <= 16384, "gguf_header_count");
    std::uint64_t alignment = 32;
    for (std::uint64_t i = 0; i < kv_count; ++i) {
        auto key = p.text(256);
        const auto type = p.u32();
        Value v = p.value(type);
        if (key == "general.alignment") {
            const auto* s = std::get_if<Scalar>(&v);
            require(s && s->type == kU32, "gguf_alignment");
            alignment = s->bits;
            require(alignment && alignment <= 4096 && !(alignment & (alignment - 1)),
                    "gguf_alignment");
        }
        require(out.metadata.emplace(std::move(key), std::move(v)).second, "gguf_duplicate_key");
    }
    std::unordered_set<std::string> names;
    for (std::uint64_t i = 0; i < tensor_count; ++i) {
        GgufTensor t;
        t.name = p.text(255);
        require(!t.name.empty() && names.insert(t.name).second, "gguf_duplicate_tensor");
        t.rank = p.u32();
        require(t.rank >= 1 && t.rank <= 3, "gguf_tensor_rank");
        std::uint64_t rows = 1;
        for (std::size_t d = 0; d < t.rank; ++d) {
            t.shape[d] = p.u64();
            require(t.shape[d] && t.shape[d] <= std::uint64_t(INT64_MAX), "gguf_tensor_shape");
            if (d)
                rows = mul(rows, t.shape[d]);
        }
        t.type = p.u32();
        std::uint64_t values = 0, bytes = 0;
        require(block_geometry(t.type, values, bytes), "gguf_tensor_type");
        require(t.shape[0] % values == 0, "gguf_tensor_block_alignment");
        t.bytes = mul(mul(t.shape[0] / values, bytes), rows);
        require(t.bytes <= std::uint64_t(INT64_MAX), "gguf_tensor_shape");
        out.offsets.push_back(p.u64());
        out.tensors.push_back(std::move(t));
    }
    out.data_begin = (p.at + alignment - 1) / alignment * alignment;
    std::vector<std::pair<std::uint64_t, std::uint64_t>> ranges;
    for (std::size_t t = 0; t < out.tensors.size(); ++t) {
        const auto off = out.offsets[t];
        const auto end = add(add(out.data_begin, off), out.tensors[t].bytes);
        require(off % alignment == 0 && end <= file.size(), "gguf_tensor_bounds");
        ranges.emplace_back(off, add(off, out.tensors[t].bytes));
    }
    std::sort(ranges.begin(), ranges.end());
    for (std::size_t t = 1; t < ranges.size(); ++t)
        require(ranges[t].first >= ranges[t - 1].second, "gguf_tensor_overlap");
    file.unchanged();
    return out;
}

const Value& find_key(const std::map<std::string, Value, std::less<>>& m, std::string_view key) {
    require(key.size() <= 256, "gguf_metadata_key");
    const auto it = m.find(key);
    require(it != m.end(), "gguf_missing_metadata");
    return it->second;
}

std::uint64_t integer_of(const Value& v) {
    const auto* s = std::get_if<Scalar>(&v);
    require(s && is_integer(s->type), "gguf_metadata_integer");
    if (s->type == kI8 || s->type == kI16 || s->type == kI32 || s->type == kI64)
        require(signed_of(*s) >= 0, "gguf_metadata_integer");
    return s->bits;
}

}  // namespace

struct GgufCheckpoint::Impl {
    struct Entry {
        GgufTensor tensor;
        std::size_t file;
        std::uint64_t begin;  // absolute byte offset in its file
    };
    std::vector<File> files;
    std::vector<Entry> tensors;  // sorted by name
    std::map<std::string, Value, std::less<>> metadata;

    const Entry& find(std::string_view name) const {
        const auto it = std::lower_bound(tensors.begin(), tensors.end(), name,
                                         [](const Entry& e, std::string_view n) {
                                             return e.tensor.name < n;
                                         });
        require(it != tensors.end() && it->tensor.name == name, "gguf_missing_tensor");
        return *it;
    }
};

GgufCheckpoint::GgufCheckpoint(const std::string& root, const std::atomic_bool& cancel)
    : impl_(std::make_unique<Impl>()) {
    static_assert(std::endian::native == std::endian::little);
    stop(cancel);
    const std::regex pattern(R"((.+)-([0-9]{5})-of-([0-9]{5})\.gguf)");
    std::vector<std::string> names;
    for (const auto& entry : std::filesystem::directory_iterator(root)) {
        stop(cancel);
        if (entry.path().extension() == ".gguf")
            names.push_back(entry.path().filename().string());
        require(names.size() <= 512, "gguf_split_count");
    }
    require(!names.empty(), "gguf_missing_files");
    std::sort(names.begin(), names.end());
    File directory(::open(root.c_str(), O_RDONLY | O_DIRECTORY | O_NOFOLLOW | O_CLOEXEC),
                   "gguf_checkpoint_changed", 0, true);
    // One unsplit file carries no split metadata; a split set is numbered from 1.
    const bool single = names.size() == 1 && !std::regex_match(names[0], pattern);
    std::string prefix;
    std::uint64_t total = 0, metadata_bytes = 0;
    for (std::size_t i = 0; i < names.size(); ++i) {
        std::smatch match;
        require(names[i].size() <= 255 && (single || std::regex_match(names[i], match, pattern)),
                "gguf_split_name");
        if (!single && i == 0)
            prefix = match[1];
        require(single || (match[1] == prefix && std::stoul(match[2]) == i + 1 &&
                           std::stoul(match[3]) == names.size()),
                "gguf_split_name");
        impl_->files.emplace_back(
            ::openat(directory.fd, names[i].c_str(), O_RDONLY | O_NOFOLLOW | O_CLOEXEC),
            "gguf_checkpoint_changed", 24);
        const File& file = impl_->files.back();
        ParsedFile parsed = parse_gguf(file, cancel);
        metadata_bytes = add(metadata_bytes, parsed.data_begin);
        require(metadata_bytes <= 64 * 1024 * 1024, "gguf_metadata_limit");
        if (!single) {
            require(integer_of(find_key(parsed.metadata, "split.no")) == i &&
                        integer_of(find_key(parsed.metadata, "split.count")) == names.size(),
                    "gguf_split_metadata");
        }
        const std::uint64_t expected =
            single ? parsed.tensors.size()
                   : integer_of(find_key(parsed.metadata, "split.tensors.count"));
        if (i == 0)
            total = expected;
        require(expected == total && total <= 200000, "gguf_split_metadata");
        for (std::size_t t = 0; t < parsed.tensors.size(); ++t)
            impl_->tensors.push_back({std::move(parsed.tensors[t]), i,
                                      add(parsed.data_begin, parsed.offsets[t])});
        if (i == 0)
            impl_->metadata = std::move(parsed.metadata);
    }
    require(impl_->tensors.size() == total, "gguf_tensor_count");
    std::sort(impl_->tensors.begin(), impl_->tensors.end(),
              [](const auto& a, const auto& b) { return a.tensor.name < b.tensor.name; });
    for (std::size_t i = 1; i < impl_->tensors.size(); ++i)
        require(impl_->tensors[i - 1].tensor.name != impl_->tensors[i].tensor.name,
                "gguf_duplicate_tensor");
    check_unchanged();
}

GgufCheckpoint::~GgufCheckpoint() = default;

std::size_t GgufCheckpoint::tensor_count() const {
    return impl_->tensors.size();
}

const GgufTensor& GgufCheckpoint::tensor(std::string_view name) const {
    return impl_->find(name).tensor;
}

const GgufTensor& GgufCheckpoint::tensor_at(std::size_t index) const {
    if (index >= impl_->tensors.size())
        throw std::out_of_range("gguf_tensor_index");
    return impl_->tensors[index].tensor;
}

void GgufCheckpoint::check_unchanged() const {
    for (const auto& f : impl_->files)
        f.unchanged();
}

WeightIdentity GgufCheckpoint::identity(std::string_view name, std::size_t expert) const {
    const auto& e = impl_->find(name);
    require(expert < e.tensor.shape[2], "gguf_expert_range");
    const File& file = impl_->files[e.file];
    file.unchanged();
    const auto bytes = e.tensor.bytes / e.tensor.shape[2];
    const auto begin = add(e.begin, mul(expert, bytes));
    return file.identity(begin, add(begin, bytes));
}

void GgufCheckpoint::read_packed_rows(std::string_view name, std::size_t expert,
                                      std::size_t first_row, std::span<std::byte> output,
                                      const std::atomic_bool& cancel) const {
    stop(cancel);
    const auto& e = impl_->find(name);
    const auto& t = e.tensor;
    std::uint64_t values = 0, bytes = 0;
    (void)block_geometry(t.type, values, bytes);
    const std::uint64_t row_bytes = t.shape[0] / values * bytes;
    require(t.rank >= 2 && expert < t.shape[2] && output.size() % row_bytes == 0 &&
                first_row <= t.shape[1] && output.size() / row_bytes <= t.shape[1] - first_row,
            "gguf_row_range");
    const File& file = impl_->files[e.file];
    file.unchanged();
    const auto first = add(mul(expert, t.shape[1]), first_row);
    const auto offset = add(e.begin, mul(first, row_bytes));
    auto raw = std::span(reinterpret_cast<std::uint8_t*>(output.data()), output.size());
    for (std::size_t at = 0; at < raw.size();) {
        stop(cancel);
        const std::size_t n = std::min<std::size_t>(1024 * 1024, raw.size() - at);
        file.read(add(offset, at), raw.subspan(at, n), &cancel);
        at += n;
    }
    file.unchanged();
    stop(cancel);
}

void GgufCheckpoint::read_vector(std::string_view name, std::span<float> output,
                                 const std::atomic_bool& cancel) const {
    stop(cancel);
    const auto& e = impl_->find(name);
    const auto& t = e.tensor;
    require(t.type == KDQ_F32 && output.size() == t.shape[0] * t.shape[1] * t.shape[2] &&
                output.size_bytes() == t.bytes,
            "gguf_vector_shape");
    const File& file = impl_->files[e.file];
    file.unchanged();
    auto raw = std::span(reinterpret_cast<std::uint8_t*>(output.data()), output.size_bytes());
    for (std::size_t at = 0; at < raw.size();) {
        stop(cancel);
        const std::size_t n = std::min<std::size_t>(65536, raw.size() - at);
        file.read(add(e.begin, at), raw.subspan(at, n), &cancel);
        at += n;
    }
    for (float v : output)
        require(std::isfinite(v), "gguf_nonfinite_weight");
    file.unchanged();
    stop(cancel);
}

void GgufCheckpoint::read_rows(std::string_view name, std::size_t expert, std::size_t first_row,
                               std::span<float> output, const std::atomic_bool& cancel,
                               HipDenseCompute& compute) const {
    stop(cancel);
    const auto& t = impl_->find(name).tensor;
    std::uint64_t values = 0, bytes = 0;
    (void)block_geometry(t.type, values, bytes);
    const std::uint64_t row_bytes = t.shape[0] / values * bytes;
    require(t.rank >= 2 && expert < t.shape[2] && output.size() % t.shape[0] == 0 &&
                first_row <= t.shape[1] && output.size() / t.shape[0] <= t.shape[1] - first_row,
            "gguf_row_range");
    const std::size_t rows = output.size() / t.shape[0];
    const std::size_t batch = std::max<std::size_t>(1, std::min<std::size_t>(
                                                           rows, (16u << 20) / row_bytes));
    std::vector<std::byte> packed(batch * row_bytes);
    for (std::size_t r = 0; r < rows; r += batch) {
        const std::size_t n = std::min(batch, rows - r);
        auto chunk = std::span(packed).first(n * row_bytes);
        read_packed_rows(name, expert, first_row + r, chunk, cancel);
        auto out = output.subspan(r * t.shape[0], n * t.shape[0]);
        if (t.type == KDQ_F32) {
            std::memcpy(out.data(), chunk.data(), chunk.size());
            for (float v : out)
                require(std::isfinite(v), "gguf_nonfinite_weight");
        } else {
            const auto enc = gguf::encoding(t.type);
            require(enc.has_value(), "gguf_tensor_type");
            compute.dequantize_rows(*enc, chunk, t.shape[0], out);  // throws when nonfinite
        }
    }
}

HipDenseCompute::GgufWeightSource GgufCheckpoint::source(std::string_view name,
                                                         std::size_t expert,
                                                         const std::atomic_bool& cancel) const {
    (void)impl_->find(name);  // the tensor exists
    std::string key(name);
    return [this, key, expert, &cancel](std::size_t first, std::span<std::byte> rows) {
        read_packed_rows(key, expert, first, rows, cancel);
    };
}

bool GgufCheckpoint::has(std::string_view key) const {
    return impl_->metadata.find(key) != impl_->metadata.end();
}

std::string GgufCheckpoint::string(std::string_view key) const {
    const auto* s = std::get_if<std::string>(&find_key(impl_->metadata, key));
    require(s != nullptr, "gguf_metadata_string");
    return *s;
}

std::uint64_t GgufCheckpoint::integer(std::string_view key) const {
    return integer_of(find_key(impl_->metadata, key));
}

double GgufCheckpoint::number(std::string_view key) const {
    const auto* s = std::get_if<Scalar>(&find_key(impl_->metadata, key));
    require(s && s->type != kBool, "gguf_metadata_number");
    return number_of(*s);
}

bool GgufCheckpoint::boolean(std::string_view key) const {
    const auto* s = std::get_if<Scalar>(&find_key(impl_->metadata, key));
    require(s && s->type == kBool, "gguf_metadata_boolean");
    return s->bits != 0;
}

std::vector<bool> GgufCheckpoint::booleans(std::string_view key) const {
    const auto* a = std::get_if<Array>(&find_key(impl_->metadata, key));
    require(a && a->element == kBool, "gguf_metadata_boolean");
    std::vector<bool> out;
    for (const auto& s : a->values)
        out.push_back(s.bits != 0);
    return out;
}

std::vector<std::string> GgufCheckpoint::strings(std::string_view key) const {
    const auto* a = std::get_if<Array>(&find_key(impl_->metadata, key));
    require(a && a->element == kString, "gguf_metadata_string");
    return a->texts;
}

std::vector<std::int64_t> GgufCheckpoint::integers(std::string_view key) const {
    const auto* a = std::get_if<Array>(&find_key(impl_->metadata, key));
    require(a && is_integer(a->element), "gguf_metadata_integer");
    std::vector<std::int64_t> out;
    for (const auto& s : a->values) {
        require(s.type != kU64 || s.bits <= std::uint64_t(INT64_MAX), "gguf_metadata_integer");
        out.push_back(signed_of(s));
    }
    return out;
}

std::vector<double> GgufCheckpoint::numbers(std::string_view key) const {
    const auto* a = std::get_if<Array>(&find_key(impl_->metadata, key));
    require(a && a->element != kBool, "gguf_metadata_number");
    std::vector<double> out;
    for (const auto& s : a->values)
        out.push_back(number_of(s));
    return out;
}

// ------------------------------------------------------------- safetensors

namespace {

// A JSON reader for safetensors headers: objects, arrays, strings, integers (and the
// literals); depth and size bounded.  Numbers other than non-negative integers are kept
// as text.
struct Json {
    enum Kind { object, array, string, number, literal } kind = literal;
    std::string text;  // string value, number text or literal
    std::vector<std::pair<std::string, Json>> members;
    std::vector<Json> items;
};

class JsonParser {
public:
    explicit JsonParser(std::string_view s) : s_(s) {}

    Json document() {
        Json v = value(0);
        space();
        require(i_ == s_.size(), "safetensors_header_json");
        return v;
    }

private:
    std::string_view s_;
    std::size_t i_ = 0;

    void space() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' ||
                                  s_[i_] == '\r'))
            ++i_;
    }
    char peek() {
        space();
        require(i_ < s_.size(), "safetensors_header_json");
        return s_[i_];
    }
    void expect(char c) {
        require(peek() == c, "safetensors_header_json");
        ++i_;
    }
    std::string str() {
        expect('"');
        std::string out;
        for (;;) {
            require(i_ < s_.size(), "safetensors_header_json");
            const char c = s_[i_++];
            if (c == '"')
                return out;
            if (c != '\\') {
                out.push_back(c);
                continue;
            }
            require(i_ < s_.size(), "safetensors_header_json");
            const char e = s_[i_++];
            switch (e) {
            case '"': case '\\': case '/': out.push_back(e); break;
            case 'b': out.push_back('\b'); break;
            case 'f': out.push_back('\f'); break;
            case 'n': out.push_back('\n'); break;
            case 'r': out.push_back('\r'); break;
            case 't': out.push_back('\t'); break;
            case 'u': {
                require(i_ + 4 <= s_.size(), "safetensors_header_json");
                const unsigned cp = unsigned(std::stoul(std::string(s_.substr(i_, 4)), nullptr, 16));
                i_ += 4;
                if (cp < 0x80) {
                    out.push_back(char(cp));
                } else if (cp < 0x800) {
                    out.push_back(char(0xC0 | (cp >> 6)));
                    out.push_back(char(0x80 | (cp & 63)));
                } else {
                    out.push_back(char(0xE0 | (cp >> 12)));
                    out.push_back(char(0x80 | ((cp >> 6) & 63)));
                    out.push_back(char(0x80 | (cp & 63)));
                }
                break;
            }
            default: throw std::invalid_argument("safetensors_header_json");
            }
        }
    }
    Json value(int depth) {
        require(depth < 16, "safetensors_header_json");
        Json v;
        const char c = peek();
        if (c == '{') {
            v.kind = Json::object;
            ++i_;
            if (peek() == '}') {
                ++i_;
                return v;
            }
            for (;;) {
                std::string k = str();
                expect(':');
                v.members.emplace_back(std::move(k), value(depth + 1));
                if (peek() == ',') {
                    ++i_;
                    continue;
                }
                expect('}');
                return v;
            }
        }
        if (c == '[') {
            v.kind = Json::array;
            ++i_;
            if (peek() == ']') {
                ++i_;
                return v;
            }
            for (;;) {
                v.items.push_back(value(depth + 1));
                if (peek() == ',') {
                    ++i_;
                    continue;
                }
                expect(']');
                return v;
            }
        }
        if (c == '"') {
            v.kind = Json::string;
            v.text = str();
            return v;
        }
        const std::size_t start = i_;
        while (i_ < s_.size() && s_[i_] != ',' && s_[i_] != '}' && s_[i_] != ']' &&
               s_[i_] != ' ' && s_[i_] != '\n' && s_[i_] != '\r' && s_[i_] != '\t')
            ++i_;
        require(i_ > start, "safetensors_header_json");
        v.text = std::string(s_.substr(start, i_ - start));
        v.kind = (v.text == "true" || v.text == "false" || v.text == "null") ? Json::literal
                                                                               : Json::number;
        return v;
    }
};

std::uint64_t json_integer(const Json& j) {
    require(j.kind == Json::number && !j.text.empty() && j.text.size() <= 19 &&
                std::all_of(j.text.begin(), j.text.end(), [](char c) { return c >= '0' && c <= '9'; }),
            "safetensors_header_integer");
    return std::stoull(j.text);
}

Dtype dtype_of(const std::string& s, std::uint64_t& width) {
    if (s == "U8") return width = 1, Dtype::u8;
    if (s == "I8") return width = 1, Dtype::i8;
    if (s == "F16") return width = 2, Dtype::f16;
    if (s == "BF16") return width = 2, Dtype::bf16;
    if (s == "F32") return width = 4, Dtype::f32;
    static const std::map<std::string, std::uint64_t> others = {
        {"BOOL", 1}, {"F8_E4M3", 1}, {"F8_E5M2", 1}, {"I16", 2}, {"U16", 2}, {"I32", 4},
        {"U32", 4}, {"I64", 8}, {"U64", 8}, {"F64", 8}};
    const auto it = others.find(s);
    require(it != others.end(), "safetensors_dtype");
    width = it->second;
    return Dtype::other;
}

}  // namespace

struct SafetensorsShard::Impl {
    std::unique_ptr<File> file;
    std::vector<SafetensorsTensor> tensors;  // sorted by name
    std::map<std::string, std::string, std::less<>> metadata;

    const SafetensorsTensor& find(std::string_view name) const {
        const auto it = std::lower_bound(tensors.begin(), tensors.end(), name,
                                         [](const SafetensorsTensor& t, std::string_view n) {
                                             return t.name < n;
                                         });
        require(it != tensors.end() && it->name == name, "missing_tensor");
        return *it;
    }
    void read(const SafetensorsTensor& t, std::uint64_t offset, std::span<std::uint8_t> out) const {
        require(offset <= t.end - t.begin && out.size() <= t.end - t.begin - offset,
                "checkpoint_read_bounds");
        file->read(t.begin + offset, out, nullptr, "checkpoint_read_bounds");
    }
};

SafetensorsShard::SafetensorsShard(const std::string& path) : impl_(std::make_unique<Impl>()) {
    impl_->file = std::make_unique<File>(::open(path.c_str(), O_RDONLY | O_NOFOLLOW | O_CLOEXEC),
                                         "checkpoint_changed", 8);
    const File& f = *impl_->file;
    std::array<std::uint8_t, 8> head{};
    f.read(0, head, nullptr, "safetensors_header");
    std::uint64_t n = 0;
    for (int i = 0; i < 8; ++i)
        n |= std::uint64_t(head[i]) << (8 * i);
    require(n <= 100 * 1024 * 1024 && n <= f.size() - 8, "safetensors_header_size");
    std::string text(std::size_t(n), '\0');
    f.read(8, {reinterpret_cast<std::uint8_t*>(text.data()), text.size()}, nullptr,
           "safetensors_header");
    const Json doc = JsonParser(text).document();
    require(doc.kind == Json::object, "safetensors_header_json");
    const std::uint64_t data = 8 + n;
    std::vector<std::pair<std::uint64_t, std::uint64_t>> ranges;
    for (const auto& [name, v] : doc.members) {
        if (name == "__metadata__") {
            require(v.kind == Json::object, "safetensors_metadata");
            for (const auto& [k, s] : v.members) {
                require(s.kind == Json::string, "safetensors_metadata");
                impl_->metadata[k] = s.text;
            }
            continue;
        }
        require(v.kind == Json::object && !name.empty() && name.size() <= 1024,
                "safetensors_tensor");
        SafetensorsTensor t;
        t.name = name;
        const Json *dtype = nullptr, *shape = nullptr, *offsets = nullptr;
        for (const auto& [k, m] : v.members) {
            if (k == "dtype")
                dtype = &m;
            else if (k == "shape")
                shape = &m;
            else if (k == "data_offsets")
                offsets = &m;
        }
        require(dtype && shape && offsets && dtype->kind == Json::string &&
                    shape->kind == Json::array && offsets->kind == Json::array &&
                    offsets->items.size() == 2 && shape->items.size() <= 8,
                "safetensors_tensor");
        std::uint64_t width = 0;
        t.dtype = dtype_of(dtype->text, width);
        std::uint64_t count = 1;
        for (const auto& d : shape->items) {
            t.shape.push_back(json_integer(d));
            count = mul(count, t.shape.back(), "safetensors_tensor_shape");
        }
        const auto a = json_integer(offsets->items[0]), b = json_integer(offsets->items[1]);
        require(a <= b && b - a == mul(count, width, "safetensors_tensor_shape") &&
                    b <= f.size() - data,
                "safetensors_tensor_bounds");
        t.begin = data + a;
        t.end = data + b;
        ranges.emplace_back(a, b);
        impl_->tensors.push_back(std::move(t));
    }
    std::sort(ranges.begin(), ranges.end());
    for (std::size_t i = 1; i < ranges.size(); ++i)
        require(ranges[i].first >= ranges[i - 1].second, "safetensors_tensor_overlap");
    std::sort(impl_->tensors.begin(), impl_->tensors.end(),
              [](const auto& x, const auto& y) { return x.name < y.name; });
    for (std::size_t i = 1; i < impl_->tensors.size(); ++i)
        require(impl_->tensors[i - 1].name != impl_->tensors[i].name, "safetensors_duplicate");
    f.unchanged();
}

SafetensorsShard::~SafetensorsShard() = default;

std::size_t SafetensorsShard::tensor_count() const {
    return impl_->tensors.size();
}

const SafetensorsTensor& SafetensorsShard::tensor(std::string_view name) const {
    return impl_->find(name);
}

WeightIdentity SafetensorsShard::identity(std::string_view name) const {
    const auto& t = impl_->find(name);
    impl_->file->unchanged();
    return impl_->file->identity(t.begin, t.end);
}

void SafetensorsShard::check_unchanged() const {
    impl_->file->unchanged();
}

std::string SafetensorsShard::metadata(std::string_view key) const {
    const auto it = impl_->metadata.find(key);
    require(it != impl_->metadata.end(), "safetensors_missing_metadata");
    return it->second;
}

Mxfp4Rows SafetensorsShard::load_mxfp4_expert_rows(std::string_view prefix, std::size_t expert,
                                                   std::size_t first, std::size_t count,
                                                   std::size_t payload_budget) const {
    require(!prefix.empty() && prefix.size() <= 480 && count != 0, "projection_range_or_name");
    const auto& blocks = impl_->find(std::string(prefix) + "_blocks");
    const auto& scales = impl_->find(std::string(prefix) + "_scales");
    require(blocks.dtype == Dtype::u8 && scales.dtype == Dtype::u8, "mxfp4_dtype");
    require(blocks.shape.size() == 4 && scales.shape.size() == 3 && blocks.shape[3] == 16 &&
                blocks.shape[2] > 0 && expert < blocks.shape[0] && first <= blocks.shape[1] &&
                count <= blocks.shape[1] - first &&
                std::equal(scales.shape.begin(), scales.shape.end(), blocks.shape.begin()),
            "mxfp4_expert_shape");
    const std::uint64_t groups = blocks.shape[2];
    const std::uint64_t scale_bytes = mul(count, groups);
    const std::uint64_t weight_bytes = mul(scale_bytes, 16);
    const std::uint64_t total = add(weight_bytes, scale_bytes);
    require(total <= payload_budget, "payload_budget");
    const std::uint64_t scale_offset = mul(add(mul(expert, blocks.shape[1]), first), groups);
    Mxfp4Rows out;
    out.rows = count;
    out.columns = std::size_t(mul(groups, 32));
    out.blocks.resize(std::size_t(weight_bytes));
    out.scales.resize(std::size_t(scale_bytes));
    impl_->file->unchanged();
    impl_->read(blocks, mul(scale_offset, 16), out.blocks);
    impl_->read(scales, scale_offset, out.scales);
    impl_->file->unchanged();
    for (auto s : out.scales)  // IW/src/weights/quantization.cpp:46-56
        require(s != 255, "invalid_block_scale");
    return out;
}

Mxfp4Rows SafetensorsShard::load_mxfp4_experts(std::string_view prefix, std::size_t& experts,
                                               std::size_t payload_budget) const {
    const auto& blocks = impl_->find(std::string(prefix) + "_blocks");
    require(blocks.shape.size() == 4 && blocks.shape[0] > 0, "mxfp4_expert_shape");
    experts = std::size_t(blocks.shape[0]);
    const std::size_t rows = std::size_t(blocks.shape[1]);
    // the experts' rows lie one after another in both tensors: one load of all of them
    const std::uint64_t per = add(mul(mul(rows, blocks.shape[2]), 16), mul(rows, blocks.shape[2]));
    require(mul(per, experts) <= payload_budget, "payload_budget");
    Mxfp4Rows all;
    for (std::size_t e = 0; e < experts; ++e) {
        Mxfp4Rows one = load_mxfp4_expert_rows(prefix, e, 0, rows, payload_budget);
        if (e == 0) {
            all.rows = rows;
            all.columns = one.columns;
            all.blocks.reserve(one.blocks.size() * experts);
            all.scales.reserve(one.scales.size() * experts);
        }
        all.blocks.insert(all.blocks.end(), one.blocks.begin(), one.blocks.end());
        all.scales.insert(all.scales.end(), one.scales.begin(), one.scales.end());
    }
    return all;
}

}  // namespace kadan_amd::checkpoint
