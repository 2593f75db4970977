// kadan_amd checkpoint readers (include/kadan_amd_checkpoint.hpp), host only.
//
// GGUF v3, as ggml's published format description (docs/gguf.md) lays it out, all
// little-endian: "GGUF", u32 version, u64 tensor count, u64 metadata count; the metadata
// pairs (string key, u32 value type, value); per tensor its name, u32 dimension count,
// the dimensions (u64, fastest first), u32 GGML type and u64 offset into the data
// section, which begins at the first multiple of general.alignment (default 32) past
// the header.  Strings are a u64 byte count and the bytes; arrays a u32 element type, a
// u64 count and the elements.
//
// safetensors, as its specification lays it out: u64 little-endian header length N, N
// bytes of JSON mapping each tensor name to {"dtype", "shape", "data_offsets": [begin,
// end]} (offsets into the payload that follows the header) plus an optional
// "__metadata__" object of strings, then the payload.
//
// Bounds are derived rather than listed: a count or length is accepted only if the
// bytes it implies fit in what is left of the header, and the header itself is capped
// (GGUF: kGgufHeaderLimit; safetensors: the specification's 100,000,000 bytes), so no
// allocation is sized by an unchecked field.
#include "kadan_amd_checkpoint.hpp"

#include <algorithm>
#include <bit>
#include <cerrno>
#include <cmath>
#include <cstring>
#include <dirent.h>
#include <fcntl.h>
#include <optional>
#include <sys/stat.h>
#include <unistd.h>

#include "kadan_amd.h"

static_assert(std::endian::native == std::endian::little,
              "the readers take file integers as they lie (both formats are little-endian)");

namespace kadan_amd::checkpoint {
namespace {

[[noreturn]] void fail(const char* code) {
    throw CheckpointError(code);
}

void expect(bool ok, const char* code) {
    if (!ok)
        fail(code);
}

std::uint64_t add_or(std::uint64_t a, std::uint64_t b, const char* code) {
    std::uint64_t r = 0;
    expect(!__builtin_add_overflow(a, b, &r), code);
    return r;
}

std::uint64_t mul_or(std::uint64_t a, std::uint64_t b, const char* code) {
    std::uint64_t r = 0;
    expect(!__builtin_mul_overflow(a, b, &r), code);
    return r;
}

// ------------------------------------------------------------------ files

// A read-only descriptor and the status the file had when it was opened.  Opened
// non-blocking so that a FIFO or device node at the path cannot stall the constructor
// (it is then refused as not a regular file).
class Descriptor {
public:
    Descriptor(const std::string& path, const char* cannot_open, const char* not_regular) {
        fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC | O_NONBLOCK);
        expect(fd_ >= 0, cannot_open);
        if (::fstat(fd_, &seen_) != 0 || !S_ISREG(seen_.st_mode)) {
            ::close(fd_);
            fd_ = -1;
            fail(not_regular);
        }
    }
    Descriptor(Descriptor&& other) noexcept : fd_(other.fd_), seen_(other.seen_) {
        other.fd_ = -1;
    }
    Descriptor(const Descriptor&) = delete;
    Descriptor& operator=(const Descriptor&) = delete;
    Descriptor& operator=(Descriptor&&) = delete;
    ~Descriptor() {
        if (fd_ >= 0)
            ::close(fd_);
    }

    std::uint64_t size() const { return std::uint64_t(seen_.st_size); }

    // Exactly out.size() bytes from byte `at`.
    void read(std::uint64_t at, std::span<std::byte> out, const char* beyond,
              const char* failed) const {
        expect(at <= size() && out.size() <= size() - at, beyond);
        std::size_t done = 0;
        while (done < out.size()) {
            const ssize_t got = ::pread(fd_, out.data() + done, out.size() - done,
                                        off_t(at + done));
            if (got < 0 && errno == EINTR)
                continue;
            expect(got > 0, failed);  // an error, or the file ended early
            done += std::size_t(got);
        }
    }

    // Whether device, inode, size, modification or status-change time differ now.
    bool moved() const {
        struct stat now {};
        if (::fstat(fd_, &now) != 0)
            return true;
        auto same_time = [](const timespec& a, const timespec& b) {
            return a.tv_sec == b.tv_sec && a.tv_nsec == b.tv_nsec;
        };
        return now.st_dev != seen_.st_dev || now.st_ino != seen_.st_ino ||
               now.st_size != seen_.st_size || !same_time(now.st_mtim, seen_.st_mtim) ||
               !same_time(now.st_ctim, seen_.st_ctim);
    }

    WeightIdentity identity(std::uint64_t begin, std::uint64_t end) const {
        WeightIdentity w;
        w.device = std::uint64_t(seen_.st_dev);
        w.inode = std::uint64_t(seen_.st_ino);
        w.file_size = size();
        w.modified_seconds = std::uint64_t(seen_.st_mtim.tv_sec);
        w.modified_nanoseconds = std::uint64_t(seen_.st_mtim.tv_nsec);
        w.changed_seconds = std::uint64_t(seen_.st_ctim.tv_sec);
        w.changed_nanoseconds = std::uint64_t(seen_.st_ctim.tv_nsec);
        w.payload_begin = begin;
        w.payload_end = end;
        return w;
    }

private:
    int fd_ = -1;
    struct stat seen_ {};
};

// Exact IEEE binary16 -> binary32 (normal, subnormal, infinity and NaN payloads).
float half_to_float(std::uint16_t h) {
    const std::uint32_t sign = std::uint32_t(h >> 15) << 31;
    std::uint32_t exponent = (h >> 10) & 31u, fraction = h & 1023u;
    std::uint32_t bits;
    if (exponent == 31) {
        bits = sign | 0x7f800000u | (fraction << 13);
    } else if (exponent) {
        bits = sign | ((exponent + 112) << 23) | (fraction << 13);
    } else if (!fraction) {
        bits = sign;
    } else {  // subnormal: shift the fraction up to a leading one
        int shift = 0;
        while (!(fraction & 1024u)) {
            fraction <<= 1;
            ++shift;
        }
        bits = sign | (std::uint32_t(113 - shift) << 23) | ((fraction & 1023u) << 13);
    }
    return std::bit_cast<float>(bits);
}

// ------------------------------------------------------------------ GGUF header

constexpr std::uint32_t kGgufMagic = 0x46554747;  // "GGUF" read as a little-endian u32
constexpr std::uint64_t kGgufHeaderLimit = std::uint64_t(256) << 20;
constexpr std::uint64_t kDefaultAlignment = 32;

// GGUF metadata value types.
enum GgufType : std::uint32_t {
    kU8, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kString, kArray, kU64, kI64, kF64
};

// Fewest header bytes one element of `type` can take (a string: its length field).
std::uint64_t least_bytes(std::uint32_t type) {
    switch (type) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    default: return 8;
    }
}

// Sequential decoding over the front of a file.  The bytes held grow on demand (at least
// doubling, at least 1 MiB at a time) up to kGgufHeaderLimit, so a header is read in a few
// large preads whatever its metadata holds.
class HeaderCursor {
public:
    explicit HeaderCursor(const Descriptor& file) : file_(file) {}

    std::uint64_t at() const { return at_; }
    // Bytes a field could still take: to the end of the file or of the header limit.
    std::uint64_t room() const { return std::min(file_.size(), kGgufHeaderLimit) - at_; }

    template <class T> T get() {
        T v;
        std::memcpy(&v, take(sizeof v), sizeof v);
        return v;
    }

    std::string text() {
        const auto n = get<std::uint64_t>();
        const auto* p = take(n);
        return std::string(reinterpret_cast<const char*>(p), std::size_t(n));
    }

private:
    const std::byte* take(std::uint64_t n) {
        const auto end = add_or(at_, n, "gguf_read_bounds");
        if (end > held_.size()) {
            expect(end <= file_.size(), "gguf_read_bounds");
            expect(end <= kGgufHeaderLimit, "gguf_metadata_limit");
            std::uint64_t want = std::max<std::uint64_t>({end, 2 * held_.size(), 1u << 20});
            want = std::min({want, file_.size(), kGgufHeaderLimit});
            const std::size_t old = held_.size();
            held_.resize(std::size_t(want));
            file_.read(old, std::span<std::byte>(held_.data() + old, held_.size() - old),
                       "gguf_read_bounds", "gguf_read_failed");
        }
        const std::byte* p = held_.data() + at_;
        at_ = end;
        return p;
    }

    const Descriptor& file_;
    std::vector<std::byte> held_;
    std::uint64_t at_ = 0;
};

GgufValue::Scalar scalar_of(HeaderCursor& c, std::uint32_t type) {
    switch (type) {
    case kU8: return std::uint64_t(c.get<std::uint8_t>());
    case kI8: return std::int64_t(c.get<std::int8_t>());
    case kU16: return std::uint64_t(c.get<std::uint16_t>());
    case kI16: return std::int64_t(c.get<std::int16_t>());
    case kU32: return std::uint64_t(c.get<std::uint32_t>());
    case kI32: return std::int64_t(c.get<std::int32_t>());
    case kU64: return c.get<std::uint64_t>();
    case kI64: return c.get<std::int64_t>();
    case kF32: return double(c.get<float>());
    case kF64: return c.get<double>();
    case kBool: {
        const auto b = c.get<std::uint8_t>();
        expect(b <= 1, "gguf_invalid_metadata");
        return b == 1;
    }
    case kString: return c.text();
    default: fail("gguf_metadata_type");
    }
}

GgufValue value_of(HeaderCursor& c) {
    const auto type = c.get<std::uint32_t>();
    if (type != kArray)
        return GgufValue(type, false, {scalar_of(c, type)});
    const auto element = c.get<std::uint32_t>();
    expect(element <= kF64 && element != kArray, "gguf_metadata_type");
    const auto n = c.get<std::uint64_t>();
    // nothing is reserved for more elements than the rest of the header could hold
    expect(n <= c.room() / least_bytes(element), "gguf_array_limit");
    std::vector<GgufValue::Scalar> items;
    items.reserve(std::size_t(n));
    for (std::uint64_t i = 0; i < n; ++i)
        items.push_back(scalar_of(c, element));
    return GgufValue(element, true, std::move(items));
}

// A key or tensor name must be non-empty and hold no NUL (names are matched as text).
void check_name(const std::string& s, const char* empty) {
    expect(!s.empty(), empty);
    expect(s.find('\0') == std::string::npos, "gguf_string_nul");
}

using Metadata = std::map<std::string, GgufValue, std::less<>>;

// One decoded GGUF file: its metadata and tensors (offsets already absolute).
struct GgufHeader {
    Metadata metadata;
    std::vector<GgufTensorInfo> tensors;
};

GgufHeader decode_header(const Descriptor& file, std::size_t file_index) {
    HeaderCursor c(file);
    expect(c.get<std::uint32_t>() == kGgufMagic, "gguf_magic");
    expect(c.get<std::uint32_t>() == 3, "gguf_version");
    const auto tensor_count = c.get<std::uint64_t>();
    const auto pair_count = c.get<std::uint64_t>();
    // a pair takes at least 14 bytes (key length, one key byte, type, one value byte), a
    // tensor record at least 33 (name length, one name byte, rank, one dimension, type,
    // offset)
    expect(pair_count <= c.room() / 14 && tensor_count <= c.room() / 33, "gguf_header_count");

    GgufHeader h;
    for (std::uint64_t i = 0; i < pair_count; ++i) {
        std::string key = c.text();
        check_name(key, "gguf_metadata_key");
        GgufValue v = value_of(c);
        expect(h.metadata.emplace(std::move(key), std::move(v)).second, "gguf_duplicate_key");
    }
    std::uint64_t alignment = kDefaultAlignment;
    if (auto it = h.metadata.find("general.alignment"); it != h.metadata.end()) {
        const GgufValue& a = it->second;
        expect(!a.is_array() && a.gguf_type() == kU32, "gguf_alignment");
        alignment = a.count();
        expect(alignment && std::has_single_bit(alignment), "gguf_alignment");
    }

    std::vector<std::uint64_t> relative;
    relative.reserve(std::size_t(tensor_count));
    for (std::uint64_t i = 0; i < tensor_count; ++i) {
        GgufTensorInfo t;
        t.name = c.text();
        check_name(t.name, "gguf_tensor_name");
        const auto rank = c.get<std::uint32_t>();
        expect(rank >= 1 && rank <= 3, "gguf_tensor_rank");
        t.rank = rank;
        std::uint64_t dims[3] = {1, 1, 1};
        for (std::uint32_t d = 0; d < rank; ++d) {
            dims[d] = c.get<std::uint64_t>();
            expect(dims[d] >= 1, "gguf_tensor_shape");
        }
        t.columns = dims[0];
        t.rows = dims[1];
        t.experts = dims[2];
        t.ggml_type = c.get<std::uint32_t>();
        const std::size_t values = kdq_block_values(int(t.ggml_type));
        expect(values != 0, "gguf_tensor_type");
        expect(t.columns % values == 0, "gguf_tensor_block_alignment");
        t.row_bytes = mul_or(t.columns / values, kdq_block_bytes(int(t.ggml_type)),
                             "gguf_size_overflow");
        t.slice_bytes = mul_or(t.rows, t.row_bytes, "gguf_size_overflow");
        t.bytes = mul_or(t.experts, t.slice_bytes, "gguf_size_overflow");
        const auto offset = c.get<std::uint64_t>();
        expect(offset % alignment == 0, "gguf_alignment");
        t.file = file_index;
        relative.push_back(offset);
        h.tensors.push_back(std::move(t));
    }

    // payloads: the data section starts at the header's end rounded up to the alignment
    const std::uint64_t data = add_or(c.at(), alignment - 1, "gguf_tensor_bounds") /
                               alignment * alignment;
    for (std::size_t i = 0; i < h.tensors.size(); ++i) {
        auto& t = h.tensors[i];
        t.offset = add_or(data, relative[i], "gguf_tensor_bounds");
        const auto end = add_or(t.offset, t.bytes, "gguf_tensor_bounds");
        expect(end <= file.size(), "gguf_tensor_bounds");
    }
    // no two payloads share a byte
    std::vector<std::size_t> order(h.tensors.size());
    for (std::size_t i = 0; i < order.size(); ++i)
        order[i] = i;
    std::sort(order.begin(), order.end(), [&](std::size_t a, std::size_t b) {
        return h.tensors[a].offset < h.tensors[b].offset;
    });
    for (std::size_t k = 1; k < order.size(); ++k) {
        const auto& before = h.tensors[order[k - 1]];
        expect(h.tensors[order[k]].offset >= before.offset + before.bytes, "gguf_tensor_overlap");
    }
    return h;
}

// ------------------------------------------------------------------ split sets

// <stem>-NNNNN-of-NNNNN.gguf: the numbered split naming of llama.cpp's gguf-split.
struct SplitPart {
    std::string stem;
    unsigned index = 0, count = 0;
};

std::optional<unsigned> five_digits(std::string_view s) {
    if (s.size() != 5)
        return std::nullopt;
    unsigned v = 0;
    for (char ch : s) {
        if (ch < '0' || ch > '9')
            return std::nullopt;
        v = 10 * v + unsigned(ch - '0');
    }
    return v;
}

std::optional<SplitPart> split_part(std::string_view name) {
    // suffix "-IIIII-of-CCCCC.gguf": 20 bytes after the stem
    constexpr std::size_t suffix = 20;
    if (name.size() <= suffix || !name.ends_with(".gguf"))
        return std::nullopt;
    const std::string_view tail = name.substr(name.size() - suffix);
    if (tail[0] != '-' || tail.substr(6, 4) != "-of-")
        return std::nullopt;
    const auto index = five_digits(tail.substr(1, 5));
    const auto count = five_digits(tail.substr(10, 5));
    if (!index || !count)
        return std::nullopt;
    return SplitPart{std::string(name.substr(0, name.size() - suffix)), *index, *count};
}

// The .gguf files of `directory` in the order the set is read: one file, or a whole
// split set by part number.
std::vector<std::string> set_members(const std::string& directory, bool& split) {
    std::vector<std::string> names;
    if (DIR* d = ::opendir(directory.c_str())) {
        while (const dirent* e = ::readdir(d)) {
            const std::string_view n = e->d_name;
            if (n.size() > 5 && n.ends_with(".gguf"))
                names.emplace_back(n);
        }
        ::closedir(d);
    }
    expect(!names.empty(), "gguf_missing_files");
    std::sort(names.begin(), names.end());
    split = false;
    if (names.size() == 1 && !split_part(names[0]))
        return {directory + "/" + names[0]};
    split = true;
    std::vector<SplitPart> parts;
    for (const auto& n : names) {
        auto p = split_part(n);
        expect(p && p->count >= 1 && p->index >= 1 && p->index <= p->count, "gguf_split_name");
        expect(parts.empty() || (p->stem == parts[0].stem && p->count == parts[0].count),
               "gguf_split_name");
        parts.push_back(*p);
    }
    expect(parts.size() == parts[0].count, "gguf_split_count");
    std::vector<std::string> ordered(parts.size());
    for (std::size_t i = 0; i < parts.size(); ++i) {
        auto& slot = ordered[parts[i].index - 1];
        expect(slot.empty(), "gguf_split_name");  // a part number twice
        slot = directory + "/" + names[i];
    }
    return ordered;
}

// An integer-valued metadata entry, or nothing when absent or of another kind.
std::optional<std::uint64_t> whole_number(const Metadata& m, std::string_view key) {
    const auto it = m.find(key);
    if (it == m.end() || it->second.is_array())
        return std::nullopt;
    try {
        return it->second.count();
    } catch (const CheckpointError&) {
        return std::nullopt;
    }
}

}  // namespace

// ------------------------------------------------------------------ GgufValue

namespace {
template <class T> bool holds(const GgufValue::Scalar& s) {
    return std::holds_alternative<T>(s);
}
}  // namespace

std::string GgufValue::text() const {
    expect(!array_ && items_.size() == 1 && holds<std::string>(items_[0]),
           "gguf_metadata_string");
    return std::get<std::string>(items_[0]);
}

std::uint64_t GgufValue::count() const {
    expect(!array_ && items_.size() == 1, "gguf_metadata_integer");
    if (holds<std::uint64_t>(items_[0]))
        return std::get<std::uint64_t>(items_[0]);
    expect(holds<std::int64_t>(items_[0]) && std::get<std::int64_t>(items_[0]) >= 0,
           "gguf_metadata_integer");
    return std::uint64_t(std::get<std::int64_t>(items_[0]));
}

double GgufValue::real() const {
    expect(!array_ && items_.size() == 1 && holds<double>(items_[0]), "gguf_metadata_number");
    return std::get<double>(items_[0]);
}

bool GgufValue::flag() const {
    expect(!array_ && items_.size() == 1 && holds<bool>(items_[0]), "gguf_metadata_boolean");
    return std::get<bool>(items_[0]);
}

std::vector<std::string> GgufValue::texts() const {
    expect(array_ && type_ == kString, "gguf_metadata_strings");
    std::vector<std::string> out;
    out.reserve(items_.size());
    for (const auto& s : items_)
        out.push_back(std::get<std::string>(s));
    return out;
}

std::vector<std::int64_t> GgufValue::integers() const {
    const bool integral = type_ == kU8 || type_ == kI8 || type_ == kU16 || type_ == kI16 ||
                          type_ == kU32 || type_ == kI32 || type_ == kU64 || type_ == kI64;
    expect(array_ && integral, "gguf_metadata_integers");
    std::vector<std::int64_t> out;
    out.reserve(items_.size());
    for (const auto& s : items_) {
        if (holds<std::int64_t>(s)) {
            out.push_back(std::get<std::int64_t>(s));
        } else {
            const auto u = std::get<std::uint64_t>(s);
            expect(u <= std::uint64_t(INT64_MAX), "gguf_metadata_integers");
            out.push_back(std::int64_t(u));
        }
    }
    return out;
}

std::vector<double> GgufValue::reals() const {
    expect(array_ && (type_ == kF32 || type_ == kF64), "gguf_metadata_numbers");
    std::vector<double> out;
    out.reserve(items_.size());
    for (const auto& s : items_)
        out.push_back(std::get<double>(s));
    return out;
}

std::vector<bool> GgufValue::flags() const {
    expect(array_ && type_ == kBool, "gguf_metadata_booleans");
    std::vector<bool> out;
    out.reserve(items_.size());
    for (const auto& s : items_)
        out.push_back(std::get<bool>(s));
    return out;
}

// ------------------------------------------------------------------ GgufFiles

struct GgufFiles::State {
    std::vector<Descriptor> files;
    std::vector<GgufTensorInfo> tensors;
    std::map<std::string, std::size_t, std::less<>> by_name;
    Metadata metadata;  // the first file's
};

GgufFiles::GgufFiles(const std::string& directory, const std::atomic_bool& cancel)
    : state_(std::make_unique<State>()) {
    auto& s = *state_;
    bool split = false;
    const auto members = set_members(directory, split);
    std::vector<Metadata> per_file;
    for (std::size_t i = 0; i < members.size(); ++i) {
        expect(!cancel.load(), "gguf_cancelled");
        s.files.emplace_back(members[i], "gguf_open_failed", "gguf_not_regular_file");
        GgufHeader h = decode_header(s.files.back(), i);
        for (auto& t : h.tensors) {
            expect(s.by_name.emplace(t.name, s.tensors.size()).second, "gguf_duplicate_tensor");
            s.tensors.push_back(std::move(t));
        }
        per_file.push_back(std::move(h.metadata));
    }
    if (split) {
        // every part names its place in the set, and any tensor total it states is the set's
        for (std::size_t i = 0; i < per_file.size(); ++i) {
            expect(whole_number(per_file[i], "split.no") == std::uint64_t(i) &&
                       whole_number(per_file[i], "split.count") == per_file.size(),
                   "gguf_split_metadata");
            const auto total = whole_number(per_file[i], "split.tensors.count");
            expect(!per_file[i].contains("split.tensors.count") || total == s.tensors.size(),
                   "gguf_split_metadata");
        }
    }
    s.metadata = std::move(per_file.front());
}

GgufFiles::~GgufFiles() = default;

std::size_t GgufFiles::size() const {
    return state_->tensors.size();
}

const GgufTensorInfo& GgufFiles::info(std::size_t index) const {
    expect(index < state_->tensors.size(), "gguf_tensor_index");
    return state_->tensors[index];
}

const GgufTensorInfo& GgufFiles::info(std::string_view name) const {
    const auto it = state_->by_name.find(name);
    expect(it != state_->by_name.end(), "gguf_missing_tensor");
    return state_->tensors[it->second];
}

WeightIdentity GgufFiles::slice_identity(std::string_view name, std::size_t expert) const {
    const auto& t = info(name);
    expect(expert < t.experts, "gguf_expert_range");
    const auto begin = t.offset + expert * t.slice_bytes;
    return state_->files[t.file].identity(begin, begin + t.slice_bytes);
}

void GgufFiles::verify_unchanged() const {
    for (const auto& f : state_->files)
        expect(!f.moved(), "gguf_checkpoint_changed");
}

void GgufFiles::copy_rows(std::string_view name, std::size_t expert, std::size_t first_row,
                          std::span<std::byte> out, const std::atomic_bool& cancel) const {
    const auto& t = info(name);
    const bool whole = t.rank >= 2 && out.size() % t.row_bytes == 0;
    const std::uint64_t rows = whole ? out.size() / t.row_bytes : 0;
    expect(whole && expert < t.experts && first_row <= t.rows && rows <= t.rows - first_row,
           "gguf_row_range");
    verify_unchanged();
    expect(!cancel.load(), "gguf_cancelled");
    if (out.empty())
        return;
    state_->files[t.file].read(t.offset + expert * t.slice_bytes + first_row * t.row_bytes, out,
                               "gguf_read_bounds", "gguf_read_failed");
}

void GgufFiles::copy_vector(std::string_view name, std::span<float> out,
                            const std::atomic_bool& cancel) const {
    const auto& t = info(name);
    expect(t.rank == 1 && t.ggml_type == KDQ_F32 && out.size() == t.columns, "gguf_vector_shape");
    verify_unchanged();
    expect(!cancel.load(), "gguf_cancelled");
    state_->files[t.file].read(t.offset, std::as_writable_bytes(out), "gguf_read_bounds",
                               "gguf_read_failed");
    for (float v : out)
        expect(std::isfinite(v), "gguf_nonfinite_weight");
}

void GgufFiles::decode_rows(std::string_view name, std::size_t expert, std::size_t first_row,
                            std::span<float> out, const std::atomic_bool& cancel,
                            HipDenseCompute& compute) const {
    const auto& t = info(name);
    expect(out.size() % t.columns == 0, "gguf_row_range");
    const std::size_t rows = out.size() / t.columns;
    std::vector<std::byte> packed(rows * t.row_bytes);
    copy_rows(name, expert, first_row, packed, cancel);
    if (t.ggml_type == KDQ_F32 || t.ggml_type == KDQ_F16) {
        for (std::size_t i = 0; i < out.size(); ++i) {
            if (t.ggml_type == KDQ_F32) {
                std::memcpy(&out[i], packed.data() + 4 * i, 4);
            } else {
                std::uint16_t h;
                std::memcpy(&h, packed.data() + 2 * i, 2);
                out[i] = half_to_float(h);
            }
            expect(std::isfinite(out[i]), "gguf_nonfinite_weight");
        }
        return;
    }
    const auto enc = gguf::encoding(t.ggml_type);
    expect(enc.has_value(), "gguf_tensor_type");
    try {
        compute.dequantize_rows(*enc, packed, t.columns, out);
    } catch (const std::runtime_error& e) {
        if (std::string_view(e.what()) == "kdq_nonfinite_weight")
            fail("gguf_nonfinite_weight");
        throw;
    }
}

HipDenseCompute::GgufWeightSource GgufFiles::row_source(std::string_view name,
                                                        std::size_t expert,
                                                        const std::atomic_bool& cancel) const {
    info(name);  // an unknown name is refused now, not at the first read
    return [this, tensor = std::string(name), expert, &cancel](std::size_t first,
                                                               std::span<std::byte> out) {
        copy_rows(tensor, expert, first, out, cancel);
    };
}

bool GgufFiles::has(std::string_view key) const {
    return state_->metadata.contains(key);
}

const GgufValue& GgufFiles::value(std::string_view key) const {
    const auto it = state_->metadata.find(key);
    expect(it != state_->metadata.end(), "gguf_missing_metadata");
    return it->second;
}

// ------------------------------------------------------------------ safetensors

namespace {

constexpr std::uint64_t kSafetensorsHeaderLimit = 100000000;  // the specification's cap

// A parsed JSON value.  Numbers keep their literal text; only the unsigned integers the
// header's fields need are ever converted.
struct Json {
    enum class Kind { null, boolean, number, string, array, object } kind = Kind::null;
    bool flag = false;
    std::string text;
    std::vector<Json> items;
    std::vector<std::pair<std::string, Json>> members;  // in file order
};

// Recursive descent over the header text.  Strings must be ASCII (raw bytes and \u
// escapes alike), escapes exactly as JSON defines them.
class JsonReader {
public:
    explicit JsonReader(std::string_view s) : s_(s) {}

    Json document() {
        Json v = value(0);
        space();
        expect(i_ == s_.size(), "safetensors_header_json");
        return v;
    }

private:
    void space() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' ||
                                  s_[i_] == '\r'))
            ++i_;
    }
    char next() {
        expect(i_ < s_.size(), "safetensors_header_json");
        return s_[i_++];
    }
    void literal(std::string_view word) {
        expect(s_.substr(i_, word.size()) == word, "safetensors_header_json");
        i_ += word.size();
    }

    Json value(int depth) {
        expect(depth < 32, "safetensors_header_json");
        space();
        expect(i_ < s_.size(), "safetensors_header_json");
        Json v;
        const char c = s_[i_];
        if (c == '{') {
            v.kind = Json::Kind::object;
            ++i_;
            space();
            if (i_ < s_.size() && s_[i_] == '}') {
                ++i_;
                return v;
            }
            for (;;) {
                space();
                expect(i_ < s_.size() && s_[i_] == '"', "safetensors_header_json");
                std::string key = string();
                space();
                expect(next() == ':', "safetensors_header_json");
                v.members.emplace_back(std::move(key), value(depth + 1));
                space();
                const char sep = next();
                if (sep == '}')
                    return v;
                expect(sep == ',', "safetensors_header_json");
            }
        }
        if (c == '[') {
            v.kind = Json::Kind::array;
            ++i_;
            space();
            if (i_ < s_.size() && s_[i_] == ']') {
                ++i_;
                return v;
            }
            for (;;) {
                v.items.push_back(value(depth + 1));
                space();
                const char sep = next();
                if (sep == ']')
                    return v;
                expect(sep == ',', "safetensors_header_json");
            }
        }
        if (c == '"') {
            v.kind = Json::Kind::string;
            v.text = string();
            return v;
        }
        if (c == 't' || c == 'f') {
            v.kind = Json::Kind::boolean;
            v.flag = c == 't';
            literal(v.flag ? "true" : "false");
            return v;
        }
        if (c == 'n') {
            literal("null");
            return v;
        }
        v.kind = Json::Kind::number;
        v.text = number();
        return v;
    }

    std::string number() {
        const std::size_t begin = i_;
        auto digits = [&] {
            const std::size_t from = i_;
            while (i_ < s_.size() && s_[i_] >= '0' && s_[i_] <= '9')
                ++i_;
            expect(i_ > from, "safetensors_header_json");
        };
        if (s_[i_] == '-')
            ++i_;
        digits();
        if (i_ < s_.size() && s_[i_] == '.') {
            ++i_;
            digits();
        }
        if (i_ < s_.size() && (s_[i_] == 'e' || s_[i_] == 'E')) {
            ++i_;
            if (i_ < s_.size() && (s_[i_] == '+' || s_[i_] == '-'))
                ++i_;
            digits();
        }
        return std::string(s_.substr(begin, i_ - begin));
    }

    std::string string() {
        ++i_;  // the opening quote
        std::string out;
        for (;;) {
            const auto c = static_cast<unsigned char>(next());
            if (c == '"')
                return out;
            expect(c >= 0x20, "safetensors_header_json");  // control characters
            expect(c < 0x80, "safetensors_header_ascii");
            if (c != '\\') {
                out.push_back(char(c));
                continue;
            }
            const char e = next();
            switch (e) {
            case '"': case '\\': case '/': out.push_back(e); break;
            case 'b': out.push_back('\b'); break;
            case 'f': out.push_back('\f'); break;
            case 'n': out.push_back('\n'); break;
            case 'r': out.push_back('\r'); break;
            case 't': out.push_back('\t'); break;
            case 'u': {
                unsigned code = 0;
                for (int k = 0; k < 4; ++k) {
                    const char h = next();
                    const unsigned digit = h >= '0' && h <= '9'   ? unsigned(h - '0')
                                           : h >= 'a' && h <= 'f' ? unsigned(h - 'a' + 10)
                                           : h >= 'A' && h <= 'F' ? unsigned(h - 'A' + 10)
                                                                  : 16u;
                    expect(digit < 16, "safetensors_header_json");
                    code = 16 * code + digit;
                }
                expect(code < 0x80, "safetensors_header_ascii");
                out.push_back(char(code));
                break;
            }
            default: fail("safetensors_header_json");
            }
        }
    }

    std::string_view s_;
    std::size_t i_ = 0;
};

// A JSON number that is a plain non-negative integer within 64 bits.
std::uint64_t unsigned_of(const Json& v) {
    expect(v.kind == Json::Kind::number && !v.text.empty(), "safetensors_header_integer");
    std::uint64_t r = 0;
    for (char c : v.text) {
        expect(c >= '0' && c <= '9', "safetensors_header_integer");
        r = add_or(mul_or(r, 10, "safetensors_header_integer"), std::uint64_t(c - '0'),
                   "safetensors_header_integer");
    }
    return r;
}

struct DtypeName {
    std::string_view name;
    Dtype dtype;
    std::uint64_t bytes;
};

constexpr DtypeName kDtypes[] = {
    {"BOOL", Dtype::boolean, 1}, {"U8", Dtype::u8, 1},        {"I8", Dtype::i8, 1},
    {"U16", Dtype::u16, 2},      {"I16", Dtype::i16, 2},      {"F16", Dtype::f16, 2},
    {"BF16", Dtype::bf16, 2},    {"U32", Dtype::u32, 4},      {"I32", Dtype::i32, 4},
    {"F32", Dtype::f32, 4},      {"U64", Dtype::u64, 8},      {"I64", Dtype::i64, 8},
    {"F64", Dtype::f64, 8},      {"F8_E4M3", Dtype::f8_e4m3, 1}, {"F8_E5M2", Dtype::f8_e5m2, 1},
};

// One tensor entry: exactly the fields dtype, shape and data_offsets, each once.
SafetensorsInfo tensor_entry(const std::string& name, const Json& entry,
                             std::uint64_t payload_at) {
    expect(entry.kind == Json::Kind::object, "safetensors_tensor");
    const Json *dtype = nullptr, *shape = nullptr, *offsets = nullptr;
    for (const auto& [field, v] : entry.members) {
        const Json** slot = field == "dtype"          ? &dtype
                            : field == "shape"        ? &shape
                            : field == "data_offsets" ? &offsets
                                                      : nullptr;
        expect(slot != nullptr, "safetensors_tensor");
        expect(*slot == nullptr, "safetensors_duplicate");
        *slot = &v;
    }
    expect(dtype && shape && offsets, "safetensors_tensor");
    expect(dtype->kind == Json::Kind::string, "safetensors_dtype");
    const DtypeName* kind = nullptr;
    for (const auto& d : kDtypes)
        if (d.name == dtype->text)
            kind = &d;
    expect(kind != nullptr, "safetensors_dtype");
    SafetensorsInfo t;
    t.name = name;
    t.dtype = kind->dtype;
    expect(shape->kind == Json::Kind::array, "safetensors_tensor_shape");
    std::uint64_t elements = 1;
    for (const auto& d : shape->items) {
        t.shape.push_back(unsigned_of(d));
        elements = mul_or(elements, t.shape.back(), "safetensors_tensor_shape");
    }
    expect(offsets->kind == Json::Kind::array && offsets->items.size() == 2,
           "safetensors_tensor");
    const auto begin = unsigned_of(offsets->items[0]), end = unsigned_of(offsets->items[1]);
    expect(begin <= end &&
               end - begin == mul_or(elements, kind->bytes, "safetensors_tensor_shape"),
           "safetensors_tensor_shape");
    t.begin = add_or(payload_at, begin, "safetensors_tensor_bounds");
    t.end = add_or(payload_at, end, "safetensors_tensor_bounds");
    return t;
}

}  // namespace

struct SafetensorsFile::State {
    Descriptor file;
    std::vector<SafetensorsInfo> tensors;
    std::map<std::string, std::size_t, std::less<>> by_name;
    std::map<std::string, std::string, std::less<>> metadata;
    explicit State(const std::string& path)
        : file(path, "checkpoint_open_failed", "checkpoint_not_regular_file") {}
};

SafetensorsFile::SafetensorsFile(const std::string& path)
    : state_(std::make_unique<State>(path)) {
    auto& s = *state_;
    std::uint64_t header = 0;
    s.file.read(0, std::as_writable_bytes(std::span<std::uint64_t>(&header, 1)),
                "safetensors_header_size", "checkpoint_read_bounds");
    expect(header <= kSafetensorsHeaderLimit && header <= s.file.size() - 8,
           "safetensors_header_size");
    std::string text(std::size_t(header), '\0');
    s.file.read(8, std::as_writable_bytes(std::span<char>(text)), "safetensors_header_size",
                "checkpoint_read_bounds");
    const Json root = JsonReader(text).document();
    expect(root.kind == Json::Kind::object, "safetensors_header");
    const std::uint64_t payload_at = 8 + header, payload = s.file.size() - payload_at;
    bool seen_metadata = false;
    for (const auto& [key, v] : root.members) {
        if (key == "__metadata__") {
            expect(!seen_metadata, "safetensors_duplicate");
            seen_metadata = true;
            expect(v.kind == Json::Kind::object, "safetensors_metadata");
            for (const auto& [k, m] : v.members) {
                expect(m.kind == Json::Kind::string, "safetensors_metadata");
                expect(s.metadata.emplace(k, m.text).second, "safetensors_duplicate");
            }
            continue;
        }
        expect(!key.empty(), "safetensors_tensor");
        expect(s.by_name.emplace(key, s.tensors.size()).second, "safetensors_duplicate");
        s.tensors.push_back(tensor_entry(key, v, payload_at));
    }
    // the tensors tile the payload: from its first byte, no overlap, no gap, to its end
    std::vector<const SafetensorsInfo*> order;
    for (const auto& t : s.tensors)
        order.push_back(&t);
    std::sort(order.begin(), order.end(), [](const auto* a, const auto* b) {
        return a->begin != b->begin ? a->begin < b->begin : a->end < b->end;
    });
    std::uint64_t covered = payload_at;
    for (const auto* t : order) {
        expect(t->begin >= covered, "safetensors_tensor_overlap");
        expect(t->begin == covered, "safetensors_tensor_gap");
        covered = t->end;
    }
    expect(covered == payload_at + payload, "safetensors_payload_coverage");
}

SafetensorsFile::~SafetensorsFile() = default;

std::size_t SafetensorsFile::size() const {
    return state_->tensors.size();
}

const SafetensorsInfo& SafetensorsFile::info(std::string_view name) const {
    const auto it = state_->by_name.find(name);
    expect(it != state_->by_name.end(), "missing_tensor");
    return state_->tensors[it->second];
}

WeightIdentity SafetensorsFile::identity(std::string_view name) const {
    const auto& t = info(name);
    return state_->file.identity(t.begin, t.end);
}

void SafetensorsFile::verify_unchanged() const {
    expect(!state_->file.moved(), "checkpoint_changed");
}

std::string SafetensorsFile::metadata(std::string_view key) const {
    const auto it = state_->metadata.find(key);
    expect(it != state_->metadata.end(), "safetensors_missing_metadata");
    return it->second;
}

namespace {

// The pair <prefix>_blocks U8 [E, R, G, 16] / <prefix>_scales U8 [E, R, G].
struct Mxfp4Pair {
    const SafetensorsInfo* blocks;
    const SafetensorsInfo* scales;
    std::uint64_t experts, rows, groups;
};

Mxfp4Pair mxfp4_pair(const SafetensorsFile& f, std::string_view prefix) {
    expect(!prefix.empty(), "projection_range_or_name");
    const std::string stem(prefix);
    const auto& b = f.info(stem + "_blocks");
    const auto& s = f.info(stem + "_scales");
    expect(b.dtype == Dtype::u8 && s.dtype == Dtype::u8, "mxfp4_dtype");
    expect(b.shape.size() == 4 && s.shape.size() == 3 && b.shape[3] == 16 && b.shape[2] > 0 &&
               std::equal(s.shape.begin(), s.shape.end(), b.shape.begin()),
           "mxfp4_expert_shape");
    return {&b, &s, b.shape[0], b.shape[1], b.shape[2]};
}

// `count` rows of scales then blocks, from row `row` of the flattened [E * R] rows; every
// scale byte checked before a block byte is read.
void read_mxfp4(const Descriptor& file, const Mxfp4Pair& p, std::uint64_t row,
                std::uint64_t count, Mxfp4Rows& out) {
    out.scales.resize(std::size_t(count * p.groups));
    out.blocks.resize(std::size_t(count * p.groups * 16));
    file.read(p.scales->begin + row * p.groups, std::as_writable_bytes(std::span(out.scales)),
              "checkpoint_read_bounds", "checkpoint_read_bounds");
    for (std::uint8_t e : out.scales)
        expect(e != 255, "invalid_block_scale");  // E8M0 255 is NaN, not a scale
    file.read(p.blocks->begin + row * p.groups * 16, std::as_writable_bytes(std::span(out.blocks)),
              "checkpoint_read_bounds", "checkpoint_read_bounds");
}

}  // namespace

Mxfp4Rows SafetensorsFile::mxfp4_rows(std::string_view prefix, std::size_t expert,
                                      std::size_t first, std::size_t count,
                                      std::size_t payload_budget) const {
    expect(count > 0, "projection_range_or_name");
    const Mxfp4Pair p = mxfp4_pair(*this, prefix);
    expect(expert < p.experts && first <= p.rows && count <= p.rows - first,
           "mxfp4_expert_shape");
    // count <= rows, so the sizes stay below the tensors' own byte counts
    const std::uint64_t bytes = count * p.groups * 17;
    expect(bytes <= payload_budget, "payload_budget");
    verify_unchanged();
    Mxfp4Rows out;
    out.rows = count;
    out.columns = std::size_t(p.groups * 32);
    read_mxfp4(state_->file, p, expert * p.rows + first, count, out);
    return out;
}

Mxfp4Rows SafetensorsFile::mxfp4_experts(std::string_view prefix, std::size_t& experts,
                                         std::size_t payload_budget) const {
    const Mxfp4Pair p = mxfp4_pair(*this, prefix);
    const std::uint64_t rows = p.experts * p.rows;  // both bounded by the tensor sizes
    expect(rows * p.groups * 17 <= payload_budget, "payload_budget");
    verify_unchanged();
    Mxfp4Rows out;
    out.rows = std::size_t(p.rows);
    out.columns = std::size_t(p.groups * 32);
    read_mxfp4(state_->file, p, 0, rows, out);
    experts = std::size_t(p.experts);
    return out;
}

}  // namespace kadan_amd::checkpoint
