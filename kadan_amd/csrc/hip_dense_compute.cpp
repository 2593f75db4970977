// kadan_amd::HipDenseCompute: the DenseCompute-compatible host layer over the C ABI.
// Restates the reference's validation and result contract (IW/src/cuda/h3_compute.cu:
// 1760-1830 validate/alias checks, :3503-3536 dense_gguf_source, :3963-4375
// dense_gguf_batch; IW = services/hikari/inference_worker) on one HIP stream.
#include "kadan_amd_dense_compute.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <condition_variable>
#include <exception>
#include <climits>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <string>

#include "kadan_amd.h"

namespace kadan_amd {
namespace {

void require(bool ok, const char* what) {
    if (!ok)
        throw std::runtime_error(what);
}

void hip_check(hipError_t e) {
    if (e != hipSuccess)
        throw std::runtime_error(std::string("kdq_hip: ") + hipGetErrorString(e));
}

void kdq_check(int status) {
    if (status == KDQ_OK)
        return;
    std::string what = kdq_status_string(status);
    if (status == KDQ_ERR_HIP)
        what += std::string(": ") + kdq_last_hip_error();
    throw std::runtime_error(what);
}

int ggml_type(gguf::Encoding e) {
    switch (e) {
    case gguf::Encoding::q4_0:
        return KDQ_Q4_0;
    case gguf::Encoding::q8_0:
        return KDQ_Q8_0;
    case gguf::Encoding::q4_k:
        return KDQ_Q4_K;
    case gguf::Encoding::q3_k:
        return KDQ_Q3_K;
    case gguf::Encoding::q6_k:
        return KDQ_Q6_K;
    case gguf::Encoding::iq4_nl:
        return KDQ_IQ4_NL;
    case gguf::Encoding::iq4_xs:
        return KDQ_IQ4_XS;
    case gguf::Encoding::bf16:
        return KDQ_BF16;
    case gguf::Encoding::iq3_xxs:
        return KDQ_IQ3_XXS;
    case gguf::Encoding::iq2_s:
        return KDQ_IQ2_S;
    case gguf::Encoding::iq3_s:
        return KDQ_IQ3_S;
    default:
        return -1;
    }
}

bool overlap(const void* a, std::size_t an, const void* b, std::size_t bn) {
    if (!an || !bn)
        return false;
    const auto x = reinterpret_cast<std::uintptr_t>(a), y = reinterpret_cast<std::uintptr_t>(b);
    return x <= y ? y - x < an : x - y < bn;
}

template <class T, class U> bool overlap(std::span<T> a, std::span<U> b) {
    return overlap(a.data(), a.size_bytes(), b.data(), b.size_bytes());
}

// Whole packed rows cross the host boundary through at most this much pinned staging
// (IW/include/kadan/device_placement.hpp:111).
constexpr std::size_t kStagingBytes = std::size_t(16) << 20;

std::size_t align16(std::size_t n) {
    return (n + 15) & ~std::size_t(15);
}

}  // namespace

namespace gguf {

std::optional<Encoding> encoding(std::uint32_t ggml_type) {
    switch (ggml_type) {
    case 2:
        return Encoding::q4_0;
    case 8:
        return Encoding::q8_0;
    case 11:
        return Encoding::q3_k;
    case 12:
        return Encoding::q4_k;
    case 14:
        return Encoding::q6_k;
    case 18:
        return Encoding::iq3_xxs;
    case 20:
        return Encoding::iq4_nl;
    case 21:
        return Encoding::iq3_s;
    case 22:
        return Encoding::iq2_s;
    case 23:
        return Encoding::iq4_xs;
    case 30:
        return Encoding::bf16;
    default:
        return std::nullopt;
    }
}

bool supported(Encoding e) {
    return ggml_type(e) >= 0;
}

std::size_t block_values(Encoding e) {
    switch (e) {
    case Encoding::bf16:
        return 1;
    case Encoding::q8_0:
    case Encoding::iq4_nl:
    case Encoding::q4_0:
        return 32;
    default:
        return 256;
    }
}

std::size_t block_bytes(Encoding e) {
    switch (e) {
    case Encoding::q3_k:
        return 110;
    case Encoding::q4_k:
        return 144;
    case Encoding::q8_0:
        return 34;
    case Encoding::q6_k:
        return 210;
    case Encoding::iq3_xxs:
        return 98;
    case Encoding::iq4_nl:
        return 18;
    case Encoding::iq4_xs:
        return 136;
    case Encoding::iq2_s:
        return 82;
    case Encoding::iq3_s:
        return 110;
    case Encoding::bf16:
        return 2;
    case Encoding::q4_0:
        return 18;
    }
    return 0;
}

}  // namespace gguf

struct HipDenseCompute::Resident {
    void* device = nullptr;
    std::size_t bytes = 0, row_bytes = 0;
    bool packed = false;  // the tile-packed layout of kdq_gguf_pack (else row-major rows)
    ~Resident() {
        if (device)
            (void)hipFree(device);
    }
};

// Three persistent host threads and the caller read one staging chunk's disjoint whole
// rows from the weight source in parallel (the source contract allows concurrent calls
// on disjoint rows, IW/include/kadan/dense_compute.hpp:174-179), as the reference's
// PackedReadTeam does (IW/include/kadan/packed_read_team.hpp:24-134).  Small chunks are
// read by the caller alone.
struct HipDenseCompute::ReadTeam {
    static constexpr std::size_t kParallelBytes = std::size_t(2) << 20;
    static constexpr int kWorkers = 3;

    ReadTeam() {
        for (int i = 0; i < kWorkers; ++i)
            threads_.emplace_back([this, i] { run(i); });
    }
    ~ReadTeam() {
        {
            std::lock_guard<std::mutex> lock(mutex_);
            closing_ = true;
        }
        ready_.notify_all();
        for (auto& t : threads_)
            t.join();
    }

    void read(const GgufWeightSource& source, std::size_t first, std::size_t row_bytes,
              std::span<std::byte> dst) {
        const std::size_t rows = dst.size() / row_bytes;
        if (dst.size() < kParallelBytes || rows < kWorkers + 1) {
            source(first, dst);
            return;
        }
        {
            std::lock_guard<std::mutex> lock(mutex_);
            source_ = &source;
            first_ = first;
            row_bytes_ = row_bytes;
            dst_ = dst;
            rows_ = rows;
            remaining_ = kWorkers;
            for (auto& e : errors_)
                e = nullptr;
            ++round_;
        }
        ready_.notify_all();
        std::exception_ptr mine;
        try {
            part(kWorkers);
        } catch (...) {
            mine = std::current_exception();
        }
        std::unique_lock<std::mutex> lock(mutex_);
        done_.wait(lock, [&] { return remaining_ == 0; });
        source_ = nullptr;
        if (mine)
            std::rethrow_exception(mine);
        for (auto& e : errors_)
            if (e)
                std::rethrow_exception(e);
    }

private:
    // part k of kWorkers + 1 contiguous row ranges
    void part(int k) {
        const std::size_t a = rows_ * std::size_t(k) / (kWorkers + 1);
        const std::size_t b = rows_ * std::size_t(k + 1) / (kWorkers + 1);
        if (b > a)
            (*source_)(first_ + a, dst_.subspan(a * row_bytes_, (b - a) * row_bytes_));
    }
    void run(int k) {
        std::uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lock(mutex_);
                ready_.wait(lock, [&] { return closing_ || round_ != seen; });
                if (closing_)
                    return;
                seen = round_;
            }
            std::exception_ptr error;
            try {
                part(k);
            } catch (...) {
                error = std::current_exception();
            }
            {
                std::lock_guard<std::mutex> lock(mutex_);
                errors_[k] = error;
                --remaining_;
            }
            done_.notify_all();
        }
    }

    std::vector<std::thread> threads_;
    std::mutex mutex_;
    std::condition_variable ready_, done_;
    bool closing_ = false;
    std::uint64_t round_ = 0;
    const GgufWeightSource* source_ = nullptr;
    std::size_t first_ = 0, row_bytes_ = 0, rows_ = 0;
    std::span<std::byte> dst_;
    int remaining_ = 0;
    std::exception_ptr errors_[kWorkers];
};

HipDenseCompute::HipDenseCompute(int device) : device_(device) {
    hip_check(hipSetDevice(device));
    hipStream_t s = nullptr;
    hip_check(hipStreamCreate(&s));  // default priority
    stream_ = s;
    for (auto& e : staged_) {
        hipEvent_t ev = nullptr;
        hip_check(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
        e = ev;
    }
    team_ = std::make_unique<ReadTeam>();
}

HipDenseCompute::~HipDenseCompute() {
    (void)hipSetDevice(device_);
    if (stream_)
        (void)hipStreamSynchronize(static_cast<hipStream_t>(stream_));
    team_.reset();
    bank_.clear();
    for (auto& b : buffers_)
        if (b.first)
            (void)hipFree(b.first);
    for (auto* p : pinned_)
        if (p)
            (void)hipHostFree(p);
    for (auto* e : staged_)
        if (e)
            (void)hipEventDestroy(static_cast<hipEvent_t>(e));
    if (stream_)
        (void)hipStreamDestroy(static_cast<hipStream_t>(stream_));
}

void HipDenseCompute::synchronize() {
    hip_check(hipStreamSynchronize(static_cast<hipStream_t>(stream_)));
}

void* HipDenseCompute::device_buffer(std::size_t slot, std::size_t bytes) {
    if (buffers_.size() <= slot)
        buffers_.resize(slot + 1, {nullptr, 0});
    auto& b = buffers_[slot];
    if (b.second < bytes) {
        synchronize();
        if (b.first)
            hip_check(hipFree(b.first));
        b = {nullptr, 0};
        const std::size_t grown = std::max<std::size_t>(bytes, 1 << 20);
        hip_check(hipMalloc(&b.first, grown));
        b.second = grown;
    }
    return b.first;
}

void HipDenseCompute::set_weight_limit(std::size_t bytes) {
    std::lock_guard<std::mutex> lock(mutex_);
    weight_limit_ = bytes;
}

std::byte* HipDenseCompute::stage_rows(unsigned b, const GgufWeightSource& source,
                                       std::size_t first, std::size_t n, std::size_t row_bytes) {
    const std::size_t need = std::max(kStagingBytes, n * row_bytes);
    if (pinned_bytes_ < need) {
        synchronize();  // no copy may still read the old buffers
        for (auto& p : pinned_) {
            if (p)
                hip_check(hipHostFree(p));
            p = nullptr;
        }
        pinned_bytes_ = 0;
        for (auto& p : pinned_)
            hip_check(hipHostMalloc(&p, need, hipHostMallocDefault));
        pinned_bytes_ = need;
        staged_pending_[0] = staged_pending_[1] = false;
    }
    if (staged_pending_[b]) {  // the upload of this buffer's previous chunk is done
        hip_check(hipEventSynchronize(static_cast<hipEvent_t>(staged_[b])));
        staged_pending_[b] = false;
    }
    auto* bytes = static_cast<std::byte*>(pinned_[b]);
    team_->read(source, first, row_bytes, std::span<std::byte>(bytes, n * row_bytes));
    return bytes;
}

void HipDenseCompute::staged(unsigned b) {
    hip_check(hipEventRecord(static_cast<hipEvent_t>(staged_[b]),
                             static_cast<hipStream_t>(stream_)));
    staged_pending_[b] = true;
}

const HipDenseCompute::Resident* HipDenseCompute::weights_for(
    const WeightIdentity& identity, int type, std::size_t in, std::size_t out,
    const GgufWeightSource& source, bool retain, const std::atomic_bool& cancel,
    std::unique_ptr<Resident>& transient, bool product, bool stream_miss) {
    // Products (decode GEMV and prefill GEMM) keep the tile-packed layout when the packed
    // GEMV takes the shape, so one resident copy serves both; the layout is part of the
    // bank key.  F32 rows are kept with each row zero-padded to a multiple of 8 values,
    // the exact product's granule.
    const bool f32 = type == KDQ_F32;
    const bool packed = product && !f32 && kdq_gemv_packed_supported(type, in);
    const BankKey key{identity, 2 * type + (packed ? 1 : 0), in, out};
    if (auto it = bank_.find(key); it != bank_.end())
        return it->second.get();
    const std::size_t source_row_bytes = kdq_row_bytes(type, in);
    const std::size_t row_bytes = f32 ? (in + 7) / 8 * 8 * sizeof(float) : source_row_bytes;
    const std::size_t bytes = packed ? kdq_gguf_packed_bytes(type, in, out) : out * row_bytes;
    if (retain && weight_limit_) {
        // the reference's envelope refusal (IW/include/kadan/device_weights.hpp:203-206):
        // a miss that would pass the limit is not admitted, and nothing is evicted for it
        std::size_t used = 0;
        for (const auto& [k, r] : bank_)
            used += r->bytes;
        retain = used <= weight_limit_ && bytes <= weight_limit_ - used;
    }
    if (!retain && stream_miss)
        return nullptr;
    auto r = std::make_unique<Resident>();
    r->row_bytes = row_bytes;
    r->packed = packed;
    r->bytes = bytes;
    hip_check(hipMalloc(&r->device, r->bytes));
    // chunks of whole 16-row tiles when packing (each chunk packs into its own tiles);
    // the reads of chunk c + 1 overlap the upload and packing of chunk c
    std::size_t rows_per_chunk = std::max<std::size_t>(1, kStagingBytes / source_row_bytes);
    if (packed)
        rows_per_chunk = std::max<std::size_t>(16, rows_per_chunk / 16 * 16);
    const std::size_t tile_bytes = packed ? kdq_gguf_packed_bytes(type, in, 16) : 0;
    auto st = static_cast<hipStream_t>(stream_);
    try {
        if (row_bytes != source_row_bytes)  // the padding of every F32 row
            hip_check(hipMemsetAsync(r->device, 0, r->bytes, st));
        unsigned b = 0;
        for (std::size_t first = 0; first < out; first += rows_per_chunk, b ^= 1) {
            require(!cancel.load(), "kdq_cancelled");
            const std::size_t n = std::min(rows_per_chunk, out - first);
            std::byte* host = stage_rows(b, source, first, n, source_row_bytes);
            if (packed) {
                auto* raw = static_cast<std::uint8_t*>(device_buffer(6 + b, n * row_bytes));
                hip_check(hipMemcpyAsync(raw, host, n * row_bytes, hipMemcpyHostToDevice, st));
                staged(b);
                kdq_check(kdq_gguf_pack(type, raw, row_bytes, in, n,
                                        static_cast<std::uint8_t*>(r->device) +
                                            first / 16 * tile_bytes,
                                        st));
            } else if (row_bytes != source_row_bytes) {
                hip_check(hipMemcpy2DAsync(static_cast<std::uint8_t*>(r->device) +
                                               first * row_bytes,
                                           row_bytes, host, source_row_bytes, source_row_bytes,
                                           n, hipMemcpyHostToDevice, st));
                staged(b);
            } else {
                hip_check(hipMemcpyAsync(static_cast<std::uint8_t*>(r->device) + first * row_bytes,
                                         host, n * row_bytes, hipMemcpyHostToDevice, st));
                staged(b);
            }
        }
    } catch (...) {
        (void)hipStreamSynchronize(st);  // nothing in flight reads what unwinding frees
        throw;
    }
    if (!retain) {
        transient = std::move(r);
        return transient.get();
    }
    auto& slot = bank_[key];
    slot = std::move(r);
    return slot.get();
}

void HipDenseCompute::stream_product(gguf::Encoding enc, std::size_t in, std::size_t out,
                                     std::size_t rows, const GgufWeightSource& source,
                                     const float* dx, float* dy, unsigned* dstatus,
                                     const std::atomic_bool& cancel, bool gemm) {
    const bool packed = kdq_gemv_packed_supported(ggml_type(enc), in);
    const std::size_t row_bytes = in / gguf::block_values(enc) * gguf::block_bytes(enc);
    std::size_t rows_per_chunk = std::max<std::size_t>(1, kStagingBytes / row_bytes);
    if (packed)
        rows_per_chunk = std::max<std::size_t>(16, rows_per_chunk / 16 * 16);
    rows_per_chunk = std::min(rows_per_chunk, out);
    auto st = static_cast<hipStream_t>(stream_);
    try {
        unsigned b = 0;
        for (std::size_t first = 0; first < out; first += rows_per_chunk, b ^= 1) {
            require(!cancel.load(), "kdq_cancelled");
            const std::size_t n = std::min(rows_per_chunk, out - first);
            std::byte* host = stage_rows(b, source, first, n, row_bytes);
            auto* raw = static_cast<std::uint8_t*>(device_buffer(6 + b, n * row_bytes));
            hip_check(hipMemcpyAsync(raw, host, n * row_bytes, hipMemcpyHostToDevice, st));
            staged(b);
            const void* w = raw;
            if (packed) {
                auto* pk = static_cast<std::uint8_t*>(
                    device_buffer(8 + b, kdq_gguf_packed_bytes(ggml_type(enc), in, n)));
                kdq_check(kdq_gguf_pack(ggml_type(enc), raw, row_bytes, in, n, pk, st));
                w = pk;
            }
            if (gemm) {  // columns [first, first + n) of y through a [rows x n] tile
                auto* tile = static_cast<float*>(device_buffer(10 + b, rows * n * 4));
                kdq_check(packed ? kdq_gemm_packed(ggml_type(enc), w, n, in, dx, rows, tile,
                                                   dstatus, st)
                                 : kdq_gemm_rows(ggml_type(enc), w, row_bytes, n, in, dx, rows,
                                                 tile, dstatus, st));
                hip_check(hipMemcpy2DAsync(dy + first, out * 4, tile, n * 4, n * 4, rows,
                                           hipMemcpyDeviceToDevice, st));
            } else {
                for (std::size_t r0 = 0; r0 < rows; r0 += gguf_batch_max_rows) {
                    const std::size_t m = std::min(gguf_batch_max_rows, rows - r0);
                    kdq_check(packed ? kdq_gemv_packed(ggml_type(enc), w, dx + r0 * in, m, in, n,
                                                       dy + r0 * out + first, out, dstatus, st)
                                     : kdq_gemv(ggml_type(enc), w, row_bytes, dx + r0 * in, m,
                                                in, n, dy + r0 * out + first, out, dstatus, st));
                }
            }
        }
    } catch (...) {
        (void)hipStreamSynchronize(st);
        throw;
    }
}

// The prefill GEMM (kdq_gemm_packed) takes packed Q4_K / Q8_0 / Q6_K rows of up to 32K
// values; the decode-time product takes batches of at most gguf_batch_rows rows (one
// weight pass serves every row anyway).
bool gemm_takes(gguf::Encoding enc, std::size_t in, std::size_t rows, bool packed) {
    return packed && rows > HipDenseCompute::gguf_batch_rows && in % 256 == 0 && in <= 32768 &&
           (enc == gguf::Encoding::q4_k || enc == gguf::Encoding::q8_0 ||
            enc == gguf::Encoding::q6_k);
}

// The prefill GEMM over row-major rows (kdq_gemm_rows) takes every other encoding kept
// row-major, so a prefill chunk reads its weights once instead of once per
// gguf_batch_rows rows.
bool rows_gemm_takes(gguf::Encoding enc, std::size_t in, std::size_t rows, bool packed) {
    const std::size_t values = kdq_gemm_rows_values(ggml_type(enc));
    return !packed && rows > HipDenseCompute::gguf_batch_rows && values && in % values == 0 &&
           in <= 65536;
}

ProjectionResult HipDenseCompute::dense_gguf_source(
    const WeightIdentity& identity, gguf::Encoding enc, const GgufWeightSource& source,
    std::span<const float> bias, std::span<const float> input, std::size_t in, std::size_t out,
    std::span<float> output, const std::atomic_bool& cancel, bool precise, bool retain_misses) {
    std::lock_guard<std::mutex> lock(mutex_);
    if (!gguf::supported(enc) || !in || in % gguf::block_values(enc) || in % 8)
        return ProjectionResult::unsupported;
    require(!cancel.load(), "kdq_cancelled");
    require(in && out && in <= std::size_t(INT_MAX) && out <= std::size_t(INT_MAX) &&
                !input.empty() && input.size() % in == 0 &&
                output.size() == input.size() / in * out && (bias.empty() || bias.size() == out),
            "kdq_projection_shape");
    for (float v : input)
        require(std::isfinite(v), "kdq_nonfinite_input");
    for (float v : bias)
        require(std::isfinite(v), "kdq_nonfinite_bias");
    require(!overlap(output, input) && !overlap(output, bias), "kdq_alias");
    hip_check(hipSetDevice(device_));
    const std::size_t rows = input.size() / in;
    auto st = static_cast<hipStream_t>(stream_);
    auto* dx = static_cast<float*>(device_buffer(0, rows * in * sizeof(float)));
    auto* dy = static_cast<float*>(device_buffer(1, rows * out * sizeof(float)));
    auto* dstatus = static_cast<unsigned*>(device_buffer(2, 256));
    hip_check(hipMemsetAsync(dstatus, 0, sizeof(unsigned), st));
    hip_check(hipMemcpyAsync(dx, input.data(), input.size_bytes(), hipMemcpyHostToDevice, st));
    // A miss that is not to be retained (or does not fit the bank's limit) is streamed: the
    // reference "keeps existing hits and streams uncached tiles" (dense_compute.hpp:174-179).
    // status into `status`, the rows into `output`, bias added; finite when every output is
    auto finish = [&](unsigned status) {
        hip_check(hipMemcpyAsync(output.data(), dy, output.size_bytes(), hipMemcpyDeviceToHost,
                                 st));
        synchronize();
        require(status == 0, "kdq_nonfinite_weight");
        bool finite = true;
        for (std::size_t r = 0; r < rows; ++r)
            for (std::size_t c = 0; c < out; ++c) {
                float& v = output[r * out + c];
                if (!bias.empty())
                    v += bias[c];
                finite = finite && std::isfinite(v);
            }
        return finite ? ProjectionResult::finite : ProjectionResult::unvalidated;
    };
    auto read_status = [&] {
        unsigned status = 0;
        hip_check(hipMemcpyAsync(&status, dstatus, sizeof status, hipMemcpyDeviceToHost, st));
        synchronize();
        return status;
    };
    std::unique_ptr<Resident> transient;
    if (precise) {
        // fp32 operands throughout: the exact-decode product (every weight decoded as
        // kdq_dequantize does, one fp32 fused multiply-add chain per output) over a
        // row-major copy, for every row count
        const Resident& rw = *weights_for(identity, ggml_type(enc), in, out, source,
                                          retain_misses, cancel, transient, false);
        for (std::size_t first = 0; first < rows; first += gguf_batch_max_rows) {
            require(!cancel.load(), "kdq_cancelled");
            const std::size_t n = std::min(gguf_batch_max_rows, rows - first);
            kdq_check(kdq_gemv_exact(ggml_type(enc), rw.device, rw.row_bytes, dx + first * in, n,
                                     in, out, dy + first * out, out, dstatus, st));
        }
        return finish(read_status());
    }
    const Resident* w = weights_for(identity, ggml_type(enc), in, out, source, retain_misses,
                                    cancel, transient, true, /*stream_miss=*/true);
    const bool packed = w ? w->packed : kdq_gemv_packed_supported(ggml_type(enc), in) != 0;
    auto decode_product = [&] {
        if (!w) {
            stream_product(enc, in, out, rows, source, dx, dy, dstatus, cancel, false);
            return;
        }
        for (std::size_t first = 0; first < rows; first += gguf_batch_max_rows) {
            require(!cancel.load(), "kdq_cancelled");
            const std::size_t n = std::min(gguf_batch_max_rows, rows - first);
            kdq_check(w->packed ? kdq_gemv_packed(ggml_type(enc), w->device, dx + first * in, n,
                                                  in, out, dy + first * out, out, dstatus, st)
                                : kdq_gemv(ggml_type(enc), w->device, w->row_bytes,
                                           dx + first * in, n, in, out, dy + first * out, out,
                                           dstatus, st));
        }
    };
    // Prefill (the reference's decode-tile + SGEMM path, h3_compute.cu:2201-2218,2451): one
    // GEMM reads each weight byte once for all rows; its status bit 2 (a dequantised weight
    // past the fp16 range) sends the rows through the decode-time product instead.
    const bool gemm = gemm_takes(enc, in, rows, packed) || rows_gemm_takes(enc, in, rows, packed);
    if (gemm && w && packed)
        kdq_check(kdq_gemm_packed(ggml_type(enc), w->device, out, in, dx, rows, dy, dstatus, st));
    else if (gemm && w)
        kdq_check(kdq_gemm_rows(ggml_type(enc), w->device, w->row_bytes, out, in, dx, rows, dy,
                                dstatus, st));
    else if (gemm)
        stream_product(enc, in, out, rows, source, dx, dy, dstatus, cancel, true);
    else
        decode_product();
    unsigned status = read_status();
    if (gemm && (status & 2u) && !(status & 1u)) {
        hip_check(hipMemsetAsync(dstatus, 0, sizeof(unsigned), st));
        decode_product();
        status = read_status();
    }
    return finish(status);
}

void HipDenseCompute::dense(std::span<const float> weights, std::span<const float> bias,
                            std::span<const float> input, std::size_t in, std::size_t out,
                            std::span<float> output, const std::atomic_bool& cancel,
                            bool precise) {
    (void)precise;  // the product is fp32 either way
    std::lock_guard<std::mutex> lock(mutex_);
    require(!cancel.load(), "kdq_cancelled");
    require(in && out && in <= std::size_t(INT_MAX) && out <= std::size_t(INT_MAX) &&
                weights.size() == in * out && !input.empty() && input.size() % in == 0 &&
                output.size() == input.size() / in * out && (bias.empty() || bias.size() == out),
            "kdq_projection_shape");
    require(!overlap(output, input) && !overlap(output, bias) && !overlap(output, weights),
            "kdq_alias");
    hip_check(hipSetDevice(device_));
    const std::size_t rows = input.size() / in;
    // F32 rows of the exact kernel need in % 8 == 0: zero-pad each row (and x) on upload
    const std::size_t padded = (in + 7) / 8 * 8;
    auto st = static_cast<hipStream_t>(stream_);
    auto* dw = static_cast<float*>(device_buffer(5, out * padded * sizeof(float)));
    auto* dx = static_cast<float*>(device_buffer(0, rows * padded * sizeof(float)));
    auto* dy = static_cast<float*>(device_buffer(1, rows * out * sizeof(float)));
    if (padded == in) {
        hip_check(hipMemcpyAsync(dw, weights.data(), weights.size_bytes(), hipMemcpyHostToDevice,
                                 st));
        hip_check(hipMemcpyAsync(dx, input.data(), input.size_bytes(), hipMemcpyHostToDevice, st));
    } else {
        hip_check(hipMemsetAsync(dw, 0, out * padded * sizeof(float), st));
        hip_check(hipMemsetAsync(dx, 0, rows * padded * sizeof(float), st));
        hip_check(hipMemcpy2DAsync(dw, padded * sizeof(float), weights.data(), in * sizeof(float),
                                   in * sizeof(float), out, hipMemcpyHostToDevice, st));
        hip_check(hipMemcpy2DAsync(dx, padded * sizeof(float), input.data(), in * sizeof(float),
                                   in * sizeof(float), rows, hipMemcpyHostToDevice, st));
    }
    for (std::size_t first = 0; first < rows; first += gguf_batch_max_rows) {
        require(!cancel.load(), "kdq_cancelled");
        const std::size_t n = std::min(gguf_batch_max_rows, rows - first);
        kdq_check(kdq_gemv(KDQ_F32, dw, padded * sizeof(float), dx + first * padded, n, padded,
                           out, dy + first * out, out, nullptr, st));
    }
    hip_check(hipMemcpyAsync(output.data(), dy, output.size_bytes(), hipMemcpyDeviceToHost, st));
    synchronize();
    if (!bias.empty())
        for (std::size_t r = 0; r < rows; ++r)
            for (std::size_t c = 0; c < out; ++c)
                output[r * out + c] += bias[c];
}

ProjectionResult HipDenseCompute::dense_source(const WeightIdentity& identity,
                                               const FloatWeightSource& source,
                                               std::span<const float> bias,
                                               std::span<const float> input, std::size_t in,
                                               std::size_t out, std::span<float> output,
                                               const std::atomic_bool& cancel, bool precise,
                                               ProjectionPolicy policy) {
    (void)precise;  // fp32 operands and accumulation whatever is asked
    (void)policy;
    std::lock_guard<std::mutex> lock(mutex_);
    require(!cancel.load(), "kdq_cancelled");
    require(in && out && in <= std::size_t(INT_MAX) && out <= std::size_t(INT_MAX) &&
                !input.empty() && input.size() % in == 0 &&
                output.size() == input.size() / in * out && (bias.empty() || bias.size() == out),
            "kdq_projection_shape");
    for (float v : input)
        require(std::isfinite(v), "kdq_nonfinite_input");
    for (float v : bias)
        require(std::isfinite(v), "kdq_nonfinite_bias");
    require(!overlap(output, input) && !overlap(output, bias), "kdq_alias");
    hip_check(hipSetDevice(device_));
    // The bank reads whole rows as bytes; the F32 source takes element offsets.
    const GgufWeightSource rows_of = [&](std::size_t first_row, std::span<std::byte> dst) {
        source(first_row * in, std::span<float>(reinterpret_cast<float*>(dst.data()),
                                                dst.size() / sizeof(float)));
    };
    std::unique_ptr<Resident> transient;
    const Resident& w =
        *weights_for(identity, KDQ_F32, in, out, rows_of, true, cancel, transient, true);
    const std::size_t rows = input.size() / in, padded = w.row_bytes / sizeof(float);
    auto st = static_cast<hipStream_t>(stream_);
    auto* dx = static_cast<float*>(device_buffer(0, rows * padded * sizeof(float)));
    auto* dy = static_cast<float*>(device_buffer(1, rows * out * sizeof(float)));
    auto* dstatus = static_cast<unsigned*>(device_buffer(2, 256));
    hip_check(hipMemsetAsync(dstatus, 0, sizeof(unsigned), st));
    if (padded == in) {
        hip_check(hipMemcpyAsync(dx, input.data(), input.size_bytes(), hipMemcpyHostToDevice, st));
    } else {
        hip_check(hipMemsetAsync(dx, 0, rows * padded * sizeof(float), st));
        hip_check(hipMemcpy2DAsync(dx, padded * sizeof(float), input.data(), in * sizeof(float),
                                   in * sizeof(float), rows, hipMemcpyHostToDevice, st));
    }
    for (std::size_t first = 0; first < rows; first += gguf_batch_max_rows) {
        require(!cancel.load(), "kdq_cancelled");
        const std::size_t n = std::min(gguf_batch_max_rows, rows - first);
        kdq_check(kdq_gemv(KDQ_F32, w.device, w.row_bytes, dx + first * padded, n, padded, out,
                           dy + first * out, out, dstatus, st));
    }
    unsigned status = 0;
    hip_check(hipMemcpyAsync(&status, dstatus, sizeof status, hipMemcpyDeviceToHost, st));
    hip_check(hipMemcpyAsync(output.data(), dy, output.size_bytes(), hipMemcpyDeviceToHost, st));
    synchronize();
    require(status == 0, "kdq_nonfinite_weight");
    bool finite = true;
    for (std::size_t r = 0; r < rows; ++r)
        for (std::size_t c = 0; c < out; ++c) {
            float& v = output[r * out + c];
            if (!bias.empty())
                v += bias[c];
            finite = finite && std::isfinite(v);
        }
    return finite ? ProjectionResult::finite : ProjectionResult::unvalidated;
}

void HipDenseCompute::dequantize_rows(gguf::Encoding enc, std::span<const std::byte> packed,
                                      std::size_t in, std::span<float> output) {
    std::lock_guard<std::mutex> lock(mutex_);
    require(gguf::supported(enc) && in && in % gguf::block_values(enc) == 0,
            "kdq_projection_shape");
    const std::size_t row_bytes = in / gguf::block_values(enc) * gguf::block_bytes(enc);
    require(packed.size() % row_bytes == 0 && output.size() == packed.size() / row_bytes * in,
            "kdq_projection_shape");
    if (packed.empty())
        return;
    hip_check(hipSetDevice(device_));
    auto st = static_cast<hipStream_t>(stream_);
    const std::size_t rows = packed.size() / row_bytes;
    auto* dw = static_cast<std::uint8_t*>(device_buffer(5, packed.size()));
    auto* dy = static_cast<float*>(device_buffer(1, output.size_bytes()));
    auto* dstatus = static_cast<unsigned*>(device_buffer(2, 256));
    hip_check(hipMemsetAsync(dstatus, 0, sizeof(unsigned), st));
    hip_check(hipMemcpyAsync(dw, packed.data(), packed.size(), hipMemcpyHostToDevice, st));
    kdq_check(kdq_dequantize(ggml_type(enc), dw, row_bytes, rows, in, dy, dstatus, st));
    unsigned status = 0;
    hip_check(hipMemcpyAsync(output.data(), dy, output.size_bytes(), hipMemcpyDeviceToHost, st));
    hip_check(hipMemcpyAsync(&status, dstatus, sizeof status, hipMemcpyDeviceToHost, st));
    synchronize();
    require(status == 0, "kdq_nonfinite_weight");
}

bool HipDenseCompute::batch_supported(std::span<const GgufBatchJob> jobs) {
    if (jobs.empty())
        return false;
    for (const auto& j : jobs) {
        if (!j.identity || !j.source || !j.in || !j.out || j.in > std::size_t(INT_MAX) ||
            j.out > std::size_t(INT_MAX) || j.input.empty() || j.input.size() % j.in ||
            j.input.size() / j.in > gguf_batch_max_rows ||
            j.output.size() != j.input.size() / j.in * j.out ||
            (j.encoding && (!gguf::supported(*j.encoding) ||
                            j.in % gguf::block_values(*j.encoding) ||
                            j.in / gguf::block_values(*j.encoding) >
                                kStagingBytes / gguf::block_bytes(*j.encoding))) ||
            (!j.encoding && j.in > kStagingBytes / sizeof(float)) || j.in % 8)
            return false;
    }
    return true;
}

ProjectionResult HipDenseCompute::dense_gguf_batch(std::span<const GgufBatchJob> jobs,
                                                   const std::atomic_bool& cancel) {
    std::lock_guard<std::mutex> lock(mutex_);
    // decided before any source read
    if (!batch_supported(jobs))
        return ProjectionResult::unsupported;
    require(!cancel.load(), "kdq_cancelled");
    for (const auto& j : jobs) {
        for (float v : j.input)
            require(std::isfinite(v), "kdq_nonfinite_input");
        for (const auto& k : jobs)
            require(!overlap(j.output, k.input), "kdq_alias");
    }
    hip_check(hipSetDevice(device_));
    auto st = static_cast<hipStream_t>(stream_);
    std::vector<std::unique_ptr<Resident>> transients(jobs.size());
    std::vector<const Resident*> weights(jobs.size());
    // F32 rows (no encoding) take the exact fp32 product, IW/src/cuda/h3_compute.cu:4076-4082
    std::vector<int> types(jobs.size());
    for (std::size_t i = 0; i < jobs.size(); ++i)
        types[i] = jobs[i].encoding ? ggml_type(*jobs[i].encoding) : int(KDQ_F32);
    for (std::size_t i = 0; i < jobs.size(); ++i)
        weights[i] = weights_for(*jobs[i].identity, types[i], jobs[i].in, jobs[i].out,
                                  *jobs[i].source, jobs[i].retain_misses, cancel, transients[i],
                                  true);
    // One upload of each distinct input span, one device output region per job.
    std::vector<std::size_t> input_at(jobs.size()), output_at(jobs.size());
    std::size_t in_bytes = 0, out_bytes = 0;
    for (std::size_t i = 0; i < jobs.size(); ++i) {
        std::size_t same = i;
        for (std::size_t k = 0; k < i; ++k)
            if (jobs[k].input.data() == jobs[i].input.data() &&
                jobs[k].input.size() == jobs[i].input.size()) {
                same = k;
                break;
            }
        if (same != i) {
            input_at[i] = input_at[same];
        } else {
            input_at[i] = in_bytes;
            in_bytes += align16(jobs[i].input.size_bytes());
        }
        output_at[i] = out_bytes;
        out_bytes += align16(jobs[i].output.size_bytes());
    }
    auto* dx = static_cast<std::uint8_t*>(device_buffer(0, in_bytes));
    auto* dy = static_cast<std::uint8_t*>(device_buffer(1, out_bytes));
    auto* dstatus = static_cast<unsigned*>(device_buffer(2, 256));
    hip_check(hipMemsetAsync(dstatus, 0, sizeof(unsigned), st));
    std::vector<kdq_matvec_job> table(jobs.size());
    for (std::size_t i = 0; i < jobs.size(); ++i) {
        const auto& j = jobs[i];
        bool first_use = true;
        for (std::size_t k = 0; k < i; ++k)
            first_use = first_use && input_at[k] != input_at[i];
        if (first_use)
            hip_check(hipMemcpyAsync(dx + input_at[i], j.input.data(), j.input.size_bytes(),
                                     hipMemcpyHostToDevice, st));
        table[i] = kdq_matvec_job{weights[i]->device,
                                  reinterpret_cast<const float*>(dx + input_at[i]),
                                  reinterpret_cast<float*>(dy + output_at[i]),
                                  dstatus,
                                  weights[i]->row_bytes,
                                  j.out,
                                  std::uint32_t(j.in),
                                  std::uint32_t(j.out),
                                  std::uint32_t(j.input.size() / j.in),
                                  types[i]};
    }
    require(!cancel.load(), "kdq_cancelled");
    // Jobs of more than gguf_batch_rows rows over packed Q4_K / Q8_0 / Q6_K (routed experts
    // at prefill) run the GEMM, one launch each; the rest go in one submission per layout
    // (jobs keep their order within each; every job writes its own output region).
    // (GEMM jobs over row-major rows, the other encodings, run kdq_gemm_rows)
    std::vector<kdq_matvec_job> packed_jobs, row_jobs, gemm_jobs, rows_gemm_jobs;
    for (std::size_t i = 0; i < jobs.size(); ++i) {
        const bool packed = weights[i]->packed;
        const bool gemm = jobs[i].encoding &&
                          gemm_takes(*jobs[i].encoding, jobs[i].in, table[i].rows, packed);
        const bool rows_gemm =
            jobs[i].encoding && rows_gemm_takes(*jobs[i].encoding, jobs[i].in, table[i].rows,
                                                packed);
        (gemm        ? gemm_jobs
         : rows_gemm ? rows_gemm_jobs
         : packed    ? packed_jobs
                     : row_jobs)
            .push_back(table[i]);
    }
    for (const auto& j : gemm_jobs)
        kdq_check(kdq_gemm_packed(j.encoding, j.weights, j.columns, j.in, j.input, j.rows,
                                  j.output, dstatus, st));
    for (const auto& j : rows_gemm_jobs)
        kdq_check(kdq_gemm_rows(j.encoding, j.weights, j.row_bytes, j.columns, j.in, j.input,
                                j.rows, j.output, dstatus, st));
    if (!packed_jobs.empty())
        kdq_check(kdq_gemv_packed_batch(packed_jobs.data(), packed_jobs.size(), st));
    if (!row_jobs.empty())
        kdq_check(kdq_gemv_batch(row_jobs.data(), row_jobs.size(), st));
    unsigned status = 0;
    hip_check(hipMemcpyAsync(&status, dstatus, sizeof status, hipMemcpyDeviceToHost, st));
    synchronize();
    if ((!gemm_jobs.empty() || !rows_gemm_jobs.empty()) && (status & 2u) && !(status & 1u)) {
        // a dequantised weight past the fp16 range: the GEMM jobs again, decode-time
        hip_check(hipMemsetAsync(dstatus, 0, sizeof(unsigned), st));
        if (!gemm_jobs.empty())
            kdq_check(kdq_gemv_packed_batch(gemm_jobs.data(), gemm_jobs.size(), st));
        if (!rows_gemm_jobs.empty())
            kdq_check(kdq_gemv_batch(rows_gemm_jobs.data(), rows_gemm_jobs.size(), st));
        hip_check(hipMemcpyAsync(&status, dstatus, sizeof status, hipMemcpyDeviceToHost, st));
    }
    for (std::size_t i = 0; i < jobs.size(); ++i)
        hip_check(hipMemcpyAsync(jobs[i].output.data(), dy + output_at[i],
                                 jobs[i].output.size_bytes(), hipMemcpyDeviceToHost, st));
    synchronize();
    require(status == 0, "kdq_nonfinite_weight");
    return ProjectionResult::unvalidated;
}

ProjectionResult HipDenseCompute::dense_gguf_q8_source(
    const WeightIdentity& identity, gguf::Encoding enc, const GgufWeightSource& source,
    std::span<const std::uint16_t> input, std::size_t in, std::size_t out,
    std::span<std::uint16_t> output, const std::atomic_bool& cancel) {
    std::lock_guard<std::mutex> lock(mutex_);
    if (enc != gguf::Encoding::q4_0 || !in || in % 256)
        return ProjectionResult::unsupported;
    require(!cancel.load(), "kdq_cancelled");
    require(out && in <= std::size_t(INT_MAX) && out <= std::size_t(INT_MAX) && !input.empty() &&
                input.size() % in == 0 && output.size() == input.size() / in * out,
            "kdq_projection_shape");
    require(!overlap(output, input), "kdq_alias");
    hip_check(hipSetDevice(device_));
    const std::size_t rows = input.size() / in;
    std::unique_ptr<Resident> transient;
    // the same resident copy (tile-packed when the decode product takes it) serves both
    const Resident& w = *weights_for(identity, ggml_type(enc), in, out, source, true, cancel,
                                     transient, true);
    auto st = static_cast<hipStream_t>(stream_);
    auto* dx = static_cast<std::uint16_t*>(device_buffer(0, input.size_bytes()));
    auto* dy = static_cast<std::uint16_t*>(device_buffer(1, output.size_bytes()));
    hip_check(hipMemcpyAsync(dx, input.data(), input.size_bytes(), hipMemcpyHostToDevice, st));
    if (w.packed)
        kdq_check(kdq_gemm_q4_0_packed(w.device, out, in, dx, rows, dy, st));
    else
        kdq_check(kdq_gemm_q4_0(w.device, out, in, dx, rows, dy, st));
    hip_check(hipMemcpyAsync(output.data(), dy, output.size_bytes(), hipMemcpyDeviceToHost, st));
    synchronize();
    return ProjectionResult::unvalidated;
}

ProjectionResult HipDenseCompute::moe_mxfp4(const Mxfp4Experts& e,
                                            std::span<const std::uint16_t> x,
                                            std::span<const float> logits, std::size_t tokens,
                                            std::size_t top_k, std::span<float> output,
                                            std::span<std::int32_t> selected,
                                            std::span<float> weights,
                                            const std::atomic_bool& cancel) {
    std::lock_guard<std::mutex> lock(mutex_);
    if (!e.identity || !e.experts || e.experts > 256 || !e.hidden || !e.inter ||
        e.hidden % 64 || e.inter % 64 || !top_k || top_k > 8 || top_k > e.experts || !tokens)
        return ProjectionResult::unsupported;
    require(!cancel.load(), "kdq_cancelled");
    const std::size_t E = e.experts, H = e.hidden, I = e.inter;
    require(e.gate_blocks.size() == E * I * H / 2 && e.up_blocks.size() == E * I * H / 2 &&
                e.gate_scales.size() == E * I * H / 32 && e.up_scales.size() == E * I * H / 32 &&
                e.down_blocks.size() == E * H * I / 2 && e.down_scales.size() == E * H * I / 32 &&
                x.size() == tokens * H && logits.size() == tokens * E &&
                output.size() == tokens * H &&
                (selected.empty() || selected.size() == tokens * top_k) &&
                (weights.empty() || weights.size() == tokens * top_k),
            "kdq_projection_shape");
    for (float v : logits)
        require(std::isfinite(v), "kdq_nonfinite_input");
    require(!overlap(output, x) && !overlap(output, logits), "kdq_alias");
    hip_check(hipSetDevice(device_));
    auto st = static_cast<hipStream_t>(stream_);
    // The expert set lives in the bank as one allocation in the packed layout of
    // kdq_moe_mxfp4_pack: gate, up, down, each 256-byte aligned.
    const std::span<const std::uint8_t> parts[6] = {e.gate_blocks, e.gate_scales, e.up_blocks,
                                                    e.up_scales,   e.down_blocks, e.down_scales};
    const std::size_t gu = (kdq_moe_mxfp4_packed_bytes(E, I, H) + 255) & ~std::size_t(255);
    const std::size_t dn = (kdq_moe_mxfp4_packed_bytes(E, H, I) + 255) & ~std::size_t(255);
    const BankKey key{*e.identity, -1, H, I * E};
    auto it = bank_.find(key);
    if (it == bank_.end()) {
        for (int i : {1, 3, 5})  // IW/src/weights/quantization.cpp:51-53: 255 is not a scale
            for (std::uint8_t s : parts[i])
                require(s != 255, "kdq_invalid_block_scale");
        auto r = std::make_unique<Resident>();
        r->bytes = 2 * gu + dn;
        hip_check(hipMalloc(&r->device, r->bytes));
        // the six arrays pass through one temporary device copy in the GPT-OSS layout
        std::size_t at[6], total = 0;
        for (int i = 0; i < 6; ++i) {
            at[i] = total;
            total += (parts[i].size() + 255) & ~std::size_t(255);
        }
        Resident raw;
        raw.bytes = total;
        hip_check(hipMalloc(&raw.device, total));
        auto* src = static_cast<std::uint8_t*>(raw.device);
        auto* dst = static_cast<std::uint8_t*>(r->device);
        for (int i = 0; i < 6; ++i)
            hip_check(hipMemcpyAsync(src + at[i], parts[i].data(), parts[i].size(),
                                     hipMemcpyHostToDevice, st));
        kdq_check(kdq_moe_mxfp4_pack(src + at[0], src + at[1], E, I, H, dst, st));
        kdq_check(kdq_moe_mxfp4_pack(src + at[2], src + at[3], E, I, H, dst + gu, st));
        kdq_check(kdq_moe_mxfp4_pack(src + at[4], src + at[5], E, H, I, dst + 2 * gu, st));
        synchronize();
        it = bank_.emplace(key, std::move(r)).first;
    }
    auto* base = static_cast<const std::uint8_t*>(it->second->device);
    auto* dx = static_cast<std::uint16_t*>(device_buffer(0, align16(x.size_bytes()) + logits.size_bytes()));
    auto* dl = reinterpret_cast<float*>(reinterpret_cast<std::uint8_t*>(dx) + align16(x.size_bytes()));
    auto* dy = static_cast<float*>(device_buffer(1, output.size_bytes()));
    auto* route = static_cast<std::uint8_t*>(device_buffer(3, align16(tokens * top_k * 4) * 2));
    auto* didx = reinterpret_cast<std::int32_t*>(route);
    auto* dw = reinterpret_cast<float*>(route + align16(tokens * top_k * 4));
    hip_check(hipMemcpyAsync(dx, x.data(), x.size_bytes(), hipMemcpyHostToDevice, st));
    hip_check(hipMemcpyAsync(dl, logits.data(), logits.size_bytes(), hipMemcpyHostToDevice, st));
    kdq_check(kdq_moe_mxfp4_packed(dx, dl, tokens, H, I, E, top_k, base, base + gu,
                                   base + 2 * gu, dy, didx, dw, nullptr, nullptr, st));
    hip_check(hipMemcpyAsync(output.data(), dy, output.size_bytes(), hipMemcpyDeviceToHost, st));
    if (!selected.empty())
        hip_check(hipMemcpyAsync(selected.data(), didx, selected.size_bytes(),
                                 hipMemcpyDeviceToHost, st));
    if (!weights.empty())
        hip_check(hipMemcpyAsync(weights.data(), dw, weights.size_bytes(), hipMemcpyDeviceToHost, st));
    synchronize();
    for (float v : output)
        if (!std::isfinite(v))
            return ProjectionResult::unvalidated;
    return ProjectionResult::finite;
}

std::size_t HipDenseCompute::release_weights(std::span<const WeightIdentity> identities) {
    std::lock_guard<std::mutex> lock(mutex_);
    synchronize();
    std::size_t freed = 0;
    for (auto it = bank_.begin(); it != bank_.end();) {
        const bool retire = std::find(identities.begin(), identities.end(),
                                      std::get<0>(it->first)) != identities.end();
        if (retire) {
            freed += it->second->bytes;
            it = bank_.erase(it);
        } else {
            ++it;
        }
    }
    return freed;
}

std::size_t HipDenseCompute::retained_weight_bytes() const {
    std::lock_guard<std::mutex> lock(mutex_);
    std::size_t total = 0;
    for (const auto& [key, r] : bank_)
        total += r->bytes;
    return total;
}

void HipDenseCompute::release_scratch() {
    std::lock_guard<std::mutex> lock(mutex_);
    synchronize();
    for (auto& b : buffers_) {
        if (b.first)
            hip_check(hipFree(b.first));
        b = {nullptr, 0};
    }
    kdq_check(kdq_release_scratch());
}

}  // namespace kadan_amd
