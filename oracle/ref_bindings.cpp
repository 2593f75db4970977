// C bindings over the COMPILED REFERENCE (test infrastructure only).
//
// oracle/Makefile compiles this file together with the reference's own sources
// where they lie under /root/reference (vendored ggml, kadan's quantization.cpp and
// cpu_matvec.cpp) into oracle/_ref/libkadan_ref.so.  Nothing here restates the
// reference: every function forwards to the reference's code, so tests can pin
// the oracle restatement (oracle.c) against it and bench.py can time the real
// reference CPU path.  Only tests/, tests/golden/ and bench.py's cpu_baseline leg
// may load the resulting library.
//
// One exception: kdr_moe_route.  The reference's router only runs inside
// MoeLayer::forward (IW/src/models/text/qwen_layers.cpp:397-425), which needs a GGUF
// file and a DenseCompute to construct; so kdr_moe_route states the same steps with
// the same standard-library calls (std::max_element, float std::exp, a double total,
// std::partial_sort with the p[a] > p[b] comparator over std::iota indices).  Its
// point is that std::partial_sort is the C++ library's own, so the order it gives
// equal probabilities is the order the reference gets.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <numeric>
#include <cstring>
#include <exception>
#include <span>
#include <stdexcept>
#include <thread>
#include <vector>

#include <ggml-cpu.h>
#include <ggml.h>

#include "cpu_matvec.hpp"
#include "kadan/gguf_quantization.hpp"
#include "kadan/quantization.hpp"

extern "C" {

// ggml_fp16_to_fp32 (G/src/ggml.c).
float kdr_half_to_float(uint16_t bits) {
    return ggml_fp16_to_fp32(ggml_fp16_t(bits));
}

// ggml to_float of one row (G/src/ggml-quants.c dequantize_row_*).
int kdr_ggml_to_float(int type, const void* row, int64_t n, float* out) {
    const auto* traits = ggml_get_type_traits(ggml_type(type));
    if (!traits || !traits->to_float || n % traits->blck_size)
        return -1;
    traits->to_float(row, out, n);
    return 0;
}

// kadan::gguf::decode (IW/include/kadan/gguf_quantization.hpp:631-762); -1 when
// the GGML type has no kadan encoding (Q4_0 has none).
int kdr_kadan_decode_block(int type, const unsigned char* block, float* out) {
    const auto encoding = kadan::gguf::encoding(std::uint32_t(type));
    if (!encoding)
        return -1;
    for (std::size_t i = 0; i < kadan::gguf::block_values(*encoding); ++i)
        out[i] = kadan::gguf::decode(*encoding, block, i);
    return 0;
}

// ggml-cpu from_float of the dot type (x86 quantize_row_q8_0 / quantize_row_q8_K).
int kdr_quantize_row(int type, const float* x, void* y, int64_t n) {
    ggml_cpu_init();
    const auto* traits = ggml_get_type_traits_cpu(ggml_type(type));
    if (!traits || !traits->from_float)
        return -1;
    traits->from_float(x, y, n);
    return 0;
}

// ggml-cpu vec_dot of a weight type against its dot type (x86 AVX2 kernels).
int kdr_vec_dot(int type, int n, const void* weights, const void* activations, float* out) {
    ggml_cpu_init();
    const auto* traits = ggml_get_type_traits_cpu(ggml_type(type));
    if (!traits || !traits->vec_dot)
        return -1;
    traits->vec_dot(n, out, 0, weights, 0, activations, 0, 1);
    return 0;
}

// kadan::text::CpuMatvec (IW/src/models/text/cpu_matvec.cpp:28-66) over 64-output-
// column units on `threads` workers, the split of GgufWeights::project
// (IW/src/models/text/gguf_weights.cpp:400-446).  y is [rows x out].
int kdr_cpu_matvec(int type, const void* weights, size_t row_bytes, const float* x,
                   size_t rows, size_t in, size_t out, float* y, int threads) {
    try {
        const kadan::text::CpuMatvec product(
            std::uint32_t(type), std::span<const float>(x, rows * in), in
        );
        std::span<float> output(y, rows * out);
        constexpr std::size_t unit = 64;
        const std::size_t units = (out + unit - 1) / unit;
        std::atomic<std::size_t> next{0};
        std::atomic<bool> failed{false};
        auto work = [&] {
            try {
                for (std::size_t u; (u = next.fetch_add(1)) < units;)
                    product.run(
                        static_cast<const std::byte*>(weights), row_bytes, u * unit,
                        std::min(out, (u + 1) * unit), output, out
                    );
            } catch (...) {
                failed = true;
            }
        };
        std::vector<std::thread> pool;
        for (int t = 1; t < threads; ++t)
            pool.emplace_back(work);
        work();
        for (auto& t : pool)
            t.join();
        return failed ? -2 : 0;
    } catch (...) {
        return -1;
    }
}

// kadan::quantization::e2m1 (IW/src/weights/quantization.cpp:102-110).
float kdr_e2m1(uint8_t code) {
    return kadan::quantization::e2m1(code);
}

// kadan::quantization::decode_rows for MXFP4 (IW/src/weights/quantization.cpp:193-205).
// Returns 0, -1 on invalid_argument, -2 on overflow_error, -3 otherwise.
int kdr_mxfp4_decode_rows(const uint8_t* blocks, const uint8_t* scales, size_t rows,
                          size_t cols, float* out) {
    try {
        const kadan::quantization::Matrix m{
            kadan::quantization::Encoding::mxfp4, rows, cols,
            std::span<const std::uint8_t>(blocks, rows * (cols / 2)),
            std::span<const std::uint8_t>(scales, rows * (cols / 32)), {}
        };
        const auto values = kadan::quantization::decode_rows(m, 0, rows, rows * cols * 4);
        std::memcpy(out, values.data(), values.size() * sizeof(float));
        return 0;
    } catch (const std::invalid_argument&) {
        return -1;
    } catch (const std::overflow_error&) {
        return -2;
    } catch (...) {
        return -3;
    }
}

// kadan::quantization::matvec for MXFP4 (IW/src/weights/quantization.cpp:207-247).
int kdr_mxfp4_matvec(const uint8_t* blocks, const uint8_t* scales, size_t rows, size_t cols,
                     const float* x, float* y) {
    try {
        const kadan::quantization::Matrix m{
            kadan::quantization::Encoding::mxfp4, rows, cols,
            std::span<const std::uint8_t>(blocks, rows * (cols / 2)),
            std::span<const std::uint8_t>(scales, rows * (cols / 32)), {}
        };
        kadan::quantization::matvec(
            m, std::span<const float>(x, cols), std::span<float>(y, rows)
        );
        return 0;
    } catch (const std::invalid_argument&) {
        return -1;
    } catch (const std::overflow_error&) {
        return -2;
    } catch (...) {
        return -3;
    }
}

// Routing as the reference's MoeLayer::forward computes it (qwen_layers.cpp:397-425),
// with the C++ library's std::partial_sort choosing and ordering the experts.
void kdr_moe_route(const float* logits, size_t tokens, size_t experts, size_t top_k,
                   int32_t* idx, float* w) {
    std::vector<float> p(experts);
    std::vector<std::size_t> order(experts);
    for (std::size_t t = 0; t < tokens; ++t) {
        const float* l = logits + t * experts;
        const float top = *std::max_element(l, l + experts);
        double total = 0;
        for (std::size_t e = 0; e < experts; ++e) {
            p[e] = std::exp(l[e] - top);
            total += p[e];
        }
        for (auto& v : p)
            v = float(v / total);
        std::iota(order.begin(), order.end(), std::size_t{0});
        std::partial_sort(order.begin(), order.begin() + top_k, order.end(),
                          [&](std::size_t a, std::size_t b) { return p[a] > p[b]; });
        float sum = 0;
        for (std::size_t i = 0; i < top_k; ++i) {
            idx[t * top_k + i] = int32_t(order[i]);
            sum += w[t * top_k + i] = p[order[i]];
        }
        sum = std::max(sum, 6.103515625e-5f);
        for (std::size_t i = 0; i < top_k; ++i)
            w[t * top_k + i] /= sum;
    }
}
}
