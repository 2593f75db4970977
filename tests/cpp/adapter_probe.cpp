// Calls the DenseCompute adapter of the integration guide's section 1 through the reference's
// own interface type, kadan::DenseCompute (IW/include/kadan/dense_compute.hpp:60-342;
// IW = services/hikari/inference_worker), compiled against the reference's headers.
// Test infrastructure: built by tests/cpp/adapter.py where the reference exists.
//
// Exit status: 0 every check passed; 3 no GPU device (construction threw kdq_hip: ...);
// 1 a check failed (the failing check is printed).
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "kadan/dense_compute.hpp"
#include "kadan/gguf_quantization.hpp"

namespace kadan {
std::shared_ptr<DenseCompute> hip_dense_compute(std::shared_ptr<Resources>, std::vector<int>,
                                                Workload);
}

namespace {

int failures = 0;

void check(bool ok, const char* what) {
    std::printf("%s %s\n", ok ? "ok  " : "FAIL", what);
    std::fflush(stdout);
    if (!ok)
        ++failures;
}

struct XorShift {
    std::uint32_t s = 0x2545F491u;
    std::uint32_t operator()() {
        s ^= s << 13;
        s ^= s >> 17;
        s ^= s << 5;
        return s;
    }
    float normal() {  // a sum of uniforms: mean 0, unit-ish spread
        float v = 0;
        for (int i = 0; i < 4; ++i)
            v += float((*this)() & 0xFFFF) / 65536.0f - 0.5f;
        return v;
    }
};

// Packed rows of random blocks whose fp16 scales are small finite values.
std::vector<std::byte> random_rows(kadan::gguf::Encoding enc, std::size_t rows, std::size_t in,
                                   XorShift& rng) {
    const std::size_t bv = kadan::gguf::block_values(enc), bb = kadan::gguf::block_bytes(enc);
    std::vector<std::byte> out(rows * in / bv * bb);
    for (auto& b : out)
        b = std::byte(rng() & 255);
    for (std::size_t blk = 0; blk < out.size() / bb; ++blk) {
        auto* p = out.data() + blk * bb;
        p[1] = std::byte(0x18 + (rng() & 3));  // d: fp16 exponent 6..7 (~1e-3)
        if (enc == kadan::gguf::Encoding::q4_k)
            p[3] = std::byte(0x14 + (rng() & 3));  // dmin
    }
    return out;
}

// y[r][c] = sum_k decode(W[c, k]) * x[r][k] in double, with the reference's decode.
std::vector<double> expected(kadan::gguf::Encoding enc, const std::vector<std::byte>& w,
                             const std::vector<float>& x, std::size_t in, std::size_t out) {
    const std::size_t bv = kadan::gguf::block_values(enc), bb = kadan::gguf::block_bytes(enc);
    const std::size_t rows = x.size() / in;
    std::vector<double> y(rows * out, 0.0);
    for (std::size_t c = 0; c < out; ++c)
        for (std::size_t k = 0; k < in; ++k) {
            const auto* block = reinterpret_cast<const unsigned char*>(w.data()) +
                                (c * (in / bv) + k / bv) * bb;
            const double v = kadan::gguf::decode(enc, block, k % bv);
            for (std::size_t r = 0; r < rows; ++r)
                y[r * out + c] += v * double(x[r * in + k]);
        }
    return y;
}

double rel_l2(const std::vector<float>& got, const std::vector<double>& want) {
    double num = 0, den = 0;
    for (std::size_t i = 0; i < want.size(); ++i) {
        num += (double(got[i]) - want[i]) * (double(got[i]) - want[i]);
        den += want[i] * want[i];
    }
    return std::sqrt(num / (den ? den : 1.0));
}

kadan::WeightIdentity identity(std::uint64_t n) {
    kadan::WeightIdentity id;
    id.inode = n;
    id.payload_end = 1000 + n;
    return id;
}

}  // namespace

int main() {
    std::shared_ptr<kadan::DenseCompute> owner;
    try {
        owner = kadan::hip_dense_compute(nullptr, {0}, kadan::Workload::llm);
    } catch (const std::runtime_error& e) {
        if (std::strncmp(e.what(), "kdq_hip", 7) == 0) {
            std::printf("no device: %s\n", e.what());
            return 3;
        }
        throw;
    }
    kadan::DenseCompute& dc = *owner;  // only the reference's interface from here on
    const std::atomic_bool cancel{false};
    XorShift rng;
    check(dc.supports_weight_sources(), "supports_weight_sources");

    // 1. unsupported before the source is read: in is not a whole number of blocks
    {
        bool read = false;
        const kadan::DenseCompute::GgufWeightSource source = [&](std::size_t,
                                                                  std::span<std::byte>) {
            read = true;
        };
        std::vector<float> x(100, 1.0f), y(4, -7.0f);
        const auto r = dc.dense_gguf_source(identity(1), kadan::gguf::Encoding::q4_k, source,
                                            {}, x, 100, 4, y, cancel);
        check(r == kadan::ProjectionResult::unsupported && !read && y[0] == -7.0f,
              "unsupported shape: no source read, no output write");
    }

    // 2. Q4_K through dense_gguf_source, 3 rows x 512 -> 40, with bias
    const std::size_t in = 512, out = 40, rows = 3;
    const auto wq = random_rows(kadan::gguf::Encoding::q4_k, out, in, rng);
    const std::size_t row_bytes = in / 256 * 144;
    std::size_t reads = 0;
    const kadan::DenseCompute::GgufWeightSource q4k = [&](std::size_t first,
                                                         std::span<std::byte> dst) {
        ++reads;
        std::memcpy(dst.data(), wq.data() + first * row_bytes, dst.size());
    };
    std::vector<float> x(rows * in), bias(out), y(rows * out);
    for (auto& v : x)
        v = rng.normal();
    for (auto& v : bias)
        v = rng.normal();
    auto want = expected(kadan::gguf::Encoding::q4_k, wq, x, in, out);
    for (std::size_t r = 0; r < rows; ++r)
        for (std::size_t c = 0; c < out; ++c)
            want[r * out + c] += bias[c];
    auto result = dc.dense_gguf_source(identity(2), kadan::gguf::Encoding::q4_k, q4k, bias, x, in,
                                       out, y, cancel);
    check(result == kadan::ProjectionResult::finite, "q4_k dense_gguf_source finite");
    check(rel_l2(y, want) < 1e-4, "q4_k dense_gguf_source matches the reference decode");
    const std::size_t first_reads = reads;
    result = dc.dense_gguf_source(identity(2), kadan::gguf::Encoding::q4_k, q4k, bias, x, in, out,
                                  y, cancel);
    check(reads == first_reads && rel_l2(y, want) < 1e-4, "bank hit reads nothing");

    // 3. two Q8_0 jobs in one dense_gguf_batch, sharing the input
    {
        const std::size_t o1 = 24, o2 = 56;
        const auto w1 = random_rows(kadan::gguf::Encoding::q8_0, o1, in, rng);
        const auto w2 = random_rows(kadan::gguf::Encoding::q8_0, o2, in, rng);
        const std::size_t rb = in / 32 * 34;
        const kadan::DenseCompute::GgufWeightSource s1 = [&](std::size_t f,
                                                            std::span<std::byte> d) {
            std::memcpy(d.data(), w1.data() + f * rb, d.size());
        };
        const kadan::DenseCompute::GgufWeightSource s2 = [&](std::size_t f,
                                                            std::span<std::byte> d) {
            std::memcpy(d.data(), w2.data() + f * rb, d.size());
        };
        std::vector<float> xb(in), y1(o1), y2(o2);
        for (auto& v : xb)
            v = rng.normal();
        const auto id1 = identity(3), id2 = identity(4);
        const kadan::DenseCompute::GgufBatchJob jobs[2] = {
            {&id1, kadan::gguf::Encoding::q8_0, &s1, xb, in, o1, y1, true},
            {&id2, kadan::gguf::Encoding::q8_0, &s2, xb, in, o2, y2, false}};
        const auto r = dc.dense_gguf_batch(jobs, cancel);
        check(r == kadan::ProjectionResult::unvalidated, "q8_0 dense_gguf_batch unvalidated");
        check(rel_l2(y1, expected(kadan::gguf::Encoding::q8_0, w1, xb, in, o1)) < 1e-4 &&
                  rel_l2(y2, expected(kadan::gguf::Encoding::q8_0, w2, xb, in, o2)) < 1e-4,
              "q8_0 dense_gguf_batch matches the reference decode");
    }

    // 4. the pure virtual dense(): F32 weights, in = 37 (padded inside), bias
    {
        const std::size_t fin = 37, fout = 5, frows = 2;
        std::vector<float> w(fout * fin), fx(frows * fin), fb(fout), fy(frows * fout);
        for (auto& v : w)
            v = rng.normal();
        for (auto& v : fx)
            v = rng.normal();
        for (auto& v : fb)
            v = rng.normal();
        std::vector<double> fw(frows * fout);
        for (std::size_t r = 0; r < frows; ++r)
            for (std::size_t c = 0; c < fout; ++c) {
                double s = fb[c];
                for (std::size_t k = 0; k < fin; ++k)
                    s += double(w[c * fin + k]) * double(fx[r * fin + k]);
                fw[r * fout + c] = s;
            }
        dc.dense(w, fb, fx, fin, fout, fy, cancel);
        check(rel_l2(fy, fw) < 1e-6, "dense (F32) matches the double product");
    }

    // 5. MoeLayer::forward's first batch (IW/src/models/text/qwen_layers.cpp:383-389) in the
    // job form GgufWeights::project builds (IW/src/models/text/gguf_weights.cpp:456-466):
    // the F32 router ffn_gate_inp (no encoding, F32 rows from a byte source) and the Q8_0
    // shared gate and up, all three on the same input rows
    {
        const std::size_t hidden = 256, experts = 16, shared_ff = 96, mrows = 2;
        std::vector<float> router(experts * hidden), xm(mrows * hidden);
        for (auto& v : router)
            v = rng.normal() * 0.1f;
        for (auto& v : xm)
            v = rng.normal();
        const auto wg = random_rows(kadan::gguf::Encoding::q8_0, shared_ff, hidden, rng);
        const auto wu = random_rows(kadan::gguf::Encoding::q8_0, shared_ff, hidden, rng);
        const std::size_t rb = hidden / 32 * 34, fb = hidden * sizeof(float);
        std::size_t router_reads = 0;
        const kadan::DenseCompute::GgufWeightSource rs = [&](std::size_t f,
                                                            std::span<std::byte> d) {
            ++router_reads;
            std::memcpy(d.data(), reinterpret_cast<const std::byte*>(router.data()) + f * fb,
                        d.size());
        };
        const kadan::DenseCompute::GgufWeightSource gs = [&](std::size_t f,
                                                            std::span<std::byte> d) {
            std::memcpy(d.data(), wg.data() + f * rb, d.size());
        };
        const kadan::DenseCompute::GgufWeightSource us = [&](std::size_t f,
                                                            std::span<std::byte> d) {
            std::memcpy(d.data(), wu.data() + f * rb, d.size());
        };
        std::vector<float> logits(mrows * experts), gate(mrows * shared_ff),
            up(mrows * shared_ff);
        const auto ir = identity(20), ig = identity(21), iu = identity(22);
        const kadan::DenseCompute::GgufBatchJob jobs[3] = {
            {&ir, std::nullopt, &rs, xm, hidden, experts, logits, true},
            {&ig, kadan::gguf::Encoding::q8_0, &gs, xm, hidden, shared_ff, gate, true},
            {&iu, kadan::gguf::Encoding::q8_0, &us, xm, hidden, shared_ff, up, true}};
        const auto r = dc.dense_gguf_batch(jobs, cancel);
        check(r != kadan::ProjectionResult::unsupported, "moe first batch (F32 router) accepted");
        std::vector<double> want(mrows * experts, 0.0);
        for (std::size_t t = 0; t < mrows; ++t)
            for (std::size_t e = 0; e < experts; ++e)
                for (std::size_t k = 0; k < hidden; ++k)
                    want[t * experts + e] += double(router[e * hidden + k]) *
                                             double(xm[t * hidden + k]);
        check(rel_l2(logits, want) < 1e-6, "F32 router job matches the double product");
        check(rel_l2(gate, expected(kadan::gguf::Encoding::q8_0, wg, xm, hidden, shared_ff)) <
                      1e-4 &&
                  rel_l2(up, expected(kadan::gguf::Encoding::q8_0, wu, xm, hidden, shared_ff)) <
                      1e-4,
              "shared gate/up jobs match the reference decode");

        // the caller's fallback for an F32 tensor: dense_source over a FloatWeightSource
        // whose offsets are elements (first row * in), here on a fresh identity
        std::size_t float_reads = 0;
        const kadan::DenseCompute::FloatWeightSource fs = [&](std::size_t first,
                                                             std::span<float> d) {
            ++float_reads;
            std::memcpy(d.data(), router.data() + first, d.size_bytes());
        };
        std::vector<float> ls(mrows * experts, -1.0f);
        const auto r2 = dc.dense_source(identity(23), fs, {}, xm, hidden, experts, ls, cancel);
        check(r2 == kadan::ProjectionResult::finite && float_reads > 0 &&
                  rel_l2(ls, want) < 1e-6,
              "dense_source (F32 source) matches the double product");
        const std::size_t seen = float_reads;
        dc.dense_source(identity(23), fs, {}, xm, hidden, experts, ls, cancel);
        check(float_reads == seen && rel_l2(ls, want) < 1e-6, "dense_source bank hit reads nothing");

        // an F32 dense_source of any width (rows zero-padded on the device)
        const std::size_t odd = 37;
        std::vector<float> wodd(experts * odd), xo(mrows * odd), yo(mrows * experts);
        for (auto& v : wodd)
            v = rng.normal();
        for (auto& v : xo)
            v = rng.normal();
        const kadan::DenseCompute::FloatWeightSource os = [&](std::size_t first,
                                                             std::span<float> d) {
            std::memcpy(d.data(), wodd.data() + first, d.size_bytes());
        };
        std::vector<double> wo(mrows * experts, 0.0);
        for (std::size_t t = 0; t < mrows; ++t)
            for (std::size_t e = 0; e < experts; ++e)
                for (std::size_t k = 0; k < odd; ++k)
                    wo[t * experts + e] += double(wodd[e * odd + k]) * double(xo[t * odd + k]);
        dc.dense_source(identity(24), os, {}, xo, odd, experts, yo, cancel);
        check(rel_l2(yo, wo) < 1e-6, "dense_source with in = 37 matches the double product");

        // F32 batch jobs the reference's eligibility refuses (gguf_batch_partition.hpp:32-34):
        // in % 8 != 0, and a row past the 16 MiB staging; no source read, no output write
        std::vector<float> x36(36, 1.0f), y36(1, -7.0f);
        bool read = false;
        const kadan::DenseCompute::GgufWeightSource never = [&](std::size_t,
                                                               std::span<std::byte>) {
            read = true;
        };
        const auto i36 = identity(25);
        const kadan::DenseCompute::GgufBatchJob bad[1] = {
            {&i36, std::nullopt, &never, x36, 36, 1, y36, true}};
        check(dc.dense_gguf_batch(bad, cancel) == kadan::ProjectionResult::unsupported &&
                  !read && y36[0] == -7.0f,
              "F32 batch job with in % 8 != 0: unsupported, no read, no write");
        const std::size_t wide = (std::size_t(16) << 20) / sizeof(float) + 8;
        std::vector<float> xw(wide, 0.0f), yw(1, -7.0f);
        const kadan::DenseCompute::GgufBatchJob big[1] = {
            {&i36, std::nullopt, &never, xw, wide, 1, yw, true}};
        check(dc.dense_gguf_batch(big, cancel) == kadan::ProjectionResult::unsupported &&
                  !read && yw[0] == -7.0f,
              "F32 batch job over 16 MiB per row: unsupported, no read, no write");
        check(router_reads > 0, "router rows were read once for the bank");
    }

    // 6. the bank: retained bytes reported, then released
    const auto before = dc.retained_weights();
    check(before.size() == 2 && before[1] > 0, "retained_weights reports the bank");
    const kadan::WeightIdentity gone[2] = {identity(2), identity(3)};
    check(dc.release_weights(gone) > 0, "release_weights frees the entries");
    dc.release_scratch();
    std::printf("%s\n", failures ? "adapter probe FAILED" : "adapter probe passed");
    return failures ? 1 : 0;
}
