// Host check of glibc_expf (kadan_amd/csrc/kdq_expf.hpp, the restatement the device
// router runs) against the installed C library's expf: every one of the 2^32 float bit
// patterns (zeros, subnormals, the overflow and underflow ranges, infinities and NaNs
// included).  Prints the number of inputs whose result bits differ and the first few;
// exit status 1 if any.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

using std::fma;
#define KDQ_EXPF_FN inline
#include "../../kadan_amd/csrc/kdq_expf.hpp"

static uint32_t bits_of(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}

int main() {
    // every bit pattern: [+0, +NaN with all payload bits] and [-0, -NaN with all]
    const uint64_t ranges[2][2] = {{0x00000000u, 0x7fffffffu}, {0x80000000u, 0xffffffffu}};
    const unsigned workers = std::max(1u, std::thread::hardware_concurrency());
    std::vector<uint64_t> bad(workers, 0);
    std::vector<uint32_t> first(workers, 0);
    std::vector<std::thread> team;
    uint64_t total = 0;
    for (auto& r : ranges)
        total += r[1] - r[0] + 1;
    for (unsigned w = 0; w < workers; ++w)
        team.emplace_back([&, w] {
            for (auto& r : ranges) {
                const uint64_t n = r[1] - r[0] + 1;
                for (uint64_t i = r[0] + w * n / workers; i < r[0] + (w + 1) * n / workers; ++i) {
                    float x;
                    const uint32_t u = uint32_t(i);
                    std::memcpy(&x, &u, 4);
                    if (bits_of(glibc_expf(x)) != bits_of(expf(x))) {
                        if (!bad[w])
                            first[w] = u;
                        ++bad[w];
                    }
                }
            }
        });
    for (auto& t : team)
        t.join();
    uint64_t mismatches = 0;
    for (unsigned w = 0; w < workers; ++w) {
        mismatches += bad[w];
        if (bad[w])
            std::printf("first mismatch of worker %u: 0x%08x\n", w, first[w]);
    }
    std::printf("%llu inputs, %llu mismatches\n", (unsigned long long)total,
                (unsigned long long)mismatches);
    return mismatches ? 1 : 0;
}
