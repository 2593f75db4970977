// The single-precision exponential of glibc (2.27 and later), restated so that device
// code reproduces the host library bit for bit.  The reference's router takes
// std::exp(float) (IW/src/models/text/qwen_layers.cpp:404-408; IW =
// services/hikari/inference_worker), which is glibc's expf; routing picks experts by
// comparing those values, so a one-ulp difference can reorder near-equal experts.
//
// Algorithm (glibc sysdeps/ieee754/flt-32/e_expf.c, from ARM's optimized-routines by
// Szabolcs Nagy): with N = 32, z = x * N / ln2 is split as k + r (k the nearest integer,
// by adding and subtracting 1.5 * 2^52), 2^(k/N) comes from a 32-entry table of
// 2^(i/N) with k / N folded into the exponent bits, and 2^(r/N) from a cubic in r; all in
// double, rounded once to float.  The x86-64 build runs its FMA variant on CPUs with FMA
// (glibc's ifunc picks __expf_fma): the range reduction is then contracted, z + 1.5 * 2^52
// and z - kd each one fused multiply-add of (N / ln2) * x, and so is the cubic.  This
// restatement equals that glibc's expf on every float (checked exhaustively on the host
// against the installed library).  Without the fused range
// reduction two inputs differ (-0x1.f8cbb2p5 is one).
//
// The includer defines KDQ_EXPF_FN (for example `__device__ __forceinline__` in HIP
// code, `inline` in host code) and provides uint32_t / uint64_t and
// fma(double, double, double); the header may be included inside a namespace.
#pragma once

namespace kdq_expf {

// 2^(i/32) rounded to the nearest double, minus i << 47 (the i/32 that k / N adds to
// the exponent field when k's low five bits index the table).
constexpr uint64_t kTable[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};
constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;  // N / ln2
constexpr double kShift = 0x1.8p+52;                       // rounds z to an integer
// the cubic for 2^(r/N): ln2^3/6, ln2^2/2 and ln2 as fitted by the library, over N^3, N^2, N
constexpr double kC0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;

}  // namespace kdq_expf

// glibc_expf with the table of 2^(i/32) read from `table` (kdq_expf::kTable or a copy of
// it, e.g. in LDS, where a latency-bound caller has staged it ahead of time).
KDQ_EXPF_FN float glibc_expf_with(float x, const uint64_t* table) {
    using namespace kdq_expf;
    // the general path for every input, then the library's special cases chosen by
    // selection (no branches: a taken branch costs a latency-bound wavefront tens of
    // clocks); outside the range the general path's value is discarded
    const uint32_t bits = __builtin_bit_cast(uint32_t, x);
    const uint32_t top = (bits >> 20) & 0x7ffu;
    const double xd = double(x);
    double kd = fma(kInvLn2N, xd, kShift);
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= kShift;
    const double r = fma(kInvLn2N, xd, -kd);
    const double s = __builtin_bit_cast(double, table[ki % 32] + (ki << 47));
    const double z = fma(kC0, r, kC1);
    const double r2 = r * r;
    double y = fma(kC2, r, 1.0);
    y = fma(z, r2, y);
    float result = float(y * s);
    // |x| >= 88 (top 12 bits of 88.0f), or x is not finite
    const bool large = top >= 0x42bu;
    result = large && x < -0x1.9fe368p6f ? 0.0f : result;            // below log(2^-150)
    result = large && x > 0x1.62e42ep6f ? __builtin_inff() : result;  // past log(2^128)
    result = top >= 0x7f8u ? x + x : result;                          // +inf, NaN
    result = bits == 0xff800000u ? 0.0f : result;                     // -inf
    return result;
}

KDQ_EXPF_FN float glibc_expf(float x) {
    return glibc_expf_with(x, kdq_expf::kTable);
}
