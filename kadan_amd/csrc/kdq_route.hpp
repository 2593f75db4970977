// Expert routing, by one wavefront (route_select) or by a whole workgroup for one token's
// latency (route_select_wg), shared by the MoE layers (moe_mxfp4.hip, and the GGUF
// layer's fused decode in gguf_gemv.hip): the softmax of the reference's
// MoeLayer::forward (IW/src/models/text/qwen_layers.cpp:397-425; IW =
// services/hikari/inference_worker) with the host library's expf and the total in expert
// order, then its std::partial_sort top-k and the renormalised weights.  Included inside
// namespace kdq's anonymous namespace of each translation unit, after kdq_common.hpp.
#pragma once

#define KDQ_EXPF_FN __device__ __forceinline__
#include "kdq_expf.hpp"
#undef KDQ_EXPF_FN

// Routing reductions by DPP row operations (no LDS round trips): within each row of 16
// lanes by pair, quad, half-row and row permutations, then the four rows in a fixed order
// through readlane.  Every lane returns the same bits; all 64 lanes must be active.
template <int CTRL>
__device__ __forceinline__ double dpp_read_double(double v) {
    const unsigned long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, int(b), CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, int(b >> 32), CTRL, 0xf, 0xf, false);
    return __longlong_as_double((static_cast<long long>(hi) << 32) | unsigned(lo));
}

__device__ __forceinline__ double readlane_double(double v, int lane) {
    const unsigned long long b = __double_as_longlong(v);
    const unsigned lo = __builtin_amdgcn_readlane(int(b), lane);
    const unsigned hi = __builtin_amdgcn_readlane(int(b >> 32), lane);
    return __longlong_as_double((static_cast<long long>(hi) << 32) | lo);
}

__device__ __forceinline__ double wave_sum_double(double v) {
    v += dpp_read_double<0xb1>(v);   // quad_perm [1,0,3,2]
    v += dpp_read_double<0x4e>(v);   // quad_perm [2,3,0,1]
    v += dpp_read_double<0x141>(v);  // row_half_mirror
    v += dpp_read_double<0x140>(v);  // row_mirror: every lane holds its row's sum
    return (readlane_double(v, 0) + readlane_double(v, 16)) +
           (readlane_double(v, 32) + readlane_double(v, 48));
}

// Maximum over the 64 lanes of any floats (fmaxf: a NaN loses to a number).
__device__ __forceinline__ float wave_max_rows(float v) {
    v = fmaxf(v, dpp_read<0xb1, 0xf>(v));
    v = fmaxf(v, dpp_read<0x4e, 0xf>(v));
    v = fmaxf(v, dpp_read<0x141, 0xf>(v));
    v = fmaxf(v, dpp_read<0x140, 0xf>(v));
    auto at = [&](int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); };
    return fmaxf(fmaxf(at(0), at(16)), fmaxf(at(32), at(48)));
}

// libstdc++'s std::partial_sort (std::__heap_select, then std::__sort_heap, both over
// std::__adjust_heap: the published binary-heap algorithm) of experts 0..E-1 by
// p[a] > p[b], for the first k, run by a whole wavefront with wave-uniform control:
// heap slot i lives in lane i's register.  Returns lane i's selection (i < k).  Only
// called when probabilities tie or are NaN; otherwise the order is the descending one.
template <class POf>
__device__ __forceinline__ int heap_route(POf p_of, unsigned experts, unsigned k,
                                          unsigned lane) {
    int slot = int(lane);  // order = iota
    auto get = [&](int i) { return __builtin_amdgcn_readlane(slot, i); };
    auto put = [&](int i, int v) {
        if (lane == unsigned(i))
            slot = v;
    };
    auto before = [&](int a, int b) { return p_of(a) > p_of(b); };
    auto adjust = [&](int hole, int len, int value) {
        const int top = hole;
        int child = hole;
        while (child < (len - 1) / 2) {
            child = 2 * (child + 1);
            if (before(get(child), get(child - 1)))
                --child;
            put(hole, get(child));
            hole = child;
        }
        if ((len & 1) == 0 && child == (len - 2) / 2) {
            child = 2 * (child + 1);
            put(hole, get(child - 1));
            hole = child - 1;
        }
        while (hole > top) {
            const int parent = (hole - 1) / 2;
            if (!before(get(parent), value))
                break;
            put(hole, get(parent));
            hole = parent;
        }
        put(hole, value);
    };
    const int len = int(k);
    if (len >= 2)  // make_heap
        for (int parent = (len - 2) / 2; parent >= 0; --parent)
            adjust(parent, len, get(parent));
    for (int i = len; i < int(experts); ++i)  // heap select; position i still holds i
        if (before(i, get(0)))
            adjust(0, len, i);
    for (int last = len - 1; last > 0; --last) {  // sort_heap
        const int value = get(last);
        put(last, get(0));
        adjust(0, last, value);
    }
    return slot;
}

// Token t by one whole wavefront (lane = its lane): lane i < top_k gets the i-th selected
// expert and its renormalised weight.  R probabilities per lane (experts <= 64 R).
// COHERENT reads the logits at device scope (another workgroup of the same launch wrote
// them with device-scope stores).
template <int R, bool COHERENT = false>
__device__ __forceinline__ void route_select_r(const float* __restrict__ logits, unsigned t,
                                               unsigned experts, unsigned top_k, unsigned lane,
                                               int& selected, float& selected_weight) {
    const float* l = logits + size_t(t) * experts;
    float v[R], p[R];
    float maximum = -INFINITY;
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const unsigned e = lane + 64 * j;
        if constexpr (COHERENT)
            v[j] = e < experts ? __hip_atomic_load(l + e, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT)
                               : -INFINITY;
        else
            v[j] = e < experts ? l[e] : -INFINITY;
        maximum = fmaxf(maximum, v[j]);
    }
    maximum = wave_max_rows(maximum);
    auto value_of = [&](const float (&a)[R], unsigned e) {  // a of expert e (wave-uniform)
        const unsigned j = e / 64;
        float aj = a[0];
#pragma unroll
        for (int r = 1; r < R; ++r)
            aj = j == unsigned(r) ? a[r] : aj;
        return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(aj), e % 64));
    };
    // p = the host library's expf (glibc_expf reproduces it bit for bit) and the total in
    // double, summed in expert order as the reference's loop does.  When every p is a
    // multiple of 2^-45 every partial sum is exact (all stay below 2^8), so any order
    // gives that total and one wavefront reduction computes it; otherwise (p below
    // 2^-22 with low bits set, NaN) the wavefront adds them one by one in expert order,
    // e = lane + 64 j, every lane of every register: experts past the last hold +0,
    // which leaves a total that started at +0 unchanged.
    double total = 0.0;
    bool exact = true;
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const unsigned e = lane + 64 * j;
        p[j] = e < experts ? glibc_expf(v[j] - maximum) : 0.f;
        const double scaled = double(p[j]) * 0x1p45;
        exact = exact && scaled == __builtin_trunc(scaled);
        total += double(p[j]);
    }
    if (__ballot(!exact) == 0) {
        total = wave_sum_double(total);
    } else {
        total = 0.0;
#pragma unroll
        for (int j = 0; j < R; ++j)
#pragma unroll
            for (int l = 0; l < 64; ++l)
                total += double(__int_as_float(
                    __builtin_amdgcn_readlane(__float_as_int(p[j]), l)));
    }
#pragma unroll
    for (int j = 0; j < R; ++j)
        p[j] = float(double(p[j]) / total);

    // Selection.  The reference takes the first k of std::partial_sort over experts
    // 0..E-1 by p[a] > p[b] (qwen_layers.cpp:409-416).  When the k largest p are distinct
    // and above every other p, that is simply the k largest in descending order: one DPP
    // maximum and a ballot per register per pick.  Equal probabilities (and NaN ones,
    // which compare false both ways) come out in the order of libstdc++'s heap
    // selection; then the wavefront reruns that heap algorithm (heap_route below).
    bool valid[R];
    bool nan_seen = false;
#pragma unroll
    for (int j = 0; j < R; ++j) {
        valid[j] = lane + 64 * j < experts;
        nan_seen |= __ballot(valid[j] && isnan(p[j])) != 0;
    }
    auto p_of = [&](int e) { return value_of(p, unsigned(e)); };  // p of expert e
    int chosen_e = 0;  // lane i < top_k: the i-th selection
    bool ambiguous = nan_seen;
    if (!nan_seen) {
        unsigned taken = 0;
        float previous = INFINITY;
        for (unsigned i = 0; i <= top_k && i < experts; ++i) {
            float c = 0.f;  // every probability is >= 0 here
#pragma unroll
            for (int j = 0; j < R; ++j)
                if (valid[j] && !((taken >> j) & 1u))
                    c = fmaxf(c, p[j]);
            c = wave_max_nonneg(c);
            ambiguous |= c == previous;  // equal to the last pick: a tie
            previous = c;
            if (i == top_k)
                break;  // only the largest unselected p was needed
            int best = -1;
#pragma unroll
            for (int j = 0; j < R; ++j) {
                const bool open = valid[j] && !((taken >> j) & 1u);
                const unsigned long long hit = __ballot(open && p[j] == c);
                if (best < 0 && hit)
                    best = 64 * j + __builtin_ctzll(hit);
            }
            if (lane == unsigned(best % 64))
                taken |= 1u << (best / 64);
            if (lane == i)
                chosen_e = best;
        }
    }
    if (ambiguous)
        chosen_e = heap_route(p_of, experts, top_k, lane);
    float sum = 0.f, chosen_p = 0.f;
    for (unsigned i = 0; i < top_k; ++i) {  // sequential, in selection order
        const float pi = p_of(__builtin_amdgcn_readlane(chosen_e, i));
        sum += pi;
        if (lane == i)
            chosen_p = pi;
    }
    sum = fmaxf(sum, 6.103515625e-5f);
    selected = chosen_e;
    selected_weight = chosen_p / sum;
}

template <bool COHERENT = false>
__device__ __forceinline__ void route_select(const float* __restrict__ logits, unsigned t,
                                             unsigned experts, unsigned top_k, unsigned lane,
                                             int& selected, float& selected_weight) {
    if (experts <= 64)
        route_select_r<1, COHERENT>(logits, t, experts, top_k, lane, selected, selected_weight);
    else if (experts <= 128)
        route_select_r<2, COHERENT>(logits, t, experts, top_k, lane, selected, selected_weight);
    else
        route_select_r<4, COHERENT>(logits, t, experts, top_k, lane, selected, selected_weight);
}

// LDS of route_select_wg (16-byte aligned, in the caller's LDS).
struct RouteScratch {
    uint64_t exp_table[32];  // kdq_expf::kTable, staged while the logits load
    float p[320];            // expf(v - max) (+0 past the experts)
    float q[320];            // probabilities (NaN past the experts: compares false)
    unsigned rank[256];      // per expert: probabilities above it | equal ones << 16
    double part[16];         // per wavefront: its p total
    float wave_max[16];
    unsigned inexact, ambiguous;
    int sel[64];
    float sel_p[64];
};

// route_select_r's result for one token, bit for bit, computed by a whole workgroup of
// 64 W threads (4 <= W <= 16; experts <= 256, top_k <= KMAX <= 64): thread i < top_k gets
// the i-th selected expert and its renormalised weight.  Thread e takes expert e's
// probability; the total is exact in any order when every p is a multiple of 2^-45, and
// otherwise every wavefront adds the p in expert order.  The selection ranks every expert
// by counting the probabilities above it and equal to it: a task is 64 experts (one a
// lane) against a chunk of 32 probabilities, which every lane of the wavefront reads at
// the same LDS address.  With the top_k + 1 largest distinct, expert e's count is its
// position in the descending order, which is std::partial_sort's; equal or NaN
// probabilities there go to heap_route by wavefront 0.  The code is straight-line where
// it can be (selections rather than branches, loops of fixed length): one wavefront per
// SIMD has nothing to hide a taken branch behind.  Every thread must call it.
template <int W, int KMAX, bool COHERENT>
__device__ __forceinline__ void route_select_wg(const float* __restrict__ logits,
                                                unsigned experts, unsigned top_k,
                                                RouteScratch& s, int& selected,
                                                float& selected_weight) {
    static_assert(W >= 4 && W <= 16 && KMAX <= 64, "route_select_wg: 4..16 waves");
    constexpr unsigned kThreads = W * 64;
    const unsigned t = threadIdx.x, lane = t % 64, wave = t / 64;
    const bool mine = t < experts;
    const float* at = logits + min(t, experts - 1);
    float v;
    if constexpr (COHERENT)
        v = __hip_atomic_load(at, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        v = *at;
    if (t < 32)  // a global load, in flight with the logits
        s.exp_table[t] = kdq_expf::kTable[t];
    v = mine ? v : -INFINITY;
    const float wave_max = wave_max_rows(v);
    if (lane == 0)
        s.wave_max[wave] = wave_max;
    if (t < 256)
        s.rank[t] = 0u;
    if (t == 0) {
        s.inexact = 0u;
        s.ambiguous = 0u;
    }
    __syncthreads();
    // the maximum of a set by fmaxf is the same in any order (up to the sign of a zero,
    // which leaves every v - maximum, and so every p, unchanged)
    float maximum = s.wave_max[0];
#pragma unroll
    for (int i = 1; i < W; ++i)
        maximum = fmaxf(maximum, s.wave_max[i]);
    const float e_v = glibc_expf_with(v - maximum, s.exp_table);
    const float p = mine ? e_v : 0.f;
    const double scaled = double(p) * 0x1p45;
    const bool exact = scaled == __builtin_trunc(scaled);
#pragma unroll
    for (unsigned i = 0; i < 320; i += kThreads)
        if (i + t < 320)
            s.p[i + t] = i == 0 ? p : 0.f;  // +0 past the experts leaves the in-order total
    const double wave_total = wave_sum_double(double(p));
    const bool wave_inexact = __ballot(!exact) != 0;
    if (lane == 0) {
        s.part[wave] = wave_total;
        atomicOr(&s.inexact, wave_inexact ? 1u : 0u);
    }
    __syncthreads();
    double total = s.part[0];
#pragma unroll
    for (int i = 1; i < W; ++i)
        total += s.part[i];  // exact: every partial sum a multiple of 2^-45 below 2^9
    if (s.inexact) {
        // every lane of every wavefront adds the same p in expert order, 64 at a time
        // (reading past the experts adds +0); no barrier needed for the result
        const float4* q4 = reinterpret_cast<const float4*>(s.p);
        double in_order = 0.0;
        for (unsigned b = 0; b < experts; b += 64) {
            float4 f[16];
#pragma unroll
            for (int j = 0; j < 16; ++j)
                f[j] = q4[b / 4 + j];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                in_order += double(f[j].x);
                in_order += double(f[j].y);
                in_order += double(f[j].z);
                in_order += double(f[j].w);
            }
        }
        total = in_order;
    }
    const float pf = float(double(p) / total);
    const bool nan_here = mine && isnan(pf);
#pragma unroll
    for (unsigned i = 0; i < 320; i += kThreads)
        if (i + t < 320)
            s.q[i + t] = i + t < experts ? pf : __builtin_nanf("");
    const bool wave_nan = __ballot(nan_here) != 0;
    if (lane == 0)
        atomicOr(&s.ambiguous, wave_nan ? 1u : 0u);
    __syncthreads();

    // tasks (chunk c of 32 probabilities, experts 64 g .. 64 g + 63), by wavefronts
    const unsigned chunks = (experts + 31) / 32, tasks = chunks * ((experts + 63) / 64);
    for (unsigned task = wave; task < tasks; task += W) {
        const unsigned c = task % chunks, e = (task / chunks) * 64 + lane;
        const float pe = s.q[e];  // NaN past the experts: counts nothing
        const float4* q4 = reinterpret_cast<const float4*>(s.q + 32 * c);
        float4 f[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            f[j] = q4[j];
        unsigned count = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            count += unsigned(f[j].x > pe) + unsigned(f[j].y > pe) + unsigned(f[j].z > pe) +
                     unsigned(f[j].w > pe);
            count += (unsigned(f[j].x == pe) + unsigned(f[j].y == pe) +
                      unsigned(f[j].z == pe) + unsigned(f[j].w == pe)) << 16;
        }
        atomicAdd(&s.rank[e], count);
    }
    __syncthreads();
    const unsigned rank = s.rank[min(t, 255u)];
    const unsigned greater = rank & 0xffffu, equal = rank >> 16;  // equal counts t itself
    const bool top = mine && greater < top_k;
    const bool tie = top && (isnan(pf) || equal > 1);
    if (top && !tie) {
        s.sel[greater] = int(t);
        s.sel_p[greater] = pf;
    }
    const bool wave_tie = __ballot(tie) != 0;
    if (lane == 0)
        atomicOr(&s.ambiguous, wave_tie ? 1u : 0u);
    __syncthreads();
    if (s.ambiguous) {
        if (wave == 0) {
            const int slot =
                heap_route([&](int i) { return s.q[i]; }, experts, top_k, lane);
            if (lane < top_k) {
                s.sel[lane] = slot;
                s.sel_p[lane] = s.q[slot];
            }
        }
        __syncthreads();
    }
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < KMAX; ++i) {  // sequential, in selection order (+0 past top_k)
        const float pi = s.sel_p[i];
        sum += unsigned(i) < top_k ? pi : 0.f;
    }
    sum = fmaxf(sum, 6.103515625e-5f);
    if (t < top_k) {
        selected = s.sel[t];
        selected_weight = s.sel_p[t] / sum;
    }
}
