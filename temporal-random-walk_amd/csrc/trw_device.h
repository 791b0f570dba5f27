// trw_device.h -- device-side building blocks of the MI355X temporal random
// walk engine: counter-based RNG, the draw-slot layout, and the pickers.
//
// Everything here is CDNA4 device code (gfx950, wave64).  The arithmetic of the
// pickers restates random/pickers.cuh:15-126 of the reference exactly (same
// operation order; the library is built with -ffp-contract=off so no FMA
// contraction changes a rounding), which is what makes replay-mode walks
// bit-exact against the reference CPU path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace trw {

// ---------------------------------------------------------------------------
// Picker ids (data/enums.cuh:4-15 of the reference).
// ---------------------------------------------------------------------------
enum Picker : int {
    kUniform = 0,
    kLinear = 1,
    kExponentialIndex = 2,
    kExponentialWeight = 3,
    kTemporalNode2Vec = 4,
    kTestFirst = 5,
    kTestLast = 6,
};

__host__ __device__ inline bool is_index_picker(int p) {
    return p == kUniform || p == kLinear || p == kExponentialIndex || p == kTestFirst ||
           p == kTestLast;
}

constexpr int64_t kNoCutoff = -1;     // common/const.cuh:24
constexpr int kNode2VecMaxRetries = 64;  // common/const.cuh:37

// ---------------------------------------------------------------------------
// Philox4x32-10 (Salmon, Moraes, Dror, Shaw: "Parallel random numbers: as easy
// as 1, 2, 3", SC'11).  Round: (c0,c1,c2,c3) ->
//   (hi(M1*c2) ^ c1 ^ k0, lo(M1*c2), hi(M0*c0) ^ c3 ^ k1, lo(M0*c0)),
// key bumped by the Weyl constants between rounds.
// ---------------------------------------------------------------------------
struct U4 {
    uint32_t x, y, z, w;
};

__device__ __forceinline__ U4 philox4x32_10(U4 c, uint32_t k0, uint32_t k1) {
    constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
    constexpr uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        // one 32 x 32 -> 64-bit multiply per product (v_mad_u64_u32) gives
        // both halves
        const uint64_t p0 = static_cast<uint64_t>(M0) * c.x;
        const uint64_t p1 = static_cast<uint64_t>(M1) * c.z;
        const uint32_t lo0 = static_cast<uint32_t>(p0), hi0 = static_cast<uint32_t>(p0 >> 32);
        const uint32_t lo1 = static_cast<uint32_t>(p1), hi1 = static_cast<uint32_t>(p1 >> 32);
        c = U4{hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0};
        k0 += W0;
        k1 += W1;
    }
    return c;
}

// 52 random bits -> a double strictly inside (0, 1): (m + 0.5) * 2^-52, built
// from the bits: 1 + m * 2^-52 has m as its mantissa, subtracting 1 is exact
// (Sterbenz), and adding 2^-53 is exact because (2m + 1) * 2^-53 fits 53 bits.
__device__ __forceinline__ double bits_to_unit(uint32_t lo, uint32_t hi) {
    const uint64_t m = ((static_cast<uint64_t>(hi) << 32) | lo) >> 12;
    const double one_m = __longlong_as_double(static_cast<long long>(0x3ff0000000000000ull | m));
    return (one_m - 1.0) + 1.1102230246251565404236316680908203125e-16;
}

// ---------------------------------------------------------------------------
// Draw slots.  The reference CPU path consumes, per walk, 1 + 2L uniforms laid
// out as: slot 0 = start group, slot 1 = start edge, slot 2 = endpoint of an
// undirected unconstrained start, slots 2k+1 / 2k+2 = group / edge of hop k
// (core/temporal_random_walk_cpu.cuh:32-33, 43-44, 84, 94-96).
//
// Replay mode reads those slots from an injected buffer.  Normal mode derives
// them from Philox keyed by the seed with counter (pair, walk): pair 0 holds
// slot 0, pair p >= 1 holds slots 2p-1 and 2p, so each hop costs exactly one
// Philox evaluation and every draw is a pure function of (seed, walk, slot) --
// independent of how walks are scheduled on the device.
// ---------------------------------------------------------------------------
struct DrawSource {
    const double* replay;  // nullptr => Philox
    uint32_t k0, k1;       // Philox key (the 64-bit seed)
    uint32_t stride;       // 1 + 2L
};

struct DrawPair {
    double a, b;
};

// Draws for slots (2p-1, 2p) of walk w (p >= 1).
__device__ __forceinline__ DrawPair draw_pair(const DrawSource& ds, uint64_t w, uint32_t p) {
    if (ds.replay) {
        const double* r = ds.replay + w * ds.stride;
        return DrawPair{r[2 * p - 1], r[2 * p]};
    }
    const U4 o = philox4x32_10(U4{p, static_cast<uint32_t>(w), static_cast<uint32_t>(w >> 32), 0u},
                               ds.k0, ds.k1);
    return DrawPair{bits_to_unit(o.x, o.y), bits_to_unit(o.z, o.w)};
}

__device__ __forceinline__ double draw_slot0(const DrawSource& ds, uint64_t w) {
    if (ds.replay) return ds.replay[w * ds.stride];
    const U4 o = philox4x32_10(U4{0u, static_cast<uint32_t>(w), static_cast<uint32_t>(w >> 32), 0u},
                               ds.k0, ds.k1);
    return bits_to_unit(o.x, o.y);
}

// ---------------------------------------------------------------------------
// Pickers (random/pickers.cuh:15-126).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int pick_linear(int start, int end, bool prioritize_end, double r) {
    if (start >= end) return -1;
    const int len = end - start;
    const double total = static_cast<double>(len) * (static_cast<double>(len) + 1.0) / 2.0;
    const double scaled = total * r;
    const double disc = 1.0 + 8.0 * scaled;
    const double root = (-1.0 + sqrt(disc)) / 2.0;
    const int index = static_cast<int>(floor(root));
    if (prioritize_end) return start + min(index, len - 1);
    return start + max(0, len - 1 - index);
}

// Lengths below this take the expm1 branch of the exponential index picker.
constexpr int kExpm1Table = 710;

// em1: expm1(len) for len in [0, kExpm1Table) (the same values expm1 returns
// here), or nullptr to evaluate it.
__device__ __forceinline__ int pick_exponential_index(int start, int end, bool prioritize_end,
                                                      double r, const double* em1 = nullptr) {
    if (start >= end) return -1;
    const int len = end - start;
    double k;
    if (len < kExpm1Table) {
        k = log1p(r * (em1 ? em1[len] : expm1(static_cast<double>(len)))) - 1;
    } else {
        k = len + log(r) - 1;
    }
    const int ri = max(0, min(static_cast<int>(k + 1), len - 1));
    return prioritize_end ? start + ri : start + (len - 1 - ri);
}

__device__ __forceinline__ int pick_uniform(int start, int end, double r) {
    if (start >= end) return -1;
    return start + static_cast<int>(r * (end - start));
}

__device__ __forceinline__ int pick_index(int picker, int start, int end, bool prioritize_end,
                                          double r, const double* em1 = nullptr) {
    switch (picker) {
        case kLinear: return pick_linear(start, end, prioritize_end, r);
        case kExponentialIndex: return pick_exponential_index(start, end, prioritize_end, r, em1);
        case kUniform: return pick_uniform(start, end, r);
        case kTestFirst: return start;
        case kTestLast: return end - 1;
        default: return -1;
    }
}

// Cumulative-weight inverse-CDF picker over [gs, ge) of a piecewise CDF whose
// segment starts at slice_start (random/pickers.cuh:84-126).
__device__ __forceinline__ int pick_exponential_weights(const double* w, uint64_t wsize,
                                                        uint64_t gs, uint64_t ge, double r,
                                                        uint64_t slice_start) {
    if (gs >= ge || ge > wsize) return -1;
    const double start_sum = gs > slice_start ? w[gs - 1] : 0.0;
    const double end_sum = w[ge - 1];
    if (end_sum < start_sum) return -1;
    const double target = start_sum + r * (end_sum - start_sum);
    uint64_t lo = gs, hi = ge;
    while (lo < hi) {
        const uint64_t mid = lo + ((hi - lo) >> 1);
        if (w[mid] < target) lo = mid + 1;
        else hi = mid;
    }
    return static_cast<int>(lo);
}

// splitmix64-style retry draws of the node2vec rejection loop
// (graph/temporal_node2vec_helpers.cuh:57-70).
__device__ __forceinline__ double derive_uniform(double a, double b, int counter) {
    uint64_t s = static_cast<uint64_t>(__double_as_longlong(a)) * 0x9E3779B97F4A7C15ULL;
    s ^= static_cast<uint64_t>(__double_as_longlong(b)) + 0xBF58476D1CE4E5B9ULL;
    s += static_cast<uint64_t>(counter) * 0x94D049BB133111EBULL;
    s ^= s >> 30;
    s *= 0xBF58476D1CE4E5B9ULL;
    s ^= s >> 27;
    s *= 0x94D049BB133111EBULL;
    s ^= s >> 31;
    return static_cast<double>(s >> 11) * (1.0 / 9007199254740992.0);
}

}  // namespace trw
