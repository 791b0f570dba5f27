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

// Normal-mode draws for slots (2p-1, 2p) of walk w (p >= 1).
__device__ __forceinline__ DrawPair philox_pair(const DrawSource& ds, uint64_t w, uint32_t p) {
    const U4 o = philox4x32_10(U4{p, static_cast<uint32_t>(w), static_cast<uint32_t>(w >> 32), 0u},
                               ds.k0, ds.k1);
    return DrawPair{bits_to_unit(o.x, o.y), bits_to_unit(o.z, o.w)};
}

// Replay-mode draws for slots (2p-1, 2p) of walk w (p >= 1).
__device__ __forceinline__ DrawPair replay_pair(const DrawSource& ds, uint64_t w, uint32_t p) {
    const double* r = ds.replay + w * ds.stride;
    return DrawPair{r[2 * p - 1], r[2 * p]};
}

// Draws for slots (2p-1, 2p) of walk w (p >= 1).
__device__ __forceinline__ DrawPair draw_pair(const DrawSource& ds, uint64_t w, uint32_t p) {
    return ds.replay ? replay_pair(ds, w, p) : philox_pair(ds, w, p);
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
// exp(-j) for j in [0, kExpNegTable), after the expm1 values.
constexpr int kExpNegTable = 40;
constexpr int kExpTables = kExpm1Table + kExpNegTable;

// Fills the exponential index picker's tables: xt[i] = expm1(i) for i <
// kExpm1Table, then xt[kExpm1Table + j] = exp(-j).  Threads tid of nthreads
// share the work.
__device__ __forceinline__ void fill_exp_tables(double* xt, int tid, int nthreads) {
    for (int i = tid; i < kExpTables; i += nthreads)
        xt[i] = i < kExpm1Table ? expm1(static_cast<double>(i))
                                : exp(-static_cast<double>(i - kExpm1Table));
}

// The exponential index picker's ri (random/pickers.cuh:47-71): with k =
// log1p(r * expm1(len)) - 1 for len < kExpm1Table and k = len + log(r) - 1
// above, ri = clamp((int)(k + 1), 0, len - 1).
__device__ __forceinline__ int exp_index_ri_ref(int len, double r, const double* xt) {
    double k;
    if (len < kExpm1Table) {
        k = log1p(r * (xt ? xt[len] : expm1(static_cast<double>(len)))) - 1;
    } else {
        k = len + log(r) - 1;
    }
    return max(0, min(static_cast<int>(k + 1), len - 1));
}

// The same ri from the tables, without a logarithm.  In exact arithmetic
// ri = floor(log1p(x)) with x = r * expm1(len), the number of i in [1, len)
// with expm1(i) <= x; above the table ri = len - 1 - j with j = floor(-log r),
// where exp(-(j+1)) < r <= exp(-j).  The exponent of 1 + x (of r) brackets
// the answer to two neighbours, one table entry decides between them.  The
// reference's rounded log1p / log and sum agree with the exact floor unless
// the exact value lies within a few ulps of an integer, i.e. unless x (r)
// lies within a small relative margin of a table threshold: such a draw, or
// one the estimate did not bracket (the margin test then fails too), takes
// the reference expression itself.  Margins: log1p and log err by at most 2
// ulps (<= 2^-41.5 absolute below 710, <= 2^-45 below 64), the sum len +
// log(r) rounds by at most len * 2^-52, the table entries by 2^-52
// relative; the margins below exceed their sum eightfold.
__device__ __forceinline__ int exp_index_ri(int len, double r, const double* xt) {
    if (xt == nullptr) return exp_index_ri_ref(len, r, xt);
    constexpr float kLn2 = 0.693147182f;
    if (len < kExpm1Table) {
        const double x = r * xt[len];
        const int e = __builtin_amdgcn_frexp_exp(1.0 + x) - 1;  // 1 + x in [2^e, 2^(e+1))
        const int est = min(static_cast<int>(static_cast<float>(e) * kLn2), len - 1);
        const double t1 = xt[min(est + 1, kExpm1Table - 1)];
        const bool up = est + 1 < len && x >= t1;
        const int i = est + (up ? 1 : 0);
        const double lo = up ? t1 : xt[est];
        const double hi = xt[min(i + 1, kExpm1Table - 1)];
        const double m = 0x1p-38;
        const bool near_lo = i > 0 && x - lo < m * (1.0 + lo);
        const bool near_hi = i + 1 < len && hi - x < m * (1.0 + hi);
        if (near_lo || near_hi || !(x >= 0.0)) return exp_index_ri_ref(len, r, xt);
        return i;
    }
    const double* en = xt + kExpm1Table;
    const int e = __builtin_amdgcn_frexp_exp(r);  // r in [2^(e-1), 2^e)
    // -log r lies in (-e ln2, (1 - e) ln2]; r >= 2^-54 keeps the entries read
    // inside the table
    if (!(r >= 0x1p-54 && r < 1.0)) return exp_index_ri_ref(len, r, xt);
    const int est = static_cast<int>(static_cast<float>(-e) * kLn2);
    const double t1 = en[est + 1];
    const bool up = r <= t1;
    const int j = est + (up ? 1 : 0);
    const double lo = up ? en[est + 2] : t1;  // exp(-(j+1))
    const double hi = up ? t1 : en[est];      // exp(-j)
    const double m = static_cast<double>(len + 64) * 0x1p-48;
    const bool near_lo = r - lo < m * lo;
    const bool near_hi = j > 0 && hi - r < m * hi;
    if (near_lo || near_hi) return exp_index_ri_ref(len, r, xt);
    return len - 1 - j;
}

// xt: the tables of fill_exp_tables, or nullptr to evaluate the reference
// expression directly.
__device__ __forceinline__ int pick_exponential_index(int start, int end, bool prioritize_end,
                                                      double r, const double* xt = nullptr) {
    if (start >= end) return -1;
    const int len = end - start;
    const int ri = exp_index_ri(len, r, xt);
    return prioritize_end ? start + ri : start + (len - 1 - ri);
}

__device__ __forceinline__ int pick_uniform(int start, int end, double r) {
    if (start >= end) return -1;
    return start + static_cast<int>(r * (end - start));
}

__device__ __forceinline__ int pick_index(int picker, int start, int end, bool prioritize_end,
                                          double r, const double* xt = nullptr) {
    switch (picker) {
        case kLinear: return pick_linear(start, end, prioritize_end, r);
        case kExponentialIndex: return pick_exponential_index(start, end, prioritize_end, r, xt);
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
