// pickers.hip -- the standalone pickers of the reference's RandomPicker
// proxies (proxies/RandomPicker.cu:11-313) on the device.
//
// The reference launches one single-thread kernel per pick, with a cudaMalloc,
// two copies and a cudaFree around it.  Here one launch serves a whole batch of
// picks (one lane each): the same picker arithmetic as the walk kernel
// (trw_device.h, random/pickers.cuh:15-126), with either caller-given uniforms
// (pick_random_with_provided_number) or in-kernel Philox4x32-10 draws keyed by
// a seed (pick_random, which the reference feeds from a fresh generator).
#include "engine.h"
#include "trw_device.h"

namespace trw {
namespace {

constexpr int kB = 256;

// Counter word 2 of the pickers' Philox stream (the walks use the slot pair).
constexpr uint32_t kPickStream = 0x5049434bu;

__device__ __forceinline__ double pick_draw(const double* draws, uint64_t i, uint32_t k0,
                                            uint32_t k1) {
    if (draws) return draws[i];
    const U4 o = philox4x32_10(U4{static_cast<uint32_t>(i), static_cast<uint32_t>(i >> 32),
                                  kPickStream, 0u},
                               k0, k1);
    return bits_to_unit(o.x, o.y);
}

__global__ void pick_index_kernel(int picker, const int32_t* __restrict__ start,
                                  const int32_t* __restrict__ end, uint64_t n, int prioritize_end,
                                  const double* __restrict__ draws, uint32_t k0, uint32_t k1,
                                  int32_t* __restrict__ out) {
    __shared__ double s_xt[kExpTables];
    const bool use_xt = picker == kExponentialIndex;
    if (use_xt) {
        fill_exp_tables(s_xt, threadIdx.x, kB);
        __syncthreads();
    }
    const uint64_t i = blockIdx.x * static_cast<uint64_t>(kB) + threadIdx.x;
    if (i >= n) return;
    out[i] = pick_index(picker, start[i], end[i], prioritize_end != 0, pick_draw(draws, i, k0, k1),
                        use_xt ? s_xt : nullptr);
}

// WeightBasedRandomPicker::pick_random over one cumulative array (slice start
// 0, as the proxy passes it).
__global__ void pick_weights_kernel(const double* __restrict__ w, uint64_t size,
                                    const uint64_t* __restrict__ gs,
                                    const uint64_t* __restrict__ ge, uint64_t n,
                                    const double* __restrict__ draws, uint32_t k0, uint32_t k1,
                                    int32_t* __restrict__ out) {
    const uint64_t i = blockIdx.x * static_cast<uint64_t>(kB) + threadIdx.x;
    if (i >= n) return;
    out[i] = pick_exponential_weights(w, size, gs[i], ge[i], pick_draw(draws, i, k0, k1), 0);
}

// Device copy of a host array, freed at scope exit.
template <typename T>
struct Staged {
    DBuf<T> buf;
    Staged(const T* host, size_t n) {
        buf.resize(n);
        if (n && host) check_hip(hipMemcpy(buf.p, host, n * sizeof(T), hipMemcpyHostToDevice), "H2D");
    }
};

void check_draws(const double* draws, uint64_t n) {
    if (!draws) return;
    for (uint64_t i = 0; i < n; ++i)
        if (!(draws[i] >= 0.0 && draws[i] < 1.0))
            throw InvalidArgument("random numbers must lie in [0, 1)");
}

inline unsigned grid(uint64_t n) {
    return static_cast<unsigned>((n + kB - 1) / kB);
}

}  // namespace

void pick_index_batch(int picker, const int32_t* start, const int32_t* end, uint64_t n,
                      bool prioritize_end, const double* draws, uint64_t seed, int32_t* out) {
    if (!is_index_picker(picker)) throw InvalidArgument("Invalid picker type");
    if (n && (!start || !end || !out)) throw InvalidArgument("null argument");
    if (n >= (1ull << 32) - kB) throw InvalidArgument("too many picks (limit 2^32 - 256)");
    check_draws(draws, n);
    if (n == 0) return;
    Staged<int32_t> s(start, n), e(end, n);
    Staged<double> d(draws, draws ? n : 0);
    DBuf<int32_t> o;
    o.resize(n);
    hipLaunchKernelGGL(pick_index_kernel, dim3(grid(n)), dim3(kB), 0, nullptr, picker, s.buf.p,
                       e.buf.p, n, prioritize_end ? 1 : 0, draws ? d.buf.p : nullptr,
                       static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32), o.p);
    check_hip(hipGetLastError(), "picker launch");
    check_hip(hipMemcpy(out, o.p, n * sizeof(int32_t), hipMemcpyDeviceToHost), "D2H");
}

void pick_weights_batch(const double* cumulative, uint64_t size, const uint64_t* group_start,
                        const uint64_t* group_end, uint64_t n, const double* draws, uint64_t seed,
                        int32_t* out) {
    if (n && (!group_start || !group_end || !out)) throw InvalidArgument("null argument");
    if (size && !cumulative) throw InvalidArgument("null argument");
    if (n >= (1ull << 32) - kB) throw InvalidArgument("too many picks (limit 2^32 - 256)");
    check_draws(draws, n);
    if (n == 0) return;
    Staged<double> w(cumulative, size);
    Staged<uint64_t> gs(group_start, n), ge(group_end, n);
    Staged<double> d(draws, draws ? n : 0);
    DBuf<int32_t> o;
    o.resize(n);
    hipLaunchKernelGGL(pick_weights_kernel, dim3(grid(n)), dim3(kB), 0, nullptr, w.buf.p, size,
                       gs.buf.p, ge.buf.p, n, draws ? d.buf.p : nullptr,
                       static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32), o.p);
    check_hip(hipGetLastError(), "picker launch");
    check_hip(hipMemcpy(out, o.p, n * sizeof(int32_t), hipMemcpyDeviceToHost), "D2H");
}

}  // namespace trw
