// probe.hip -- a measurement aid for bench.py, built into its own library
// (libtrw_probe.so) and not part of the engine or its C ABI: the rate at which
// this GPU serves random 8-byte gathers from a table of a given size, as
// independent loads or as chains in which every address depends on the value
// the previous load returned.
//
// The walk kernels run one lane per walk, and every hop reads an edge record
// (and a panel entry, a node header) at a place no other lane of the wave
// shares: each such load is one L1 miss.  This probe issues nothing but such
// misses, so its rate is the ceiling the walk kernels' L1 -> L2 read rate is
// compared with (bench.py reports both).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <stdexcept>
#include <string>

namespace trw {
namespace {

constexpr int kPB = 256;

// splitmix64's output function (Steele, Lea, Flood 2014): a bijective mixer
// whose outputs serve as random table contents and indices.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(kPB) void probe_fill_kernel(uint64_t* __restrict__ t, uint64_t n,
                                                         uint64_t seed) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kPB;
    for (uint64_t i = blockIdx.x * static_cast<uint64_t>(kPB) + threadIdx.x; i < n; i += stride)
        t[i] = mix64(seed + i);
}

// `rounds` gathers per lane from t[0, mask]; every index is masked into the
// table.  Chained: the next index is the loaded value plus a per-lane,
// per-round offset, so a lane has one load in flight, as a walk has, and lanes
// that load the same word do not continue on one path (plain value chains
// merge and end in short cycles, whose lines then hit in the caches).
// Independent: indices from a counter hash, so the compiler issues several
// loads of a lane ahead of their use.
template <bool Chained>
__global__ __launch_bounds__(kPB) void probe_gather_kernel(const uint64_t* __restrict__ t,
                                                           uint64_t mask, uint32_t rounds,
                                                           uint64_t seed,
                                                           uint64_t* __restrict__ out) {
    const uint64_t id = blockIdx.x * static_cast<uint64_t>(kPB) + threadIdx.x;
    uint64_t x = mix64(seed ^ id), acc = 0;
    if (Chained) {
        const uint64_t salt = mix64(~id ^ seed);
        for (uint32_t r = 0; r < rounds; ++r) {
            x = t[(x + salt * (r + 1)) & mask];
            acc += x;
        }
    } else {
#pragma unroll 8
        for (uint32_t r = 0; r < rounds; ++r) acc += t[mix64(x + r) & mask];
    }
    out[id] = acc;  // keeps the loads
}

}  // namespace
}  // namespace trw

namespace {

thread_local std::string g_err;

struct ProbeError : std::runtime_error {
    int code;
    ProbeError(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

void ck(hipError_t e, const char* what) {
    if (e != hipSuccess) throw ProbeError(2, std::string(what) + ": " + hipGetErrorString(e));
}

// Device buffer freed on scope exit.
struct Buf {
    uint64_t* p = nullptr;
    explicit Buf(uint64_t n) {
        if (hipMalloc(&p, n * 8) != hipSuccess) {
            (void)hipGetLastError();
            p = nullptr;
            throw ProbeError(3, "out of device memory");
        }
    }
    ~Buf() {
        if (p) (void)hipFree(p);
    }
};

}  // namespace

extern "C" {

// The message of the calling thread's last failed call.
const char* trwp_last_error() { return g_err.c_str(); }

// `lanes` (a multiple of 256) each make `rounds` gathers (at most 2^36 in all)
// from a table of table_bytes (a power of two in [4 KiB, 64 GiB], filled with
// random words), independent (chained 0) or chained; one warm-up launch, then
// `reps` timed launches on the null stream.  out[0]: ms per launch, out[1]:
// gathers per second, out[2]: gathers per launch.  Returns 0, 1 (invalid
// argument), 2 (HIP error) or 3 (out of memory).
int trwp_gather(uint64_t table_bytes, uint32_t lanes, uint32_t rounds, int32_t chained,
                int32_t reps, double* out) {
    using namespace trw;
    try {
        if (!out) throw ProbeError(1, "null argument");
        if (table_bytes < 4096 || table_bytes > (uint64_t{1} << 36) ||
            (table_bytes & (table_bytes - 1)) != 0)
            throw ProbeError(1, "table_bytes must be a power of two in [4 KiB, 64 GiB]");
        if (lanes == 0 || lanes % kPB != 0)
            throw ProbeError(1, "lanes must be a positive multiple of 256");
        if (rounds == 0 || reps <= 0) throw ProbeError(1, "rounds and reps must be positive");
        // a launch of at most 2^36 gathers: about a second at the slowest rate
        if (static_cast<uint64_t>(lanes) * rounds > (uint64_t{1} << 36))
            throw ProbeError(1, "lanes * rounds must not exceed 2^36 gathers per launch");
        const uint64_t n = table_bytes / 8;
        Buf table(n), sink(lanes);
        hipLaunchKernelGGL(probe_fill_kernel, dim3(4096), dim3(kPB), 0, nullptr, table.p, n,
                           uint64_t{0x243f6a8885a308d3ull});
        const dim3 grid(lanes / kPB);
        auto launch = [&](uint64_t seed) {
            if (chained)
                hipLaunchKernelGGL(probe_gather_kernel<true>, grid, dim3(kPB), 0, nullptr, table.p,
                                   n - 1, rounds, seed, sink.p);
            else
                hipLaunchKernelGGL(probe_gather_kernel<false>, grid, dim3(kPB), 0, nullptr,
                                   table.p, n - 1, rounds, seed, sink.p);
        };
        launch(1);  // warm-up: code load, table in the caches it fits
        ck(hipGetLastError(), "probe launch");
        hipEvent_t ev[2];
        ck(hipEventCreate(&ev[0]), "event");
        if (hipEventCreate(&ev[1]) != hipSuccess) {
            (void)hipEventDestroy(ev[0]);
            throw ProbeError(2, "hipEventCreate failed");
        }
        float ms = 0;
        hipError_t err = hipEventRecord(ev[0], nullptr);
        for (int r = 0; r < reps && err == hipSuccess; ++r) {
            launch(2 + static_cast<uint64_t>(r));
            err = hipGetLastError();
        }
        if (err == hipSuccess) err = hipEventRecord(ev[1], nullptr);
        if (err == hipSuccess) err = hipEventSynchronize(ev[1]);
        if (err == hipSuccess) err = hipEventElapsedTime(&ms, ev[0], ev[1]);
        (void)hipEventDestroy(ev[0]);
        (void)hipEventDestroy(ev[1]);
        ck(err, "probe timing");
        const uint64_t gathers = static_cast<uint64_t>(lanes) * rounds;
        out[0] = static_cast<double>(ms) / reps;
        out[1] = out[0] > 0 ? static_cast<double>(gathers) / (out[0] * 1e-3) : 0.0;
        out[2] = static_cast<double>(gathers);
        return 0;
    } catch (const ProbeError& e) {
        g_err = e.what();
        return e.code;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 2;
    }
}

}  // extern "C"
