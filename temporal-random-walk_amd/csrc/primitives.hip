// primitives.hip -- device-wide scan, stable LSD radix sort and reductions.
// See primitives.h for the design notes.
#include "primitives.h"

#include <type_traits>

#include <stdexcept>
#include <string>

namespace trw {

void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        throw std::runtime_error(std::string("HIP error in ") + what + ": " +
                                 hipGetErrorString(e));
    }
}

namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;

// Scan operators: a sum, and a running maximum (identity -inf).
struct OpSum {
    template <typename T>
    __device__ static T identity() { return T(0); }
    template <typename T>
    __device__ static T apply(T a, T b) { return a + b; }
};
struct OpMax {
    template <typename T>
    __device__ static T identity() { return -__builtin_huge_val(); }
    template <typename T>
    __device__ static T apply(T a, T b) { return a > b ? a : b; }
};

// ---------------------------------------------------------------------------
// block-level helpers (256 threads = 4 wave64)
// ---------------------------------------------------------------------------
template <typename T, typename Op = OpSum>
__device__ __forceinline__ T wave_inclusive_scan(T x, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const T y = __shfl_up(x, off, 64);
        if (lane >= off) x = Op::apply(x, y);
    }
    return x;
}

// Exclusive block scan of one value per thread; *total receives the block
// total.  The exclusive value is built from the wave prefix and the shifted
// inclusive scan, so it is exact for the maximum as well as for integers.
template <typename T, typename Op = OpSum>
__device__ __forceinline__ T block_exclusive_scan(T v, T* total, T* s_wave) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const T inc = wave_inclusive_scan<T, Op>(v, lane);
    const T below = __shfl_up(inc, 1, 64);
    if (lane == 63) s_wave[wave] = inc;
    __syncthreads();
    T wp = Op::template identity<T>(), tot = Op::template identity<T>();
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const T sw = s_wave[w];
        if (w < wave) wp = Op::apply(wp, sw);
        tot = Op::apply(tot, sw);
    }
    __syncthreads();
    *total = tot;
    return lane == 0 ? wp : Op::apply(wp, below);
}

template <typename T, typename Op = OpSum>
__device__ __forceinline__ T block_sum(T v, T* s_wave) {
    T tot;
    (void)block_exclusive_scan<T, Op>(v, &tot, s_wave);
    return tot;
}

// ---------------------------------------------------------------------------
// scan: tile = 256 threads x 16 consecutive items per thread
// ---------------------------------------------------------------------------
constexpr int kScanItems = 16;
constexpr size_t kScanTile = static_cast<size_t>(kBlock) * kScanItems;

template <typename T, typename Op>
__global__ __launch_bounds__(kBlock) void scan_reduce_kernel(const T* __restrict__ in, size_t n,
                                                             T* __restrict__ sums) {
    __shared__ T s_wave[kWaves];
    const size_t base = blockIdx.x * kScanTile + static_cast<size_t>(threadIdx.x) * kScanItems;
    T acc = Op::template identity<T>();
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        const size_t i = base + j;
        if (i < n) acc = Op::apply(acc, in[i]);
    }
    const T tot = block_sum<T, Op>(acc, s_wave);
    if (threadIdx.x == 0) sums[blockIdx.x] = tot;
}

// Single block: exclusive scan of sums[0..nb) in place; sums[nb] = total.
template <typename T, typename Op>
__global__ __launch_bounds__(kBlock) void scan_sums_kernel(T* __restrict__ sums, size_t nb) {
    __shared__ T s_wave[kWaves];
    T carry = Op::template identity<T>();
    for (size_t chunk = 0; chunk < nb; chunk += kScanTile) {
        const size_t base = chunk + static_cast<size_t>(threadIdx.x) * kScanItems;
        T v[kScanItems];
        T acc = Op::template identity<T>();
#pragma unroll
        for (int j = 0; j < kScanItems; ++j) {
            const size_t i = base + j;
            v[j] = i < nb ? sums[i] : Op::template identity<T>();
            acc = Op::apply(acc, v[j]);
        }
        T tot;
        T run = Op::apply(carry, block_exclusive_scan<T, Op>(acc, &tot, s_wave));
#pragma unroll
        for (int j = 0; j < kScanItems; ++j) {
            const size_t i = base + j;
            if (i < nb) sums[i] = run;
            run = Op::apply(run, v[j]);
        }
        carry = Op::apply(carry, tot);
        __syncthreads();
    }
    if (threadIdx.x == 0) sums[nb] = carry;
}

template <typename T, bool Inclusive, typename Op>
__global__ __launch_bounds__(kBlock) void scan_apply_kernel(const T* in, T* out, size_t n,
                                                            const T* __restrict__ sums) {
    __shared__ T s_wave[kWaves];
    const size_t base = blockIdx.x * kScanTile + static_cast<size_t>(threadIdx.x) * kScanItems;
    T v[kScanItems];
    T acc = Op::template identity<T>();
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        const size_t i = base + j;
        v[j] = i < n ? in[i] : Op::template identity<T>();
        acc = Op::apply(acc, v[j]);
    }
    T tot;
    T run = Op::apply(sums[blockIdx.x], block_exclusive_scan<T, Op>(acc, &tot, s_wave));
#pragma unroll
    for (int j = 0; j < kScanItems; ++j) {
        const size_t i = base + j;
        if (Inclusive) run = Op::apply(run, v[j]);
        if (i < n) out[i] = run;
        if (!Inclusive) run = Op::apply(run, v[j]);
    }
    if (!Inclusive && blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) out[n] = sums[gridDim.x];
}

// ---------------------------------------------------------------------------
// uint32 exclusive scan with coalesced accesses: the same 4096-item tiles, but
// wave w of a tile owns items [1024 w, 1024 w + 1024) as four rows of 256, and
// lane l holds items 4l..4l+3 of each row (one 16-byte access per lane and
// row, 1 KiB contiguous per wave access).  Integer sums are exact in any
// order, so the tile totals equal the blocked kernels'.
// ---------------------------------------------------------------------------
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ u32x4_t load_u32x4(const uint32_t* in, size_t i, size_t n) {
    if (i + 4 <= n) return *reinterpret_cast<const u32x4_t*>(in + i);
    u32x4_t v = {0u, 0u, 0u, 0u};
    if (i < n) v.x = in[i];
    if (i + 1 < n) v.y = in[i + 1];
    if (i + 2 < n) v.z = in[i + 2];
    return v;
}

__global__ __launch_bounds__(kBlock) void scan_reduce_u32_kernel(const uint32_t* __restrict__ in,
                                                                 size_t n,
                                                                 uint32_t* __restrict__ sums) {
    __shared__ uint32_t s_wave[kWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t wbase = blockIdx.x * kScanTile + static_cast<size_t>(wave) * 1024 + lane * 4;
    uint32_t acc = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const u32x4_t v = load_u32x4(in, wbase + r * 256, n);
        acc += v.x + v.y + v.z + v.w;
    }
    const uint32_t tot = block_sum<uint32_t, OpSum>(acc, s_wave);
    if (threadIdx.x == 0) sums[blockIdx.x] = tot;
}

__global__ __launch_bounds__(kBlock) void scan_apply_u32_kernel(const uint32_t* in,
                                                                uint32_t* out, size_t n,
                                                                const uint32_t* __restrict__ sums) {
    __shared__ uint32_t s_wave[kWaves];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t wbase = blockIdx.x * kScanTile + static_cast<size_t>(wave) * 1024 + lane * 4;
    u32x4_t v[4];
    uint32_t excl[4], row_tot[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = load_u32x4(in, wbase + r * 256, n);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t ls = v[r].x + v[r].y + v[r].z + v[r].w;
        const uint32_t inc = wave_inclusive_scan<uint32_t, OpSum>(ls, lane);
        excl[r] = inc - ls;
        row_tot[r] = __shfl(inc, 63, 64);
    }
    const uint32_t wave_tot = row_tot[0] + row_tot[1] + row_tot[2] + row_tot[3];
    if (lane == 0) s_wave[wave] = wave_tot;
    __syncthreads();
    uint32_t carry = sums[blockIdx.x];
#pragma unroll
    for (int w = 0; w < kWaves; ++w)
        if (w < wave) carry += s_wave[w];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const size_t i = wbase + r * 256;
        u32x4_t o;
        o.x = carry + excl[r];
        o.y = o.x + v[r].x;
        o.z = o.y + v[r].y;
        o.w = o.z + v[r].z;
        if (i + 4 <= n) {
            *reinterpret_cast<u32x4_t*>(out + i) = o;
        } else {
            if (i < n) out[i] = o.x;
            if (i + 1 < n) out[i + 1] = o.y;
            if (i + 2 < n) out[i + 2] = o.z;
        }
        carry += row_tot[r];
    }
    if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) out[n] = sums[gridDim.x];
}

template <typename T, bool Inclusive, typename Op = OpSum>
void scan_impl(const T* in, T* out, size_t n, T* scratch, hipStream_t s) {
    if (n == 0) {
        if (!Inclusive) check_hip(hipMemsetAsync(out, 0, sizeof(T), s), "scan memset");
        return;
    }
    const size_t nb = (n + kScanTile - 1) / kScanTile;
    hipLaunchKernelGGL((scan_reduce_kernel<T, Op>), dim3(nb), dim3(kBlock), 0, s, in, n, scratch);
    hipLaunchKernelGGL((scan_sums_kernel<T, Op>), dim3(1), dim3(kBlock), 0, s, scratch, nb);
    hipLaunchKernelGGL((scan_apply_kernel<T, Inclusive, Op>), dim3(nb), dim3(kBlock), 0, s, in,
                       out, n, scratch);
    check_hip(hipGetLastError(), "scan launch");
}

// ---------------------------------------------------------------------------
// radix sort: a sort of B key bits takes the fewest passes of at most
// kMaxDigitBits bits, the bits split evenly (27 bits: three 9-bit passes, 20
// bits: two 10-bit passes); tile = 4 waves x 8 rows x 64 keys = 2048 keys; a
// workgroup owns kTilesPerBlock consecutive tiles, so the digit-major
// histogram has one column per workgroup (fewer scattered histogram writes and
// a shorter histogram scan per pass)
// ---------------------------------------------------------------------------
constexpr int kMaxDigitBits = 10;
constexpr int kMaxRadix = 1 << kMaxDigitBits;
constexpr int kRows = 8;
constexpr size_t kSortTile = static_cast<size_t>(kBlock) * kRows;
constexpr int kTilesPerBlock = 4;
constexpr size_t kSortSpan = kSortTile * kTilesPerBlock;

__device__ __forceinline__ uint64_t lanes_below(int lane) {
    return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Mask of the valid lanes of this wave whose digit (of db bits) equals mine.
__device__ __forceinline__ uint64_t match_digit(uint32_t d, bool valid, int db) {
    uint64_t m = __ballot(valid);
    for (int b = 0; b < db; ++b) {
        const bool bit = (d >> b) & 1u;
        const uint64_t vote = __ballot(bit);
        m &= bit ? vote : ~vote;
    }
    return m;
}

// Per-workgroup digit counts of keys[...] >> bit (db-bit digits, the digit
// masked to dmask), digit-major into hist, and the digit totals.  Dynamic
// LDS: kWaves << db counters.
template <typename K>
__global__ __launch_bounds__(kBlock) void radix_upsweep_kernel(const K* __restrict__ keys,
                                                               size_t n, int bit, int db,
                                                               uint32_t dmask,
                                                               uint32_t* __restrict__ hist,
                                                               size_t nb) {
    extern __shared__ uint32_t s_cnt[];  // [kWaves][R]
    const int R = 1 << db;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < kWaves * R; i += kBlock) s_cnt[i] = 0;
    __syncthreads();
    for (int t = 0; t < kTilesPerBlock; ++t) {
        const size_t wave_base = blockIdx.x * kSortSpan + t * kSortTile +
                                 static_cast<size_t>(wave) * kRows * 64;
        if (wave_base >= n) break;  // uniform over the wave
        K key[kRows];
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const size_t i = wave_base + static_cast<size_t>(r) * 64 + lane;
            key[r] = i < n ? keys[i] : K(0);
        }
        // counts only (no ranks): an LDS atomic per key, which a wave's
        // same-digit lanes serialise among themselves -- the row's lanes with
        // its first lane's digit add their count in one atomic (a hub's
        // node id fills half the rows of a power-law graph's node sort, and
        // their serialised atomics slowed that pass's histogram by 60 %)
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const size_t i = wave_base + static_cast<size_t>(r) * 64 + lane;
            const uint32_t d = static_cast<uint32_t>(key[r] >> bit) & dmask;
            const bool valid = i < n;
            const uint64_t vm = __ballot(valid);
            if (vm == 0) continue;
            const int first = __ffsll(static_cast<long long>(vm)) - 1;
            const uint32_t d0 = __shfl(d, first, 64);
            const uint64_t m0 = __ballot(valid && d == d0);
            if (lane == first) atomicAdd(&s_cnt[wave * R + d0], static_cast<uint32_t>(__popcll(m0)));
            if (valid && d != d0) atomicAdd(&s_cnt[wave * R + d], 1u);
        }
    }
    __syncthreads();
    for (int d = threadIdx.x; d < R; d += kBlock) {
        uint32_t tot = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) tot += s_cnt[w * R + d];
        hist[static_cast<size_t>(d) * nb + blockIdx.x] = tot;
    }
}

// One workgroup per digit d: the digit's total over the workgroups' counts
// (its contiguous histogram row).
__global__ __launch_bounds__(kBlock) void radix_digit_totals_kernel(const uint32_t* __restrict__ hist,
                                                                    size_t nb,
                                                                    uint32_t* __restrict__ digit_tot) {
    __shared__ uint32_t s_wave[kWaves];
    const uint32_t* row = hist + static_cast<size_t>(blockIdx.x) * nb;
    uint32_t acc = 0;
    for (size_t i = threadIdx.x; i < nb; i += kBlock) acc += row[i];
    const uint32_t tot = block_sum<uint32_t, OpSum>(acc, s_wave);
    if (threadIdx.x == 0) digit_tot[blockIdx.x] = tot;
}

// One workgroup per digit d: the exclusive scan of the workgroups' counts of
// digit d (hist[d * nb + b], in place), offset by the number of keys with a
// smaller digit -- the scatter positions of every (workgroup, digit).
__global__ __launch_bounds__(kBlock) void radix_offsets_kernel(uint32_t* __restrict__ hist,
                                                               size_t nb,
                                                               const uint32_t* __restrict__ digit_tot) {
    __shared__ uint32_t s_wave[kWaves];
    const int d = blockIdx.x;
    uint32_t below = 0;
    for (int i = threadIdx.x; i < d; i += kBlock) below += digit_tot[i];
    uint32_t carry = block_sum<uint32_t, OpSum>(below, s_wave);
    __syncthreads();
    uint32_t* row = hist + static_cast<size_t>(d) * nb;
    for (size_t chunk = 0; chunk < nb; chunk += kScanTile) {
        const size_t base = chunk + static_cast<size_t>(threadIdx.x) * kScanItems;
        uint32_t v[kScanItems];
        uint32_t acc = 0;
#pragma unroll
        for (int j = 0; j < kScanItems; ++j) {
            const size_t i = base + j;
            v[j] = i < nb ? row[i] : 0u;
            acc += v[j];
        }
        uint32_t tot;
        uint32_t run = carry + block_exclusive_scan<uint32_t, OpSum>(acc, &tot, s_wave);
#pragma unroll
        for (int j = 0; j < kScanItems; ++j) {
            const size_t i = base + j;
            if (i < nb) row[i] = run;
            run += v[j];
        }
        carry += tot;
        __syncthreads();
    }
}

// Stable scatter of one digit pass.  A tile's keys are first placed in LDS in
// their sorted order within the tile (digit, then wave, then rank), then
// written out by consecutive threads: the keys of one digit leave as one
// contiguous run instead of one scattered store per key.  Dynamic LDS
// (radix_scatter_lds): kWaves << db counters, 1 << db running positions,
// 1 << db output bases, then the tile's staged keys and values.
// Store: the last pass of an edge-store sort writes the store (st) instead of
// keys_out / vals_out.
template <typename K, typename V, bool Store = false>
__global__ __launch_bounds__(kBlock) void radix_scatter_kernel(
    const K* __restrict__ keys_in, const V* __restrict__ vals_in, K* __restrict__ keys_out,
    V* __restrict__ vals_out, size_t n, int bit, int db, uint32_t dmask,
    const uint32_t* __restrict__ offsets, size_t nb, SortedStore st = SortedStore{}) {
    extern __shared__ __align__(16) uint32_t s_lds[];
    __shared__ uint32_t s_wave[kWaves];
    const int R = 1 << db;
    uint32_t* s_cnt = s_lds;                // [kWaves][R]: counts, then tile-local offsets
    uint32_t* s_run = s_cnt + kWaves * R;   // the workgroup's next output position per digit
    uint32_t* s_base = s_run + R;           // output position of tile-local position 0, per digit
    K* s_key = reinterpret_cast<K*>(s_base + R);
    V* s_val = reinterpret_cast<V*>(s_key + kSortTile);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // digits [d0, d0 + per) of this thread in the tile epilogue
    const int per = (R + kBlock - 1) / kBlock;
    const int d0 = threadIdx.x * per;
    for (int d = threadIdx.x; d < R; d += kBlock)
        s_run[d] = offsets[static_cast<size_t>(d) * nb + blockIdx.x];
    for (int t = 0; t < kTilesPerBlock; ++t) {
        const size_t tile_base = blockIdx.x * kSortSpan + t * kSortTile;
        if (tile_base >= n) break;  // uniform over the workgroup
        for (int i = threadIdx.x; i < kWaves * R; i += kBlock) s_cnt[i] = 0;
        __syncthreads();
        const size_t wave_base = tile_base + static_cast<size_t>(wave) * kRows * 64;
        K key[kRows];
        V val[kRows];
        uint32_t dig[kRows];
        uint32_t rank[kRows];
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const size_t i = wave_base + static_cast<size_t>(r) * 64 + lane;
            const bool valid = i < n;
            key[r] = valid ? keys_in[i] : K(0);
            val[r] = (valid && vals_in) ? vals_in[i] : V(0);
        }
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const size_t i = wave_base + static_cast<size_t>(r) * 64 + lane;
            const bool valid = i < n;
            const uint32_t d = static_cast<uint32_t>(key[r] >> bit) & dmask;
            dig[r] = d;
            const uint64_t m = match_digit(d, valid, db);
            const uint32_t before = __popcll(m & lanes_below(lane));
            const uint32_t prior = s_cnt[wave * R + d];
            rank[r] = prior + before;
            if (valid && before == 0) s_cnt[wave * R + d] = prior + __popcll(m);
        }
        __syncthreads();
        {
            // tile epilogue: the tile-local start of every digit (an exclusive
            // scan of the tile's digit counts), its waves' offsets after it,
            // and the output position of local position 0 for the digit
            uint32_t cnt_mine = 0;
            for (int j = 0; j < per; ++j) {
                const int d = d0 + j;
                if (d < R) {
#pragma unroll
                    for (int w = 0; w < kWaves; ++w) cnt_mine += s_cnt[w * R + d];
                }
            }
            uint32_t tot;
            uint32_t start = block_exclusive_scan<uint32_t, OpSum>(cnt_mine, &tot, s_wave);
            for (int j = 0; j < per; ++j) {
                const int d = d0 + j;
                if (d < R) {
                    const uint32_t first = start;
#pragma unroll
                    for (int w = 0; w < kWaves; ++w) {
                        const uint32_t c = s_cnt[w * R + d];
                        s_cnt[w * R + d] = start;
                        start += c;
                    }
                    s_base[d] = s_run[d] - first;  // wraps back in pos = base + local
                    s_run[d] += start - first;
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const size_t i = wave_base + static_cast<size_t>(r) * 64 + lane;
            if (i < n) {
                const uint32_t lp = s_cnt[wave * R + dig[r]] + rank[r];
                s_key[lp] = key[r];
                if (vals_out || Store) s_val[lp] = val[r];  // the store pass writes no vals_out
            }
        }
        __syncthreads();
        const size_t tile_n = n - tile_base < kSortTile ? n - tile_base : kSortTile;
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const uint32_t lp = static_cast<uint32_t>(r) * kBlock + threadIdx.x;
            if (lp < tile_n) {
                const K k = s_key[lp];
                const uint32_t d = static_cast<uint32_t>(k >> bit) & dmask;
                const uint32_t pos = s_base[d] + lp;
                if constexpr (Store) {
                    const uint64_t v = s_val[lp];
                    st.src[pos] = static_cast<int32_t>(static_cast<uint32_t>(v));
                    st.dst[pos] = static_cast<int32_t>(static_cast<uint32_t>(v >> 32));
                    st.ts[pos] = static_cast<int64_t>(static_cast<uint64_t>(k) +
                                                      static_cast<uint64_t>(st.tmin));
                } else {
                    keys_out[pos] = k;
                    if (vals_out) vals_out[pos] = s_val[lp];
                }
            }
        }
        __syncthreads();  // s_cnt and the staging are reused by the next tile
    }
}

template <typename K, typename V>
size_t radix_scatter_lds(int R) {
    return (static_cast<size_t>(kWaves) + 2) * R * sizeof(uint32_t) +
           kSortTile * (sizeof(K) + sizeof(V));
}

// hist layout: nb * kMaxRadix per-workgroup counts, then kMaxPasses *
// kMaxRadix digit totals (one row per pass, cleared once per sort).
constexpr int kMaxPasses = (64 + kMaxDigitBits - 1) / kMaxDigitBits;

// Passes and digit width of a sort of `bits` key bits.
int sort_passes(int bits) { return (bits + kMaxDigitBits - 1) / kMaxDigitBits; }
int sort_digit_bits(int bits) {
    const int p = sort_passes(bits);
    return (bits + p - 1) / p;
}

template <typename K, typename V = uint32_t>
int radix_sort_impl(K* keys0, V* vals0, K* keys1, V* vals1, size_t n,
                    int begin_bit, int end_bit, uint32_t* hist, hipStream_t s,
                    const SortedStore* store = nullptr) {
    if (n <= 1 || end_bit <= begin_bit) return 0;
    const size_t nb = (n + kSortSpan - 1) / kSortSpan;
    const int passes = sort_passes(end_bit - begin_bit);
    const int db = sort_digit_bits(end_bit - begin_bit);
    const int R = 1 << db;
    uint32_t* totals = hist + nb * kMaxRadix;
    const size_t lds_up = static_cast<size_t>(kWaves) * R * sizeof(uint32_t);
    const size_t lds_sc = radix_scatter_lds<K, V>(R);
    int cur = 0;
    K* kb[2] = {keys0, keys1};
    V* vb[2] = {vals0, vals1};
    for (int pass = 0; pass < passes; ++pass) {
        const int bit = begin_bit + pass * db;
        // the last digit stops at end_bit
        const int w = end_bit - bit < db ? end_bit - bit : db;
        const uint32_t dmask = (1u << w) - 1u;
        uint32_t* tot = totals + pass * R;
        hipLaunchKernelGGL((radix_upsweep_kernel<K>), dim3(nb), dim3(kBlock), lds_up, s, kb[cur],
                           n, bit, db, dmask, hist, nb);
        hipLaunchKernelGGL(radix_digit_totals_kernel, dim3(R), dim3(kBlock), 0, s, hist, nb, tot);
        hipLaunchKernelGGL(radix_offsets_kernel, dim3(R), dim3(kBlock), 0, s, hist, nb, tot);
        if constexpr (std::is_same<V, uint64_t>::value) {
            if (store && pass == passes - 1) {
                hipLaunchKernelGGL((radix_scatter_kernel<K, V, true>), dim3(nb), dim3(kBlock),
                                   lds_sc, s, kb[cur], vb[cur], nullptr, nullptr, n, bit, db,
                                   dmask, hist, nb, *store);
                check_hip(hipGetLastError(), "radix sort launch");
                return cur ^ 1;
            }
        }
        hipLaunchKernelGGL((radix_scatter_kernel<K, V>), dim3(nb), dim3(kBlock), lds_sc, s,
                           kb[cur], vb[cur], kb[cur ^ 1], vb[cur ^ 1], n, bit, db, dmask, hist,
                           nb);
        check_hip(hipGetLastError(), "radix sort launch");
        cur ^= 1;
    }
    return cur;
}

// ---------------------------------------------------------------------------
// reductions (grid-stride, per-block partials, then one block)
// ---------------------------------------------------------------------------
constexpr int kReduceBlocks = 1024;

// min and max of v, and the smallest of the ids a[i], b[i] (INT64_MAX for
// n == 0): one pass over a batch's timestamps and endpoints
struct MinMaxId {
    int64_t mn, mx, id, idmax;
};

__device__ __forceinline__ MinMaxId minmax_id_join(MinMaxId x, MinMaxId y) {
    return {y.mn < x.mn ? y.mn : x.mn, y.mx > x.mx ? y.mx : x.mx, y.id < x.id ? y.id : x.id,
            y.idmax > x.idmax ? y.idmax : x.idmax};
}

__device__ __forceinline__ MinMaxId block_minmax_id(MinMaxId v, int64_t* sm) {
    int64_t* m = sm + 4 * threadIdx.x;
    m[0] = v.mn;
    m[1] = v.mx;
    m[2] = v.id;
    m[3] = v.idmax;
    __syncthreads();
    for (int st = kBlock / 2; st > 0; st >>= 1) {
        if (static_cast<int>(threadIdx.x) < st) {
            const int64_t* o = sm + 4 * (threadIdx.x + st);
            const MinMaxId r = minmax_id_join({m[0], m[1], m[2], m[3]}, {o[0], o[1], o[2], o[3]});
            m[0] = r.mn;
            m[1] = r.mx;
            m[2] = r.id;
            m[3] = r.idmax;
        }
        __syncthreads();
    }
    return {sm[0], sm[1], sm[2], sm[3]};
}

__global__ __launch_bounds__(kBlock) void minmax_partial_kernel(const int64_t* __restrict__ v,
                                                                const int32_t* __restrict__ a,
                                                                const int32_t* __restrict__ b,
                                                                size_t n, int64_t* part) {
    __shared__ int64_t sm[4 * kBlock];
    MinMaxId acc{INT64_MAX, INT64_MIN, INT64_MAX, INT64_MIN};
    for (size_t i = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * kBlock) {
        const int64_t x = v[i];
        const int32_t p = a[i], q = b[i];
        acc = minmax_id_join(acc, {x, x, min(p, q), max(p, q)});
    }
    const MinMaxId r = block_minmax_id(acc, sm);
    if (threadIdx.x == 0) {
        int64_t* o = part + 4 * blockIdx.x;
        o[0] = r.mn;
        o[1] = r.mx;
        o[2] = r.id;
        o[3] = r.idmax;
    }
}

__global__ __launch_bounds__(kBlock) void minmax_final_kernel(const int64_t* part, int np,
                                                              int64_t* out) {
    __shared__ int64_t sm[4 * kBlock];
    MinMaxId acc{INT64_MAX, INT64_MIN, INT64_MAX, INT64_MIN};
    for (int i = threadIdx.x; i < np; i += kBlock) {
        const int64_t* p = part + 4 * i;
        acc = minmax_id_join(acc, {p[0], p[1], p[2], p[3]});
    }
    const MinMaxId r = block_minmax_id(acc, sm);
    if (threadIdx.x == 0) {
        out[0] = r.mn;
        out[1] = r.mx;
        out[2] = r.id;
        out[3] = r.idmax;
    }
}

__global__ __launch_bounds__(kBlock) void max_pair_kernel(const int32_t* __restrict__ a,
                                                          const int32_t* __restrict__ b, size_t n,
                                                          int32_t* out) {
    __shared__ int32_t s[kBlock];
    int32_t mx = -1;
    for (size_t i = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * kBlock) {
        mx = max(mx, max(a[i], b[i]));
    }
    s[threadIdx.x] = mx;
    __syncthreads();
    for (int st = kBlock / 2; st > 0; st >>= 1) {
        if (static_cast<int>(threadIdx.x) < st) s[threadIdx.x] = max(s[threadIdx.x], s[threadIdx.x + st]);
        __syncthreads();
    }
    if (threadIdx.x == 0) atomicMax(out, s[0]);
}

__global__ void set_i32_kernel(int32_t* p, int32_t v) { *p = v; }

__global__ __launch_bounds__(kBlock) void sum_partial_kernel(const double* __restrict__ v,
                                                             size_t n, double* part) {
    __shared__ double s_wave[kWaves];
    double acc = 0.0;
    for (size_t i = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * kBlock) {
        acc += v[i];
    }
    const double tot = block_sum(acc, s_wave);
    if (threadIdx.x == 0) part[blockIdx.x] = tot;
}

__global__ __launch_bounds__(kBlock) void sum_final_kernel(const double* part, int np,
                                                           double* out) {
    __shared__ double s_wave[kWaves];
    double acc = 0.0;
    for (int i = threadIdx.x; i < np; i += kBlock) acc += part[i];
    const double tot = block_sum(acc, s_wave);
    if (threadIdx.x == 0) out[0] = tot;
}

int reduce_blocks(size_t n) {
    const size_t b = (n + kBlock - 1) / kBlock;
    return static_cast<int>(b < kReduceBlocks ? (b ? b : 1) : kReduceBlocks);
}

}  // namespace

size_t scan_scratch_elems(size_t n) { return (n + kScanTile - 1) / kScanTile + 1; }
size_t radix_hist_elems(size_t n) {
    return ((n + kSortSpan - 1) / kSortSpan) * kMaxRadix + kMaxPasses * kMaxRadix;
}

void exclusive_scan_u32(const uint32_t* in, uint32_t* out, size_t n, uint32_t* scratch,
                        hipStream_t s) {
    // the coalesced kernels need 16-byte aligned arrays
    if (n == 0 || (reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) % 16) {
        scan_impl<uint32_t, false>(in, out, n, scratch, s);
        return;
    }
    const size_t nb = (n + kScanTile - 1) / kScanTile;
    hipLaunchKernelGGL(scan_reduce_u32_kernel, dim3(nb), dim3(kBlock), 0, s, in, n, scratch);
    hipLaunchKernelGGL((scan_sums_kernel<uint32_t, OpSum>), dim3(1), dim3(kBlock), 0, s, scratch,
                       nb);
    hipLaunchKernelGGL(scan_apply_u32_kernel, dim3(nb), dim3(kBlock), 0, s, in, out, n, scratch);
    check_hip(hipGetLastError(), "scan launch");
}
void exclusive_scan_u64(const uint64_t* in, uint64_t* out, size_t n, uint64_t* scratch,
                        hipStream_t s) {
    scan_impl<uint64_t, false>(in, out, n, scratch, s);
}
void inclusive_scan_f64(double* data, size_t n, double* scratch, hipStream_t s) {
    scan_impl<double, true>(data, data, n, scratch, s);
}
void running_max_f64(double* data, size_t n, double* scratch, hipStream_t s) {
    scan_impl<double, true, OpMax>(data, data, n, scratch, s);
}

int radix_sort_u64(uint64_t* keys0, uint32_t* vals0, uint64_t* keys1, uint32_t* vals1, size_t n,
                   int begin_bit, int end_bit, uint32_t* hist, hipStream_t s) {
    return radix_sort_impl<uint64_t>(keys0, vals0, keys1, vals1, n, begin_bit, end_bit, hist, s);
}
int radix_sort_u32(uint32_t* keys0, uint32_t* vals0, uint32_t* keys1, uint32_t* vals1, size_t n,
                   int begin_bit, int end_bit, uint32_t* hist, hipStream_t s) {
    return radix_sort_impl<uint32_t>(keys0, vals0, keys1, vals1, n, begin_bit, end_bit, hist, s);
}
int radix_sort_u64_v64(uint64_t* keys0, uint64_t* vals0, uint64_t* keys1, uint64_t* vals1,
                       size_t n, int begin_bit, int end_bit, uint32_t* hist, hipStream_t s) {
    return radix_sort_impl<uint64_t, uint64_t>(keys0, vals0, keys1, vals1, n, begin_bit, end_bit,
                                               hist, s);
}
int radix_sort_u32_v64(uint32_t* keys0, uint64_t* vals0, uint32_t* keys1, uint64_t* vals1,
                       size_t n, int begin_bit, int end_bit, uint32_t* hist, hipStream_t s) {
    return radix_sort_impl<uint32_t, uint64_t>(keys0, vals0, keys1, vals1, n, begin_bit, end_bit,
                                               hist, s);
}
int radix_passes(int begin_bit, int end_bit) {
    return end_bit > begin_bit ? sort_passes(end_bit - begin_bit) : 0;
}
bool radix_sort_u32_v64_store(uint32_t* keys0, uint64_t* vals0, uint32_t* keys1, uint64_t* vals1,
                              size_t n, int begin_bit, int end_bit, uint32_t* hist, hipStream_t s,
                              const SortedStore& out) {
    if (n <= 1 || end_bit <= begin_bit) return false;
    radix_sort_impl<uint32_t, uint64_t>(keys0, vals0, keys1, vals1, n, begin_bit, end_bit, hist, s,
                                        &out);
    return true;
}
bool radix_sort_u64_v64_store(uint64_t* keys0, uint64_t* vals0, uint64_t* keys1, uint64_t* vals1,
                              size_t n, int begin_bit, int end_bit, uint32_t* hist, hipStream_t s,
                              const SortedStore& out) {
    if (n <= 1 || end_bit <= begin_bit) return false;
    radix_sort_impl<uint64_t, uint64_t>(keys0, vals0, keys1, vals1, n, begin_bit, end_bit, hist, s,
                                        &out);
    return true;
}

// Scratch for the reductions lives in a small per-call static device buffer
// provided by the caller through `out` (2 * kReduceBlocks int64 / doubles
// beyond out[0..1]).
void minmax_ts_min_id(const int64_t* v, const int32_t* a, const int32_t* b, size_t n, int64_t* out,
                      hipStream_t s) {
    const int nb = reduce_blocks(n);
    int64_t* part = out + 4;
    hipLaunchKernelGGL(minmax_partial_kernel, dim3(nb), dim3(kBlock), 0, s, v, a, b, n, part);
    hipLaunchKernelGGL(minmax_final_kernel, dim3(1), dim3(kBlock), 0, s, part, nb, out);
    check_hip(hipGetLastError(), "minmax launch");
}

void max_i32_pair(const int32_t* a, const int32_t* b, size_t n, int32_t* out, hipStream_t s) {
    hipLaunchKernelGGL(set_i32_kernel, dim3(1), dim3(1), 0, s, out, -1);
    if (n) {
        hipLaunchKernelGGL(max_pair_kernel, dim3(reduce_blocks(n)), dim3(kBlock), 0, s, a, b, n,
                           out);
    }
    check_hip(hipGetLastError(), "max launch");
}

void sum_f64(const double* v, size_t n, double* out, hipStream_t s) {
    const int nb = reduce_blocks(n);
    double* part = out + 2;
    hipLaunchKernelGGL(sum_partial_kernel, dim3(nb), dim3(kBlock), 0, s, v, n, part);
    hipLaunchKernelGGL(sum_final_kernel, dim3(1), dim3(kBlock), 0, s, part, nb, out);
    check_hip(hipGetLastError(), "sum launch");
}

}  // namespace trw
