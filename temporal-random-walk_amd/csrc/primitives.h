// primitives.h -- device-wide scan and stable radix sort for the index build.
//
// Hand-written for CDNA4 (wave64): no rocPRIM / hipCUB.  The radix sort is a
// classic LSD sort with four launches per digit pass (tile histograms; the
// digit totals, one workgroup per digit summing its histogram row; one
// workgroup per digit scanning that row; stable scatter); a sort of B key
// bits takes the fewest passes of at most 10-bit
// digits, the bits split evenly.  Stable ranking inside a tile uses wave-level
// multisplit: one 64-lane ballot per digit bit gives every lane the mask of
// lanes holding the same digit, so the in-row rank is a popcount and a single
// leader lane per digit bumps the wave's LDS counter.  Waves own
// consecutive rows of the tile, so the scatter keeps input order among equal
// digits -- which is what makes the edge-store order "stable by (timestamp,
// insertion position)" and the node index "stable by (node, position)".
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace trw {

void check_hip(hipError_t e, const char* what);

// ---- scan ------------------------------------------------------------------
// Exclusive scan of n values given by an input functor; writes n + 1 outputs,
// out[n] = total.  `scratch` must hold scan_scratch_elems(n) elements of T.
size_t scan_scratch_elems(size_t n);

// Exclusive scan of a plain array: out[0..n] (out may alias in only if
// out != in is not required: in-place is supported).
void exclusive_scan_u32(const uint32_t* in, uint32_t* out, size_t n, uint32_t* scratch,
                        hipStream_t s);
void exclusive_scan_u64(const uint64_t* in, uint64_t* out, size_t n, uint64_t* scratch,
                        hipStream_t s);
// Inclusive scan of doubles in place (out[i] = in[0] + ... + in[i]).
void inclusive_scan_f64(double* data, size_t n, double* scratch, hipStream_t s);
// Running maximum of doubles in place (out[i] = max(in[0..i])): makes a
// cumulative array non-decreasing to the last ulp, whatever order its partial
// sums were rounded in.
void running_max_f64(double* data, size_t n, double* scratch, hipStream_t s);

// ---- radix sort --------------------------------------------------------------
// Stable sort of (key, value) pairs by key bits [begin_bit, end_bit).  Values
// may be null (keys only).  Buffers are ping-ponged; the function returns 0 if
// the sorted result ended in (keys0, vals0) and 1 if in (keys1, vals1).
// `hist` must hold radix_hist_elems(n) uint32.
size_t radix_hist_elems(size_t n);
int radix_sort_u64(uint64_t* keys0, uint32_t* vals0, uint64_t* keys1, uint32_t* vals1, size_t n,
                   int begin_bit, int end_bit, uint32_t* hist, hipStream_t s);
int radix_sort_u32(uint32_t* keys0, uint32_t* vals0, uint32_t* keys1, uint32_t* vals1, size_t n,
                   int begin_bit, int end_bit, uint32_t* hist, hipStream_t s);
// 64- and 32-bit keys with 64-bit values (a record carried through the sort).
int radix_sort_u64_v64(uint64_t* keys0, uint64_t* vals0, uint64_t* keys1, uint64_t* vals1,
                       size_t n, int begin_bit, int end_bit, uint32_t* hist, hipStream_t s);
int radix_sort_u32_v64(uint32_t* keys0, uint64_t* vals0, uint32_t* keys1, uint64_t* vals1,
                       size_t n, int begin_bit, int end_bit, uint32_t* hist, hipStream_t s);
// Digit passes of a sort of bits [begin_bit, end_bit): the result lands in
// buffer set (passes % 2) when n > 1.
int radix_passes(int begin_bit, int end_bit);

// The edge store as the last pass of a sort of (timestamp key, packed
// endpoints) writes it: src = low half, dst = high half of the value, ts =
// key + tmin, each at the record's sorted position.
struct SortedStore {
    int32_t* src;
    int32_t* dst;
    int64_t* ts;
    int64_t tmin;
};
// radix_sort_u32_v64 / radix_sort_u64_v64 whose last digit pass writes `out`
// instead of the sorted keys and values (no pass of the store over them
// afterwards).  Returns false, writing nothing, when the sort has no pass
// (n <= 1 or no key bits): the input is then already in order.
bool radix_sort_u32_v64_store(uint32_t* keys0, uint64_t* vals0, uint32_t* keys1, uint64_t* vals1,
                              size_t n, int begin_bit, int end_bit, uint32_t* hist, hipStream_t s,
                              const SortedStore& out);
bool radix_sort_u64_v64_store(uint64_t* keys0, uint64_t* vals0, uint64_t* keys1, uint64_t* vals1,
                              size_t n, int begin_bit, int end_bit, uint32_t* hist, hipStream_t s,
                              const SortedStore& out);

// ---- reductions ---------------------------------------------------------------
// out[0], out[1] = min and max of v[0..n); out[2], out[3] = the smallest and
// the largest of a[i], b[i] (INT64_MAX / INT64_MIN when n == 0); out must hold
// minmax_scratch_elems() values
void minmax_ts_min_id(const int64_t* v, const int32_t* a, const int32_t* b, size_t n, int64_t* out,
                      hipStream_t s);
inline size_t minmax_scratch_elems() { return 4 + 4 * 1024; }
// max of two int32 arrays -> *out (device memory); -1 when n == 0.
void max_i32_pair(const int32_t* a, const int32_t* b, size_t n, int32_t* out, hipStream_t s);
// sum of doubles -> *out (device memory).
void sum_f64(const double* v, size_t n, double* out, hipStream_t s);

}  // namespace trw
