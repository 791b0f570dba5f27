// build.hip -- edge store and index build on the device.
//
// One ingest = one pass of this pipeline over the store (reference order,
// graph/temporal_graph.cu:158-220):
//   1. stable LSD radix sort of (ts - ts_min, position) over the old store
//      followed by the batch -- identical to the reference's "sort the batch,
//      stable-merge it after the old store" (temporal_graph.cu:67-134) because
//      the old store is already sorted and precedes the batch;
//   2. window eviction as an upper_bound on the sorted keys, folded into the
//      gather so evicted edges are never copied (temporal_graph.cu:136-156);
//   3. gather of src/dst/ts/features;
//   4. max node id, dense active flags (edge_data.cu:256-296);
//   5. timestamp groups by flag + scan + scatter (edge_data.cu:394-438);
//   6. per direction: stable radix sort of entries by node id, CSR offsets by
//      lower_bound, node-timestamp groups by flag + scan, per-node group counts
//      read straight off the flag scan at each node's first entry
//      (node_edge_index.cu:254-494);
//   7. node2vec adjacency (edge_data.cu:298-392) and weights
//      (edge_data.cu:440-514, node_edge_index.cu:500-684) when enabled.
// All of it is integer/byte work bound by HBM bandwidth; no MFMA.
#include <math.h>

#include <algorithm>

#include "engine.h"

namespace trw {
namespace {

constexpr int kB = 256;

inline unsigned grid_for(size_t n) {
    const size_t g = (n + kB - 1) / kB;
    return static_cast<unsigned>(g ? g : 1);
}

inline int bit_length_u64(uint64_t v) { return v ? 64 - __builtin_clzll(v) : 0; }

// Sort keys (ts - ts_min, 32-bit when the store's key range fits), positions,
// and each edge's endpoints packed into one 8-byte word, so that the gather
// after the sort costs one random load per edge instead of three.
template <typename K>
__global__ void make_ts_keys_kernel(const int64_t* __restrict__ old_ts,
                                    const int32_t* __restrict__ old_src,
                                    const int32_t* __restrict__ old_dst, size_t e_old,
                                    const int64_t* __restrict__ new_ts,
                                    const int32_t* __restrict__ new_src,
                                    const int32_t* __restrict__ new_dst, size_t n_new,
                                    int64_t tmin, K* __restrict__ keys,
                                    uint32_t* __restrict__ vals, uint64_t* __restrict__ ends) {
    const size_t i = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (i >= e_old + n_new) return;
    const bool old = i < e_old;
    const size_t k = old ? i : i - e_old;
    const int64_t t = old ? old_ts[k] : new_ts[k];
    const int32_t a = old ? old_src[k] : new_src[k];
    const int32_t b = old ? old_dst[k] : new_dst[k];
    keys[i] = static_cast<K>(static_cast<uint64_t>(t) - static_cast<uint64_t>(tmin));
    if (vals) vals[i] = static_cast<uint32_t>(i);
    ends[i] = static_cast<uint64_t>(static_cast<uint32_t>(a)) |
              (static_cast<uint64_t>(static_cast<uint32_t>(b)) << 32);
}

// out[0] = number of sorted keys <= target (upper_bound), out[1] = key at
// that position (or 0), out[2] = last key.  target < 0 means "none".
template <typename K>
__global__ void evict_search_kernel(const K* __restrict__ keys, size_t n, int64_t target,
                                    int64_t* out) {
    size_t del = 0;
    if (target >= 0) {
        size_t lo = 0, hi = n;
        const uint64_t t = static_cast<uint64_t>(target);
        while (lo < hi) {
            const size_t mid = lo + ((hi - lo) >> 1);
            if (t < static_cast<uint64_t>(keys[mid])) hi = mid;
            else lo = mid + 1;
        }
        del = lo;
    }
    out[0] = static_cast<int64_t>(del);
    out[1] = del < n ? static_cast<int64_t>(keys[del]) : 0;
    out[2] = n ? static_cast<int64_t>(keys[n - 1]) : 0;
}

// The kept suffix [del, del + kept) of the sorted order: the timestamp is the
// sorted key plus ts_min (exact in 64-bit wrap-around arithmetic), the
// endpoints one packed load at the edge's old position.
template <typename K>
__global__ void gather_store_kernel(const K* __restrict__ keys, const uint32_t* __restrict__ perm,
                                    const uint64_t* __restrict__ ends, size_t del, size_t kept,
                                    int64_t tmin, int32_t* __restrict__ s,
                                    int32_t* __restrict__ d, int64_t* __restrict__ t) {
    const size_t j = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (j >= kept) return;
    const uint64_t sd = ends[perm[del + j]];
    s[j] = static_cast<int32_t>(static_cast<uint32_t>(sd));
    d[j] = static_cast<int32_t>(static_cast<uint32_t>(sd >> 32));
    t[j] = static_cast<int64_t>(static_cast<uint64_t>(keys[del + j]) + static_cast<uint64_t>(tmin));
}

// The kept suffix when the endpoints travelled through the sort as its values:
// every read is in order.
template <typename K>
__global__ void store_from_sorted_kernel(const K* __restrict__ keys,
                                         const uint64_t* __restrict__ ends, size_t del,
                                         size_t kept, int64_t tmin, int32_t* __restrict__ s,
                                         int32_t* __restrict__ d, int64_t* __restrict__ t) {
    const size_t j = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (j >= kept) return;
    const uint64_t sd = ends[del + j];
    s[j] = static_cast<int32_t>(static_cast<uint32_t>(sd));
    d[j] = static_cast<int32_t>(static_cast<uint32_t>(sd >> 32));
    t[j] = static_cast<int64_t>(static_cast<uint64_t>(keys[del + j]) + static_cast<uint64_t>(tmin));
}

// Grid-stride over kept * dim values (can exceed one dispatch's 32-bit
// work-item count).
__global__ void gather_feat_kernel(const uint32_t* __restrict__ perm, size_t del, size_t kept,
                                   size_t dim, const float* __restrict__ of, size_t e_old,
                                   const float* __restrict__ nf, float* __restrict__ f) {
    const size_t total = kept * dim;
    const size_t stride = static_cast<size_t>(gridDim.x) * kB;
    for (size_t x = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x; x < total; x += stride) {
        const size_t j = x / dim, c = x - j * dim;
        const uint32_t id = perm[del + j];
        f[x] = id < e_old ? of[static_cast<size_t>(id) * dim + c]
                          : nf[(static_cast<size_t>(id) - e_old) * dim + c];
    }
}

// Same, 16 bytes per work-item for rows of dim % 4 == 0 floats in 16-byte
// aligned arrays: a workgroup of V * R threads (V = dim / 4 vectors per row,
// R = 256 / V rows) covers R consecutive rows, grid-stride over rows.
typedef float f32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void gather_feat_vec_kernel(
    const uint32_t* __restrict__ perm, size_t del, size_t kept, uint32_t V,
    const f32x4* __restrict__ of, size_t e_old, const f32x4* __restrict__ nf,
    f32x4* __restrict__ f) {
    const uint32_t R = blockDim.x / V;
    const uint32_t c = threadIdx.x % V, r = threadIdx.x / V;
    if (r >= R) return;
    for (size_t j = blockIdx.x * static_cast<size_t>(R) + r; j < kept;
         j += static_cast<size_t>(gridDim.x) * R) {
        const uint32_t id = perm[del + j];
        const f32x4 v = id < e_old ? of[static_cast<size_t>(id) * V + c]
                                   : nf[(static_cast<size_t>(id) - e_old) * V + c];
        f[j * V + c] = v;
    }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline unsigned grid_capped(size_t n) {
    const size_t g = (n + kB - 1) / kB;
    return static_cast<unsigned>(g == 0 ? 1 : (g > (1u << 20) ? (1u << 20) : g));
}

__global__ void ts_group_flags_kernel(const int64_t* __restrict__ ts, size_t n,
                                      uint32_t* __restrict__ flags) {
    const size_t i = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (i >= n) return;
    flags[i] = (i == 0 || ts[i] != ts[i - 1]) ? 1u : 0u;
}

__global__ void ts_group_scatter_kernel(const int64_t* __restrict__ ts, size_t n,
                                        const uint32_t* __restrict__ flags,
                                        const uint32_t* __restrict__ scan,
                                        uint32_t* __restrict__ off, int64_t* __restrict__ uq,
                                        uint32_t* __restrict__ erank) {
    const size_t i = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (i >= n) return;
    // exclusive scan of the group-start flags: the group index of position i
    erank[i] = scan[i] + flags[i] - 1u;
    if (flags[i]) {
        off[scan[i]] = static_cast<uint32_t>(i);
        uq[scan[i]] = ts[i];
    }
    if (i == n - 1) off[scan[n]] = static_cast<uint32_t>(n);
}

// Rank of timestamp -1 among the unique timestamps, or -2 when no edge has it:
// the walk compares ranks with it for the reference's `ts == -1` tests.
__global__ void neg1_rank_kernel(const int64_t* __restrict__ uq, uint32_t T,
                                 int32_t* __restrict__ out) {
    uint32_t lo = 0, hi = T;
    while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        if (uq[mid] < -1) lo = mid + 1;
        else hi = mid;
    }
    *out = (lo < T && uq[lo] == -1) ? static_cast<int32_t>(lo) : -2;
}

// Node-index entries: key = the list's node, value = the entry's walk record
// (neighbour in the low word, edge id in the high word: EdgeRec's layout),
// carried through the node sort so no record needs a gather afterwards.
// mode 0: out-lists (node = source, neighbour = target); 1: in-lists (node =
// target, neighbour = source); 2: undirected, entry 2i = (src_i; dst_i) and
// entry 2i+1 = (dst_i; src_i) (node_edge_index.cu:306-321) -- the neighbour is
// the reference's pick_other_number (utils/utils.cuh:102-104) seen from the
// entry's node.
__device__ __forceinline__ uint64_t pack_rec(int32_t nbr, uint32_t eid) {
    return static_cast<uint64_t>(static_cast<uint32_t>(nbr)) | (static_cast<uint64_t>(eid) << 32);
}

// The edges are src/dst[0, e); their edge ids (store positions) start at id0.
// With erank given, a value packs the neighbour, the edge id and the edge's
// timestamp rank into one word (nbr | eid << nb | rank << (nb + eb); the caller
// checks that they fit), so that the entries leave the node sort with their
// ranks and the group flags need no gather of erank in node order.
__global__ void node_entries_kernel(const int32_t* __restrict__ src,
                                    const int32_t* __restrict__ dst, size_t e, int mode,
                                    uint32_t id0, const uint32_t* __restrict__ erank, int nb,
                                    int eb, uint32_t* __restrict__ keys,
                                    uint64_t* __restrict__ vals) {
    const size_t i = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (i >= e) return;
    const int32_t a = src[i], b = dst[i];
    const uint32_t id = id0 + static_cast<uint32_t>(i);
    uint64_t va, vb;
    if (erank) {
        const uint64_t hi = (static_cast<uint64_t>(id) << nb) |
                            (static_cast<uint64_t>(erank[id]) << (nb + eb));
        va = hi | static_cast<uint32_t>(b);  // entry of a (out / first), neighbour b
        vb = hi | static_cast<uint32_t>(a);
    } else {
        va = pack_rec(b, id);
        vb = pack_rec(a, id);
    }
    if (mode == 0) {
        keys[i] = static_cast<uint32_t>(a);
        vals[i] = va;
    } else if (mode == 1) {
        keys[i] = static_cast<uint32_t>(b);
        vals[i] = vb;
    } else {
        keys[2 * i] = static_cast<uint32_t>(a);
        vals[2 * i] = va;
        keys[2 * i + 1] = static_cast<uint32_t>(b);
        vals[2 * i + 1] = vb;
    }
}

// off[u] = first sorted position whose node >= u, u in [0, vc).
__global__ void lower_bound_offsets_kernel(const uint32_t* __restrict__ keys, size_t n, size_t vc,
                                           uint32_t* __restrict__ off) {
    const size_t u = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (u >= vc) return;
    size_t lo = 0, hi = n;
    while (lo < hi) {
        const size_t mid = lo + ((hi - lo) >> 1);
        if (keys[mid] < u) lo = mid + 1;
        else hi = mid;
    }
    off[u] = static_cast<uint32_t>(lo);
}

// ---- append path: a batch whose timestamps are all >= the store's ----------
// The stable order by (timestamp, position) then puts the batch, sorted, after
// the store's kept edges, and every node's list keeps its old entries first:
// the store and the node index are updated by copies and scatters instead of
// sorts of the whole window.

// Eviction over the store old[0, e_old) followed by the sorted batch (keys +
// tmin): out[0] = evicted store edges, out[1] = evicted batch edges, out[2] /
// out[3] = the first / last kept timestamp.  cutoff: drop ts <= cutoff.
template <typename K>
__global__ void append_evict_kernel(const int64_t* __restrict__ old_ts, size_t e_old,
                                    const K* __restrict__ keys, size_t n, int64_t tmin,
                                    int64_t cutoff, int has_cutoff, int64_t* __restrict__ out) {
    size_t del_old = 0, del_new = 0;
    if (has_cutoff) {
        size_t lo = 0, hi = e_old;  // upper_bound
        while (lo < hi) {
            const size_t mid = lo + ((hi - lo) >> 1);
            if (cutoff < old_ts[mid]) hi = mid;
            else lo = mid + 1;
        }
        del_old = lo;
        if (del_old == e_old && cutoff >= tmin) {
            const uint64_t t = static_cast<uint64_t>(cutoff) - static_cast<uint64_t>(tmin);
            lo = 0;
            hi = n;
            while (lo < hi) {
                const size_t mid = lo + ((hi - lo) >> 1);
                if (t < static_cast<uint64_t>(keys[mid])) hi = mid;
                else lo = mid + 1;
            }
            del_new = lo;
        }
    }
    out[0] = static_cast<int64_t>(del_old);
    out[1] = static_cast<int64_t>(del_new);
    const int64_t last_new = static_cast<int64_t>(static_cast<uint64_t>(keys[n - 1]) +
                                                  static_cast<uint64_t>(tmin));
    // the cut can empty the batch too (a window ending before every timestamp)
    out[2] = del_old < e_old ? old_ts[del_old]
             : del_new < n   ? static_cast<int64_t>(static_cast<uint64_t>(keys[del_new]) +
                                                    static_cast<uint64_t>(tmin))
                             : 0;
    out[3] = del_new < n ? last_new : 0;
}

// ev[u] = entries of node u in the old index whose edge was evicted (edge id
// < del).  A node's list is ordered by edge id, so they are a prefix of it, and
// the prefix's last entry writes the count (nodes without one keep the 0 of
// the fill; no atomics, so a hub costs one write).
__global__ void evicted_prefix_kernel(const uint32_t* __restrict__ keys,
                                      const EdgeRec* __restrict__ rec, size_t n, uint32_t del,
                                      const uint32_t* __restrict__ off, uint32_t* __restrict__ ev) {
    const size_t k = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (k >= n || rec[k].eid >= del) return;
    const uint32_t u = keys[k];
    if (k + 1 == n || keys[k + 1] != u || rec[k + 1].eid >= del)
        ev[u] = static_cast<uint32_t>(k + 1) - off[u];
}

// Kept old entries of node u (0 past the old index's nodes).
__device__ __forceinline__ uint32_t kept_old(const uint32_t* off_old, size_t v_old,
                                             const uint32_t* ev, size_t u) {
    return u < v_old ? off_old[u + 1] - off_old[u] - ev[u] : 0u;
}

// Entries of node u in the updated index, u in [0, v): its kept old entries
// plus its batch entries (bstart: the batch's sorted-key offsets).
__global__ void append_counts_kernel(const uint32_t* __restrict__ off_old, size_t v_old,
                                     const uint32_t* __restrict__ ev,
                                     const uint32_t* __restrict__ bstart, size_t v,
                                     uint32_t* __restrict__ cnt) {
    const size_t u = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (u >= v) return;
    cnt[u] = kept_old(off_old, v_old, ev, u) + bstart[u + 1] - bstart[u];
}

// Old entry k of node u, if its edge is kept, moves to
// off[u] + (k - off_old[u] - ev[u]) with its edge id lowered by del.
__global__ void append_old_entries_kernel(const uint32_t* __restrict__ keys_old,
                                          const EdgeRec* __restrict__ rec_old, size_t n_old,
                                          uint32_t del, const uint32_t* __restrict__ off_old,
                                          const uint32_t* __restrict__ ev,
                                          const uint32_t* __restrict__ off,
                                          uint32_t* __restrict__ keys, EdgeRec* __restrict__ rec) {
    const size_t k = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (k >= n_old) return;
    const EdgeRec r = rec_old[k];
    if (r.eid < del) return;
    const uint32_t u = keys_old[k];
    const uint32_t d = off[u] + (static_cast<uint32_t>(k) - off_old[u] - ev[u]);
    keys[d] = u;
    rec[d] = EdgeRec{r.nbr, r.eid - del};
}

// Batch entry j (sorted stably by node) of node u follows u's kept old
// entries: off[u] + kept_old(u) + (j - bstart[u]).
__global__ void append_new_entries_kernel(const uint32_t* __restrict__ bkeys,
                                          const uint64_t* __restrict__ brec, size_t m,
                                          const uint32_t* __restrict__ bstart,
                                          const uint32_t* __restrict__ off_old, size_t v_old,
                                          const uint32_t* __restrict__ ev,
                                          const uint32_t* __restrict__ off,
                                          uint32_t* __restrict__ keys, EdgeRec* __restrict__ rec) {
    const size_t j = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (j >= m) return;
    const uint32_t u = bkeys[j];
    const uint32_t d = off[u] + kept_old(off_old, v_old, ev, u) + (static_cast<uint32_t>(j) - bstart[u]);
    keys[d] = u;
    const uint64_t b = brec[j];
    rec[d] = EdgeRec{static_cast<int32_t>(static_cast<uint32_t>(b)), static_cast<uint32_t>(b >> 32)};
}

// ---- merge path: a batch reaching back before the store's last timestamp ----
// The stable (timestamp, position) order of store + batch interleaves the two
// sorted runs -- the store's and the batch's, sorted alone -- with a store edge
// first on equal timestamps.  Each kept edge finds its place by counting the
// other run's kept edges before it (one binary search), so the store moves by
// one scatter instead of a sort of the whole window.  (The node index is
// rebuilt: the same co-rank merge of every node's old and batch entries took
// longer than the node sort it replaces.)

// Number of sorted batch keys k[lo, hi) (timestamp - btmin) whose timestamp is
// below t (strict: lower_bound) or at most t (upper_bound).
template <typename K>
__device__ __forceinline__ size_t batch_rank(const K* __restrict__ k, size_t lo, size_t hi,
                                             int64_t btmin, int64_t t, bool strict) {
    if (t < btmin || (strict && t == btmin)) return lo;
    const uint64_t x = static_cast<uint64_t>(t) - static_cast<uint64_t>(btmin);
    while (lo < hi) {
        const size_t mid = lo + ((hi - lo) >> 1);
        const uint64_t y = static_cast<uint64_t>(k[mid]);
        if (strict ? y < x : y <= x) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// Upper_bound of t over the store's timestamps ts[lo, hi).
__device__ __forceinline__ size_t store_rank(const int64_t* __restrict__ ts, size_t lo, size_t hi,
                                             int64_t t) {
    while (lo < hi) {
        const size_t mid = lo + ((hi - lo) >> 1);
        if (ts[mid] <= t) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// Eviction of the merge: out[0] / out[1] = evicted store / batch edges (those
// with ts <= cutoff: a prefix of each run), out[2] / out[3] = first / last kept
// timestamp (0 when nothing is kept).
template <typename K>
__global__ void merge_evict_kernel(const int64_t* __restrict__ old_ts, size_t e_old,
                                   const K* __restrict__ keys, size_t n, int64_t btmin,
                                   int64_t cutoff, int64_t* __restrict__ out) {
    const size_t del_old = store_rank(old_ts, 0, e_old, cutoff);
    const size_t del_new = batch_rank(keys, 0, n, btmin, cutoff, false);
    const auto bts = [&](size_t j) {
        return static_cast<int64_t>(static_cast<uint64_t>(keys[j]) + static_cast<uint64_t>(btmin));
    };
    int64_t first = 0, last = 0;
    if (del_old < e_old && del_new < n) {
        first = old_ts[del_old] <= bts(del_new) ? old_ts[del_old] : bts(del_new);
        last = old_ts[e_old - 1] >= bts(n - 1) ? old_ts[e_old - 1] : bts(n - 1);
    } else if (del_old < e_old) {
        first = old_ts[del_old];
        last = old_ts[e_old - 1];
    } else if (del_new < n) {
        first = bts(del_new);
        last = bts(n - 1);
    }
    out[0] = static_cast<int64_t>(del_old);
    out[1] = static_cast<int64_t>(del_new);
    out[2] = first;
    out[3] = last;
}

// Kept store edge i goes to (i - del_old) + (kept batch edges with a smaller
// timestamp).  perm (the feature gather's source, store ids first) is written
// when given.
template <typename K>
__global__ void merge_old_kernel(const int64_t* __restrict__ old_ts,
                                 const int32_t* __restrict__ old_src,
                                 const int32_t* __restrict__ old_dst, size_t del_old, size_t e_old,
                                 const K* __restrict__ keys, size_t del_new, size_t n,
                                 int64_t btmin, int32_t* __restrict__ s, int32_t* __restrict__ d,
                                 int64_t* __restrict__ t, uint32_t* __restrict__ perm) {
    const size_t i = del_old + blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (i >= e_old) return;
    const int64_t ti = old_ts[i];
    const size_t p = (i - del_old) + (batch_rank(keys, del_new, n, btmin, ti, true) - del_new);
    s[p] = old_src[i];
    d[p] = old_dst[i];
    t[p] = ti;
    if (perm) perm[p] = static_cast<uint32_t>(i);
}

// Kept batch edge j (sorted position) goes to (j - del_new) + (kept store
// edges with a timestamp <= its own).  Its endpoints come packed: sorted with
// the keys (bpos == nullptr), or by batch position bpos[j].
template <typename K>
__global__ void merge_new_kernel(const int64_t* __restrict__ old_ts, size_t del_old, size_t e_old,
                                 const K* __restrict__ keys, const uint64_t* __restrict__ ends,
                                 const uint32_t* __restrict__ bpos, size_t del_new, size_t n,
                                 int64_t btmin, int32_t* __restrict__ s, int32_t* __restrict__ d,
                                 int64_t* __restrict__ t, uint32_t* __restrict__ perm) {
    const size_t j = del_new + blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (j >= n) return;
    const int64_t tj =
        static_cast<int64_t>(static_cast<uint64_t>(keys[j]) + static_cast<uint64_t>(btmin));
    const size_t p = (j - del_new) + (store_rank(old_ts, del_old, e_old, tj) - del_old);
    const uint64_t sd = bpos ? ends[bpos[j]] : ends[j];
    s[p] = static_cast<int32_t>(static_cast<uint32_t>(sd));
    d[p] = static_cast<int32_t>(static_cast<uint32_t>(sd >> 32));
    t[p] = tj;
    if (perm) perm[p] = static_cast<uint32_t>(e_old) + bpos[j];
}

// Group-start flags of the sorted entries (a new node, or a new timestamp
// rank within a node) and the sorted edge ids (node_ts_sorted_*_indices).  The
// previous entry's node and rank come from the lane below.
__global__ __launch_bounds__(kB) void node_group_flags_kernel(const uint32_t* __restrict__ keys,
                                                              const EdgeRec* __restrict__ rec,
                                                              const uint32_t* __restrict__ erank,
                                                              size_t n,
                                                              uint32_t* __restrict__ flags,
                                                              uint32_t* __restrict__ idx,
                                                              uint32_t* __restrict__ rank) {
    const size_t k = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (k >= n) return;  // the active lanes of a wave are a prefix
    const uint32_t key = keys[k];
    const uint32_t e = rec[k].eid;
    const uint32_t r = erank[e];
    idx[k] = e;
    rank[k] = r;
    uint32_t kp = __shfl_up(key, 1, 64), rp = __shfl_up(r, 1, 64);
    if ((threadIdx.x & 63) == 0 && k > 0) {
        kp = keys[k - 1];
        rp = erank[rec[k - 1].eid];
    }
    flags[k] = (k == 0 || key != kp || r != rp) ? 1u : 0u;
}

// node_group_flags_kernel for entries whose sorted values carry their ranks
// (node_entries_kernel with erank): also unpacks the walk records.
__global__ __launch_bounds__(kB) void node_group_flags_packed_kernel(
    const uint32_t* __restrict__ keys, const uint64_t* __restrict__ packed, size_t n, int nb,
    int eb, uint32_t* __restrict__ flags, uint32_t* __restrict__ idx,
    uint32_t* __restrict__ rank, EdgeRec* __restrict__ rec) {
    const size_t k = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (k >= n) return;  // the active lanes of a wave are a prefix
    const uint32_t key = keys[k];
    const uint64_t v = packed[k];
    const uint32_t e = static_cast<uint32_t>((v >> nb) & ((1ull << eb) - 1ull));
    const uint32_t r = static_cast<uint32_t>(v >> (nb + eb));
    rec[k] = EdgeRec{static_cast<int32_t>(static_cast<uint32_t>(v & ((1ull << nb) - 1ull))), e};
    idx[k] = e;
    rank[k] = r;
    uint32_t kp = __shfl_up(key, 1, 64), rp = __shfl_up(r, 1, 64);
    if ((threadIdx.x & 63) == 0 && k > 0) {
        kp = keys[k - 1];
        rp = static_cast<uint32_t>(packed[k - 1] >> (nb + eb));
    }
    flags[k] = (k == 0 || key != kp || r != rp) ? 1u : 0u;
}

// Group starts, panel records and (for the weights, when first_ts is given)
// each group's timestamp, from the flags, their scan and the entries' ranks
// (all read in entry order).
__global__ void node_group_scatter_kernel(const uint32_t* __restrict__ flags,
                                          const uint32_t* __restrict__ scan,
                                          const uint32_t* __restrict__ rank,
                                          const int64_t* __restrict__ uniq_ts, size_t n,
                                          uint32_t* __restrict__ grp,
                                          int64_t* __restrict__ first_ts,
                                          PanelRec* __restrict__ pan) {
    const size_t k = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (k >= n) return;
    if (flags[k]) {
        const uint32_t g = scan[k];
        const uint32_t r = rank[k];
        grp[g] = static_cast<uint32_t>(k);
        if (first_ts) first_ts[g] = uniq_ts[r];
        pan[g] = PanelRec{r, static_cast<uint32_t>(k)};
    }
    if (k == n - 1) {
        grp[scan[n]] = static_cast<uint32_t>(n);
        pan[scan[n]] = PanelRec{0xffffffffu, static_cast<uint32_t>(n)};
    }
}

// cnt[u] = number of groups of nodes < u = flag scan at u's first entry.
__global__ void node_group_counts_kernel(const uint32_t* __restrict__ off,
                                         const uint32_t* __restrict__ scan, size_t vc,
                                         uint32_t* __restrict__ cnt) {
    const size_t u = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (u >= vc) return;
    cnt[u] = scan[off[u]];
}

// Bucket shift of a node with G > kTabMin groups whose ranks span `span`:
// the smallest power-of-two bucket width giving at most kTabBucketsPerGroup * G
// buckets.  A hub holding most ranks of its span gets width 1.
__device__ __forceinline__ uint32_t table_shift(uint32_t G, uint32_t span) {
    const uint64_t target = static_cast<uint64_t>(G) * kTabBucketsPerGroup;
    uint32_t shift = 0;
    while ((span >> shift) + 1ull > target) ++shift;
    return shift;
}

__global__ void node_headers_kernel(const uint32_t* __restrict__ cnt,
                                    const PanelRec* __restrict__ pan, size_t vc,
                                    NodeHdr* __restrict__ hdr) {
    const size_t u = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (u >= vc) return;
    const uint32_t gb = cnt[u];
    NodeHdr h{gb, 0, 0, 0};
    if (u + 1 < vc) {
        const uint32_t G = cnt[u + 1] - gb;
        uint32_t shift = 0, dense = 0;
        if (G > kTabMin) {
            h.r0 = pan[gb].rank;
            const uint32_t span = pan[gb + G - 1].rank - h.r0;
            shift = table_shift(G, span);
            h.nb = (span >> shift) + 1;
            // ranks are distinct and increasing, so G == span + 1 means every
            // rank of the span has a group: group i has rank r0 + i
            if (span == G - 1) dense = kHdrDense;
        }
        h.meta = (G < kHdrGMask ? G : kHdrGMask) | (shift << 24) | dense;
    }
    hdr[u] = h;
}

// One thread per group: group i of node u (local index) fills the buckets
// from the one after its predecessor's bucket up to its own; the last group
// also writes the closing entry G.
__global__ void node_table_fill_kernel(const uint32_t* __restrict__ key,
                                       const uint32_t* __restrict__ grp,
                                       const NodeHdr* __restrict__ hdr,
                                       const PanelRec* __restrict__ pan, size_t ng,
                                       uint32_t* __restrict__ tab) {
    const size_t g = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (g >= ng) return;
    const uint32_t u = key[grp[g]];
    const NodeHdr h = hdr[u];
    const uint32_t G = hdr[u + 1].gb - h.gb;
    if (G <= kTabMin || (h.meta & kHdrDense)) return;  // dense nodes need no table
    const uint32_t shift = hdr_shift(h);
    uint32_t* t = tab + hdr_tab_base(h, u);
    const uint32_t i = static_cast<uint32_t>(g) - h.gb;
    const uint32_t bi = (pan[g].rank - h.r0) >> shift;
    const uint32_t from = i == 0 ? 0u : ((pan[g - 1].rank - h.r0) >> shift) + 1;
    for (uint32_t b = from; b <= bi; ++b) t[b] = i;
    if (i == G - 1) t[bi + 1] = G;
}

// Guide parameters (index_layout.h) of the segment c[0, G): the smallest
// bucket shift (at least 4, so the first bucket's key fits 58 bits) that gives
// at most kWgBucketsPerGroup * G buckets over the segment's keys.
__device__ __forceinline__ WGuide make_guide(const double* c, uint32_t G, bool decaying) {
    WGuide gd{0, G ? c[G - 1] : 0.0};
    if (G > kWGuideMin) {
        const int64_t kf = wg_key(c[0], decaying), kl = wg_key(c[G - 1], decaying);
        const int64_t lim = std::min<int64_t>(static_cast<int64_t>(G) * kWgBucketsPerGroup,
                                              0xfffffffeLL);
        int sh = 4;
        while ((kl >> sh) - (kf >> sh) + 1 > lim) ++sh;
        gd.bs = (static_cast<uint64_t>(kf >> sh) << 6) | static_cast<uint64_t>(sh);
    }
    return gd;
}

// The weight pickers' node headers: the walk header of every node and the
// guide of its cumulative weights (the terminator entry V_c - 1 has none).
__global__ void whdr_kernel(const double* __restrict__ w, const uint32_t* __restrict__ cnt,
                            const NodeHdr* __restrict__ hdr, size_t vc, int decaying,
                            WNodeHdr* __restrict__ out) {
    const size_t u = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (u >= vc) return;
    const uint32_t gb = cnt[u];
    const uint32_t G = u + 1 < vc ? cnt[u + 1] - gb : 0u;
    out[u] = WNodeHdr{hdr[u], make_guide(w + gb, G, decaying != 0)};
}

// The guide of a global cumulative array (one segment).
__global__ void global_guide_kernel(const double* __restrict__ w, size_t n, int decaying,
                                    WGuide* __restrict__ out) {
    out[0] = make_guide(w, static_cast<uint32_t>(n), decaying != 0);
}

// The weighted panel: every group's panel record with its end, cumulative
// weight and first edge record (with that entry's next slice bound).  rsh:
// the weighted records' shift (1: each followed by its forward start sum).
// wide (shift 1; forward weights, over such records): each panel record is
// followed by its slot (index_layout.h, WPanelSlot): the start sum of its first
// entry's next slice, copied from that entry's record, and the group's second
// entry.
__global__ void wpan_kernel(const PanelRec* __restrict__ pan, const double* __restrict__ w,
                            const WEdgeRec* __restrict__ wrec, int rsh, size_t ng, int wide,
                            WPanelRec* __restrict__ out) {
    const size_t g = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (g >= ng) return;
    const PanelRec p = pan[g];
    const WEdgeRec* rp = wrec + (static_cast<size_t>(p.start) << rsh);
    const WEdgeRec r = *rp;
    const uint32_t end = pan[g + 1].start;
    out[g << wide] = WPanelRec{p.rank, p.start, end, r.nxt, w[g], EdgeRec{r.nbr, r.eid}};
    if (wide) {
        WPanelSlot sl{*reinterpret_cast<const double*>(rp + 1), EdgeRec{0, 0}, kNoNext, 0u, kNoSum};
        if (end - p.start >= 2) {
            const WEdgeRec r1 = rp[2];  // entry start + 1 and its sum
            sl.rec1 = EdgeRec{r1.nbr, r1.eid};
            sl.nxt1 = r1.nxt;
            sl.bs1 = *reinterpret_cast<const double*>(rp + 3);
        }
        *reinterpret_cast<WPanelSlot*>(out + (g << 1) + 1) = sl;
    }
}

// The forward start sums of the out direction's wide records (index_layout.h):
// each entry's next slice's c[vb - 1] in the forward weights w.
__global__ void entry_sums_kernel(WEdgeRec* __restrict__ wrec, const double* __restrict__ w,
                                  size_t n) {
    const size_t k = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (k >= n) return;
    const uint32_t nxt = wrec[k << 1].nxt;
    double bs = kNoSum;
    if (nxt != kNoNext) bs = next_bound_first<true>(nxt) ? 0.0 : w[next_bound<true>(nxt) - 1];
    *reinterpret_cast<double*>(wrec + (k << 1) + 1) = bs;
}

// The weighted records of a direction (index_layout.h, WEdgeRec): entry k's
// record, and the lower_bound of its timestamp rank among its neighbour's
// groups -- the walk's own time search (first_ge) over the direction's
// finished headers, bucket tables and panel -- with the flag of a group at
// that rank.  rank: the entries' timestamp ranks.
__global__ __launch_bounds__(kB) void entry_bounds_kernel(
    const EdgeRec* __restrict__ rec, const uint32_t* __restrict__ rank,
    const NodeHdr* __restrict__ hdr, const uint32_t* __restrict__ tab,
    const PanelRec* __restrict__ pan, size_t n, size_t vc, int sh, WEdgeRec* __restrict__ out) {
    const size_t k = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (k >= n) return;
    const EdgeRec r = rec[k];
    const uint32_t x = rank[k];
    const uint32_t v = static_cast<uint32_t>(r.nbr);
    uint32_t nxt = kNoNext;
    if (static_cast<size_t>(v) + 1 < vc) {
        const NodeHdr h = hdr[v];
        uint32_t G = h.meta & kHdrGMask;
        if (G == kHdrGMask) G = hdr[v + 1].gb - h.gb;
        const PanelRec* f = pan + h.gb;
        // first_ge's answer b, with the flag read where it costs no line: a
        // dense node has a group at every rank of its span, and a
        // single-rank bucket's next entry moves past b exactly when one of
        // the node's groups has rank x (the 8-byte load the walk's search
        // makes anyway; the closing entry follows the last bucket)
        int b;
        bool at;
        const uint32_t shift = hdr_shift(h);
        if (G > kTabMin && x > h.r0 && !(h.meta & kHdrDense) && shift == 0) {
            const uint32_t bk = x - h.r0;
            if (bk >= h.nb) {
                b = static_cast<int>(G);
                at = false;
            } else {
                const u32x2_a4 br =
                    *reinterpret_cast<const u32x2_a4*>(tab + hdr_tab_base(h, v) + bk);
                b = static_cast<int>(br.x);
                at = br.y > br.x;
            }
        } else if (G > kTabMin && x >= h.r0 && (h.meta & kHdrDense)) {
            b = static_cast<int>(min(x - h.r0, G));
            at = x - h.r0 < G;
        } else {
            b = first_ge(tab, h, v, static_cast<int>(G), f, x);
            at = b < static_cast<int>(G) && f[b].rank == x;
        }
        const uint64_t gl = static_cast<uint64_t>(h.gb) + static_cast<uint32_t>(b);
        if (gl <= kNextMax)
            nxt = static_cast<uint32_t>(gl) | (b == 0 ? kNextFirst : 0u) | (at ? kNextAt : 0u);
    }
    out[k << sh] = WEdgeRec{r.nbr, r.eid, nxt, 0u};
}

// The buckets [from, to] of group g (local index i of a segment of G): those
// after its predecessor's bucket up to its own, all of which first reach group
// i.  Segments are the nodes of a direction (key, grp, cnt, whdr) or, with
// key == nullptr, the whole array under the guide gg.
struct WgRun {
    uint32_t* t;  // the segment's table (nullptr: none)
    uint32_t i, from, to, G;
};
__device__ __forceinline__ WgRun wg_run(const double* w, const uint32_t* key, const uint32_t* grp,
                                        const uint32_t* cnt, const WNodeHdr* whdr,
                                        const WGuide* gg, size_t ng, int decaying, uint32_t* tab,
                                        size_t g) {
    uint32_t u = 0, gb = 0, G = static_cast<uint32_t>(ng);
    uint64_t bs;
    if (key) {
        u = key[grp[g]];
        gb = cnt[u];
        G = cnt[u + 1] - gb;
        bs = whdr[u].g.bs;
    } else {
        bs = gg->bs;
    }
    WgRun r{nullptr, 0, 0, 0, G};
    if (G <= kWGuideMin) return r;
    r.t = tab + (key ? 2ull * (static_cast<uint64_t>(gb) + u) : 0ull);
    r.i = static_cast<uint32_t>(g) - gb;
    r.to = wg_bucket(bs, wg_key(w[g], decaying != 0));
    r.from = r.i == 0 ? 0u : wg_bucket(bs, wg_key(w[g - 1], decaying != 0)) + 1;
    return r;
}

// One thread per group writes its run of buckets, or -- for a run longer than
// kWgRun -- lists the group for wg_long_kernel; the segment's last group also
// writes the closing entry G after its own bucket, the last.
__global__ void wg_fill_kernel(const double* __restrict__ w, const uint32_t* __restrict__ key,
                               const uint32_t* __restrict__ grp, const uint32_t* __restrict__ cnt,
                               const WNodeHdr* __restrict__ whdr, const WGuide* __restrict__ gg,
                               size_t ng, int decaying, uint32_t* __restrict__ tab,
                               uint32_t* __restrict__ longs) {
    const size_t g = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (g >= ng) return;
    const WgRun r = wg_run(w, key, grp, cnt, whdr, gg, ng, decaying, tab, g);
    if (r.t == nullptr) return;
    // the wave's long runs join the list with one atomic (a device-scope
    // atomic per run on one counter serialises beyond the XCDs' L2s)
    const bool is_long = r.to + 1 > r.from + kWgRun;
    const uint64_t lm = __ballot(is_long);
    if (lm != 0) {
        const int lane = __lane_id(), leader = __ffsll(static_cast<long long>(lm)) - 1;
        uint32_t base = 0;
        if (lane == leader) base = atomicAdd(longs, static_cast<uint32_t>(__popcll(lm)));
        base = __shfl(base, leader, 64);
        const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
        if (is_long) longs[1 + base + __popcll(lm & below)] = static_cast<uint32_t>(g);
    }
    if (!is_long)
        for (uint32_t b = r.from; b <= r.to; ++b) r.t[b] = r.i;
    if (r.i == r.G - 1) r.t[r.to + 1] = r.G;
}

// The listed long runs (longs[0] holds the count): with fewer runs than
// waves, each run is cut into equal parts, one wave each, so that a run of
// millions of buckets does not hold one wave for the whole launch; the
// wave's lanes write consecutive buckets.
constexpr unsigned kWgLongBlocks = 1024;
__global__ __launch_bounds__(256) void wg_long_kernel(
    const double* __restrict__ w, const uint32_t* __restrict__ key, const uint32_t* __restrict__ grp,
    const uint32_t* __restrict__ cnt, const WNodeHdr* __restrict__ whdr,
    const WGuide* __restrict__ gg, size_t ng, int decaying, uint32_t* __restrict__ tab,
    const uint32_t* __restrict__ longs) {
    const uint32_t n = longs[0];
    if (n == 0) return;
    const uint32_t waves = gridDim.x * (blockDim.x / 64);
    const uint32_t parts = n < waves ? waves / n : 1u;
    const uint64_t items = static_cast<uint64_t>(n) * parts;
    const uint32_t lane = threadIdx.x & 63;
    for (uint64_t it = blockIdx.x * (blockDim.x / 64) + (threadIdx.x >> 6); it < items;
         it += waves) {
        const uint32_t k = static_cast<uint32_t>(it / parts), part = static_cast<uint32_t>(it % parts);
        const WgRun r = wg_run(w, key, grp, cnt, whdr, gg, ng, decaying, tab, longs[1 + k]);
        const uint64_t len = static_cast<uint64_t>(r.to) - r.from + 1;
        const uint64_t lo = r.from + len * part / parts, hi = r.from + len * (part + 1) / parts;
        for (uint64_t b = lo + lane; b < hi; b += 64) r.t[b] = r.i;
    }
}

__global__ void active_flags_kernel(const uint32_t* __restrict__ out_off,
                                    const uint32_t* __restrict__ in_off, size_t v,
                                    uint8_t* __restrict__ active) {
    const size_t u = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (u >= v) return;
    bool a = out_off[u + 1] > out_off[u];
    if (in_off) a = a || in_off[u + 1] > in_off[u];
    active[u] = a ? 1 : 0;
}

// node2vec adjacency: key = owner << b | neighbour for both directions of
// every edge; sorting it orders lists by owner and each list ascending.
__global__ void adj_keys_kernel(const int32_t* __restrict__ s, const int32_t* __restrict__ d,
                                size_t e, int b, uint64_t* __restrict__ keys) {
    const size_t i = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (i >= e) return;
    const uint64_t u = static_cast<uint32_t>(s[i]), v = static_cast<uint32_t>(d[i]);
    keys[2 * i] = (u << b) | v;
    keys[2 * i + 1] = (v << b) | u;
}

__global__ void adj_finish_kernel(const uint64_t* __restrict__ keys, size_t n, uint64_t mask,
                                  int32_t* __restrict__ nbr) {
    const size_t k = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (k >= n) return;
    nbr[k] = static_cast<int32_t>(keys[k] & mask);
}

__global__ void adj_offsets_kernel(const uint64_t* __restrict__ keys, size_t n, int b, size_t cnt,
                                   uint32_t* __restrict__ off) {
    const size_t u = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (u >= cnt) return;
    const uint64_t target = static_cast<uint64_t>(u) << b;
    size_t lo = 0, hi = n;
    while (lo < hi) {
        const size_t mid = lo + ((hi - lo) >> 1);
        if (keys[mid] < target) lo = mid + 1;
        else hi = mid;
    }
    off[u] = static_cast<uint32_t>(lo);
}

// The adjacency pair set (open addressing, linear probing, Fibonacci hash; at
// most half full, so every probe sequence reaches a free slot), filled from
// the pair keys sorted with their duplicates adjacent: one insertion per
// distinct pair.  (Inserting every edge's two pairs straight from the store
// touched the table 2E times at random -- 1.4 ms at cfg5's 9M edges, against
// 42 us for the distinct pairs.)  Keys of active-id ranks (ranked != nullptr:
// ids[] maps a rank back to its node) or of node ids.
__device__ __forceinline__ void adj_set_insert(uint64_t k, int shift, uint64_t mask,
                                               uint64_t* tab) {
    uint64_t h = (k * kAdjHashMul) >> shift;
    while (atomicCAS(reinterpret_cast<unsigned long long*>(tab + h),
                     static_cast<unsigned long long>(kAdjEmpty),
                     static_cast<unsigned long long>(k)) != kAdjEmpty)
        h = (h + 1) & mask;
}

__global__ void adj_hash_insert_ranked_kernel(const uint32_t* __restrict__ keys, size_t n, int rb,
                                              const uint32_t* __restrict__ ids, int b, int shift,
                                              uint64_t mask, uint64_t* __restrict__ tab) {
    const size_t i = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (i >= n) return;
    const uint32_t k = keys[i];
    if (i > 0 && keys[i - 1] == k) return;  // a repeated pair
    const uint64_t u = ids[k >> rb], v = ids[k & ((1u << rb) - 1u)];
    adj_set_insert((u << b) | v, shift, mask, tab);
}

__global__ void adj_hash_insert_kernel(const uint64_t* __restrict__ keys, size_t n, int shift,
                                       uint64_t mask, uint64_t* __restrict__ tab) {
    const size_t i = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (i >= n) return;
    const uint64_t k = keys[i];
    if (i > 0 && keys[i - 1] == k) return;  // a repeated pair
    adj_set_insert(k, shift, mask, tab);
}

// Ranks of the active node ids (the exclusive scan of these flags) and the
// ids by rank.
__global__ void active_u32_kernel(const uint8_t* __restrict__ active, size_t v,
                                  uint32_t* __restrict__ f) {
    const size_t u = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (u < v) f[u] = active[u];
}

__global__ void active_ids_kernel(const uint8_t* __restrict__ active,
                                  const uint32_t* __restrict__ rank, size_t v,
                                  uint32_t* __restrict__ ids) {
    const size_t u = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (u < v && active[u]) ids[rank[u]] = static_cast<uint32_t>(u);
}

// The pair set holds every edge once, as its endpoints in increasing order
// (the walks ask about both orders, and adjacency is symmetric): keys of
// active-id ranks, rank(smaller) << rb | rank(larger) -- ranks keep the ids'
// order -- or of the ids themselves.
__global__ void adj_rank_keys_kernel(const int32_t* __restrict__ s, const int32_t* __restrict__ d,
                                     size_t e, const uint32_t* __restrict__ rank, int rb,
                                     uint32_t* __restrict__ keys) {
    const size_t i = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (i >= e) return;
    const uint32_t ru = rank[s[i]], rv = rank[d[i]];
    keys[i] = (min(ru, rv) << rb) | max(ru, rv);
}

__global__ void adj_pair_keys_kernel(const int32_t* __restrict__ s, const int32_t* __restrict__ d,
                                     size_t e, int b, uint64_t* __restrict__ keys) {
    const size_t i = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (i >= e) return;
    const uint64_t u = static_cast<uint32_t>(s[i]), v = static_cast<uint32_t>(d[i]);
    keys[i] = (min(u, v) << b) | max(u, v);
}

__global__ void distinct_flags_kernel(const uint32_t* __restrict__ keys, size_t n,
                                      uint32_t* __restrict__ flags) {
    const size_t i = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (i < n) flags[i] = (i == 0 || keys[i] != keys[i - 1]) ? 1u : 0u;
}

// Global per-timestamp-group weights before normalisation
// (edge_data.cu:477-492).
__global__ void global_weights_kernel(const uint32_t* __restrict__ off,
                                      const int64_t* __restrict__ uq, size_t t_groups,
                                      int64_t tmin, int64_t tmax, double bound, double scale,
                                      double* __restrict__ fwd, double* __restrict__ bwd) {
    const size_t g = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (g >= t_groups) return;
    const double size = static_cast<double>(off[g + 1] - off[g]);
    const int64_t t = uq[g];
    const double tf = static_cast<double>(tmin - t);
    const double tb = static_cast<double>(t - tmax);
    const double fs = bound > 0 ? tf * scale : tf;
    const double bs = bound > 0 ? tb * scale : tb;
    fwd[g] = size * exp(fs);
    bwd[g] = size * exp(bs);
}

__global__ void divide_kernel(double* __restrict__ a, double* __restrict__ b, size_t n,
                              const double* __restrict__ sums_a, const double* __restrict__ sums_b) {
    const size_t i = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (i >= n) return;
    a[i] = a[i] / sums_a[0];
    b[i] = b[i] / sums_b[0];
}

// Per-node cumulative exponential weights (node_edge_index.cu:500-640).
// Raw weights: group size * exp(scaled distance to the node's pivot):
// backward pivots on the node's latest time, forward on its earliest.
struct NodeWeightParams {
    int64_t mn, mx;
    double scale;
};

__device__ __forceinline__ NodeWeightParams node_weight_params(const int64_t* first_ts,
                                                               uint32_t s, uint32_t e,
                                                               double bound) {
    const int64_t mn = first_ts[s], mx = first_ts[e - 1];
    const double diff = static_cast<double>(mx - mn);
    return NodeWeightParams{mn, mx, (bound > 0 && diff > 0) ? bound / diff : 1.0};
}

__device__ __forceinline__ void raw_node_weights(const NodeWeightParams& q, const uint32_t* grp,
                                                 const int64_t* first_ts, uint32_t p,
                                                 double bound, double* f, double* b) {
    const double sz = static_cast<double>(grp[p + 1] - grp[p]);
    const int64_t t = first_ts[p];
    const double bsc = bound > 0 ? static_cast<double>(t - q.mx) * q.scale
                                 : static_cast<double>(t - q.mx);
    const double fsc = bound > 0 ? static_cast<double>(q.mn - t) * q.scale
                                 : static_cast<double>(q.mn - t);
    *b = sz * exp(bsc);
    *f = sz * exp(fsc);
}

// Nodes with at most kHeavyGroups groups: one thread per node; the normalised
// weights are accumulated sequentially in group order, exactly as the
// reference does (node_edge_index.cu:617-639).  A wave of such threads waits
// for its largest node's two loops, so larger nodes take the tile path (one
// workgroup per kHeavyTile groups).
constexpr uint32_t kHeavyGroups = 32;

__global__ void node_weights_light_kernel(const uint32_t* __restrict__ cnt,
                                          const uint32_t* __restrict__ grp,
                                          const int64_t* __restrict__ first_ts, size_t nodes,
                                          double bound, int compute_forward,
                                          double* __restrict__ wf, double* __restrict__ wb) {
    const size_t u = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (u >= nodes) return;
    const uint32_t s = cnt[u], e = cnt[u + 1];
    if (s >= e || e - s > kHeavyGroups) return;
    const NodeWeightParams q = node_weight_params(first_ts, s, e, bound);
    double fsum = 0.0, bsum = 0.0;
    for (uint32_t p = s; p < e; ++p) {
        double f, b;
        raw_node_weights(q, grp, first_ts, p, bound, &f, &b);
        wb[p] = b;
        bsum += b;
        if (compute_forward) {
            wf[p] = f;
            fsum += f;
        }
    }
    double fc = 0.0, bc = 0.0;
    for (uint32_t p = s; p < e; ++p) {
        bc += wb[p] / bsum;
        wb[p] = bc;
        if (compute_forward) {
            fc += wf[p] / fsum;
            wf[p] = fc;
        }
    }
}

__global__ void heavy_node_flags_kernel(const uint32_t* __restrict__ cnt, size_t nodes,
                                        uint32_t* __restrict__ flags) {
    const size_t u = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (u < nodes) flags[u] = (cnt[u + 1] - cnt[u] > kHeavyGroups) ? 1u : 0u;
}

// Heavy nodes are cut into tiles of kHeavyTile groups (256 threads x 16); the
// i-th heavy node (in id order) owns tiles [tile_base[i], tile_base[i + 1]).
constexpr int kHeavyItems = 16;
constexpr uint32_t kHeavyTile = 256 * kHeavyItems;
// Workgroups of the tile kernels, each taking tiles in turn.
constexpr size_t kHeavyGrid = 2048;

__global__ void fill_u32_kernel(uint32_t* __restrict__ p, size_t n, uint32_t v) {
    const size_t i = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void compact_heavy_kernel(const uint32_t* __restrict__ flags,
                                     const uint32_t* __restrict__ scan,
                                     const uint32_t* __restrict__ cnt, size_t nodes,
                                     uint32_t* __restrict__ heavy, uint32_t* __restrict__ tiles) {
    const size_t u = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (u < nodes && flags[u]) {
        heavy[scan[u]] = static_cast<uint32_t>(u);
        tiles[scan[u]] = (cnt[u + 1] - cnt[u] + kHeavyTile - 1) / kHeavyTile;
    }
}

// Exclusive block scan (sum or max) of one value per thread.
template <bool Max>
__device__ double block_excl_scan_f64(double v, double* s4, double* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    double x = v;
    for (int off = 1; off < 64; off <<= 1) {
        const double y = __shfl_up(x, off, 64);
        if (lane >= off) x = Max ? fmax(x, y) : x + y;
    }
    if (lane == 63) s4[wave] = x;
    __syncthreads();
    double before = Max ? -1.0 : 0.0, tot = Max ? -1.0 : 0.0;
    for (int w = 0; w < 4; ++w) {
        const double sw = s4[w];
        if (w < wave) before = Max ? fmax(before, sw) : before + sw;
        tot = Max ? fmax(tot, sw) : tot + sw;
    }
    __syncthreads();
    *total = tot;
    const double excl_in_wave = __shfl_up(x, 1, 64);
    if (Max) return lane == 0 ? before : fmax(before, excl_in_wave);
    return before + (lane == 0 ? 0.0 : excl_in_wave);
}

// The heavy node and the tile's first group of tile t (-1: past the last tile).
__device__ __forceinline__ int heavy_tile_node(const uint32_t* tile_base, uint32_t nh, uint32_t t) {
    if (t >= tile_base[nh]) return -1;
    uint32_t lo = 0, hi = nh;  // last i with tile_base[i] <= t
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (tile_base[mid] <= t) lo = mid;
        else hi = mid;
    }
    return static_cast<int>(lo);
}

// Pass 1 of a heavy node's weights, one workgroup per tile: the raw weights
// of the tile's groups and their running sum within the tile -- per-thread
// sequential sums of 16, a block scan, then a block running maximum so the
// tile's values are non-decreasing -- written in place; the tile's last
// value goes to tsum.  Both directions (f is skipped when wf is null).
__global__ __launch_bounds__(256) void heavy_tile_scan_kernel(
    const uint32_t* __restrict__ heavy, const uint32_t* __restrict__ tile_base,
    const uint32_t* __restrict__ nh_dev, const uint32_t* __restrict__ cnt,
    const uint32_t* __restrict__ grp, const int64_t* __restrict__ first_ts, double bound,
    double* __restrict__ wf, double* __restrict__ wb, double* __restrict__ tsum_f,
    double* __restrict__ tsum_b) {
    __shared__ double s4[4];
    const uint32_t nh = *nh_dev;
    for (uint32_t t = blockIdx.x;; t += gridDim.x) {
        const int i = heavy_tile_node(tile_base, nh, t);
        if (i < 0) return;  // uniform over the workgroup
        const uint32_t u = heavy[i];
        const uint32_t s = cnt[u], e = cnt[u + 1];
        const NodeWeightParams q = node_weight_params(first_ts, s, e, bound);
        const uint32_t t0 = s + (t - tile_base[i]) * kHeavyTile;
        const uint32_t p0 = t0 + threadIdx.x * kHeavyItems;
        double vf[kHeavyItems], vb[kHeavyItems];
        double rf = 0.0, rb = 0.0;
#pragma unroll
        for (int j = 0; j < kHeavyItems; ++j) {
            const uint32_t p = p0 + j;
            double f = 0.0, b = 0.0;
            if (p < e) raw_node_weights(q, grp, first_ts, p, bound, &f, &b);
            rf += f;
            rb += b;
            vf[j] = rf;
            vb[j] = rb;
        }
        for (int dir = 0; dir < (wf ? 2 : 1); ++dir) {
            double* v = dir == 0 ? vb : vf;
            double* w = dir == 0 ? wb : wf;
            double tot;
            const double before = block_excl_scan_f64<false>(dir == 0 ? rb : rf, s4, &tot);
            double mx = 0.0;
#pragma unroll
            for (int j = 0; j < kHeavyItems; ++j) {
                v[j] = before + v[j];
                mx = fmax(mx, v[j]);
            }
            double mtot;
            double m = block_excl_scan_f64<true>(mx, s4, &mtot);
            m = fmax(m, 0.0);
#pragma unroll
            for (int j = 0; j < kHeavyItems; ++j) {
                const uint32_t p = p0 + j;
                m = fmax(m, v[j]);
                if (p < e) w[p] = m;
            }
            if (threadIdx.x == 0) (dir == 0 ? tsum_b : tsum_f)[t] = mtot;
        }
    }
}

// Pass 2, one thread per heavy node: its tiles' exclusive prefixes, each the
// previous prefix plus the previous tile's last value, so consecutive tiles
// stay non-decreasing across their boundary; the node's total follows.
__global__ void heavy_tile_prefix_kernel(const uint32_t* __restrict__ tile_base,
                                         const uint32_t* __restrict__ nh_dev,
                                         double* __restrict__ tsum_f, double* __restrict__ tsum_b,
                                         double* __restrict__ total_f,
                                         double* __restrict__ total_b, int compute_forward) {
    const uint32_t i = blockIdx.x * kB + threadIdx.x;
    if (i >= *nh_dev) return;
    for (int dir = 0; dir < (compute_forward ? 2 : 1); ++dir) {
        double* ts = dir == 0 ? tsum_b : tsum_f;
        double run = 0.0;
        uint32_t t = tile_base[i];
        const uint32_t te = tile_base[i + 1];
        // 16 tile sums are loaded before the running sum consumes them, so the
        // loads are in flight together; the additions keep tile order
        constexpr int kBatch = 16;
        for (; t + kBatch <= te; t += kBatch) {
            double x[kBatch];
#pragma unroll
            for (int j = 0; j < kBatch; ++j) x[j] = ts[t + j];
#pragma unroll
            for (int j = 0; j < kBatch; ++j) {
                ts[t + j] = run;
                run = run + x[j];
            }
        }
        for (; t < te; ++t) {
            const double x = ts[t];
            ts[t] = run;
            run = run + x;
        }
        (dir == 0 ? total_b : total_f)[i] = run;
    }
}

// Pass 3, one workgroup per tile: cumulative = (tile prefix + running sum) /
// node total, the normalisation of node_edge_index.cu:617-639 applied to the
// prefix sums (non-decreasing, the node's last value exactly 1).
__global__ __launch_bounds__(256) void heavy_tile_finish_kernel(
    const uint32_t* __restrict__ heavy, const uint32_t* __restrict__ tile_base,
    const uint32_t* __restrict__ nh_dev, const uint32_t* __restrict__ cnt,
    const double* __restrict__ tsum_f, const double* __restrict__ tsum_b,
    const double* __restrict__ total_f, const double* __restrict__ total_b,
    double* __restrict__ wf, double* __restrict__ wb) {
    const uint32_t nh = *nh_dev;
    for (uint32_t t = blockIdx.x;; t += gridDim.x) {
        const int i = heavy_tile_node(tile_base, nh, t);
        if (i < 0) return;
        const uint32_t u = heavy[i];
        const uint32_t s = cnt[u], e = cnt[u + 1];
        const uint32_t t0 = s + (t - tile_base[i]) * kHeavyTile;
        for (int dir = 0; dir < (wf ? 2 : 1); ++dir) {
            double* w = dir == 0 ? wb : wf;
            const double pre = (dir == 0 ? tsum_b : tsum_f)[t];
            const double tot = (dir == 0 ? total_b : total_f)[i];
            for (uint32_t p = t0 + threadIdx.x; p < e && p < t0 + kHeavyTile; p += 256)
                w[p] = (pre + w[p]) / tot;
        }
    }
}

}  // namespace

void validate_batch(const Engine& e, const void* feat, size_t n, size_t dim) {
    // graph/edge_data.cu:71-89
    if (feat != nullptr && dim == 0)
        throw std::runtime_error("edge_features provided but feature_dim is 0");
    if (e.E != 0 && dim != e.feat_dim)
        throw std::runtime_error("feature_dim mismatch with existing data.feature_dim");
    const size_t eff = e.E == 0 ? dim : e.feat_dim;
    if (feat == nullptr && dim != 0)
        throw std::runtime_error("feature_dim must be 0 when edge_features is not provided");
    if (eff > 0 && feat == nullptr && n > 0)
        throw std::runtime_error(
            "edge features enabled; non-empty ingestion must provide edge_features");
    if (e.E + n > 0x7fffffffull)
        throw std::runtime_error("edge store would exceed 2^31-1 edges");
}

namespace {

// Sorted node-index entries whose values carry their timestamp ranks
// (node_entries_kernel with erank), or none (vals == nullptr: dir.rec holds
// the records and the ranks are gathered from erank).
struct PackedEntries {
    const uint64_t* vals;
    int nb, eb;
};

void finish_direction(Engine& e, DirIndex& dir, size_t n, size_t vc, int64_t* host_scratch,
                      const PackedEntries& pe);

// Stable per-direction node index of the store's n entries (mode: see
// node_entries_kernel).
void build_direction(Engine& e, DirIndex& dir, size_t n, int key_bits, size_t vc, int mode,
                     int64_t* host_scratch) {
    hipStream_t s = e.stream;
    dir.present = true;
    dir.n_entries = n;
    // values carry the timestamp rank when neighbour, edge id and rank fit
    // in 64 bits (cfg2: 20 + 25 + 17)
    const int nb = key_bits;
    const int eb = std::max(1, bit_length_u64(e.E ? e.E - 1 : 0));
    const int rb = std::max(1, bit_length_u64(e.T ? e.T - 1 : 0));
    const bool packed = nb + eb + rb <= 64;
    dir.rec.resize(n);
    e.k32a.ensure(n);
    e.k32b.ensure(n);
    e.k64a.ensure(n);
    if (packed) e.k64b.ensure(n);
    e.hist.ensure(radix_hist_elems(n));
    const int passes = n > 1 ? radix_passes(0, key_bits) : 0;
    // unpacked, the sorted records land in dir.rec: start in the buffer set
    // the last digit pass does not write into
    uint64_t* recs = reinterpret_cast<uint64_t*>(dir.rec.p);
    uint64_t* v0 = packed ? e.k64a.p : (passes % 2 == 0 ? recs : e.k64a.p);
    uint64_t* v1 = packed ? e.k64b.p : (passes % 2 == 0 ? e.k64a.p : recs);
    const size_t edges = mode == 2 ? n / 2 : n;
    if (edges)
        hipLaunchKernelGGL(node_entries_kernel, dim3(grid_for(edges)), dim3(kB), 0, s, e.src.p,
                           e.dst.p, edges, mode, 0u, packed ? e.erank.p : nullptr, nb, eb,
                           e.k32a.p, v0);
    const int which = radix_sort_u32_v64(e.k32a.p, v0, e.k32b.p, v1, n, 0, key_bits, e.hist.p, s);
    // the sorted keys become the direction's (the scratch takes the old
    // buffer, which every user sizes again before writing)
    dir.key.swap(which ? e.k32b : e.k32a);
    dir.key.n = n;
    dir.off.resize(vc);
    hipLaunchKernelGGL(lower_bound_offsets_kernel, dim3(grid_for(vc)), dim3(kB), 0, s, dir.key.p,
                       n, vc, dir.off.p);
    PackedEntries pe{packed ? (which ? v1 : v0) : nullptr, nb, eb};
    finish_direction(e, dir, n, vc, host_scratch, pe);
}

// The node index of one direction after an append (Engine::append_store):
// every node's list is its old entries whose edges were kept (edge ids
// lowered by the evicted count), then its batch entries in batch order -- the
// stable (node, position) order of the new store, because the kept old edges
// precede the batch.  Only the batch's entries are sorted; the old entries
// move by one scatter.  mode as node_entries_kernel.
void append_direction(Engine& e, DirIndex& dir, int mode, int key_bits, size_t vc,
                      int64_t* host_scratch) {
    hipStream_t s = e.stream;
    const size_t per = mode == 2 ? 2 : 1;
    const size_t n_old = dir.n_entries;
    const size_t v_old = dir.off.n ? dir.off.n - 1 : 0;
    const size_t v = vc - 1;
    const size_t m = per * e.append_kept_new;
    const size_t n = per * e.E;
    const uint32_t del = static_cast<uint32_t>(e.append_del);
    dir.present = true;
    dir.n_entries = n;
    // the batch's entries (the store's tail), sorted stably by node
    e.k32a.ensure(m);
    e.k32b.ensure(m);
    e.k64a.ensure(m);
    e.k64b.ensure(m);
    e.hist.ensure(radix_hist_elems(m));
    const uint32_t id0 = static_cast<uint32_t>(e.append_kept_old);
    if (e.append_kept_new)
        hipLaunchKernelGGL(node_entries_kernel, dim3(grid_for(e.append_kept_new)), dim3(kB), 0, s,
                           e.src.p + id0, e.dst.p + id0, e.append_kept_new, mode, id0, nullptr, 0,
                           0, e.k32a.p, e.k64a.p);
    const int w = radix_sort_u32_v64(e.k32a.p, e.k64a.p, e.k32b.p, e.k64b.p, m, 0, key_bits,
                                     e.hist.p, s);
    const uint32_t* bkeys = w ? e.k32b.p : e.k32a.p;
    const uint64_t* brec = w ? e.k64b.p : e.k64a.p;
    e.inc_bstart.resize(vc);
    uint32_t* bstart = e.inc_bstart.p;
    hipLaunchKernelGGL(lower_bound_offsets_kernel, dim3(grid_for(vc)), dim3(kB), 0, s, bkeys, m,
                       vc, bstart);
    // evicted prefix of every old node, then the new offsets
    e.inc_ev.resize(std::max<size_t>(v_old, 1));
    check_hip(hipMemsetAsync(e.inc_ev.p, 0, e.inc_ev.n * 4, s), "evicted counts clear");
    if (del && n_old)
        hipLaunchKernelGGL(evicted_prefix_kernel, dim3(grid_for(n_old)), dim3(kB), 0, s, dir.key.p,
                           dir.rec.p, n_old, del, dir.off.p, e.inc_ev.p);
    e.inc_cnt.resize(vc);
    hipLaunchKernelGGL(append_counts_kernel, dim3(grid_for(v)), dim3(kB), 0, s, dir.off.p, v_old,
                       e.inc_ev.p, bstart, v, e.inc_cnt.p);
    e.off_next.resize(vc);
    e.scan_scratch.ensure(scan_scratch_elems(vc));
    exclusive_scan_u32(e.inc_cnt.p, e.off_next.p, v, e.scan_scratch.p, s);
    // the entries at their new places
    e.key_next.resize(n);
    e.rec_next.resize(n);
    if (n_old)
        hipLaunchKernelGGL(append_old_entries_kernel, dim3(grid_for(n_old)), dim3(kB), 0, s,
                           dir.key.p, dir.rec.p, n_old, del, dir.off.p, e.inc_ev.p, e.off_next.p,
                           e.key_next.p, e.rec_next.p);
    if (m)
        hipLaunchKernelGGL(append_new_entries_kernel, dim3(grid_for(m)), dim3(kB), 0, s, bkeys,
                           brec, m, bstart, dir.off.p, v_old, e.inc_ev.p, e.off_next.p,
                           e.key_next.p, e.rec_next.p);
    check_hip(hipGetLastError(), "append index launch");
    dir.key.swap(e.key_next);
    dir.rec.swap(e.rec_next);
    dir.off.swap(e.off_next);
    dir.key.n = n;
    dir.rec.n = n;
    dir.off.n = vc;
    // the old entries' ranks changed with the eviction: gathered from erank
    finish_direction(e, dir, n, vc, host_scratch, PackedEntries{nullptr, 0, 0});
}

// The rest of a direction's index from its sorted entries (dir.key, dir.rec)
// and CSR offsets (dir.off): edge ids, node-timestamp groups, per-node group
// counts, walk headers and bucket tables.
void finish_direction(Engine& e, DirIndex& dir, size_t n, size_t vc, int64_t* host_scratch,
                      const PackedEntries& pe) {
    hipStream_t s = e.stream;
    dir.idx.resize(n);
    e.v32a.ensure(n);  // the entries' timestamp ranks
    if (pe.vals)
        hipLaunchKernelGGL(node_group_flags_packed_kernel, dim3(grid_for(n)), dim3(kB), 0, s,
                           dir.key.p, pe.vals, n, pe.nb, pe.eb, e.flags.p, dir.idx.p, e.v32a.p,
                           dir.rec.p);
    else
        hipLaunchKernelGGL(node_group_flags_kernel, dim3(grid_for(n)), dim3(kB), 0, s, dir.key.p,
                           dir.rec.p, e.erank.p, n, e.flags.p, dir.idx.p, e.v32a.p);
    exclusive_scan_u32(e.flags.p, e.scan.p, n, e.scan_scratch.p, s);
    uint32_t g = 0;
    check_hip(hipMemcpyAsync(host_scratch, e.scan.p + n, 4, hipMemcpyDeviceToHost, s), "read g");
    e.sync();
    std::memcpy(&g, host_scratch, 4);
    dir.n_groups = g;
    dir.grp.resize(static_cast<size_t>(g) + 1);
    // group timestamps feed only the per-node weights
    const bool weights = e.cfg.enable_weight_computation || e.cfg.enable_temporal_node2vec;
    dir.first_ts.resize(weights ? g : 0);
    dir.pan.resize(static_cast<size_t>(g) + 1);
    if (n) {
        hipLaunchKernelGGL(node_group_scatter_kernel, dim3(grid_for(n)), dim3(kB), 0, s,
                           e.flags.p, e.scan.p, e.v32a.p, e.uniq_ts.p, n, dir.grp.p,
                           weights ? dir.first_ts.p : nullptr, dir.pan.p);
    } else {
        check_hip(hipMemsetAsync(dir.grp.p, 0, 4, s), "grp terminator");
        check_hip(hipMemsetAsync(dir.pan.p, 0, sizeof(PanelRec), s), "panel terminator");
    }
    dir.cnt.resize(vc);
    hipLaunchKernelGGL(node_group_counts_kernel, dim3(grid_for(vc)), dim3(kB), 0, s, dir.off.p,
                       e.scan.p, vc, dir.cnt.p);

    // walk search headers and bucket tables
    dir.hdr.resize(vc);
    hipLaunchKernelGGL(node_headers_kernel, dim3(grid_for(vc)), dim3(kB), 0, s, dir.cnt.p,
                       dir.pan.p, vc, dir.hdr.p);
    dir.tab.resize(2 * (static_cast<size_t>(g) + vc));
    if (g)
        hipLaunchKernelGGL(node_table_fill_kernel, dim3(grid_for(g)), dim3(kB), 0, s, dir.key.p,
                           dir.grp.p, dir.hdr.p, dir.pan.p, static_cast<size_t>(g), dir.tab.p);
    // the weight pickers' records: every entry's next slice bound, searched
    // once here instead of at every hop that takes the entry
    // wide in the out direction when the ExponentialWeight weights were asked for
    dir.wrec_shift = weights && e.cfg.enable_weight_computation && &dir == &e.out ? 1 : 0;
    dir.wrec.resize(weights ? n << dir.wrec_shift : 0);
    if (weights && n)
        hipLaunchKernelGGL(entry_bounds_kernel, dim3(grid_for(n)), dim3(kB), 0, s, dir.rec.p,
                           e.v32a.p, dir.hdr.p, dir.tab.p, dir.pan.p, n, vc, dir.wrec_shift,
                           dir.wrec.p);
    check_hip(hipGetLastError(), "direction index launch");
}

void node_weights(Engine& e, DirIndex& dir, size_t v, double bound, bool compute_forward,
                  int64_t* host_scratch) {
    hipStream_t s = e.stream;
    double* wf = compute_forward ? dir.w_fwd.p : nullptr;
    hipLaunchKernelGGL(node_weights_light_kernel, dim3(grid_for(v)), dim3(kB), 0, s, dir.cnt.p,
                       dir.grp.p, dir.first_ts.p, v, bound, compute_forward ? 1 : 0, wf,
                       dir.w_bwd.p);
    // heavier nodes: list them on the device, then tiles of kHeavyTile groups
    e.flags.ensure(v + 1);
    e.scan.ensure(v + 1);
    e.scan_scratch.ensure(scan_scratch_elems(v + 1));
    hipLaunchKernelGGL(heavy_node_flags_kernel, dim3(grid_for(v)), dim3(kB), 0, s, dir.cnt.p, v,
                       e.flags.p);
    exclusive_scan_u32(e.flags.p, e.scan.p, v, e.scan_scratch.p, s);
    // the heavy count stays on the device (scan[v]): the buffers are sized
    // for the most heavy nodes the groups allow, and the kernels read it
    (void)host_scratch;
    const size_t nh_max = std::min<size_t>(v, dir.n_groups / (kHeavyGroups + 1));
    if (nh_max) {
        const uint32_t* nh_dev = e.scan.p + v;
        // heavy ids in k32b, their tile counts (zero past the last) then tile
        // bases in v32b
        e.k32b.ensure(nh_max);
        e.v32b.ensure(nh_max + 1);
        e.v32a.ensure(nh_max + 1);
        hipLaunchKernelGGL(fill_u32_kernel, dim3(grid_for(nh_max + 1)), dim3(kB), 0, s, e.v32a.p,
                           nh_max + 1, 0u);
        hipLaunchKernelGGL(compact_heavy_kernel, dim3(grid_for(v)), dim3(kB), 0, s, e.flags.p,
                           e.scan.p, dir.cnt.p, v, e.k32b.p, e.v32a.p);
        e.scan_scratch.ensure(scan_scratch_elems(nh_max + 1));
        exclusive_scan_u32(e.v32a.p, e.v32b.p, nh_max, e.scan_scratch.p, s);
        // at most g / kHeavyTile + nh tiles, taken in turn by a fixed grid
        const size_t tiles = dir.n_groups / kHeavyTile + nh_max + 1;
        e.dscratch.ensure(4 * tiles + 2 * nh_max);
        double* tsum_f = e.dscratch.p;
        double* tsum_b = tsum_f + tiles;
        double* total_f = tsum_b + tiles;
        double* total_b = total_f + nh_max;
        const unsigned grid = static_cast<unsigned>(std::min<size_t>(tiles, kHeavyGrid));
        hipLaunchKernelGGL(heavy_tile_scan_kernel, dim3(grid), dim3(256), 0, s, e.k32b.p,
                           e.v32b.p, nh_dev, dir.cnt.p, dir.grp.p, dir.first_ts.p, bound, wf,
                           dir.w_bwd.p, tsum_f, tsum_b);
        hipLaunchKernelGGL(heavy_tile_prefix_kernel, dim3(grid_for(nh_max)), dim3(kB), 0, s,
                           e.v32b.p, nh_dev, tsum_f, tsum_b, total_f, total_b,
                           compute_forward ? 1 : 0);
        hipLaunchKernelGGL(heavy_tile_finish_kernel, dim3(grid), dim3(256), 0, s, e.k32b.p,
                           e.v32b.p, nh_dev, dir.cnt.p, tsum_f, tsum_b, total_f, total_b, wf,
                           dir.w_bwd.p);
    }
    check_hip(hipGetLastError(), "node weights launch");
}

// Guide tables of one cumulative weight array (index_layout.h), its guides
// already written: per node of a direction (key, grp, cnt, whdr) or, with
// key == nullptr, the whole array under the guide gg.  Each bucket is written
// once: by its group's thread, or for a run of more than kWgRun buckets (the
// weights jumping by orders of magnitude) by a wave of wg_long_kernel.
void fill_weight_guides(hipStream_t s, DBuf<uint32_t>& longs, const double* w, size_t ng,
                        const uint32_t* key, const uint32_t* grp, const uint32_t* cnt,
                        const WNodeHdr* whdr, const WGuide* gg, bool decaying, uint32_t* tab,
                        size_t tsize) {
    if (ng == 0) return;
    longs.ensure(tsize / kWgRun + 2);
    check_hip(hipMemsetAsync(longs.p, 0, 4, s), "guide long-run count");
    hipLaunchKernelGGL(wg_fill_kernel, dim3(grid_for(ng)), dim3(kB), 0, s, w, key, grp, cnt, whdr,
                       gg, ng, decaying ? 1 : 0, tab, longs.p);
    hipLaunchKernelGGL(wg_long_kernel, dim3(kWgLongBlocks), dim3(256), 0, s, w, key, grp, cnt,
                       whdr, gg, ng, decaying ? 1 : 0, tab, longs.p);
}

// The weight pickers' view of one direction's cumulative weights w (forward
// weights decay, backward weights grow: node_edge_index.cu:540-575).
void build_walk_weights(Engine& e, DirIndex& dir, size_t v, const DBuf<double>& w, bool decaying,
                        WalkWeights& ww) {
    hipStream_t s = e.stream;
    const size_t vc = v + 1, g = dir.n_groups;
    ww.hdr.resize(vc);
    // a wide panel (index_layout.h) for forward walks where the ExponentialWeight
    // weights were asked for, over the out direction's wide records
    ww.shift = dir.wrec_shift && decaying ? 1 : 0;
    ww.pan.resize(g << ww.shift);
    ww.tab.resize(2 * (g + v));
    hipLaunchKernelGGL(whdr_kernel, dim3(grid_for(vc)), dim3(kB), 0, s, w.p, dir.cnt.p, dir.hdr.p,
                       vc, decaying ? 1 : 0, ww.hdr.p);
    // the records' start sums first: the wide panel copies its first entries'
    const size_t n = dir.wrec.n >> dir.wrec_shift;
    if (ww.shift && n)
        hipLaunchKernelGGL(entry_sums_kernel, dim3(grid_for(n)), dim3(kB), 0, s, dir.wrec.p, w.p, n);
    if (g)
        hipLaunchKernelGGL(wpan_kernel, dim3(grid_for(g)), dim3(kB), 0, s, dir.pan.p, w.p,
                           dir.wrec.p, dir.wrec_shift, g, ww.shift, ww.pan.p);
    fill_weight_guides(e.stream, e.wg_long, w.p, g, dir.key.p, dir.grp.p, dir.cnt.p, ww.hdr.p,
                       nullptr, decaying, ww.tab.p, ww.tab.n);
    check_hip(hipGetLastError(), "walk weights launch");
}

// The guide of a global cumulative array (one segment of n).
void build_global_guide(Engine& e, hipStream_t s, const DBuf<double>& w, size_t n, bool decaying,
                        DBuf<WGuide>& gd, DBuf<uint32_t>& tab) {
    gd.resize(1);
    tab.resize(2 * n + 1);
    hipLaunchKernelGGL(global_guide_kernel, dim3(1), dim3(1), 0, s, w.p, n, decaying ? 1 : 0,
                       gd.p);
    fill_weight_guides(s, e.wg_long_g, w.p, n, nullptr, nullptr, nullptr, nullptr, gd.p, decaying,
                       tab.p, tab.n);
    check_hip(hipGetLastError(), "global guide launch");
}

// The batch alone, sorted stably by timestamp: keys ts - btmin (32-bit when the
// batch's range fits).  Without edge features the packed endpoints travel as
// the sort's values (ends sorted, bpos null); with them the batch positions do
// (bpos), the endpoints staying in batch order (ends).
struct SortedBatch {
    bool keys32;
    const uint32_t* k32;
    const uint64_t* k64;
    const uint64_t* ends;
    const uint32_t* bpos;
};

SortedBatch sort_batch(Engine& e, const int32_t* d_src, const int32_t* d_dst, const int64_t* d_ts,
                       size_t n, int64_t btmin, int64_t btmax) {
    hipStream_t s = e.stream;
    const int bits = bit_length_u64(static_cast<uint64_t>(btmax) - static_cast<uint64_t>(btmin));
    const bool keys32 = bits <= 32;
    const bool carry_ends = e.feat_dim == 0;
    e.k64a.ensure(n);
    e.k64b.ensure(n);
    e.ends64.ensure(n);
    if (carry_ends) e.ends64b.ensure(n);
    e.v32a.ensure(n);
    e.v32b.ensure(n);
    e.hist.ensure(radix_hist_elems(n));
    uint32_t* k32s[2] = {reinterpret_cast<uint32_t*>(e.k64a.p), reinterpret_cast<uint32_t*>(e.k64b.p)};
    uint32_t* pos0 = carry_ends ? nullptr : e.v32a.p;
    int which;
    if (keys32) {
        hipLaunchKernelGGL((make_ts_keys_kernel<uint32_t>), dim3(grid_for(n)), dim3(kB), 0, s,
                           e.ts.p, e.src.p, e.dst.p, size_t{0}, d_ts, d_src, d_dst, n, btmin,
                           k32s[0], pos0, e.ends64.p);
        which = carry_ends ? radix_sort_u32_v64(k32s[0], e.ends64.p, k32s[1], e.ends64b.p, n, 0,
                                                bits, e.hist.p, s)
                           : radix_sort_u32(k32s[0], e.v32a.p, k32s[1], e.v32b.p, n, 0, bits,
                                            e.hist.p, s);
    } else {
        hipLaunchKernelGGL((make_ts_keys_kernel<uint64_t>), dim3(grid_for(n)), dim3(kB), 0, s,
                           e.ts.p, e.src.p, e.dst.p, size_t{0}, d_ts, d_src, d_dst, n, btmin,
                           e.k64a.p, pos0, e.ends64.p);
        which = carry_ends ? radix_sort_u64_v64(e.k64a.p, e.ends64.p, e.k64b.p, e.ends64b.p, n, 0,
                                                bits, e.hist.p, s)
                           : radix_sort_u64(e.k64a.p, e.v32a.p, e.k64b.p, e.v32b.p, n, 0, bits,
                                            e.hist.p, s);
    }
    SortedBatch b;
    b.keys32 = keys32;
    b.k32 = k32s[which];
    b.k64 = which ? e.k64b.p : e.k64a.p;
    b.ends = carry_ends ? (which ? e.ends64b.p : e.ends64.p) : e.ends64.p;
    b.bpos = carry_ends ? nullptr : (which ? e.v32b.p : e.v32a.p);
    return b;
}

}  // namespace

void Engine::build(const int32_t* d_src, const int32_t* d_dst, const int64_t* d_ts,
                   const float* d_feat, size_t n, size_t dim) {
    if (n == 0) return;
    hipStream_t s = stream;
    int64_t* hs = reinterpret_cast<int64_t*>(host_scalars);
    check_hip(hipEventRecord(ev[0], s), "event");

    // ---- 1. key range, latest timestamp, and the batch's smallest node id:
    // the node index is keyed by ids in [0, max_node_id], so a negative id
    // is rejected here, before the store changes
    red64.ensure(minmax_scratch_elems());
    minmax_ts_min_id(d_ts, d_src, d_dst, n, red64.p, s);
    check_hip(hipMemcpyAsync(hs, red64.p, 32, hipMemcpyDeviceToHost, s), "read minmax");
    sync();
    if (hs[2] < 0) throw InvalidArgument("node ids must be non-negative");
    // A windowed store settles at about the edges one window of time holds:
    // this batch's rate times the window.  Buffers that grow while it fills
    // are sized for that at once (at most kMaxGrowthHint times what the
    // store after this batch asks).
    struct HintScope {
        double prev = g_growth_hint;
        ~HintScope() { g_growth_hint = prev; }
    } hint_scope;
    if (cfg.max_time_capacity > 0) {
        const double span = static_cast<double>(hs[1] - hs[0]) + 1.0;
        const double window = static_cast<double>(cfg.max_time_capacity) + 1.0;
        const double settled = static_cast<double>(n) * std::max(1.0, window / span);
        const double after = static_cast<double>(E + n);
        g_growth_hint = std::min(kMaxGrowthHint, std::max(1.0, settled / after));
    }
    try {
        batch_max_id = static_cast<int32_t>(hs[3]);
        build_accepted(d_src, d_dst, d_ts, d_feat, n, dim, hs[0], hs[1]);
    } catch (...) {
        // the store, its index and the last batch may disagree: start empty,
        // and hand back the blocks the failed ingest's growth retired
        (void)hipStreamSynchronize(stream);
        (void)hipStreamSynchronize(side);
        clear();
        free_retired();
        throw;
    }
}

// Steps 2-4 of an ingest, general case: one stable LSD radix sort of
// (ts - tmin, position) over the old store followed by the batch -- identical
// to the reference's "sort the batch, stable-merge it after the old store"
// (temporal_graph.cu:67-134) because the old store is already sorted and
// precedes the batch -- then the window eviction as an upper_bound on the
// sorted keys (temporal_graph.cu:136-156) and the gather of the kept suffix.
// tmin / tmax span the store and the batch.
void Engine::sort_store(const int32_t* d_src, const int32_t* d_dst, const int64_t* d_ts,
                        const float* d_feat, size_t n, int64_t tmin, int64_t tmax) {
    hipStream_t s = stream;
    int64_t* hs = reinterpret_cast<int64_t*>(host_scalars);
    const size_t e_old = E, etot = E + n;
    // ---- 2. stable radix sort by (ts, position); 32-bit keys when the key
    // range fits (4-byte key traffic per pass instead of 8).  Without edge
    // features the sort's values are the packed endpoints themselves, so the
    // store is written from the sorted values in order; with features they are
    // the positions the feature rows are gathered by.
    const int bits = bit_length_u64(static_cast<uint64_t>(tmax) - static_cast<uint64_t>(tmin));
    const bool keys32 = bits <= 32;
    const bool carry_ends = feat_dim == 0;
    k64a.ensure(etot);
    k64b.ensure(etot);
    ends64.ensure(etot);
    if (carry_ends) ends64b.ensure(etot);
    v32a.ensure(std::max(etot, 2 * etot));
    v32b.ensure(std::max(etot, 2 * etot));
    hist.ensure(radix_hist_elems(2 * etot));
    uint32_t* k32s[2] = {reinterpret_cast<uint32_t*>(k64a.p), reinterpret_cast<uint32_t*>(k64b.p)};
    uint32_t* pos0 = carry_ends ? nullptr : v32a.p;
    // the window's cut (step 3), known before the sort: when it keeps every
    // edge and the endpoints ride as values, the sort's last pass writes the
    // new store itself (step 4 then has nothing to do)
    int64_t target = -1;
    if (cfg.max_time_capacity > 0) {
        const int64_t cutoff = latest_ts - cfg.max_time_capacity;
        if (cutoff >= tmin) target = static_cast<int64_t>(static_cast<uint64_t>(cutoff) -
                                                          static_cast<uint64_t>(tmin));
    }
    const bool fold = carry_ends && target < 0;
    if (fold) {
        src2.resize(etot);
        dst2.resize(etot);
        ts2.resize(etot);
    }
    const SortedStore st{src2.p, dst2.p, ts2.p, tmin};
    bool folded = false;
    int which = 0;
    if (keys32) {
        hipLaunchKernelGGL((make_ts_keys_kernel<uint32_t>), dim3(grid_for(etot)), dim3(kB), 0, s,
                           ts.p, src.p, dst.p, e_old, d_ts, d_src, d_dst, n, tmin, k32s[0], pos0,
                           ends64.p);
        if (fold)
            folded = radix_sort_u32_v64_store(k32s[0], ends64.p, k32s[1], ends64b.p, etot, 0, bits,
                                              hist.p, s, st);
        else
            which = carry_ends
                        ? radix_sort_u32_v64(k32s[0], ends64.p, k32s[1], ends64b.p, etot, 0, bits,
                                             hist.p, s)
                        : radix_sort_u32(k32s[0], v32a.p, k32s[1], v32b.p, etot, 0, bits, hist.p,
                                         s);
    } else {
        hipLaunchKernelGGL((make_ts_keys_kernel<uint64_t>), dim3(grid_for(etot)), dim3(kB), 0, s,
                           ts.p, src.p, dst.p, e_old, d_ts, d_src, d_dst, n, tmin, k64a.p, pos0,
                           ends64.p);
        if (fold)
            folded = radix_sort_u64_v64_store(k64a.p, ends64.p, k64b.p, ends64b.p, etot, 0, bits,
                                              hist.p, s, st);
        else
            which = carry_ends
                        ? radix_sort_u64_v64(k64a.p, ends64.p, k64b.p, ends64b.p, etot, 0, bits,
                                             hist.p, s)
                        : radix_sort_u64(k64a.p, v32a.p, k64b.p, v32b.p, etot, 0, bits, hist.p, s);
    }
    uint32_t* perm = which ? v32b.p : v32a.p;
    const uint64_t* sorted_ends = which ? ends64b.p : ends64.p;

    // ---- 3. window eviction: drop ts <= latest - capacity
    size_t del = 0;
    if (target >= 0) {
        if (keys32)
            hipLaunchKernelGGL((evict_search_kernel<uint32_t>), dim3(1), dim3(1), 0, s,
                               k32s[which], etot, target, red64.p);
        else
            hipLaunchKernelGGL((evict_search_kernel<uint64_t>), dim3(1), dim3(1), 0, s,
                               which ? k64b.p : k64a.p, etot, target, red64.p);
        check_hip(hipMemcpyAsync(hs, red64.p, 24, hipMemcpyDeviceToHost, s), "read evict");
        sync();
        del = static_cast<size_t>(hs[0]);
        store_tmin = static_cast<int64_t>(static_cast<uint64_t>(tmin) + static_cast<uint64_t>(hs[1]));
        store_tmax = static_cast<int64_t>(static_cast<uint64_t>(tmin) + static_cast<uint64_t>(hs[2]));
    } else {
        // nothing is evicted: the store spans the merged key range
        store_tmin = tmin;
        store_tmax = tmax;
    }
    const size_t kept = etot - del;

    // ---- 4. gather the kept suffix into the new store
    src2.resize(kept);
    dst2.resize(kept);
    ts2.resize(kept);
    if (folded) {
        // written by the sort
    } else if (kept && carry_ends) {
        if (keys32)
            hipLaunchKernelGGL((store_from_sorted_kernel<uint32_t>), dim3(grid_for(kept)), dim3(kB),
                               0, s, k32s[which], sorted_ends, del, kept, tmin, src2.p, dst2.p,
                               ts2.p);
        else
            hipLaunchKernelGGL((store_from_sorted_kernel<uint64_t>), dim3(grid_for(kept)), dim3(kB),
                               0, s, which ? k64b.p : k64a.p, sorted_ends, del, kept, tmin,
                               src2.p, dst2.p, ts2.p);
    } else if (kept) {
        if (keys32)
            hipLaunchKernelGGL((gather_store_kernel<uint32_t>), dim3(grid_for(kept)), dim3(kB), 0,
                               s, k32s[which], perm, ends64.p, del, kept, tmin, src2.p, dst2.p,
                               ts2.p);
        else
            hipLaunchKernelGGL((gather_store_kernel<uint64_t>), dim3(grid_for(kept)), dim3(kB), 0,
                               s, which ? k64b.p : k64a.p, perm, ends64.p, del, kept, tmin,
                               src2.p, dst2.p, ts2.p);
    }
    if (feat_dim > 0) {
        feat2.resize(kept * feat_dim);
        const uint32_t V = static_cast<uint32_t>(feat_dim / 4);
        if (feat_dim % 4 == 0 && V <= 256 && aligned16(d_feat)) {
            const uint32_t R = 256 / V;
            const size_t blocks = std::min<size_t>((kept + R - 1) / R, 65536);
            hipLaunchKernelGGL(gather_feat_vec_kernel, dim3(blocks ? blocks : 1), dim3(V * R), 0, s,
                               perm, del, kept, V, reinterpret_cast<const f32x4*>(feat.p), e_old,
                               reinterpret_cast<const f32x4*>(d_feat),
                               reinterpret_cast<f32x4*>(feat2.p));
        } else {
            hipLaunchKernelGGL(gather_feat_kernel, dim3(grid_capped(kept * feat_dim)), dim3(kB), 0,
                               s, perm, del, kept, feat_dim, feat.p, e_old, d_feat, feat2.p);
        }
        feat.swap(feat2);
    }
    src.swap(src2);
    dst.swap(dst2);
    ts.swap(ts2);
    E = kept;
    check_hip(hipGetLastError(), "gather launch");

}

// Steps 2-4 of an ingest whose batch timestamps are all >= the store's last
// (btmin >= store_tmax): in the stable (ts, position) order the batch then
// follows the store's edges, ties included (old before new), so the new
// store is the old store's kept suffix followed by the batch sorted alone --
// no pass over the old store but one copy.  The eviction cut can fall in the
// old store or, when it empties it, in the batch.
void Engine::append_store(const int32_t* d_src, const int32_t* d_dst, const int64_t* d_ts,
                          const float* d_feat, size_t n, int64_t btmin, int64_t btmax) {
    hipStream_t s = stream;
    int64_t* hs = reinterpret_cast<int64_t*>(host_scalars);
    const size_t e_old = E;
    const bool carry_ends = feat_dim == 0;
    const SortedBatch sb = sort_batch(*this, d_src, d_dst, d_ts, n, btmin, btmax);
    const bool keys32 = sb.keys32;
    const uint32_t* perm = sb.bpos;
    const uint64_t* sorted_ends = sb.ends;
    const uint32_t* sk32 = sb.k32;
    const uint64_t* sk64 = sb.k64;

    // eviction: drop ts <= latest - capacity, from the store first
    size_t del_old = 0, del_new = 0;
    const int64_t cutoff = latest_ts - cfg.max_time_capacity;
    if (cfg.max_time_capacity > 0 && cutoff >= store_tmin) {
        if (keys32)
            hipLaunchKernelGGL((append_evict_kernel<uint32_t>), dim3(1), dim3(1), 0, s, ts.p,
                               e_old, sk32, n, btmin, cutoff, 1, red64.p);
        else
            hipLaunchKernelGGL((append_evict_kernel<uint64_t>), dim3(1), dim3(1), 0, s, ts.p,
                               e_old, sk64, n, btmin, cutoff, 1, red64.p);
        check_hip(hipMemcpyAsync(hs, red64.p, 32, hipMemcpyDeviceToHost, s), "read evict");
        sync();
        del_old = static_cast<size_t>(hs[0]);
        del_new = static_cast<size_t>(hs[1]);
        store_tmin = hs[2];
        store_tmax = hs[3];
    } else {
        store_tmax = btmax;  // store_tmin stays
    }
    const size_t kept_old = e_old - del_old, kept_new = n - del_new, kept = kept_old + kept_new;
    append_del = del_old;
    append_kept_old = kept_old;
    append_kept_new = kept_new;

    src2.resize(kept);
    dst2.resize(kept);
    ts2.resize(kept);
    if (kept_old) {
        check_hip(hipMemcpyAsync(src2.p, src.p + del_old, kept_old * 4, hipMemcpyDeviceToDevice, s),
                  "store copy");
        check_hip(hipMemcpyAsync(dst2.p, dst.p + del_old, kept_old * 4, hipMemcpyDeviceToDevice, s),
                  "store copy");
        check_hip(hipMemcpyAsync(ts2.p, ts.p + del_old, kept_old * 8, hipMemcpyDeviceToDevice, s),
                  "store copy");
    }
    if (kept_new && carry_ends) {
        if (keys32)
            hipLaunchKernelGGL((store_from_sorted_kernel<uint32_t>), dim3(grid_for(kept_new)),
                               dim3(kB), 0, s, sk32, sorted_ends, del_new, kept_new, btmin,
                               src2.p + kept_old, dst2.p + kept_old, ts2.p + kept_old);
        else
            hipLaunchKernelGGL((store_from_sorted_kernel<uint64_t>), dim3(grid_for(kept_new)),
                               dim3(kB), 0, s, sk64, sorted_ends, del_new, kept_new, btmin,
                               src2.p + kept_old, dst2.p + kept_old, ts2.p + kept_old);
    } else if (kept_new) {
        if (keys32)
            hipLaunchKernelGGL((gather_store_kernel<uint32_t>), dim3(grid_for(kept_new)), dim3(kB),
                               0, s, sk32, perm, ends64.p, del_new, kept_new, btmin,
                               src2.p + kept_old, dst2.p + kept_old, ts2.p + kept_old);
        else
            hipLaunchKernelGGL((gather_store_kernel<uint64_t>), dim3(grid_for(kept_new)), dim3(kB),
                               0, s, sk64, perm, ends64.p, del_new, kept_new, btmin,
                               src2.p + kept_old, dst2.p + kept_old, ts2.p + kept_old);
    }
    if (feat_dim > 0) {
        feat2.resize(kept * feat_dim);
        if (kept_old)
            check_hip(hipMemcpyAsync(feat2.p, feat.p + del_old * feat_dim,
                                     kept_old * feat_dim * sizeof(float), hipMemcpyDeviceToDevice,
                                     s),
                      "feature copy");
        float* fdst = feat2.p + kept_old * feat_dim;
        const uint32_t V = static_cast<uint32_t>(feat_dim / 4);
        if (kept_new && feat_dim % 4 == 0 && V <= 256 && aligned16(d_feat) && aligned16(fdst)) {
            const uint32_t R = 256 / V;
            const size_t blocks = std::min<size_t>((kept_new + R - 1) / R, 65536);
            hipLaunchKernelGGL(gather_feat_vec_kernel, dim3(blocks ? blocks : 1), dim3(V * R), 0, s,
                               perm, del_new, kept_new, V, nullptr, size_t{0},
                               reinterpret_cast<const f32x4*>(d_feat),
                               reinterpret_cast<f32x4*>(fdst));
        } else if (kept_new) {
            hipLaunchKernelGGL(gather_feat_kernel, dim3(grid_capped(kept_new * feat_dim)), dim3(kB),
                               0, s, perm, del_new, kept_new, feat_dim, nullptr, size_t{0}, d_feat,
                               fdst);
        }
        feat.swap(feat2);
    }
    src.swap(src2);
    dst.swap(dst2);
    ts.swap(ts2);
    E = kept;
    check_hip(hipGetLastError(), "append launch");
}

// Steps 2-4 of an ingest of a batch that reaches back before the store's last
// timestamp: the batch is sorted alone and merged with the store (the merge
// kernels above), which gives the same order as the reference's "sort the
// batch, stable-merge it after the old store" (temporal_graph.cu:67-134);
// the window's cut (temporal_graph.cu:136-156) drops a prefix of each run.
void Engine::merge_store(const int32_t* d_src, const int32_t* d_dst, const int64_t* d_ts,
                         const float* d_feat, size_t n, int64_t btmin, int64_t btmax) {
    hipStream_t s = stream;
    int64_t* hs = reinterpret_cast<int64_t*>(host_scalars);
    const size_t e_old = E;
    const SortedBatch sb = sort_batch(*this, d_src, d_dst, d_ts, n, btmin, btmax);
    size_t del_old = 0, del_new = 0;
    if (cfg.max_time_capacity > 0) {
        const int64_t cutoff = latest_ts - cfg.max_time_capacity;
        if (sb.keys32)
            hipLaunchKernelGGL((merge_evict_kernel<uint32_t>), dim3(1), dim3(1), 0, s, ts.p, e_old,
                               sb.k32, n, btmin, cutoff, red64.p);
        else
            hipLaunchKernelGGL((merge_evict_kernel<uint64_t>), dim3(1), dim3(1), 0, s, ts.p, e_old,
                               sb.k64, n, btmin, cutoff, red64.p);
        check_hip(hipMemcpyAsync(hs, red64.p, 32, hipMemcpyDeviceToHost, s), "read evict");
        sync();
        del_old = static_cast<size_t>(hs[0]);
        del_new = static_cast<size_t>(hs[1]);
        store_tmin = hs[2];
        store_tmax = hs[3];
    } else {
        store_tmin = std::min(store_tmin, btmin);
        store_tmax = std::max(store_tmax, btmax);
    }
    const size_t kept_old = e_old - del_old, kept_new = n - del_new, kept = kept_old + kept_new;
    src2.resize(kept);
    dst2.resize(kept);
    ts2.resize(kept);
    uint32_t* perm = nullptr;
    if (feat_dim > 0) {
        merge_perm.resize(std::max<size_t>(kept, 1));
        perm = merge_perm.p;
    }
    if (kept_old) {
        if (sb.keys32)
            hipLaunchKernelGGL((merge_old_kernel<uint32_t>), dim3(grid_for(kept_old)), dim3(kB), 0, s,
                               ts.p, src.p, dst.p, del_old, e_old, sb.k32, del_new, n, btmin,
                               src2.p, dst2.p, ts2.p, perm);
        else
            hipLaunchKernelGGL((merge_old_kernel<uint64_t>), dim3(grid_for(kept_old)), dim3(kB), 0, s,
                               ts.p, src.p, dst.p, del_old, e_old, sb.k64, del_new, n, btmin,
                               src2.p, dst2.p, ts2.p, perm);
    }
    if (kept_new) {
        if (sb.keys32)
            hipLaunchKernelGGL((merge_new_kernel<uint32_t>), dim3(grid_for(kept_new)), dim3(kB), 0, s,
                               ts.p, del_old, e_old, sb.k32, sb.ends, sb.bpos, del_new, n, btmin,
                               src2.p, dst2.p, ts2.p, perm);
        else
            hipLaunchKernelGGL((merge_new_kernel<uint64_t>), dim3(grid_for(kept_new)), dim3(kB), 0, s,
                               ts.p, del_old, e_old, sb.k64, sb.ends, sb.bpos, del_new, n, btmin,
                               src2.p, dst2.p, ts2.p, perm);
    }
    if (feat_dim > 0) {
        feat2.resize(kept * feat_dim);
        const uint32_t V = static_cast<uint32_t>(feat_dim / 4);
        if (kept && feat_dim % 4 == 0 && V <= 256 && aligned16(d_feat)) {
            const uint32_t R = 256 / V;
            const size_t blocks = std::min<size_t>((kept + R - 1) / R, 65536);
            hipLaunchKernelGGL(gather_feat_vec_kernel, dim3(blocks), dim3(V * R), 0, s, perm,
                               size_t{0}, kept, V, reinterpret_cast<const f32x4*>(feat.p), e_old,
                               reinterpret_cast<const f32x4*>(d_feat),
                               reinterpret_cast<f32x4*>(feat2.p));
        } else if (kept) {
            hipLaunchKernelGGL(gather_feat_kernel, dim3(grid_capped(kept * feat_dim)), dim3(kB), 0,
                               s, perm, size_t{0}, kept, feat_dim, feat.p, e_old, d_feat, feat2.p);
        }
        feat.swap(feat2);
    }
    src.swap(src2);
    dst.swap(dst2);
    ts.swap(ts2);
    E = kept;
    check_hip(hipGetLastError(), "merge launch");
}

void Engine::build_accepted(const int32_t* d_src, const int32_t* d_dst, const int64_t* d_ts,
                            const float* d_feat, size_t n, size_t dim, int64_t tmin,
                            int64_t tmax) {
    hipStream_t s = stream;
    int64_t* hs = reinterpret_cast<int64_t*>(host_scalars);
    const size_t e_old = E;
    const int64_t batch_tmin = tmin, batch_tmax = tmax;
    if (E == 0) feat_dim = dim;

    // the batch's endpoints, for ..._for_last_batch: copied on the side
    // stream beside the build; the build's end waits for them
    last_src.resize(n);
    last_dst.resize(n);
    check_hip(hipMemcpyAsync(last_src.p, d_src, n * 4, hipMemcpyDeviceToDevice, side), "last src");
    check_hip(hipMemcpyAsync(last_dst.p, d_dst, n * 4, hipMemcpyDeviceToDevice, side), "last dst");
    check_hip(hipEventRecord(side_done, side), "event");
    last_n = n;
    if (e_old) {
        tmin = std::min(tmin, store_tmin);
        tmax = std::max(tmax, store_tmax);
    }
    latest_ts = std::max(latest_ts, batch_tmax);

    // ---- 2-4. the new store: sorted stable by (ts, position), the window's
    // old edges evicted.  A batch whose timestamps are all >= the store's
    // (streaming) goes after the store's kept edges as it is, sorted alone;
    // any other batch is sorted together with the store.
    append_mode = e_old > 0 && batch_tmin >= store_tmax;
    merge_mode = e_old > 0 && !append_mode;
    if (append_mode)
        append_store(d_src, d_dst, d_ts, d_feat, n, batch_tmin, batch_tmax);
    else if (merge_mode)
        merge_store(d_src, d_dst, d_ts, d_feat, n, batch_tmin, batch_tmax);
    else
        sort_store(d_src, d_dst, d_ts, d_feat, n, tmin, tmax);
    check_hip(hipEventRecord(ev[1], s), "event");

    // ---- 5. max node id, timestamp groups.  Without an eviction the store
    // is the old store plus the batch, whose largest id the batch's reduction
    // found; an eviction can remove the largest id, so the store is reduced
    const bool evicted = E != e_old + n;
    if (evicted) {
        red32.ensure(4);
        max_i32_pair(src.p, dst.p, E, red32.p, s);
    }
    flags.ensure(2 * E + 1);
    scan.ensure(2 * E + 1);
    scan_scratch.ensure(scan_scratch_elems(2 * E + 1));
    hipLaunchKernelGGL(ts_group_flags_kernel, dim3(grid_for(E)), dim3(kB), 0, s, ts.p, E, flags.p);
    exclusive_scan_u32(flags.p, scan.p, E, scan_scratch.p, s);
    if (evicted) check_hip(hipMemcpyAsync(hs, red32.p, 4, hipMemcpyDeviceToHost, s), "read max id");
    check_hip(hipMemcpyAsync(hs + 1, scan.p + E, 4, hipMemcpyDeviceToHost, s), "read T");
    sync();
    int32_t mx = std::max(max_node_id, batch_max_id);
    uint32_t tg;
    if (evicted) std::memcpy(&mx, hs, 4);
    std::memcpy(&tg, hs + 1, 4);
    max_node_id = mx;
    T = tg;
    tsg_off.resize(T + 1);
    uniq_ts.resize(T);
    erank.resize(E);
    hipLaunchKernelGGL(ts_group_scatter_kernel, dim3(grid_for(E)), dim3(kB), 0, s, ts.p, E,
                       flags.p, scan.p, tsg_off.p, uniq_ts.p, erank.p);
    update_neg1_rank(*this);

    // ---- 5b. global cumulative weights (edge_data.cu:440-514) on the side
    // stream, beside the node index: they read only the timestamp groups.
    // Pivots are the store's min/max ts.  Their buffers are the side's own.
    weights_ready = false;
    const bool weights = cfg.enable_weight_computation || cfg.enable_temporal_node2vec;
    if (weights) {
        hipStream_t sd = side;
        check_hip(hipEventRecord(ts_ready, s), "event");
        check_hip(hipStreamWaitEvent(sd, ts_ready, 0), "wait timestamp groups");
        const double bound = cfg.timescale_bound;
        const double diff = static_cast<double>(store_tmax - store_tmin);
        const double scale = (bound > 0 && diff > 0) ? bound / diff : 1.0;
        fwd_cum.resize(T);
        bwd_cum.resize(T);
        hipLaunchKernelGGL(global_weights_kernel, dim3(grid_for(T)), dim3(kB), 0, sd, tsg_off.p,
                           uniq_ts.p, T, store_tmin, store_tmax, bound, scale, fwd_cum.p,
                           bwd_cum.p);
        gsum.ensure(2 * (2 + 1024));
        sum_f64(fwd_cum.p, T, gsum.p, sd);
        sum_f64(bwd_cum.p, T, gsum.p + 2 + 1024, sd);
        hipLaunchKernelGGL(divide_kernel, dim3(grid_for(T)), dim3(kB), 0, sd, fwd_cum.p,
                           bwd_cum.p, T, gsum.p, gsum.p + 2 + 1024);
        fscan_scratch.ensure(scan_scratch_elems(T));
        inclusive_scan_f64(fwd_cum.p, T, fscan_scratch.p, sd);
        inclusive_scan_f64(bwd_cum.p, T, fscan_scratch.p, sd);
        // the weight search counts entries below its target, which is the
        // lower_bound only on a non-decreasing array
        running_max_f64(fwd_cum.p, T, fscan_scratch.p, sd);
        running_max_f64(bwd_cum.p, T, fscan_scratch.p, sd);
        build_global_guide(*this, sd, fwd_cum, T, true, gwg_fwd, gwt_fwd);
        build_global_guide(*this, sd, bwd_cum, T, false, gwg_bwd, gwt_bwd);
        check_hip(hipEventRecord(side_done, sd), "event");
    }

    // ---- 6. node index
    const size_t v = static_cast<size_t>(max_node_id) + 1;  // active_node_ids size
    const size_t vc = v + 1;                                // node_index_capacity
    const int key_bits = std::max(1, bit_length_u64(static_cast<uint64_t>(max_node_id)));
    if (append_mode) {
        append_direction(*this, out, cfg.is_directed ? 0 : 2, key_bits, vc, hs);
        if (cfg.is_directed) append_direction(*this, in, 1, key_bits, vc, hs);
        else in.clear();
    } else if (cfg.is_directed) {
        build_direction(*this, out, E, key_bits, vc, 0, hs);
        build_direction(*this, in, E, key_bits, vc, 1, hs);
    } else {
        build_direction(*this, out, 2 * E, key_bits, vc, 2, hs);
        in.clear();
    }
    active.resize(v);
    hipLaunchKernelGGL(active_flags_kernel, dim3(grid_for(v)), dim3(kB), 0, s, out.off.p,
                       cfg.is_directed ? in.off.p : nullptr, v, active.p);
    check_hip(hipGetLastError(), "index launch");
    check_hip(hipEventRecord(ev[2], s), "event");

    // ---- 7. node2vec adjacency (edge_data.cu:298-392).  The walks' test "is
    // a candidate adjacent to the previous node?" probes a hash set of the
    // node pairs joined by an edge, each once in increasing order -- about
    // one line -- instead of binary-searching a hub's list of millions of
    // neighbours.  The sorted neighbour lists themselves are only read
    // through trw_get_array, which builds them on first request after an
    // ingest (build_adjacency_lists).
    adj_ready = adj_lists_ready = false;
    if (cfg.enable_temporal_node2vec) {
        const int b = key_bits;
        const size_t m2 = E;  // one pair key per edge
        // the pairs sorted with duplicates adjacent: as 32-bit keys of the
        // active ids' ranks when two ranks fit (a streaming window of a
        // power-law graph touches few of its ids: cfg5's 15k of 1M ids make
        // 28-bit keys, three passes of 4-byte keys instead of four of
        // 8-byte ones), else as 64-bit keys of the ids
        flags.ensure(v + 1);
        scan.ensure(v + 1);
        scan_scratch.ensure(scan_scratch_elems(std::max(v + 1, m2 + 1)));
        hipLaunchKernelGGL(active_u32_kernel, dim3(grid_for(v)), dim3(kB), 0, s, active.p, v,
                           flags.p);
        exclusive_scan_u32(flags.p, scan.p, v, scan_scratch.p, s);
        check_hip(hipMemcpyAsync(hs, scan.p + v, 4, hipMemcpyDeviceToHost, s), "read active count");
        sync();
        uint32_t n_active;
        std::memcpy(&n_active, hs, 4);
        const int rb = std::max(1, bit_length_u64(n_active ? n_active - 1 : 0));
        const bool ranked = 2 * rb <= 32;
        hist.ensure(radix_hist_elems(m2));
        const uint32_t* rkeys = nullptr;
        const uint64_t* fkeys = nullptr;
        if (ranked) {
            adj_rank.resize(v + 1);
            check_hip(hipMemcpyAsync(adj_rank.p, scan.p, (v + 1) * 4, hipMemcpyDeviceToDevice, s),
                      "rank copy");
            adj_ids.resize(std::max<size_t>(n_active, 1));
            hipLaunchKernelGGL(active_ids_kernel, dim3(grid_for(v)), dim3(kB), 0, s, active.p,
                               adj_rank.p, v, adj_ids.p);
            k32a.ensure(m2);
            k32b.ensure(m2);
            if (E)
                hipLaunchKernelGGL(adj_rank_keys_kernel, dim3(grid_for(E)), dim3(kB), 0, s, src.p,
                                   dst.p, E, adj_rank.p, rb, k32a.p);
            const int w = radix_sort_u32(k32a.p, nullptr, k32b.p, nullptr, m2, 0, 2 * rb, hist.p, s);
            rkeys = w ? k32b.p : k32a.p;
        } else {
            k64a.ensure(m2);
            k64b.ensure(m2);
            if (E)
                hipLaunchKernelGGL(adj_pair_keys_kernel, dim3(grid_for(E)), dim3(kB), 0, s, src.p,
                                   dst.p, E, b, k64a.p);
            const int w = radix_sort_u64(k64a.p, nullptr, k64b.p, nullptr, m2, 0, 2 * b, hist.p, s);
            fkeys = w ? k64b.p : k64a.p;
        }
        // a set at most half full of the distinct pairs
        size_t distinct = m2;
        if (ranked && m2) {
            flags.ensure(m2 + 1);
            scan.ensure(m2 + 1);
            hipLaunchKernelGGL(distinct_flags_kernel, dim3(grid_for(m2)), dim3(kB), 0, s, rkeys, m2,
                               flags.p);
            exclusive_scan_u32(flags.p, scan.p, m2, scan_scratch.p, s);
            check_hip(hipMemcpyAsync(hs, scan.p + m2, 4, hipMemcpyDeviceToHost, s), "read pairs");
            sync();
            uint32_t dcount;
            std::memcpy(&dcount, hs, 4);
            distinct = dcount;
        }
        int lg = 10;
        while ((size_t{1} << lg) < 2 * distinct) ++lg;
        adj_hash.resize(size_t{1} << lg);
        check_hip(hipMemsetAsync(adj_hash.p, 0xff, (size_t{1} << lg) * sizeof(uint64_t), s),
                  "adjacency set clear");
        if (m2 && ranked)
            hipLaunchKernelGGL(adj_hash_insert_ranked_kernel, dim3(grid_for(m2)), dim3(kB), 0, s,
                               rkeys, m2, rb, adj_ids.p, b, 64 - lg, (uint64_t{1} << lg) - 1,
                               adj_hash.p);
        else if (m2)
            hipLaunchKernelGGL(adj_hash_insert_kernel, dim3(grid_for(m2)), dim3(kB), 0, s, fkeys,
                               m2, 64 - lg, (uint64_t{1} << lg) - 1, adj_hash.p);
        adj_hash_log = lg;
        adj_bits = b;
        adj_nodes = v;
        check_hip(hipGetLastError(), "adjacency launch");
        adj_ready = true;
    }

    // ---- 8. per-node weights (node_edge_index.cu:644-684): outbound
    // forward + backward, inbound backward (directed); the global ones run
    // on the side stream (5b)
    if (weights) {
        const double bound = cfg.timescale_bound;
        out.w_fwd.resize(out.n_groups);
        out.w_bwd.resize(out.n_groups);
        node_weights(*this, out, v, bound, true, hs);
        if (cfg.is_directed) {
            in.w_bwd.resize(in.n_groups);
            node_weights(*this, in, v, bound, false, hs);
        }
        // the weight pickers' views: forward walks read out's forward
        // weights, backward walks in's backward weights (out's if undirected)
        build_walk_weights(*this, out, v, out.w_fwd, true, out.wf);
        if (cfg.is_directed) build_walk_weights(*this, in, v, in.w_bwd, false, in.wb);
        else build_walk_weights(*this, out, v, out.w_bwd, false, out.wb);
        check_hip(hipGetLastError(), "weights launch");
        weights_ready = true;
    }

    check_hip(hipStreamWaitEvent(s, side_done, 0), "wait side");
    check_hip(hipEventRecord(ev[3], s), "event");
    sync();
    float ms = 0;
    check_hip(hipEventElapsedTime(&ms, ev[0], ev[3]), "elapsed");
    timings.build_ms = ms;
    check_hip(hipEventElapsedTime(&ms, ev[0], ev[1]), "elapsed");
    timings.sort_ms = ms;
    check_hip(hipEventElapsedTime(&ms, ev[1], ev[2]), "elapsed");
    timings.index_ms = ms;
}

void Engine::build_adjacency_lists() {
    // edge_data.cu:298-392: every edge adds v to N(u) and u to N(v),
    // duplicates kept, each list ascending -- one radix sort of the 2E keys
    // owner << b | neighbour
    if (!adj_ready || adj_lists_ready) return;
    hipStream_t s = stream;
    const int b = adj_bits;
    const size_t m2 = 2 * E, v = adj_nodes;
    k64a.ensure(m2);
    k64b.ensure(m2);
    hist.ensure(radix_hist_elems(m2));
    if (E)
        hipLaunchKernelGGL(adj_keys_kernel, dim3(grid_for(E)), dim3(kB), 0, s, src.p, dst.p, E, b,
                           k64a.p);
    const int w = radix_sort_u64(k64a.p, nullptr, k64b.p, nullptr, m2, 0, 2 * b, hist.p, s);
    uint64_t* ak = w ? k64b.p : k64a.p;
    adj_nbr.resize(m2);
    if (m2)
        hipLaunchKernelGGL(adj_finish_kernel, dim3(grid_for(m2)), dim3(kB), 0, s, ak, m2,
                           (1ull << b) - 1, adj_nbr.p);
    adj_off.resize(v + 1);
    hipLaunchKernelGGL(adj_offsets_kernel, dim3(grid_for(v + 1)), dim3(kB), 0, s, ak, m2, b,
                       v + 1, adj_off.p);
    check_hip(hipGetLastError(), "adjacency lists launch");
    sync();
    adj_lists_ready = true;
}

void Engine::clear() {
    // core/temporal_random_walk.cu:358-373: a fresh store with the same config
    E = 0;
    feat_dim = 0;
    latest_ts = 0;
    T = 0;
    max_node_id = -1;
    store_tmin = store_tmax = 0;
    src.n = dst.n = ts.n = feat.n = tsg_off.n = uniq_ts.n = erank.n = neg1_rank.n = active.n = 0;
    fwd_cum.n = bwd_cum.n = adj_off.n = adj_nbr.n = adj_hash.n = 0;
    gwg_fwd.n = gwg_bwd.n = gwt_fwd.n = gwt_bwd.n = 0;
    weights_ready = adj_ready = adj_lists_ready = false;
    adj_nodes = 0;
    out.clear();
    in.clear();
    last_n = 0;
    last_src.n = last_dst.n = 0;
}

void update_neg1_rank(Engine& e) {
    e.neg1_rank.resize(1);
    launch_neg1_rank(e, e.neg1_rank.p);
}

void launch_neg1_rank(Engine& e, int32_t* out) {
    hipLaunchKernelGGL(neg1_rank_kernel, dim3(1), dim3(1), 0, e.stream, e.uniq_ts.p,
                       static_cast<uint32_t>(e.E ? e.T : 0), out);
    check_hip(hipGetLastError(), "neg1 rank launch");
}

}  // namespace trw
