// index_layout.h -- the device-side layout of the walk's index: the records,
// headers and search structures the walk kernels read, and the constants
// that shape them (the kernels and the index build both include it).
//
// HBM layout (all arrays resident on the device; 32-bit positions because the
// reference itself caps the edge store at INT_MAX entries -- its sort uses
// `int` positions, graph/temporal_graph.cu:77-87):
//
//   edge store (sorted stable by (ts, insertion position))
//     src, dst      int32[E]      ts   int64[E]      feat fp32[E*dim]
//   timestamp groups
//     tsg_off       uint32[T+1]   uniq_ts int64[T]
//     erank         uint32[E]     rank of every stored edge's timestamp
//   node map        active uint8[max_id+1]   (dense flags, as the reference)
//   per direction (out = by source / both endpoints if undirected, in = by target)
//     off           uint32[V_c]    CSR offsets, V_c = max_id + 2
//     idx           uint32[n]      edge ids ordered stably by (node, position)
//     rec           EdgeRec[n]     (neighbour, edge id) in the same order
//     cnt           uint32[V_c]    exclusive prefix of per-node group counts
//     hdr           NodeHdr[V_c]   the walk's per-node header: first group,
//                                  group count, bucket shift, first rank,
//                                  bucket count
//     tab           uint32[2(g+V_c)] bucket tables of nodes with > kTabMin
//                                  groups, node u's at 2 (gb + u): bucket b
//                                  covers the ranks [r0 + (b << shift),
//                                  r0 + ((b + 1) << shift)) and holds the
//                                  first of u's groups that reaches it; a
//                                  closing entry G follows the last bucket
//     grp           uint32[g+1]    group starts into idx, plus a terminator
//     first_ts      int64[g]       timestamp of every node-timestamp group
//     pan           PanelRec[g+1]  (ts rank, start) of every group, plus a
//                                  terminator: the walk's search panel; the
//                                  rank is the group's timestamp's position
//                                  among the unique timestamps, so it orders
//                                  exactly as the timestamp does, and the
//                                  picked group's range usually shares the
//                                  line of the search's last probe
//     w_fwd, w_bwd  fp64[g]        per-node cumulative exponential weights
//     wrec          WEdgeRec[n << s] (neighbour, edge id, the walk's next
//                                  slice bound at the neighbour) in idx
//                                  order, built with the weights (below); in
//                                  the out direction with the ExponentialWeight
//                                  weights (s = 1) every record is followed by
//                                  a 16-byte slot: the forward start sum of
//                                  its next slice
//   per walk direction with weights (forward walks: out with w_fwd; backward
//   walks: in with w_bwd, or out with w_bwd if undirected)
//     whdr          WNodeHdr[V_c]  node header + guide parameters and weight
//                                  total of the node's cumulative weights
//     wpan          WPanelRec[g << s] (ts rank, start, end, the first entry's
//                                  next slice bound, cumulative weight, first
//                                  edge record) of every group; forward views
//                                  with the ExponentialWeight weights (s = 1)
//                                  follow every record with a 32-byte slot:
//                                  its first entry's next slice's start sum
//                                  and its second entry (WPanelSlot)
//     wgt           uint32[2(g+V_c)] guide tables of nodes with > kWGuideMin
//                                  groups, node u's at 2 (gb + u) (below)
//   global weights  fwd_cum, bwd_cum fp64[T] (+ their guides: one segment)
//   node2vec        adj_hash uint64[2^k >= 2 x distinct edge pairs] (the
//                   endpoints of every edge, smaller first: a membership set,
//                   built with the index); adj_off uint32[max_id+2], adj_nbr
//                   int32[2E] (sorted lists, built when first requested)
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace trw {

// One entry of a node's list as the walk reads it: the node reached over the
// edge and the edge id, one 8-byte load.  Its timestamp is the
// group's (every entry of a node-timestamp group shares it), carried by the
// walk as the group's rank.
struct alignas(8) EdgeRec {
    int32_t nbr;
    uint32_t eid;
};
static_assert(sizeof(EdgeRec) == 8, "EdgeRec must be 8 bytes");

// Segments of more than this many cumulative weights get a guide table (below);
// shorter ones are binary-searched directly (at most two lines of a weighted
// panel).
constexpr uint32_t kWGuideMin = 16;

// Adjacency pair set: an empty slot, and the multiplier of its Fibonacci
// hash (slot = key * kAdjHashMul >> (64 - log2 slots)).
constexpr uint64_t kAdjEmpty = ~0ull;
constexpr uint64_t kAdjHashMul = 0x9E3779B97F4A7C15ull;

// ---- weight guide tables ----------------------------------------------------
// An inverse-CDF guide table (Chen & Asau, "On generating random variates
// from an empirical distribution", AIIE Trans. 6, 1974) over each segment of
// more than kWGuideMin cumulative weights, keyed not by the weight but by
// wg_key(weight): an integer that never decreases as the weight grows and is
// spaced about evenly in the logarithm of the weight's distance from the end
// its picks crowd towards.  Bucket b of a segment holds the first local index
// whose key bucket is >= b, followed by a closing entry G; since the key is
// monotone, the lower_bound of any target (at most the segment's last weight)
// whose key falls in bucket b lies in [tab[b], tab[b + 1]] -- exact, whatever
// the weights look like.
//
// The key of a decaying segment (forward weights: most mass at its start, so
// a late slice's sums sit within a few ulps of 1) is the bit pattern of
// 1 - c, negated: 1 - c is monotone under round-to-nearest, and the bits of a
// positive double order as its value, so the key is monotone and grows by
// 2^52 per halving of 1 - c.  A growing segment (backward weights) keys on
// the bits of c itself.  Either way an exponential weight profile maps to
// keys that are close to linear in the group index.
constexpr uint32_t kWgBucketsPerGroup = 2;
// A segment of G weights has at most kWgBucketsPerGroup * G buckets plus the
// closing entry; node u's table at 2 (gb + u) has room for 2 G + 2 of them,
// and a global segment's table holds 2 G + 1.
static_assert(kWgBucketsPerGroup <= 2, "guide tables have room for 2 buckets per group");
// Runs of more buckets than this between two consecutive groups are filled by
// a wave each rather than by the group's thread.
constexpr uint32_t kWgRun = 16;

__host__ __device__ inline uint64_t wg_double_bits(double x) {
#ifdef __HIP_DEVICE_COMPILE__
    return static_cast<uint64_t>(__double_as_longlong(x));
#else
    uint64_t b;
    __builtin_memcpy(&b, &x, 8);
    return b;
#endif
}
// Monotone key of a cumulative weight c (see above); never negative for
// c >= 0, negative only for a negative decaying target.
__host__ __device__ inline int64_t wg_key(double c, bool decaying) {
    if (decaying) {
        double u = 1.0 - c;
        if (!(u >= 0x1p-54)) u = 0x1p-54;  // c at or above 1 (and NaN)
        return static_cast<int64_t>(wg_double_bits(1.0)) - static_cast<int64_t>(wg_double_bits(u));
    }
    return c > 0.0 ? static_cast<int64_t>(wg_double_bits(c)) : 0;
}

// A segment's guide parameters and its last (largest) cumulative weight.
struct alignas(16) WGuide {
    uint64_t bs;   // bucket shift (bits 0-5) and the first bucket's key >> shift
                   // (bits 6-63); unused for a segment of at most kWGuideMin
    double total;  // the segment's last cumulative weight
};
static_assert(sizeof(WGuide) == 16, "WGuide must be 16 bytes");
// Bucket of the key of a target no larger than the segment's total (so at
// most the last bucket); keys below the first bucket go to bucket 0.
__host__ __device__ inline uint32_t wg_bucket(uint64_t bs, int64_t key) {
    const int sh = static_cast<int>(bs & 63u);
    const int64_t kb = key >> sh, base = static_cast<int64_t>(bs >> 6);
    return kb <= base ? 0u : static_cast<uint32_t>(kb - base);
}

// Nodes with more groups than this get a bucket table for the walk's search;
// smaller ones are binary-searched directly (at most two panel lines).
constexpr uint32_t kTabMin = 16;
// A node's table has at most this many buckets per group: hubs whose groups
// cover most ranks of their span get single-rank buckets, whose entry is the
// search's answer.
constexpr uint32_t kTabBucketsPerGroup = 2;

// Per-node header of the walk's group search, read with one 16-byte load.
// Node u's bucket table starts at entry 2 * (gb + u) of `tab` (room for the
// 2 * G + 1 entries its at most 2 * G buckets need, so no base is stored).
struct alignas(16) NodeHdr {
    uint32_t gb;    // first group of the node
    uint32_t meta;  // G (bits 0-23, kHdrGMask if larger: read the next gb),
                    // bucket shift (bits 24-28), dense flag (bit 31: a
                    // tabled node with a group at every rank of its span)
    uint32_t r0;    // rank of its first group (tabled nodes)
    uint32_t nb;    // number of buckets (tabled nodes)
};
constexpr uint32_t kHdrGMask = 0xffffffu;
constexpr uint32_t kHdrDense = 1u << 31;
__host__ __device__ inline uint32_t hdr_shift(const NodeHdr& h) { return (h.meta >> 24) & 31u; }
__host__ __device__ inline uint64_t hdr_tab_base(const NodeHdr& h, uint32_t u) {
    return 2ull * (static_cast<uint64_t>(h.gb) + u);
}
static_assert(sizeof(NodeHdr) == 16, "NodeHdr must be 16 bytes");

// One node-timestamp group in the walk's search panel.
struct alignas(8) PanelRec {
    uint32_t rank;   // index of the group's timestamp in uniq_ts
    uint32_t start;  // first entry (position in idx / rec); the next record's
                     // start ends the group
};
static_assert(sizeof(PanelRec) == 8, "PanelRec must be 8 bytes");

// The weight pickers' view of a node: its header and the guide of its
// cumulative weights, one 32-byte load.
struct alignas(32) WNodeHdr {
    NodeHdr h;
    WGuide g;
};
static_assert(sizeof(WNodeHdr) == 32, "WNodeHdr must be 32 bytes");

// One node-timestamp group in the weight pickers' panel: its panel record, its
// end, its cumulative weight and its first edge record (with that entry's
// next slice bound, below), so the weight search, the slice's sums, the
// picked group's range and -- for a group of one edge -- the edge itself read
// one aligned 32-byte record.
struct alignas(32) WPanelRec {
    uint32_t rank;
    uint32_t start;
    uint32_t end;   // the next group's start
    uint32_t nxt0;  // wrec[start].nxt
    double c;
    EdgeRec rec0;  // rec[start]
};
static_assert(sizeof(WPanelRec) == 32, "WPanelRec must be 32 bytes");
// A forward view's panel whose records are followed by a 32-byte slot (wide,
// shift 1) holds there, as its first double, the start sum of rec0's next
// slice: c[vb - 1] in the view's cumulative weights c at rec0's neighbour v,
// vb the bound nxt0 carries (0 when vb is 0); kNoSum where nxt0 holds no
// bound.  A forward walk that takes rec0 then starts its next weight pick
// without loading the record before its slice.  The rest of the slot holds the
// group's second entry (its record, next slice bound and start sum; rec1 =
// {0, 0}, bs1 = kNoSum for a group of one entry), so a pick of either of a
// group's first two entries reads no edge record.  The forward view's edge
// records (WEdgeRec, the out direction's) are wide alike, a 16-byte slot after
// each holding the same start sum for that entry.  Panels and records are
// wide only for the ExponentialWeight weights' forward walks (node2vec's
// retries pay for the larger arrays in cache; backward walks keep the build's
// gathers).
struct alignas(32) WPanelSlot {
    double bs0;
    EdgeRec rec1;  // rec[start + 1]
    uint32_t nxt1;
    uint32_t pad;
    double bs1;
};
static_assert(sizeof(WPanelSlot) == 32, "WPanelSlot must be 32 bytes");
constexpr double kNoSum = -1.0;  // the sums are >= 0

// The records of a direction with weights: an entry (u, v, r) -- neighbour v
// reached at timestamp rank r -- also holds where the walk's next valid slice
// at v begins or ends.  A walk that takes the entry continues from v at time
// r, and its time search there is the lower_bound b of r among v's group
// ranks (backward: the slice ends at b) or of r + 1 (forward: it starts at b,
// plus one when v has a group at r itself).  nxt holds v's first group plus b
// (a global panel index) in bits 0-30 and that "group at r" flag in bit 31,
// so one record serves both walk directions of an undirected index; kNoNext
// where the index is too large for 30 bits.  Bit 30 flags b == 0.  The search
// it replaces reads a node's bucket table and panel: one random line less per
// hop at a hub.
struct alignas(16) WEdgeRec {
    int32_t nbr;
    uint32_t eid;
    uint32_t nxt;
    uint32_t pad;
};
static_assert(sizeof(WEdgeRec) == 16, "WEdgeRec must be 16 bytes");
constexpr uint32_t kNoNext = 0xffffffffu;
constexpr uint32_t kNextMax = 0x3ffffffeu;  // largest global bound nxt holds
constexpr uint32_t kNextFirst = 1u << 30;   // nxt: b is 0
constexpr uint32_t kNextAt = 1u << 31;      // nxt: v has a group at r

// The global bound a walk of direction Fwd reads from nxt (kNoNext: search).
template <bool Fwd>
__host__ __device__ inline uint32_t next_bound(uint32_t nxt) {
    if (nxt == kNoNext) return kNoNext;
    return (nxt & (kNextFirst - 1u)) + (Fwd ? (nxt >> 31) : 0u);
}
// Whether that bound is v's first group (local index 0): no weight bounds
// the slice there.
template <bool Fwd>
__host__ __device__ inline bool next_bound_first(uint32_t nxt) {
    return (nxt & kNextFirst) && !(Fwd && (nxt & kNextAt));
}

typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));
typedef uint32_t u32x4_a8 __attribute__((ext_vector_type(4), aligned(8)));

// First local index i in [0, G) whose group rank is >= x, G if none: a
// lower_bound over the node's sorted panel, so the answer is unique and the
// way it is found does not change any result.  A node with more than kTabMin
// groups that has a group at every rank of its span (dense) answers from the
// rank itself.  Another such node looks up x's bucket b in its table: a
// single-rank bucket holds the answer itself; a wider one gives the bracket
// [tab[b], tab[b + 1]] (about one group).  The rest is a binary search over
// at most kTabMin groups.
template <class Pan>
__device__ __forceinline__ int first_ge(const uint32_t* tab, const NodeHdr& h, uint32_t u, int G,
                                        const Pan& f, uint32_t x) {
    int lo = 0, hi = G;
    if (G > static_cast<int>(kTabMin)) {
        if (x <= h.r0) return 0;
        if (h.meta & kHdrDense) return static_cast<int>(min(x - h.r0, static_cast<uint32_t>(G)));
        const uint32_t shift = hdr_shift(h);
        const uint32_t b = (x - h.r0) >> shift;
        if (b >= h.nb) return G;  // past the last bucket
        const uint32_t* t = tab + hdr_tab_base(h, u) + b;
        if (shift == 0) return static_cast<int>(t[0]);
        const u32x2_a4 br = *reinterpret_cast<const u32x2_a4*>(t);  // one 8-byte load
        lo = static_cast<int>(br.x);
        hi = static_cast<int>(br.y);
    }
    while (lo < hi) {
        const int mid = lo + ((hi - lo) >> 1);
        if (f[mid].rank >= x) hi = mid;
        else lo = mid + 1;
    }
    return lo;
}


}  // namespace trw
