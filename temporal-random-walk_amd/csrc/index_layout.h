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
//     wx_off        uint32[V_c]    each node's base in the weight search index
//     wx_fwd/wx_bwd fp64[..]       weight search index of nodes with > kWIdxMin
//                                  groups: level k (k = 1..K) holds every
//                                  16^k-th cumulative weight, K the first level
//                                  of at most 16 entries; every level padded
//                                  with +inf to whole 16-entry (128-byte)
//                                  blocks; top level first
//   global weights  fwd_cum, bwd_cum fp64[T] (+ gwx_fwd, gwx_bwd: their
//                   search index, one segment of T)
//   node2vec        adj_hash uint64[2^k >= 4E] (pair membership set, built
//                   with the index); adj_off uint32[max_id+2], adj_nbr
//                   int32[2E] (sorted lists, built when first requested)
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace trw {

// One entry of a node's edge list in walk order: the node reached over the
// edge, the edge id and its timestamp -- everything a hop needs from the edge
// in one aligned 16-byte load (instead of idx -> dst -> ts, three dependent
// cache-line misses).
// One entry of a node's list as the walk reads it.  Its timestamp is the
// group's (every entry of a node-timestamp group shares it), carried by the
// walk as the group's rank.
struct alignas(8) EdgeRec {
    int32_t nbr;
    uint32_t eid;
};
static_assert(sizeof(EdgeRec) == 8, "EdgeRec must be 8 bytes");

// Cumulative-weight segments longer than this get a search index (levels of
// every 16^k-th value); shorter ones are binary-searched directly.
constexpr uint32_t kWIdxMin = 16;

// Adjacency pair set: an empty slot, and the multiplier of its Fibonacci
// hash (slot = key * kAdjHashMul >> (64 - log2 slots)).
constexpr uint64_t kAdjEmpty = ~0ull;
constexpr uint64_t kAdjHashMul = 0x9E3779B97F4A7C15ull;

// Geometry of the weight search index of a segment of G cumulative weights:
// level k has ceil(G / 16^k) entries; the top level K is the first with at
// most 16; each level is padded to whole 16-entry blocks.
__host__ __device__ inline uint32_t wx_level_entries(uint32_t G, uint64_t span) {
    return static_cast<uint32_t>((G + span - 1) / span);
}
__host__ __device__ inline uint32_t wx_pad16(uint32_t n) { return (n + 15u) & ~15u; }
__host__ __device__ inline uint64_t wx_top_span(uint32_t G) {
    uint64_t span = 16;
    while ((G + span - 1) / span > 16) span <<= 4;
    return span;
}
__host__ __device__ inline uint32_t wx_size(uint32_t G) {
    if (G <= kWIdxMin) return 0;
    uint32_t total = 0;
    for (uint64_t span = 16;; span <<= 4) {
        const uint32_t n = wx_level_entries(G, span);
        total += wx_pad16(n);
        if (n <= 16) break;
    }
    return total;
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

}  // namespace trw
