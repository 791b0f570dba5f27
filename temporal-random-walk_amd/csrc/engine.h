// engine.h -- internal state of one engine instance (one device, one stream).
//
// HBM layout (all arrays resident on the device; 32-bit positions because the
// reference itself caps the edge store at INT_MAX entries -- its sort uses
// `int` positions, graph/temporal_graph.cu:77-87):
//
//   edge store (sorted stable by (ts, insertion position))
//     src, dst      int32[E]      ts   int64[E]      feat fp32[E*dim]
//   timestamp groups
//     tsg_off       uint32[T+1]   uniq_ts int64[T]
//   node map        active uint8[max_id+1]   (dense flags, as the reference)
//   per direction (out = by source / both endpoints if undirected, in = by target)
//     off           uint32[V_c]    CSR offsets, V_c = max_id + 2
//     idx           uint32[n]      edge ids ordered stably by (node, position)
//     rec           EdgeRec[n]     (neighbour, edge id, ts) in the same order
//     cnt           uint32[V_c]    exclusive prefix of per-node group counts
//     grp           uint32[g+1]    group starts into idx, plus a terminator
//     first_ts      int64[g]       timestamp of every node-timestamp group
//                                  (the binary-search panel: one load/probe)
//     w_fwd, w_bwd  fp64[g]        per-node cumulative exponential weights
//   global weights  fwd_cum, bwd_cum fp64[T]
//   node2vec        adj_off uint32[max_id+2], adj_nbr int32[2E]
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/trw_engine.h"
#include "primitives.h"

namespace trw {

struct InvalidArgument : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};

// Grow-only device buffer; growth discards the contents.
template <typename T>
struct DBuf {
    T* p = nullptr;
    size_t n = 0;
    size_t cap = 0;

    DBuf() = default;
    DBuf(const DBuf&) = delete;
    DBuf& operator=(const DBuf&) = delete;
    ~DBuf() { release(); }

    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = cap = 0;
    }
    void ensure(size_t k) {
        if (k > cap) {
            release();
            const size_t c = k + k / 4 + 64;
            check_hip(hipMalloc(&p, c * sizeof(T)), "hipMalloc");
            cap = c;
        }
    }
    void resize(size_t k) {
        ensure(k);
        n = k;
    }
    void swap(DBuf& o) {
        std::swap(p, o.p);
        std::swap(n, o.n);
        std::swap(cap, o.cap);
    }
    size_t bytes() const { return n * sizeof(T); }
};

// One entry of a node's edge list in walk order: the node reached over the
// edge, the edge id and its timestamp -- everything a hop needs from the edge
// in one aligned 16-byte load (instead of idx -> dst -> ts, three dependent
// cache-line misses).
struct alignas(16) EdgeRec {
    int32_t nbr;
    uint32_t eid;
    int64_t ts;
};
static_assert(sizeof(EdgeRec) == 16, "EdgeRec must be 16 bytes");

struct DirIndex {
    DBuf<uint32_t> off;      // V_c
    DBuf<uint32_t> idx;      // n entries
    DBuf<EdgeRec> rec;       // n entries, same order as idx
    DBuf<uint32_t> key;      // node of every entry (sorted)
    DBuf<uint32_t> cnt;      // V_c
    DBuf<uint32_t> grp;      // g + 1
    DBuf<int64_t> first_ts;  // g
    DBuf<double> w_fwd;      // g (outbound only)
    DBuf<double> w_bwd;      // g
    size_t n_entries = 0;
    size_t n_groups = 0;
    bool present = false;

    void clear() {
        off.n = idx.n = rec.n = key.n = cnt.n = grp.n = first_ts.n = w_fwd.n = w_bwd.n = 0;
        n_entries = n_groups = 0;
        present = false;
    }
};

// One device -> host span of a handoff.
struct HostCopy {
    void* dst;
    const void* src;
    size_t bytes;
};

// Per-thread resources of the host handoff: a stream and two pinned staging
// buffers (double buffering), created on first use.
struct HostLane {
    hipStream_t stream = nullptr;
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    HostLane() = default;
    HostLane(const HostLane&) = delete;
    HostLane& operator=(const HostLane&) = delete;
    ~HostLane();
    void init();
};

// Caller-owned host output buffer (released with free()).
void* host_output_alloc(size_t bytes);

struct Engine {
    trw_config cfg{};
    int device = 0;
    hipStream_t stream = nullptr;

    // edge store (+ the second half of a ping-pong pair for the gather)
    DBuf<int32_t> src, dst, src2, dst2;
    DBuf<int64_t> ts, ts2;
    DBuf<float> feat, feat2;
    size_t E = 0;
    int64_t store_tmin = 0, store_tmax = 0;
    size_t feat_dim = 0;
    int64_t latest_ts = 0;  // TemporalGraphData::latest_timestamp starts at 0

    // timestamp groups
    DBuf<uint32_t> tsg_off;
    DBuf<int64_t> uniq_ts;
    size_t T = 0;

    // node map
    int32_t max_node_id = -1;
    DBuf<uint8_t> active;

    // global weights
    DBuf<double> fwd_cum, bwd_cum;
    bool weights_ready = false;

    // node2vec adjacency
    DBuf<uint32_t> adj_off;
    DBuf<int32_t> adj_nbr;
    bool adj_ready = false;

    DirIndex out, in;

    // last ingested batch (for ..._for_last_batch)
    DBuf<int32_t> last_src, last_dst;
    size_t last_n = 0;

    // scratch
    DBuf<uint64_t> k64a, k64b;
    DBuf<uint32_t> k32a, k32b, v32a, v32b;
    DBuf<uint32_t> hist, hist_scratch, flags, scan, scan_scratch;
    DBuf<uint64_t> scan64_scratch;
    DBuf<double> dscratch, fscan_scratch;
    DBuf<int64_t> red64;    // reduction results + partials
    DBuf<int32_t> red32;
    DBuf<int32_t> stage_src, stage_dst;
    DBuf<int64_t> stage_ts;
    DBuf<float> stage_feat;
    DBuf<int32_t> starts;
    DBuf<int64_t> cutoffs;
    DBuf<double> replay;
    DBuf<uint64_t> acc64;

    // walks (device): slot-major scratch written by the walk kernel, then the
    // row-major output [num_walks, L] the reference's API returns
    DBuf<int32_t> sw_nodes;
    DBuf<int64_t> sw_ts, sw_eids;
    DBuf<int32_t> w_nodes;
    DBuf<int64_t> w_ts, w_eids;
    DBuf<uint64_t> w_lens;
    DBuf<float> w_feat;
    uint64_t w_num = 0;
    int w_len = 0;
    int w_dir_forward = 1;

    // pinned host scalars for the few readbacks that size allocations
    void* host_scalars = nullptr;

    // host handoff lanes
    std::vector<std::unique_ptr<HostLane>> lanes;

    // timings
    hipEvent_t ev[8] = {};
    trw_timings timings{};

    explicit Engine(const trw_config& c);
    ~Engine();

    void sync() { check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize"); }

    // ingest: batch arrays in device memory
    void build(const int32_t* d_src, const int32_t* d_dst, const int64_t* d_ts,
               const float* d_feat, size_t n, size_t dim);
    void clear();

    // sampling into w_* buffers
    void sample(const trw_sample_params& p);

    size_t memory_used() const;

    // Waits for the engine stream, then copies every span to the host
    // (pinned staging, several threads); records timings.handoff_*.
    void copy_to_host(const HostCopy* segs, size_t nseg);
};

// ---- launchers implemented in build.hip / walk.hip -------------------------
void validate_batch(const Engine& e, const void* feat, size_t n, size_t dim);
void walk_stats(Engine& e, trw_walk_stats* out);

}  // namespace trw
