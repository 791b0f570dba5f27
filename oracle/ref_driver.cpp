// ref_driver.cpp -- TEST INFRASTRUCTURE ONLY.
//
// A thin C-ABI driver around the reference's OWN CPU code, compiled from the
// reference sources where they lie (oracle/Makefile, target `ref`) into
// oracle/_ref/libtrw_ref.so.  Used only by tests/ to pin oracle/trw_oracle.c.
//
// What it runs from the reference (v1.8.6, temporal_random_walk/src/):
//   node_edge_index::rebuild                  graph/node_edge_index.cu:1329-1400
//   node_edge_index::update_temporal_weights_std  graph/node_edge_index.cu:644-684
//   temporal_random_walk::launch_random_walk_cpu_new
//                                            core/temporal_random_walk_cpu.cuh:155-197
//   (selectors, pickers and node2vec are header-only and come with it)
//
// What it cannot run: graph/edge_data.cu (needs <tbb/parallel_scan.h>, absent
// from this image) and therefore temporal_graph.cu's ingest pipeline.  The
// edge store, timestamp groups, active-node flags, global weights and the
// node2vec adjacency are taken from the oracle and injected here.
#include <cstring>
#include <string>

#include "core/temporal_random_walk_cpu.cuh"
#include "data/temporal_graph_view.cuh"
#include "graph/node_edge_index.cuh"

namespace {

struct RefGraph {
    TemporalGraphData data{false};
};

template <typename T>
void load(Buffer<T>& b, const void* src, size_t n) {
    b.resize(n);
    if (n) std::memcpy(b.data(), src, n * sizeof(T));
}

}  // namespace

extern "C" {

void* ref_create(int is_directed, int enable_weight, int enable_tn2v,
                 double timescale_bound, double p, double q) {
    auto* g = new RefGraph();
    TemporalGraphData& d = g->data;
    d.is_directed = is_directed != 0;
    d.timescale_bound = timescale_bound;
    d.node2vec_p = p;
    d.node2vec_q = q;
    d.inv_p = 1.0 / p;
    d.inv_q = 1.0 / q;
    d.enable_temporal_node2vec = enable_tn2v != 0;
    d.enable_weight_computation = enable_weight != 0 || enable_tn2v != 0;
    return g;
}

void ref_destroy(void* h) { delete static_cast<RefGraph*>(h); }

void ref_set_edge_store(void* h, const int* src, const int* dst, const int64_t* ts,
                        size_t E, const size_t* ts_group_offsets,
                        const int64_t* unique_ts, size_t T, const int* active,
                        size_t active_size, int max_node_id, const double* fwd_cum,
                        const double* bwd_cum, size_t w_size, const size_t* adj_off,
                        size_t adj_off_size, const int* adj_nbr, size_t adj_nbr_size) {
    TemporalGraphData& d = static_cast<RefGraph*>(h)->data;
    load(d.sources, src, E);
    load(d.targets, dst, E);
    load(d.timestamps, ts, E);
    load(d.timestamp_group_offsets, ts_group_offsets, T ? T + 1 : 0);
    load(d.unique_timestamps, unique_ts, T);
    load(d.active_node_ids, active, active_size);
    d.max_node_id = max_node_id;
    load(d.forward_cumulative_weights_exponential, fwd_cum, w_size);
    load(d.backward_cumulative_weights_exponential, bwd_cum, w_size);
    load(d.node_adj_offsets, adj_off, adj_off_size);
    load(d.node_adj_neighbors, adj_nbr, adj_nbr_size);
}

void ref_rebuild(void* h) {
    TemporalGraphData& d = static_cast<RefGraph*>(h)->data;
    node_edge_index::rebuild(d);
    if (d.enable_weight_computation) {
        node_edge_index::update_temporal_weights_std(d, d.timescale_bound);
    }
}

const void* ref_array(void* h, const char* name, size_t* len, size_t* es) {
    TemporalGraphData& d = static_cast<RefGraph*>(h)->data;
    const std::string n(name);
#define REF_ARR(nm, buf, sz)                 \
    if (n == nm) {                           \
        *len = (buf).size();                 \
        *es = (sz);                          \
        return (buf).data();                 \
    }
    REF_ARR("node_group_outbound_offsets", d.node_group_outbound_offsets, 8)
    REF_ARR("node_group_inbound_offsets", d.node_group_inbound_offsets, 8)
    REF_ARR("node_ts_sorted_outbound_indices", d.node_ts_sorted_outbound_indices, 8)
    REF_ARR("node_ts_sorted_inbound_indices", d.node_ts_sorted_inbound_indices, 8)
    REF_ARR("count_ts_group_per_node_outbound", d.count_ts_group_per_node_outbound, 8)
    REF_ARR("count_ts_group_per_node_inbound", d.count_ts_group_per_node_inbound, 8)
    REF_ARR("node_ts_group_outbound_offsets", d.node_ts_group_outbound_offsets, 8)
    REF_ARR("node_ts_group_inbound_offsets", d.node_ts_group_inbound_offsets, 8)
    REF_ARR("outbound_forward_cumulative_weights_exponential",
            d.outbound_forward_cumulative_weights_exponential, 8)
    REF_ARR("outbound_backward_cumulative_weights_exponential",
            d.outbound_backward_cumulative_weights_exponential, 8)
    REF_ARR("inbound_backward_cumulative_weights_exponential",
            d.inbound_backward_cumulative_weights_exponential, 8)
#undef REF_ARR
    *len = 0;
    *es = 0;
    return nullptr;
}

// Replay-mode walks through the reference's CPU walk loop.  Output buffers
// are filled the way WalkSetHost's constructor fills them
// (data/walk_set/walk_set_host.cu:10-30) before the loop runs.
void ref_walks(void* h, int max_walk_len, int walk_bias, int start_bias, int forward,
               const int* start_nodes, const int64_t* cutoffs, size_t num_walks,
               const double* draws, int pad, int* nodes, int64_t* timestamps,
               size_t* lens, int64_t* edge_ids) {
    TemporalGraphData& d = static_cast<RefGraph*>(h)->data;
    const size_t L = static_cast<size_t>(max_walk_len);
    for (size_t i = 0; i < num_walks * L; ++i) {
        nodes[i] = pad;
        timestamps[i] = EMPTY_TIMESTAMP_VALUE;
    }
    const size_t ecount = num_walks * (L == 0 ? 0 : L - 1);
    for (size_t i = 0; i < ecount; ++i) edge_ids[i] = EMPTY_EDGE_ID;
    for (size_t i = 0; i < num_walks; ++i) lens[i] = 0;
    std::vector<int64_t> cut(num_walks, NO_WALK_CUTOFF);
    if (cutoffs) std::memcpy(cut.data(), cutoffs, num_walks * sizeof(int64_t));

    WalkSetView ws{};
    ws.nodes = nodes;
    ws.timestamps = timestamps;
    ws.walk_lens = lens;
    ws.edge_ids = edge_ids;
    ws.cutoffs = cut.data();
    ws.num_walks = num_walks;
    ws.max_len = L;
    ws.walk_padding_value = pad;

    const TemporalGraphView view = make_temporal_graph_view(d);
    temporal_random_walk::launch_random_walk_cpu_new(
        view, d.is_directed, ws, max_walk_len, start_nodes, num_walks,
        static_cast<RandomPickerType>(walk_bias),
        static_cast<RandomPickerType>(start_bias),
        forward ? WalkDirection::Forward_In_Time : WalkDirection::Backward_In_Time,
        draws);
}

}  // extern "C"
