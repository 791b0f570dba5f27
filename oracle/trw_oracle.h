/*
 * trw_oracle.h -- CPU restatement of the reference's temporal random walk
 * hot path (edge store + index build + replay-mode walk sampler).
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP engine, the C-ABI
 * library, the host C++ class or the Python module) links, loads or calls
 * this code.  It is the parity checker used by tests/, by smoke() and by the
 * CPU-baseline leg of bench.py.
 *
 * Reference: ashfaq1701/temporal-random-walk v1.8.6, CPU ("_std") path.
 * Each function in trw_oracle.c cites the reference file:line it restates.
 * Paths are relative to temporal_random_walk/src/ of the reference.
 *
 * Canonical tie order: the reference CPU path sorts a batch with an unstable
 * std::sort (temporal_graph.cu:89-91) and then stable-merges it after the old
 * store (temporal_graph.cu:93-97).  The only reproducible order is stable by
 * (timestamp, insertion position); this oracle uses that order.
 */
#ifndef TRW_ORACLE_H
#define TRW_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Picker ids follow RandomPickerType (data/enums.cuh:4-15). */
enum {
    ORC_UNIFORM = 0,
    ORC_LINEAR = 1,
    ORC_EXPONENTIAL_INDEX = 2,
    ORC_EXPONENTIAL_WEIGHT = 3,
    ORC_TEMPORAL_NODE2VEC = 4,
    ORC_TEST_FIRST = 5,
    ORC_TEST_LAST = 6
};

typedef struct orc_graph orc_graph;

orc_graph* orc_create(int is_directed, int64_t max_time_capacity,
                      int enable_weight_computation, int enable_temporal_node2vec,
                      double timescale_bound, double node2vec_p, double node2vec_q);
void orc_destroy(orc_graph* g);

/* Returns 0 on success, nonzero on a validation error (message in
 * orc_last_error()).  temporal_graph.cu:158-220 */
/* OpenMP threads of later ingests (1 = serial, the default); the result is
 * the same for every count. */
void orc_set_threads(orc_graph* g, int threads);
int orc_add_edges(orc_graph* g, const int32_t* src, const int32_t* dst,
                  const int64_t* ts, size_t n, const float* features,
                  size_t feature_dim);
const char* orc_last_error(void);

/* Named array snapshot.  *elem_size is 4 (int32/float) or 8 (int64, uint64,
 * double).  Returns NULL with *len = 0 for an empty or unknown array.
 * Names: sources targets timestamps timestamp_group_offsets unique_timestamps
 * active_node_ids node_group_outbound_offsets node_group_inbound_offsets
 * node_ts_sorted_outbound_indices node_ts_sorted_inbound_indices
 * count_ts_group_per_node_outbound count_ts_group_per_node_inbound
 * node_ts_group_outbound_offsets node_ts_group_inbound_offsets
 * forward_cumulative_weights_exponential backward_cumulative_weights_exponential
 * outbound_forward_cumulative_weights_exponential
 * outbound_backward_cumulative_weights_exponential
 * inbound_backward_cumulative_weights_exponential
 * node_adj_offsets node_adj_neighbors edge_features */
const void* orc_array(const orc_graph* g, const char* name, size_t* len,
                      size_t* elem_size);
/* Replace a cumulative-weight array by name (length must match); 0 on
 * success.  Lets a test run the walk loop on another engine's weights. */
int orc_set_weights(orc_graph* g, const char* name, const double* data, size_t len);
int64_t orc_latest_timestamp(const orc_graph* g);
int32_t orc_max_node_id(const orc_graph* g);
size_t orc_feature_dim(const orc_graph* g);

/* Replay-mode walks (core/temporal_random_walk_cpu.cuh:19-197).
 * start_nodes[w] == -1 means an unconstrained start.  cutoffs may be NULL
 * (all NO_WALK_CUTOFF = -1).  draws holds num_walks*(1+2L) uniforms in the
 * reference layout.  Outputs must be pre-sized: nodes/ts [num_walks*L],
 * edge_ids [num_walks*(L-1)], lens [num_walks]; they are fully written
 * (padding included).  num_threads <= 0 uses the OpenMP default. */
void orc_walks(const orc_graph* g, int max_walk_len, int walk_bias,
               int start_bias, int forward, const int32_t* start_nodes,
               const int64_t* cutoffs, size_t num_walks, const double* draws,
               int walk_padding_value, int32_t* nodes, int64_t* timestamps,
               uint64_t* lens, int64_t* edge_ids, int num_threads);

/* Single selector calls with given draws (graph/edge_selectors.cuh:177-443);
 * out = {u, i, ts, edge_id}, all -1 when no edge. */
void orc_node_edge_at(const orc_graph* g, int forward, int picker, int node, int64_t t,
                      int64_t cutoff, int prev, double rg, double re, int64_t* out);
void orc_edge_at(const orc_graph* g, int forward, int picker, double rg, double re,
                 int64_t* out);

/* Pickers (random/pickers.cuh:15-126). */
int orc_pick_linear(int start, int end, int prioritize_end, double r);
int orc_pick_exponential_index(int start, int end, int prioritize_end, double r);
int orc_pick_uniform(int start, int end, double r);
int orc_pick_exponential_weights(const double* weights, size_t weights_size,
                                 size_t group_start, size_t group_end, double r,
                                 size_t slice_start);
double orc_derive_uniform(double a, double b, int counter);

/* ---- the engine's normal-mode draw stream --------------------------------
 * Not a reference function: the reference CPU path draws from std::mt19937
 * seeded by random_device and is not reproducible.  The engine instead derives
 * every draw from Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random
 * numbers: as easy as 1, 2, 3", SC'11) keyed by the 64-bit seed; these
 * restate that derivation so normal-mode walks can be replayed here. */

/* One Philox4x32-10 block: 10 rounds, key bumped by the Weyl constants
 * (0x9E3779B9, 0xBB67AE85) between rounds. */
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* The draws of walks [walk0, walk0 + n) in the replay layout (1 + 2L per
 * walk): counter (pair, walk_lo, walk_hi, 0), key (seed_lo, seed_hi); pair 0
 * gives slot 0 from words (x, y), pair p >= 1 slots 2p-1 from (x, y) and 2p
 * from (z, w); 64 bits (hi:lo) >> 12 = m map to (m + 0.5) * 2^-52. */
void orc_philox_draws(uint64_t seed, uint64_t walk0, uint64_t n, int max_walk_len, double* out);

/* Keys of the walk-order shuffle: word x of counter (i_lo, i_hi, 0x5348, 0);
 * the shuffled order is a stable sort of positions by key. */
void orc_philox_shuffle_keys(uint64_t seed, uint64_t n, uint32_t* out);

#ifdef __cplusplus
}
#endif
#endif
