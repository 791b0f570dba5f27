/*
 * trw_engine.h -- C ABI of the MI355X temporal random walk engine.
 *
 * This is the seam under the reference's public C++ class: every
 * `#ifdef HAS_CUDA / if (use_gpu)` branch of core::TemporalRandomWalk
 * (reference: temporal_random_walk/src/core/temporal_random_walk.cu:920-1104)
 * becomes one call below.  Plain C types only: pointers, sizes, enums and POD
 * structs; no C++ or torch types cross this boundary.
 *
 * Conventions
 *  - Every function returns trw_status; on failure trw_last_error() gives the
 *    message (thread-local).  TRW_ERR_INVALID_ARGUMENT maps to the reference's
 *    std::invalid_argument / ValueError, TRW_ERR_RUNTIME to std::runtime_error.
 *  - One handle = one device + one HIP stream.  Calls are synchronous on
 *    return.  Concurrent calls on one handle are not supported (as in the
 *    reference).  The caller's current device is restored on return.
 *  - Host-pointer entry points copy their inputs before returning.  Output
 *    host buffers are allocated with malloc() and owned by the caller
 *    (release with trw_walks_free or free()), matching the reference's
 *    HostRelease capsules (py_interface/buffer_to_numpy.cuh:13-22).
 */
#ifndef TRW_ENGINE_H
#define TRW_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TRW_ABI_VERSION 7

typedef enum trw_status {
    TRW_OK = 0,
    TRW_ERR_INVALID_ARGUMENT = 1,
    TRW_ERR_RUNTIME = 2,
    TRW_ERR_OUT_OF_MEMORY = 3,
    TRW_ERR_NO_DEVICE = 4
} trw_status;

/* RandomPickerType (reference: src/data/enums.cuh:4-15). */
typedef enum trw_picker {
    TRW_PICKER_UNIFORM = 0,
    TRW_PICKER_LINEAR = 1,
    TRW_PICKER_EXPONENTIAL_INDEX = 2,
    TRW_PICKER_EXPONENTIAL_WEIGHT = 3,
    TRW_PICKER_TEMPORAL_NODE2VEC = 4,
    TRW_PICKER_TEST_FIRST = 5,
    TRW_PICKER_TEST_LAST = 6
} trw_picker;

/* WalkDirection (reference: src/data/enums.cuh:17-20). */
typedef enum trw_direction {
    TRW_FORWARD_IN_TIME = 0,
    TRW_BACKWARD_IN_TIME = 1
} trw_direction;

/* Which of the reference's four samplers builds the start array. */
typedef enum trw_start_mode {
    TRW_START_TOTAL = 0,      /* get_random_walks_and_times: n unconstrained walks */
    TRW_START_ALL_NODES = 1,  /* ..._for_all_nodes: active ids x num_walks_per_node */
    TRW_START_LAST_BATCH = 2, /* ..._for_last_batch: last batch's unique endpoints */
    TRW_START_NODES = 3       /* ..._for_nodes: given seeds (+ optional cutoffs) */
} trw_start_mode;

/* Constructor arguments of the reference's TemporalRandomWalk
 * (src/proxies/TemporalRandomWalk.cuh:21-36). */
typedef struct trw_config {
    int32_t is_directed;
    int32_t enable_weight_computation;
    int32_t enable_temporal_node2vec;
    int32_t walk_padding_value;
    int64_t max_time_capacity; /* <= 0: no window */
    double timescale_bound;    /* <= 0: unscaled */
    double node2vec_p;
    double node2vec_q;
    uint64_t global_seed;      /* UINT64_MAX: fresh seed per call */
    int32_t shuffle_walk_order;
    int32_t device_id;
} trw_config;

typedef struct trw_sample_params {
    int32_t mode;               /* trw_start_mode */
    int32_t max_walk_len;
    int32_t walk_bias;          /* trw_picker */
    int32_t initial_edge_bias;  /* trw_picker, or -1 = same as walk_bias */
    int32_t direction;          /* trw_direction */
    int32_t num_walks_per_node; /* ALL_NODES, LAST_BATCH, NODES */
    int64_t num_walks_total;    /* TOTAL */
    const int32_t* seed_nodes;  /* NODES: host array of num_seed_nodes ids */
    const int64_t* cutoff_times;/* NODES: host array or NULL (exclusive upper bounds) */
    uint64_t num_seed_nodes;
    /* Replay mode: host array of num_walks * (1 + 2 * max_walk_len) uniforms
     * in the reference CPU layout (slot 0/1 start group/edge, slot 2
     * undirected start endpoint, slots 2k+1/2k+2 hop k).  NULL = in-kernel
     * Philox4x32-10 keyed by the seed. */
    const double* replay_draws;
    uint64_t replay_draws_len;
    int32_t shuffle;            /* -1 = the handle's shuffle_walk_order, 0/1 = override */
    /* Order the walks run in on the device; the output is the same in every
     * order (each walk depends only on the graph and its own draws).
     * 0 = automatic (TRW_ORDER_START_TIME from 2^16 walks on), 1 = walk id
     * order, 2 = sorted by the time of the start edge, so that walks running
     * side by side read the same parts of the index, 3 = node-grouped: every
     * 8 hops the live walks are regrouped by their current node on the device
     * (measured slower than 2; kept for comparison). */
    int32_t walk_order;
    /* How walks become the row-major output arrays (the output is the same
     * either way).  0 = automatic: forward walks of the index pickers or
     * TemporalNode2Vec whose node id, timestamp rank and edge id pack into
     * 64 bits are written as rows by the walk kernel itself, which buffers
     * each wave's next 16 slots in LDS; other samples go through walk scratch
     * and a layout pass.  1 = always scratch and the layout pass. */
    int32_t walk_layout;
} trw_sample_params;

typedef enum trw_walk_layout {
    TRW_LAYOUT_AUTO = 0,
    TRW_LAYOUT_SCRATCH = 1
} trw_walk_layout;

typedef enum trw_walk_order {
    TRW_ORDER_AUTO = 0,
    TRW_ORDER_WALK_ID = 1,
    TRW_ORDER_START_TIME = 2,
    TRW_ORDER_NODE_GROUPED = 3
} trw_walk_order;

/* Walk output.  nodes/timestamps: [num_walks, max_walk_len]; edge_ids:
 * [num_walks, max_walk_len - 1]; walk_lens: [num_walks]; edge_features:
 * [num_walks, max_walk_len - 1, feature_dim] or NULL when feature_dim == 0.
 * Host results: malloc'd, caller-owned.  Device results (trw_sample_device):
 * device pointers owned by the handle, valid until its next sample call. */
typedef struct trw_walks {
    uint64_t num_walks;
    int32_t max_walk_len;
    int32_t feature_dim;
    int32_t* nodes;
    int64_t* timestamps;
    uint64_t* walk_lens;
    int64_t* edge_ids;
    float* edge_features;
} trw_walks;

/* Device-side timings of the last call, in milliseconds (HIP events on the
 * handle's stream). */
typedef struct trw_timings {
    double build_ms;       /* whole device-side ingest of the last add_edges */
    double sort_ms;        /* timestamp sort + gather inside it */
    double index_ms;       /* node index (sort, groups, offsets) inside it */
    double sample_ms;      /* whole device-side sample of the last sample call */
    double walk_kernel_ms; /* the walk kernel(s) inside it */
    uint64_t walk_kernel_launches;
    double handoff_ms;     /* host wall time of trw_sample's copy into host
                              arrays (allocation, PCIe and host copy) */
    uint64_t handoff_bytes; /* bytes that copy delivered */
} trw_timings;

/* Array ids for trw_get_array.  Values are widened to the reference's
 * element types: size_t arrays come back as uint64, int arrays as int32,
 * timestamps as int64, weights as double, features as float.  The layout and
 * sizes are those of TemporalGraphData (src/data/temporal_graph_data.cuh). */
typedef enum trw_array_id {
    TRW_ARR_SOURCES = 0,
    TRW_ARR_TARGETS = 1,
    TRW_ARR_TIMESTAMPS = 2,
    TRW_ARR_TIMESTAMP_GROUP_OFFSETS = 3,
    TRW_ARR_UNIQUE_TIMESTAMPS = 4,
    TRW_ARR_ACTIVE_NODE_IDS = 5,
    TRW_ARR_NODE_GROUP_OUTBOUND_OFFSETS = 6,
    TRW_ARR_NODE_GROUP_INBOUND_OFFSETS = 7,
    TRW_ARR_NODE_TS_SORTED_OUTBOUND_INDICES = 8,
    TRW_ARR_NODE_TS_SORTED_INBOUND_INDICES = 9,
    TRW_ARR_COUNT_TS_GROUP_PER_NODE_OUTBOUND = 10,
    TRW_ARR_COUNT_TS_GROUP_PER_NODE_INBOUND = 11,
    TRW_ARR_NODE_TS_GROUP_OUTBOUND_OFFSETS = 12,
    TRW_ARR_NODE_TS_GROUP_INBOUND_OFFSETS = 13,
    TRW_ARR_FORWARD_CUMULATIVE_WEIGHTS = 14,
    TRW_ARR_BACKWARD_CUMULATIVE_WEIGHTS = 15,
    TRW_ARR_OUTBOUND_FORWARD_CUMULATIVE_WEIGHTS = 16,
    TRW_ARR_OUTBOUND_BACKWARD_CUMULATIVE_WEIGHTS = 17,
    TRW_ARR_INBOUND_BACKWARD_CUMULATIVE_WEIGHTS = 18,
    TRW_ARR_NODE_ADJ_OFFSETS = 19,
    TRW_ARR_NODE_ADJ_NEIGHBORS = 20,
    TRW_ARR_EDGE_FEATURES = 21,
    TRW_ARR_COUNT = 22
} trw_array_id;

/* ---- lifecycle -------------------------------------------------------- */

/* Replaces the constructor: core/temporal_random_walk.cu:38-82. */
trw_status trw_create(const trw_config* config, void** out_handle);
/* Replaces the destructor: core/temporal_random_walk.cu:84-102. */
trw_status trw_destroy(void* handle);
/* Message of the last failed call on this thread. */
const char* trw_last_error(void);
int32_t trw_abi_version(void);

/* ---- ingest ------------------------------------------------------------ */

/* Replaces temporal_random_walk::add_multiple_edges
 * (core/temporal_random_walk.cu:276-329): append, stable sort by
 * (timestamp, insertion position), window eviction, full index rebuild,
 * optional weights, last-batch uniques.  A failure after the batch passed its
 * checks (device out of memory, a HIP error) leaves the handle empty, as after
 * trw_clear.  Host pointers; features are
 * [n, feature_dim] row-major or NULL.  Validation messages follow
 * graph/edge_data.cu:71-89.  A batch holding a negative node id is rejected
 * with TRW_ERR_INVALID_ARGUMENT before the store changes (the reference
 * indexes its dense node arrays by id and has no such check). */
trw_status trw_add_edges(void* handle, const int32_t* sources, const int32_t* targets,
                         const int64_t* timestamps, uint64_t n, const float* edge_features,
                         uint64_t feature_dim);
/* Same, with the batch already resident in device memory (HBM). */
trw_status trw_add_edges_device(void* handle, const int32_t* d_sources,
                                const int32_t* d_targets, const int64_t* d_timestamps,
                                uint64_t n, const float* d_edge_features,
                                uint64_t feature_dim);

/* Ingestion front-end: the host -> device copy of the next batch overlapped
 * with other calls.  trw_prefetch_edges starts copying a host batch into
 * engine-owned device buffers on a thread and lanes of its own, and returns;
 * the caller may then sample (or make any other call) while it copies, and
 * must keep the arrays alive and unchanged until trw_add_prefetched_edges
 * returns.  trw_add_prefetched_edges waits for the copy and ingests the batch
 * exactly as trw_add_edges would have at that point (same validation, same
 * store and index).  One batch may be pending at a time; trw_destroy waits
 * for a pending copy.  The reference has no such call: its ingest copies each
 * batch array with one blocking cudaMemcpy inside add_multiple_edges
 * (data/buffer.cuh:135-149, core/temporal_random_walk.cu:276-329). */
trw_status trw_prefetch_edges(void* handle, const int32_t* sources, const int32_t* targets,
                              const int64_t* timestamps, uint64_t n, const float* edge_features,
                              uint64_t feature_dim);
trw_status trw_add_prefetched_edges(void* handle);

/* ---- sampling ------------------------------------------------------------ */

/* Replaces the four get_random_walks_and_times*_cuda samplers
 * (core/temporal_random_walk.cu:657-916) and finalize_host_walks (:381-390):
 * outputs are copied to malloc'd host buffers owned by the caller. */
trw_status trw_sample(void* handle, const trw_sample_params* params, trw_walks* out);
/* Same, leaving the walks in device memory owned by the handle. */
trw_status trw_sample_device(void* handle, const trw_sample_params* params, trw_walks* out);
/* Same as trw_sample_device, into caller-owned device buffers, allocating
 * nothing: no hipMalloc, hipFree or allocating library call.  No counterpart
 * in the reference; it is for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation).
 *
 * On entry out->nodes, ->timestamps, ->walk_lens, ->edge_ids and, when the
 * store has edge features, ->edge_features point to 16-byte aligned device
 * buffers with room for capacity_walks walks (rows of max_walk_len,
 * max_walk_len - 1 and (max_walk_len - 1) * feature_dim values); on return
 * num_walks, max_walk_len and feature_dim are set.  Every per-call buffer
 * (start keys and states, draws, processing order, walk scratch) comes from a
 * fixed device array of 128 MiB per device, held until the process ends: a
 * sample needing more (about 40 B per walk, plus 8 B per slot of walk scratch
 * -- 640 B per walk at max_walk_len 80 -- where a layout pass writes the
 * rows), more walks than capacity_walks, or misaligned buffers, is rejected
 * with TRW_ERR_INVALID_ARGUMENT.  Calls on one
 * device share that array: calls of any handles on one device run one at a
 * time (a per-device lock held for the whole call; a call returns with its
 * walks written), and the array keeps the last call's contents.
 * trw_get_walk_stats does not describe these walks. */
trw_status trw_sample_device_noalloc(void* handle, const trw_sample_params* params,
                                     uint64_t capacity_walks, trw_walks* out);
/* free() of the host buffers of a trw_walks returned by trw_sample. */
void trw_walks_free(trw_walks* walks);

/* ---- queries (core/temporal_random_walk.cu:331-377) ------------------------ */

trw_status trw_get_node_count(void* handle, uint64_t* out);
trw_status trw_get_edge_count(void* handle, uint64_t* out);
/* Active node ids ascending (graph/edge_data.cu:144-208).  If out is NULL only
 * *len is set. */
trw_status trw_get_node_ids(void* handle, int32_t* out, uint64_t cap, uint64_t* len);
/* Degrees of the given nodes (graph/node_edge_index.cu:89-145). */
trw_status trw_get_node_degrees(void* handle, const int32_t* nodes, uint64_t n,
                                int32_t direction, int64_t* out);
/* Edge store as three arrays (graph/edge_data.cu:101-142); NULL outputs query
 * the length only. */
trw_status trw_get_edges(void* handle, int32_t* sources, int32_t* targets, int64_t* timestamps,
                         uint64_t cap, uint64_t* len);
trw_status trw_get_is_directed(void* handle, int32_t* out);
trw_status trw_get_memory_used(void* handle, uint64_t* out);
trw_status trw_get_feature_dim(void* handle, uint64_t* out);
trw_status trw_get_latest_timestamp(void* handle, int64_t* out);
/* Replaces temporal_random_walk::clear (core/temporal_random_walk.cu:358-373). */
trw_status trw_clear(void* handle);

/* Snapshot of one index array, widened to the reference's element type
 * (size in bytes: 8 except int32/float arrays: 4).  dst NULL = query *len. */
trw_status trw_get_array(void* handle, int32_t array_id, void* dst, uint64_t cap_elems,
                         uint64_t* len, uint32_t* elem_size);

/* ---- measurement ----------------------------------------------------------- */

trw_status trw_get_timings(void* handle, trw_timings* out);
/* The handle's HIP stream (a hipStream_t), for callers that time or order
 * work against it. */
trw_status trw_get_stream(void* handle, void** out_stream);
/* Statistics of the last sample, computed on the device after the fact (not
 * part of any timing).  Both byte counts are compulsory traffic of the walk
 * path, summed over the walks of the last sample; G_u is the number of
 * timestamp groups of the node u a hop is selected at, in the sampled
 * direction, and p_u = ceil(log2(G_u + 1)) the probes of a binary search over
 * them.
 *
 * reference_bytes uses the reference's element types (size_t offsets and
 * indices, int64 timestamps): per hop 72 + 8 p_u B (the node's group range
 * 16, one 8 B timestamp per probe, the picked group's edge range 16, the
 * sorted edge index 8, next node + timestamp 12, the hop's output node 4 +
 * timestamp 8 + edge id 8); per walk 8 B for the length, the start (32 B
 * unconstrained: timestamp-group range 16, edge endpoints and time 16; 52 B
 * from a given node: group range 16, edge range 16, edge index 8, next node
 * and time 12) and the output of slot 0 (12 B) and slot 1 (20 B) when
 * written.
 *
 * algorithmic_bytes is the same sum restated for this engine's 4-byte
 * positions and timestamp ranks: per walk 24 B (start-edge reads + length);
 * 8 B for slot 0 and 12 B for slot 1 when written (node, timestamp rank,
 * 32-bit edge id); per hop 36 + 4 p_u B (the node's group range 8 B, one 4 B
 * rank per probe, the picked group's range 8 B, the edge record 8 B and that
 * hop's 12 B of output).  Padding and the int64 widening are the layout
 * pass's, not the walk kernel's.  Both are demand bytes: every walk's reads
 * count, also where walks running side by side read the same lines.
 *
 * compulsory_read_bytes / compulsory_write_bytes are the bytes one launch of
 * the walk kernel must move at least once between HBM and the chip: every
 * input read once -- per walk its 16 B start state, 4 B of processing order
 * when the walks ran sorted by start time, 8 B of cutoff; the sampled
 * direction's index arrays the launched kernel reads (node headers, bucket
 * tables, panel, edge records; per-node weights and their search index for
 * weight pickers; the adjacency pair set for TemporalNode2Vec), each counted
 * whole; injected draws at 16 B per selection -- and every output written
 * once: the walk scratch (8 B per written slot packed, else 4 B node + 4 B
 * rank per slot and 4 B per edge id) and 8 B of length per walk. */
typedef struct trw_walk_stats {
    uint64_t total_len;         /* sum of walk_lens: walk steps (reference metric) */
    uint64_t transitions;       /* sum of max(len - 1, 0) */
    uint64_t nonempty_walks;
    uint64_t algorithmic_bytes;
    uint64_t reference_bytes;
    uint64_t compulsory_read_bytes;
    uint64_t compulsory_write_bytes;
    uint64_t rows_by_walk_kernel; /* 1: the walk kernel wrote the output rows
                                   * (no scratch, no layout pass); 0: scratch
                                   * and the layout pass */
    uint64_t slot_word_format;    /* what a walk slot's 64-bit word held: 0 node,
                                   * timestamp rank and edge id; 1 node and edge
                                   * id (the three do not fit in 64 bits) */
} trw_walk_stats;
trw_status trw_get_walk_stats(void* handle, trw_walk_stats* out);

/* ---- test hooks ---------------------------------------------------------- */

/* After this call, the next n device allocations of any handle succeed and the
 * one after them fails as out of memory (TRW_ERR_OUT_OF_MEMORY), its retry
 * included; n < 0 disarms.  For tests of the failure paths: an ingest that
 * fails after its batch was accepted leaves the handle empty, as after
 * trw_clear.  No counterpart in the reference. */
void trw_debug_fail_allocation(int64_t n);
/* The same, but only the allocation's first attempt fails: an allocation that
 * runs out of memory while blocks of grown buffers are held (they are kept
 * until trw_clear, a failed ingest or destruction, and counted by
 * trw_get_memory_used) releases them and tries once more, which then
 * succeeds; with none held it fails.  No counterpart in the reference. */
void trw_debug_fail_allocation_transient(int64_t n);

/* ---- standalone pickers (proxies/RandomPicker.cu:11-313) --------------------- */

/* n picks of an index picker (Uniform, Linear, ExponentialIndex, or the test
 * pickers) over [start[i], end[i]), -1 for an empty range, each with one
 * uniform draw: draws[i] (host, in [0, 1); pick_random_with_provided_number),
 * or, with draws NULL, Philox4x32-10 keyed by seed (pick_random).  Host
 * arrays; one launch on device_id (-1: the current device).  Replaces
 * {Linear,ExponentialIndex,Uniform}RandomPicker (proxies/RandomPicker.cu:
 * 11-215), which launch one single-thread kernel per pick. */
trw_status trw_pick_index(int32_t device_id, int32_t picker, const int32_t* start,
                          const int32_t* end, uint64_t n, int32_t prioritize_end,
                          const double* draws, uint64_t seed, int32_t* out);
/* n picks of WeightBasedRandomPicker (proxies/RandomPicker.cu:218-313) over one
 * cumulative-weight array of `size` values: the lower_bound of
 * start_sum + r * (end_sum - start_sum) in [group_start[i], group_end[i])
 * (random/pickers.cuh:84-126), -1 for an invalid range.  Draws as above. */
trw_status trw_pick_weights(int32_t device_id, const double* cumulative, uint64_t size,
                            const uint64_t* group_start, const uint64_t* group_end, uint64_t n,
                            const double* draws, uint64_t seed, int32_t* out);

#ifdef __cplusplus
}
#endif
#endif /* TRW_ENGINE_H */
