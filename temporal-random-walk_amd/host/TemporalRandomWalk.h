// TemporalRandomWalk.h -- the reference's public C++ class, rebuilt over the
// engine's C ABI (include/trw_engine.h).
//
// Same class name, constructor arguments, method names, argument meaning and
// error behaviour as the reference's proxy
// (temporal_random_walk/src/proxies/TemporalRandomWalk.cuh:17-112), so C++
// callers and the pybind11 module switch over without changes.  Differences:
//  - `use_gpu`, `kernel_launch_type`, `block_dim` and `w_threshold_warp` are
//    accepted and validated but every call runs the one MI355X engine;
//  - failures surface as std::invalid_argument / std::runtime_error /
//    std::bad_alloc with the engine's message, like the reference's.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <string>
#include <tuple>
#include <vector>

#include "trw_engine.h"

// data/enums.cuh:4-30 of the reference
enum RandomPickerType {
    Uniform,
    Linear,
    ExponentialIndex,
    ExponentialWeight,
    TemporalNode2Vec,
    TEST_FIRST,
    TEST_LAST
};

enum WalkDirection { Forward_In_Time, Backward_In_Time };

enum KernelLaunchType { FULL_WALK, NODE_GROUPED, NODE_GROUPED_GLOBAL_ONLY };

// common/const.cuh of the reference
constexpr double DEFAULT_TIMESCALE_BOUND = -1;
constexpr double DEFAULT_NODE2VEC_P = 1.0;
constexpr double DEFAULT_NODE2VEC_Q = 1.0;
constexpr int EMPTY_NODE_VALUE = -1;
constexpr uint64_t EMPTY_GLOBAL_SEED = UINT64_MAX;
constexpr bool DEFAULT_SHUFFLE_WALK_ORDER = true;
constexpr size_t BLOCK_DIM = 256;
constexpr int W_THRESHOLD_WARP = 32;

RandomPickerType picker_type_from_string(const std::string& s);
WalkDirection walk_direction_from_string(const std::string& s);
KernelLaunchType kernel_launch_type_from_string(const std::string& s);

// A malloc'd host buffer whose ownership is handed to the caller (freed with
// std::free), like the reference's HostRelease (data/buffer.cuh:214-224).
struct HostRelease {
    void* ptr = nullptr;
    size_t size = 0;
};

// Host walk set: nodes/timestamps [num_walks, max_len], walk_lens [num_walks],
// edge_ids [num_walks, max_len - 1] (data/walk_set/walk_set_host.cuh).
class WalkSetHost {
public:
    WalkSetHost() = default;
    explicit WalkSetHost(const trw_walks& w);
    ~WalkSetHost();
    WalkSetHost(const WalkSetHost&) = delete;
    WalkSetHost& operator=(const WalkSetHost&) = delete;
    WalkSetHost(WalkSetHost&& o) noexcept;
    WalkSetHost& operator=(WalkSetHost&& o) noexcept;

    size_t num_walks() const { return num_walks_; }
    size_t max_len() const { return max_len_; }
    const int* nodes_ptr() const { return nodes_; }
    const int64_t* timestamps_ptr() const { return timestamps_; }
    const size_t* walk_lens_ptr() const { return walk_lens_; }
    const int64_t* edge_ids_ptr() const { return edge_ids_; }
    size_t edge_ids_size() const { return num_walks_ * (max_len_ ? max_len_ - 1 : 0); }

    HostRelease release_nodes();
    HostRelease release_timestamps();
    HostRelease release_walk_lens();
    HostRelease release_edge_ids();

private:
    void reset();
    size_t num_walks_ = 0, max_len_ = 0;
    int* nodes_ = nullptr;
    int64_t* timestamps_ = nullptr;
    size_t* walk_lens_ = nullptr;
    int64_t* edge_ids_ = nullptr;
};

// data/walk_set/walks_with_edge_features_host.cuh
struct WalksWithEdgeFeaturesHost {
    WalkSetHost walk_set;
    int feature_dim = 0;
    float* walk_edge_features = nullptr;  // [num_walks, max_len - 1, feature_dim]

    WalksWithEdgeFeaturesHost() = default;
    explicit WalksWithEdgeFeaturesHost(const trw_walks& w);
    ~WalksWithEdgeFeaturesHost() { std::free(walk_edge_features); }
    WalksWithEdgeFeaturesHost(const WalksWithEdgeFeaturesHost&) = delete;
    WalksWithEdgeFeaturesHost& operator=(const WalksWithEdgeFeaturesHost&) = delete;
    WalksWithEdgeFeaturesHost(WalksWithEdgeFeaturesHost&& o) noexcept;

    size_t walk_edge_features_size() const {
        return walk_set.edge_ids_size() * static_cast<size_t>(feature_dim);
    }
    HostRelease release_walk_edge_features();
};

class TemporalRandomWalk {
public:
    explicit TemporalRandomWalk(bool is_directed, bool use_gpu, int64_t max_time_capacity = -1,
                                bool enable_weight_computation = false,
                                bool enable_temporal_node2vec = false,
                                double timescale_bound = DEFAULT_TIMESCALE_BOUND,
                                double node2vec_p = DEFAULT_NODE2VEC_P,
                                double node2vec_q = DEFAULT_NODE2VEC_Q,
                                int walk_padding_value = EMPTY_NODE_VALUE,
                                uint64_t global_seed = EMPTY_GLOBAL_SEED,
                                bool shuffle_walk_order = DEFAULT_SHUFFLE_WALK_ORDER,
                                int cuda_device_id = 0);
    ~TemporalRandomWalk();
    TemporalRandomWalk(const TemporalRandomWalk&) = delete;
    TemporalRandomWalk& operator=(const TemporalRandomWalk&) = delete;

    void* engine_handle() const { return handle_; }

    void add_multiple_edges(const int* sources, const int* targets, const int64_t* timestamps,
                            size_t edges_size, const float* edge_features = nullptr,
                            size_t feature_dim = 0, size_t block_dim = BLOCK_DIM) const;
    void add_multiple_edges(const std::vector<std::tuple<int, int, int64_t>>& edges,
                            const float* edge_features = nullptr, size_t feature_dim = 0,
                            size_t block_dim = BLOCK_DIM) const;
    // The next batch's host -> device copy beside other calls (trw_prefetch_edges);
    // the arrays must stay alive until add_prefetched_edges returns.
    void prefetch_edges(const int* sources, const int* targets, const int64_t* timestamps,
                        size_t edges_size, const float* edge_features = nullptr,
                        size_t feature_dim = 0) const;
    void add_prefetched_edges() const;

    WalksWithEdgeFeaturesHost get_random_walks_and_times_for_all_nodes(
        int max_walk_len, const RandomPickerType* walk_bias, int num_walks_per_node,
        const RandomPickerType* initial_edge_bias = nullptr,
        WalkDirection walk_direction = Forward_In_Time,
        KernelLaunchType kernel_launch_type = NODE_GROUPED, size_t block_dim = BLOCK_DIM,
        int w_threshold_warp = W_THRESHOLD_WARP) const;

    WalksWithEdgeFeaturesHost get_random_walks_and_times_for_last_batch(
        int max_walk_len, const RandomPickerType* walk_bias, int num_walks_per_node,
        const RandomPickerType* initial_edge_bias = nullptr,
        WalkDirection walk_direction = Forward_In_Time,
        KernelLaunchType kernel_launch_type = NODE_GROUPED, size_t block_dim = BLOCK_DIM,
        int w_threshold_warp = W_THRESHOLD_WARP) const;

    WalksWithEdgeFeaturesHost get_random_walks_and_times_for_nodes(
        const int* seed_nodes, size_t num_seed_nodes, const int64_t* cutoff_times,
        int max_walk_len, const RandomPickerType* walk_bias, int num_walks_per_node,
        const RandomPickerType* initial_edge_bias = nullptr,
        WalkDirection walk_direction = Forward_In_Time,
        KernelLaunchType kernel_launch_type = NODE_GROUPED, size_t block_dim = BLOCK_DIM,
        int w_threshold_warp = W_THRESHOLD_WARP) const;

    WalksWithEdgeFeaturesHost get_random_walks_and_times(
        int max_walk_len, const RandomPickerType* walk_bias, int num_walks_total,
        const RandomPickerType* initial_edge_bias = nullptr,
        WalkDirection walk_direction = Forward_In_Time,
        KernelLaunchType kernel_launch_type = NODE_GROUPED, size_t block_dim = BLOCK_DIM,
        int w_threshold_warp = W_THRESHOLD_WARP) const;

    void set_node_features(const int* node_ids, size_t num_nodes, const float* node_features_data,
                           size_t feature_dim) const;

    size_t get_node_count() const;
    size_t get_edge_count() const;
    std::vector<int> get_node_ids() const;
    std::vector<int64_t> get_node_degrees(const int* nodes, size_t n,
                                          WalkDirection direction = Forward_In_Time) const;
    std::vector<std::tuple<int, int, int64_t>> get_edges() const;
    bool get_is_directed() const;
    void clear() const;
    size_t get_memory_used() const;

    int node_feature_dim() const;
    int node_features_max_node_id() const;
    std::vector<float> node_features_dense() const;

private:
    WalksWithEdgeFeaturesHost sample(int mode, int max_walk_len, const RandomPickerType* walk_bias,
                                     int64_t count, const RandomPickerType* initial_edge_bias,
                                     WalkDirection walk_direction, const int* seeds,
                                     size_t num_seeds, const int64_t* cutoffs) const;
    int32_t max_node_id() const;

    void* handle_ = nullptr;
    // host-resident dense node features (graph/node_features.cu of the reference)
    mutable std::vector<float> node_features_;
    mutable size_t node_feature_dim_ = 0;
};
