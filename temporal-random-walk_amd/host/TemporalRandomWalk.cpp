// TemporalRandomWalk.cpp -- host class over the engine's C ABI.
#include "TemporalRandomWalk.h"

#include <cstring>
#include <new>
#include <stdexcept>
#include <utility>

namespace {

void check(trw_status st) {
    if (st == TRW_OK) return;
    const std::string msg = trw_last_error();
    switch (st) {
        case TRW_ERR_INVALID_ARGUMENT: throw std::invalid_argument(msg);
        case TRW_ERR_OUT_OF_MEMORY: throw std::bad_alloc();
        default: throw std::runtime_error(msg);
    }
}

int picker_id(const RandomPickerType* p) { return p ? static_cast<int>(*p) : -1; }

}  // namespace

// core/helpers.cuh:20-84 of the reference
RandomPickerType picker_type_from_string(const std::string& s) {
    if (s == "Uniform") return Uniform;
    if (s == "Linear") return Linear;
    if (s == "ExponentialIndex") return ExponentialIndex;
    if (s == "ExponentialWeight") return ExponentialWeight;
    if (s == "TemporalNode2Vec") return TemporalNode2Vec;
    throw std::invalid_argument("Invalid picker type: " + s);
}

WalkDirection walk_direction_from_string(const std::string& s) {
    if (s == "Forward_In_Time") return Forward_In_Time;
    if (s == "Backward_In_Time") return Backward_In_Time;
    throw std::invalid_argument("Invalid walk direction: " + s);
}

KernelLaunchType kernel_launch_type_from_string(const std::string& s) {
    if (s == "NODE_GROUPED") return NODE_GROUPED;
    if (s == "NODE_GROUPED_GLOBAL_ONLY") return NODE_GROUPED_GLOBAL_ONLY;
    if (s == "FULL_WALK") return FULL_WALK;
    throw std::invalid_argument("Invalid kernel_launch_type: " + s +
                                ". Expected \"NODE_GROUPED\", \"NODE_GROUPED_GLOBAL_ONLY\", or "
                                "\"FULL_WALK\".");
}

// ---- WalkSetHost ---------------------------------------------------------------

WalkSetHost::WalkSetHost(const trw_walks& w)
    : num_walks_(w.num_walks),
      max_len_(static_cast<size_t>(w.max_walk_len)),
      nodes_(w.nodes),
      timestamps_(w.timestamps),
      walk_lens_(reinterpret_cast<size_t*>(w.walk_lens)),
      edge_ids_(w.edge_ids) {}

WalkSetHost::~WalkSetHost() { reset(); }

void WalkSetHost::reset() {
    std::free(nodes_);
    std::free(timestamps_);
    std::free(walk_lens_);
    std::free(edge_ids_);
    nodes_ = nullptr;
    timestamps_ = nullptr;
    walk_lens_ = nullptr;
    edge_ids_ = nullptr;
}

WalkSetHost::WalkSetHost(WalkSetHost&& o) noexcept { *this = std::move(o); }

WalkSetHost& WalkSetHost::operator=(WalkSetHost&& o) noexcept {
    if (this != &o) {
        reset();
        num_walks_ = o.num_walks_;
        max_len_ = o.max_len_;
        nodes_ = std::exchange(o.nodes_, nullptr);
        timestamps_ = std::exchange(o.timestamps_, nullptr);
        walk_lens_ = std::exchange(o.walk_lens_, nullptr);
        edge_ids_ = std::exchange(o.edge_ids_, nullptr);
    }
    return *this;
}

HostRelease WalkSetHost::release_nodes() {
    return HostRelease{std::exchange(nodes_, nullptr), num_walks_ * max_len_};
}
HostRelease WalkSetHost::release_timestamps() {
    return HostRelease{std::exchange(timestamps_, nullptr), num_walks_ * max_len_};
}
HostRelease WalkSetHost::release_walk_lens() {
    return HostRelease{std::exchange(walk_lens_, nullptr), num_walks_};
}
HostRelease WalkSetHost::release_edge_ids() {
    return HostRelease{std::exchange(edge_ids_, nullptr), edge_ids_size()};
}

WalksWithEdgeFeaturesHost::WalksWithEdgeFeaturesHost(const trw_walks& w)
    : walk_set(w), feature_dim(w.feature_dim), walk_edge_features(w.edge_features) {}

WalksWithEdgeFeaturesHost::WalksWithEdgeFeaturesHost(WalksWithEdgeFeaturesHost&& o) noexcept
    : walk_set(std::move(o.walk_set)),
      feature_dim(o.feature_dim),
      walk_edge_features(std::exchange(o.walk_edge_features, nullptr)) {}

HostRelease WalksWithEdgeFeaturesHost::release_walk_edge_features() {
    const size_t n = walk_edge_features_size();
    return HostRelease{std::exchange(walk_edge_features, nullptr), n};
}

// ---- TemporalRandomWalk ---------------------------------------------------------

TemporalRandomWalk::TemporalRandomWalk(bool is_directed, bool /*use_gpu: one backend*/,
                                       int64_t max_time_capacity, bool enable_weight_computation,
                                       bool enable_temporal_node2vec, double timescale_bound,
                                       double node2vec_p, double node2vec_q,
                                       int walk_padding_value, uint64_t global_seed,
                                       bool shuffle_walk_order, int cuda_device_id) {
    trw_config c{};
    c.is_directed = is_directed;
    c.enable_weight_computation = enable_weight_computation;
    c.enable_temporal_node2vec = enable_temporal_node2vec;
    c.walk_padding_value = walk_padding_value;
    c.max_time_capacity = max_time_capacity;
    c.timescale_bound = timescale_bound;
    c.node2vec_p = node2vec_p;
    c.node2vec_q = node2vec_q;
    c.global_seed = global_seed;
    c.shuffle_walk_order = shuffle_walk_order;
    c.device_id = cuda_device_id;
    check(trw_create(&c, &handle_));
}

TemporalRandomWalk::~TemporalRandomWalk() {
    if (handle_) trw_destroy(handle_);
}

void TemporalRandomWalk::add_multiple_edges(const int* sources, const int* targets,
                                            const int64_t* timestamps, size_t edges_size,
                                            const float* edge_features, size_t feature_dim,
                                            size_t /*block_dim*/) const {
    check(trw_add_edges(handle_, sources, targets, timestamps, edges_size, edge_features,
                        feature_dim));
}

void TemporalRandomWalk::prefetch_edges(const int* sources, const int* targets,
                                        const int64_t* timestamps, size_t edges_size,
                                        const float* edge_features, size_t feature_dim) const {
    check(trw_prefetch_edges(handle_, sources, targets, timestamps, edges_size, edge_features,
                             feature_dim));
}

void TemporalRandomWalk::add_prefetched_edges() const { check(trw_add_prefetched_edges(handle_)); }

void TemporalRandomWalk::add_multiple_edges(
    const std::vector<std::tuple<int, int, int64_t>>& edges, const float* edge_features,
    size_t feature_dim, size_t block_dim) const {
    std::vector<int> s(edges.size()), d(edges.size());
    std::vector<int64_t> t(edges.size());
    for (size_t i = 0; i < edges.size(); ++i) {
        s[i] = std::get<0>(edges[i]);
        d[i] = std::get<1>(edges[i]);
        t[i] = std::get<2>(edges[i]);
    }
    add_multiple_edges(s.data(), d.data(), t.data(), edges.size(), edge_features, feature_dim,
                       block_dim);
}

WalksWithEdgeFeaturesHost TemporalRandomWalk::sample(
    int mode, int max_walk_len, const RandomPickerType* walk_bias, int64_t count,
    const RandomPickerType* initial_edge_bias, WalkDirection walk_direction, const int* seeds,
    size_t num_seeds, const int64_t* cutoffs) const {
    if (!walk_bias) throw std::invalid_argument("walk_bias must not be null");
    trw_sample_params p{};
    p.mode = mode;
    p.max_walk_len = max_walk_len;
    p.walk_bias = picker_id(walk_bias);
    p.initial_edge_bias = picker_id(initial_edge_bias);
    p.direction = walk_direction == Backward_In_Time ? TRW_BACKWARD_IN_TIME : TRW_FORWARD_IN_TIME;
    if (mode == TRW_START_TOTAL) p.num_walks_total = count;
    else p.num_walks_per_node = static_cast<int32_t>(count);
    p.seed_nodes = seeds;
    p.cutoff_times = cutoffs;
    p.num_seed_nodes = num_seeds;
    p.shuffle = -1;
    trw_walks w{};
    check(trw_sample(handle_, &p, &w));
    return WalksWithEdgeFeaturesHost(w);
}

WalksWithEdgeFeaturesHost TemporalRandomWalk::get_random_walks_and_times_for_all_nodes(
    int max_walk_len, const RandomPickerType* walk_bias, int num_walks_per_node,
    const RandomPickerType* initial_edge_bias, WalkDirection walk_direction, KernelLaunchType,
    size_t, int) const {
    return sample(TRW_START_ALL_NODES, max_walk_len, walk_bias, num_walks_per_node,
                  initial_edge_bias, walk_direction, nullptr, 0, nullptr);
}

WalksWithEdgeFeaturesHost TemporalRandomWalk::get_random_walks_and_times_for_last_batch(
    int max_walk_len, const RandomPickerType* walk_bias, int num_walks_per_node,
    const RandomPickerType* initial_edge_bias, WalkDirection walk_direction, KernelLaunchType,
    size_t, int) const {
    return sample(TRW_START_LAST_BATCH, max_walk_len, walk_bias, num_walks_per_node,
                  initial_edge_bias, walk_direction, nullptr, 0, nullptr);
}

WalksWithEdgeFeaturesHost TemporalRandomWalk::get_random_walks_and_times_for_nodes(
    const int* seed_nodes, size_t num_seed_nodes, const int64_t* cutoff_times, int max_walk_len,
    const RandomPickerType* walk_bias, int num_walks_per_node,
    const RandomPickerType* initial_edge_bias, WalkDirection walk_direction, KernelLaunchType,
    size_t, int) const {
    return sample(TRW_START_NODES, max_walk_len, walk_bias, num_walks_per_node,
                  initial_edge_bias, walk_direction, seed_nodes, num_seed_nodes, cutoff_times);
}

WalksWithEdgeFeaturesHost TemporalRandomWalk::get_random_walks_and_times(
    int max_walk_len, const RandomPickerType* walk_bias, int num_walks_total,
    const RandomPickerType* initial_edge_bias, WalkDirection walk_direction, KernelLaunchType,
    size_t, int) const {
    return sample(TRW_START_TOTAL, max_walk_len, walk_bias, num_walks_total, initial_edge_bias,
                  walk_direction, nullptr, 0, nullptr);
}

int32_t TemporalRandomWalk::max_node_id() const {
    uint64_t n = 0;
    check(trw_get_array(handle_, TRW_ARR_ACTIVE_NODE_IDS, nullptr, 0, &n, nullptr));
    return static_cast<int32_t>(n) - 1;
}

// graph/node_features.cu:30-66 of the reference; ids outside [0, max_node_id]
// are rejected (the reference writes past its buffer for them).
void TemporalRandomWalk::set_node_features(const int* node_ids, size_t num_nodes,
                                           const float* node_features_data,
                                           size_t feature_dim) const {
    if (num_nodes == 0) {
        node_feature_dim_ = feature_dim;
        return;
    }
    if (feature_dim == 0)
        throw std::runtime_error("feature_dim must be greater than 0 when setting node features");
    if (node_feature_dim_ != 0 && node_feature_dim_ != feature_dim)
        throw std::runtime_error(
            "feature_dim mismatch with existing TemporalGraphData node features");
    const int32_t mx = max_node_id();
    for (size_t i = 0; i < num_nodes; ++i) {
        if (node_ids[i] < 0 || node_ids[i] > mx)
            throw std::runtime_error("node id outside [0, max_node_id] in set_node_features");
    }
    node_feature_dim_ = feature_dim;
    const size_t need = static_cast<size_t>(mx + 1) * feature_dim;
    if (node_features_.size() < need) node_features_.resize(need, 0.0f);
    for (size_t i = 0; i < num_nodes; ++i) {
        std::memcpy(node_features_.data() + static_cast<size_t>(node_ids[i]) * feature_dim,
                    node_features_data + i * feature_dim, feature_dim * sizeof(float));
    }
}

size_t TemporalRandomWalk::get_node_count() const {
    uint64_t v = 0;
    check(trw_get_node_count(handle_, &v));
    return v;
}

size_t TemporalRandomWalk::get_edge_count() const {
    uint64_t v = 0;
    check(trw_get_edge_count(handle_, &v));
    return v;
}

std::vector<int> TemporalRandomWalk::get_node_ids() const {
    uint64_t n = 0;
    check(trw_get_node_ids(handle_, nullptr, 0, &n));
    std::vector<int> out(n);
    if (n) check(trw_get_node_ids(handle_, out.data(), n, &n));
    return out;
}

std::vector<int64_t> TemporalRandomWalk::get_node_degrees(const int* nodes, size_t n,
                                                          WalkDirection direction) const {
    std::vector<int64_t> out(n);
    if (n) {
        check(trw_get_node_degrees(handle_, nodes, n,
                                   direction == Backward_In_Time ? TRW_BACKWARD_IN_TIME
                                                                 : TRW_FORWARD_IN_TIME,
                                   out.data()));
    }
    return out;
}

std::vector<std::tuple<int, int, int64_t>> TemporalRandomWalk::get_edges() const {
    uint64_t n = 0;
    check(trw_get_edges(handle_, nullptr, nullptr, nullptr, 0, &n));
    std::vector<int> s(n), d(n);
    std::vector<int64_t> t(n);
    if (n) check(trw_get_edges(handle_, s.data(), d.data(), t.data(), n, &n));
    std::vector<std::tuple<int, int, int64_t>> out(n);
    for (size_t i = 0; i < n; ++i) out[i] = std::make_tuple(s[i], d[i], t[i]);
    return out;
}

bool TemporalRandomWalk::get_is_directed() const {
    int32_t v = 0;
    check(trw_get_is_directed(handle_, &v));
    return v != 0;
}

void TemporalRandomWalk::clear() const {
    check(trw_clear(handle_));
    node_features_.clear();
    node_feature_dim_ = 0;
}

size_t TemporalRandomWalk::get_memory_used() const {
    uint64_t v = 0;
    check(trw_get_memory_used(handle_, &v));
    return v + node_features_.size() * sizeof(float);
}

int TemporalRandomWalk::node_feature_dim() const { return static_cast<int>(node_feature_dim_); }

int TemporalRandomWalk::node_features_max_node_id() const { return max_node_id(); }

std::vector<float> TemporalRandomWalk::node_features_dense() const {
    const int32_t mx = max_node_id();
    std::vector<float> out(mx >= 0 ? static_cast<size_t>(mx + 1) * node_feature_dim_ : 0, 0.0f);
    std::memcpy(out.data(), node_features_.data(),
                std::min(out.size(), node_features_.size()) * sizeof(float));
    return out;
}
