// py_module.cpp -- pybind11 module `_temporal_random_walk`, the reference's
// Python surface (py_interface/_temporal_random_walk.cu:43-902) over the C++
// TemporalRandomWalk class of this engine.  Same class, method and keyword
// names, same defaults, same array shapes and dtypes, same error types.
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <algorithm>
#include <cstdlib>
#include <optional>
#include <stdexcept>

#include "RandomPicker.h"
#include "TemporalRandomWalk.h"

namespace py = pybind11;

namespace {

// numpy array owning a malloc'd buffer (py_interface/buffer_to_numpy.cuh:13-22)
py::capsule make_capsule(const HostRelease& r) {
    return py::capsule(r.ptr, [](void* p) { std::free(p); });
}

const RandomPickerType* optional_picker(const std::optional<std::string>& s,
                                        std::optional<RandomPickerType>& storage) {
    if (!s.has_value()) return nullptr;
    storage = picker_type_from_string(*s);
    return &(*storage);
}

py::tuple walks_to_numpy(WalksWithEdgeFeaturesHost& walks, int max_walk_len) {
    const auto num_walks = static_cast<py::ssize_t>(walks.walk_set.num_walks());
    const auto L = static_cast<py::ssize_t>(max_walk_len);

    auto rn = walks.walk_set.release_nodes();
    py::array_t<int> nodes({num_walks, L}, {static_cast<py::ssize_t>(sizeof(int)) * L,
                                            static_cast<py::ssize_t>(sizeof(int))},
                           static_cast<int*>(rn.ptr), make_capsule(rn));
    auto rt = walks.walk_set.release_timestamps();
    py::array_t<int64_t> ts({num_walks, L}, {static_cast<py::ssize_t>(sizeof(int64_t)) * L,
                                             static_cast<py::ssize_t>(sizeof(int64_t))},
                            static_cast<int64_t*>(rt.ptr), make_capsule(rt));
    auto rl = walks.walk_set.release_walk_lens();
    py::array_t<size_t> lens({num_walks}, {static_cast<py::ssize_t>(sizeof(size_t))},
                             static_cast<size_t*>(rl.ptr), make_capsule(rl));
    py::object feats = py::none();
    if (walks.feature_dim > 0 && walks.walk_edge_features_size() > 0) {
        const auto epw = static_cast<py::ssize_t>(std::max(0, max_walk_len - 1));
        const auto fd = static_cast<py::ssize_t>(walks.feature_dim);
        auto re = walks.release_walk_edge_features();
        feats = py::array_t<float>(
            {num_walks, epw, fd},
            {static_cast<py::ssize_t>(sizeof(float)) * epw * fd,
             static_cast<py::ssize_t>(sizeof(float)) * fd, static_cast<py::ssize_t>(sizeof(float))},
            static_cast<float*>(re.ptr), make_capsule(re));
    }
    return py::make_tuple(nodes, ts, lens, feats);
}

// numpy int32 array of a batch of picks
py::array_t<int32_t> to_numpy(const std::vector<int32_t>& v) {
    py::array_t<int32_t> out(static_cast<py::ssize_t>(v.size()));
    std::copy(v.begin(), v.end(), out.mutable_data());
    return out;
}

// Optional batch of uniforms, one per pick.
const double* optional_draws(const std::optional<py::array_t<double, py::array::c_style |
                                                                        py::array::forcecast>>& r,
                             size_t n) {
    if (!r.has_value()) return nullptr;
    if (static_cast<size_t>(r->size()) != n)
        throw std::invalid_argument("random_numbers must hold one value per pick");
    return r->data();
}

// The reference's index-picker classes (py_interface/_temporal_random_walk.cu:
// 904-984): same constructor and pick_random; pick_random_batch goes beyond it.
template <typename Picker>
void bind_index_picker(py::module& m, const char* name, const char* what) {
    using Draws = std::optional<py::array_t<double, py::array::c_style | py::array::forcecast>>;
    py::class_<Picker>(m, name)
        .def(py::init([](bool use_gpu) { return Picker(use_gpu); }),
             (std::string("Initialize ") + what + " random picker.\n\nArgs:\n    use_gpu (bool): "
              "accepted for the reference's interface; picks run on the GPU.").c_str(),
             py::arg("use_gpu") = false)
        .def("pick_random", &Picker::pick_random,
             (std::string("Pick a random index in [start, end) with ") + what +
              " probability.\n\nArgs:\n    start (int): Start index inclusive\n    end (int): "
              "End index exclusive\n    prioritize_end (bool, optional): Prioritize recent "
              "timestamps. Default: True\n\nReturns:\n    int: Selected index")
                 .c_str(),
             py::arg("start"), py::arg("end"), py::arg("prioritize_end") = true)
        .def(
            "pick_random_batch",
            [](const Picker& p, const std::vector<int32_t>& starts,
               const std::vector<int32_t>& ends, bool prioritize_end, const Draws& r) {
                return to_numpy(
                    p.pick_random_batch(starts, ends, prioritize_end, optional_draws(r, starts.size())));
            },
            "One pick per [starts[i], ends[i]) range in one GPU launch; random_numbers "
            "(uniforms in [0, 1), one per pick) replaces the in-kernel draws. Returns int32 "
            "indices, -1 for an empty range.",
            py::arg("starts"), py::arg("ends"), py::arg("prioritize_end") = true,
            py::arg("random_numbers") = py::none());
}

}  // namespace

PYBIND11_MODULE(_temporal_random_walk, m) {
    m.doc() = "MI355X temporal random walk engine (drop-in for temporal_random_walk)";

    py::class_<TemporalRandomWalk>(m, "TemporalRandomWalk", py::dynamic_attr())
        .def(py::init([](bool is_directed, bool use_gpu, std::optional<int64_t> max_time_capacity,
                         std::optional<bool> enable_weight_computation,
                         std::optional<bool> enable_temporal_node2vec,
                         std::optional<double> timescale_bound,
                         std::optional<double> temporal_node2vec_p,
                         std::optional<double> temporal_node2vec_q,
                         std::optional<int> walk_padding_value,
                         std::optional<uint64_t> global_seed,
                         std::optional<bool> shuffle_walk_order,
                         std::optional<int> cuda_device_id) {
                 return std::make_unique<TemporalRandomWalk>(
                     is_directed, use_gpu, max_time_capacity.value_or(-1),
                     enable_weight_computation.value_or(false),
                     enable_temporal_node2vec.value_or(false),
                     timescale_bound.value_or(DEFAULT_TIMESCALE_BOUND),
                     temporal_node2vec_p.value_or(DEFAULT_NODE2VEC_P),
                     temporal_node2vec_q.value_or(DEFAULT_NODE2VEC_Q),
                     walk_padding_value.value_or(EMPTY_NODE_VALUE),
                     global_seed.value_or(EMPTY_GLOBAL_SEED),
                     shuffle_walk_order.value_or(DEFAULT_SHUFFLE_WALK_ORDER),
                     cuda_device_id.value_or(0));
             }),
             "Initialize a temporal random walk generator (runs on the MI355X; use_gpu is "
             "accepted for compatibility).",
             py::arg("is_directed"), py::arg("use_gpu") = false,
             py::arg("max_time_capacity") = py::none(),
             py::arg("enable_weight_computation") = py::none(),
             py::arg("enable_temporal_node2vec") = py::none(),
             py::arg("timescale_bound") = py::none(), py::arg("temporal_node2vec_p") = py::none(),
             py::arg("temporal_node2vec_q") = py::none(),
             py::arg("walk_padding_value") = py::none(), py::arg("global_seed") = py::none(),
             py::arg("shuffle_walk_order") = py::none(), py::arg("cuda_device_id") = py::none())

        .def(
            "add_multiple_edges",
            [](TemporalRandomWalk& tw, const py::array_t<int>& sources,
               const py::array_t<int>& targets, const py::array_t<int64_t>& timestamps,
               const py::object& edge_features_obj) {
                // py_interface/_temporal_random_walk.cu:120-173
                const auto si = sources.request();
                const auto ti = targets.request();
                const auto tsi = timestamps.request();
                if (si.ndim != 1 || ti.ndim != 1 || tsi.ndim != 1)
                    throw std::runtime_error("Arrays must be 1-dimensional");
                const size_t n = static_cast<size_t>(si.shape[0]);
                if (static_cast<size_t>(ti.shape[0]) != n || static_cast<size_t>(tsi.shape[0]) != n)
                    throw std::runtime_error("All arrays must have the same length");
                const float* fptr = nullptr;
                size_t dim = 0;
                std::optional<py::array_t<float, py::array::c_style | py::array::forcecast>> f;
                if (!edge_features_obj.is_none()) {
                    f = edge_features_obj
                            .cast<py::array_t<float, py::array::c_style | py::array::forcecast>>();
                    const auto fi = f->request();
                    if (fi.ndim != 1 && fi.ndim != 2)
                        throw std::runtime_error("edge_features must be a 1D or 2D NumPy array");
                    const auto nv = static_cast<size_t>(fi.size);
                    if (n == 0 && nv > 0)
                        throw std::runtime_error("edge_features must be empty when there are no edges");
                    if (n > 0 && nv % n != 0)
                        throw std::runtime_error("edge_features size must be num_edges * feature_dim");
                    dim = n == 0 ? 0 : nv / n;
                    fptr = static_cast<const float*>(fi.ptr);
                }
                tw.add_multiple_edges(static_cast<const int*>(si.ptr),
                                      static_cast<const int*>(ti.ptr),
                                      static_cast<const int64_t*>(tsi.ptr), n, fptr, dim);
            },
            "Add multiple edges to the temporal graph.", py::arg("sources"), py::arg("targets"),
            py::arg("timestamps"), py::arg("edge_features") = py::none())

        .def(
            "prefetch_edges",
            [](py::object self, const py::array_t<int, py::array::c_style | py::array::forcecast>& sources,
               const py::array_t<int, py::array::c_style | py::array::forcecast>& targets,
               const py::array_t<int64_t, py::array::c_style | py::array::forcecast>& timestamps,
               const py::object& edge_features_obj) {
                auto& tw = self.cast<TemporalRandomWalk&>();
                const auto si = sources.request();
                const auto ti = targets.request();
                const auto tsi = timestamps.request();
                if (si.ndim != 1 || ti.ndim != 1 || tsi.ndim != 1)
                    throw std::runtime_error("Arrays must be 1-dimensional");
                const size_t n = static_cast<size_t>(si.shape[0]);
                if (static_cast<size_t>(ti.shape[0]) != n || static_cast<size_t>(tsi.shape[0]) != n)
                    throw std::runtime_error("All arrays must have the same length");
                const float* fptr = nullptr;
                size_t dim = 0;
                py::object keep_f = py::none();
                if (!edge_features_obj.is_none()) {
                    auto f = edge_features_obj
                                 .cast<py::array_t<float, py::array::c_style | py::array::forcecast>>();
                    const auto fi = f.request();
                    if (fi.ndim != 1 && fi.ndim != 2)
                        throw std::runtime_error("edge_features must be a 1D or 2D NumPy array");
                    const auto nv = static_cast<size_t>(fi.size);
                    if (n > 0 && nv % n != 0)
                        throw std::runtime_error("edge_features size must be num_edges * feature_dim");
                    dim = n == 0 ? 0 : nv / n;
                    fptr = static_cast<const float*>(fi.ptr);
                    keep_f = f;
                }
                tw.prefetch_edges(static_cast<const int*>(si.ptr), static_cast<const int*>(ti.ptr),
                                  static_cast<const int64_t*>(tsi.ptr), n, fptr, dim);
                // the copy reads these arrays until add_prefetched_edges returns
                self.attr("_prefetched_arrays") = py::make_tuple(sources, targets, timestamps, keep_f);
            },
            "Start copying the next batch to the GPU while other calls (such as sampling) run; "
            "add_prefetched_edges() then ingests it as add_multiple_edges would.",
            py::arg("sources"), py::arg("targets"), py::arg("timestamps"),
            py::arg("edge_features") = py::none())

        .def(
            "add_prefetched_edges",
            [](py::object self) {
                auto& tw = self.cast<TemporalRandomWalk&>();
                try {
                    tw.add_prefetched_edges();
                } catch (...) {
                    self.attr("_prefetched_arrays") = py::none();
                    throw;
                }
                self.attr("_prefetched_arrays") = py::none();
            },
            "Ingest the batch started by prefetch_edges().")

        .def(
            "set_node_features",
            [](TemporalRandomWalk& tw, const py::array_t<int>& node_ids,
               const py::array_t<float, py::array::c_style | py::array::forcecast>& feats) {
                const auto ni = node_ids.request();
                const auto fi = feats.request();
                if (ni.ndim != 1) throw std::runtime_error("node_ids must be a 1D NumPy array");
                if (fi.ndim != 2) throw std::runtime_error("node_features must be a 2D NumPy array");
                const auto n = static_cast<size_t>(ni.shape[0]);
                const auto dim = static_cast<size_t>(fi.shape[1]);
                if (static_cast<size_t>(fi.shape[0]) != n)
                    throw std::runtime_error("node_features row count must match node_ids length");
                if (dim == 0 && n > 0)
                    throw std::runtime_error(
                        "node_features must have at least one column when node_ids is non-empty");
                if (n == 0) return;
                tw.set_node_features(static_cast<const int*>(ni.ptr), n,
                                     static_cast<const float*>(fi.ptr), dim);
            },
            "Set dense feature vectors for specific node IDs.", py::arg("node_ids"),
            py::arg("node_features"))

        .def(
            "get_node_features",
            [](const TemporalRandomWalk& tw) {
                const int dim = tw.node_feature_dim();
                const int mx = tw.node_features_max_node_id();
                const std::vector<float> dense = tw.node_features_dense();
                if (dim == 0 || mx < 0 || dense.empty())
                    return py::array_t<float>(std::vector<py::ssize_t>{0, 0});
                py::array_t<float> out(std::vector<py::ssize_t>{mx + 1, dim});
                std::copy_n(dense.data(), dense.size(), static_cast<float*>(out.request().ptr));
                return out;
            },
            "Return dense node features for all node IDs from 0 to max_node_id.")

        .def(
            "get_random_walks_and_times_for_all_nodes",
            [](TemporalRandomWalk& tw, int max_walk_len, const std::string& walk_bias,
               int num_walks_per_node, const std::optional<std::string>& initial_edge_bias,
               const std::string& walk_direction, const std::string& kernel_launch_type) {
                const RandomPickerType wb = picker_type_from_string(walk_bias);
                std::optional<RandomPickerType> ib;
                const RandomPickerType* ibp = optional_picker(initial_edge_bias, ib);
                const WalkDirection dir = walk_direction_from_string(walk_direction);
                const KernelLaunchType klt = kernel_launch_type_from_string(kernel_launch_type);
                auto walks = tw.get_random_walks_and_times_for_all_nodes(
                    max_walk_len, &wb, num_walks_per_node, ibp, dir, klt);
                return walks_to_numpy(walks, max_walk_len);
            },
            "Generate temporal random walks with timestamps starting from all nodes.",
            py::arg("max_walk_len"), py::arg("walk_bias"), py::arg("num_walks_per_node"),
            py::arg("initial_edge_bias") = py::none(),
            py::arg("walk_direction") = "Forward_In_Time",
            py::arg("kernel_launch_type") = "NODE_GROUPED")

        .def(
            "get_random_walks_and_times_for_last_batch",
            [](TemporalRandomWalk& tw, int max_walk_len, const std::string& walk_bias,
               int num_walks_per_node, const std::optional<std::string>& initial_edge_bias,
               const std::string& walk_direction, const std::string& kernel_launch_type) {
                const RandomPickerType wb = picker_type_from_string(walk_bias);
                std::optional<RandomPickerType> ib;
                const RandomPickerType* ibp = optional_picker(initial_edge_bias, ib);
                const WalkDirection dir = walk_direction_from_string(walk_direction);
                const KernelLaunchType klt = kernel_launch_type_from_string(kernel_launch_type);
                auto walks = tw.get_random_walks_and_times_for_last_batch(
                    max_walk_len, &wb, num_walks_per_node, ibp, dir, klt);
                return walks_to_numpy(walks, max_walk_len);
            },
            "Generate temporal random walks starting from the last batch's nodes.",
            py::arg("max_walk_len"), py::arg("walk_bias"), py::arg("num_walks_per_node"),
            py::arg("initial_edge_bias") = py::none(),
            py::arg("walk_direction") = "Forward_In_Time",
            py::arg("kernel_launch_type") = "NODE_GROUPED")

        .def(
            "get_random_walks_and_times_for_nodes",
            [](TemporalRandomWalk& tw,
               const py::array_t<int, py::array::c_style | py::array::forcecast>& seed_nodes,
               int max_walk_len, const std::string& walk_bias, int num_walks_per_node,
               const std::optional<std::string>& initial_edge_bias,
               const std::string& walk_direction, const std::string& kernel_launch_type,
               const std::optional<py::array_t<int64_t, py::array::c_style | py::array::forcecast>>&
                   cutoff_times) {
                const RandomPickerType wb = picker_type_from_string(walk_bias);
                std::optional<RandomPickerType> ib;
                const RandomPickerType* ibp = optional_picker(initial_edge_bias, ib);
                const WalkDirection dir = walk_direction_from_string(walk_direction);
                const KernelLaunchType klt = kernel_launch_type_from_string(kernel_launch_type);
                const py::buffer_info si = seed_nodes.request();
                if (si.ndim != 1) throw std::runtime_error("seed_nodes must be a 1D int32 array");
                const auto ns = static_cast<size_t>(si.shape[0]);
                const int64_t* cptr = nullptr;
                py::buffer_info ci;
                if (cutoff_times.has_value()) {
                    ci = cutoff_times->request();
                    if (ci.ndim != 1) throw std::runtime_error("cutoff_times must be a 1D int64 array");
                    if (static_cast<size_t>(ci.shape[0]) != ns)
                        throw std::runtime_error(
                            "cutoff_times must have the same length as seed_nodes");
                    cptr = static_cast<const int64_t*>(ci.ptr);
                }
                auto walks = tw.get_random_walks_and_times_for_nodes(
                    static_cast<const int*>(si.ptr), ns, cptr, max_walk_len, &wb,
                    num_walks_per_node, ibp, dir, klt);
                return walks_to_numpy(walks, max_walk_len);
            },
            "Generate temporal random walks starting from the given seed nodes.",
            py::arg("seed_nodes"), py::arg("max_walk_len"), py::arg("walk_bias"),
            py::arg("num_walks_per_node"), py::arg("initial_edge_bias") = py::none(),
            py::arg("walk_direction") = "Forward_In_Time",
            py::arg("kernel_launch_type") = "NODE_GROUPED", py::arg("cutoff_times") = py::none())

        .def(
            "get_random_walks_and_times",
            [](TemporalRandomWalk& tw, int max_walk_len, const std::string& walk_bias,
               int num_walks_total, const std::optional<std::string>& initial_edge_bias,
               const std::string& walk_direction, const std::string& kernel_launch_type) {
                const RandomPickerType wb = picker_type_from_string(walk_bias);
                std::optional<RandomPickerType> ib;
                const RandomPickerType* ibp = optional_picker(initial_edge_bias, ib);
                const WalkDirection dir = walk_direction_from_string(walk_direction);
                const KernelLaunchType klt = kernel_launch_type_from_string(kernel_launch_type);
                auto walks = tw.get_random_walks_and_times(max_walk_len, &wb, num_walks_total, ibp,
                                                           dir, klt);
                return walks_to_numpy(walks, max_walk_len);
            },
            "Generate temporal random walks with timestamps.", py::arg("max_walk_len"),
            py::arg("walk_bias"), py::arg("num_walks_total"),
            py::arg("initial_edge_bias") = py::none(),
            py::arg("walk_direction") = "Forward_In_Time",
            py::arg("kernel_launch_type") = "NODE_GROUPED")

        .def("get_node_count", &TemporalRandomWalk::get_node_count,
             "Get total number of nodes in the graph.")
        .def("get_edge_count", &TemporalRandomWalk::get_edge_count,
             "Returns the total number of directed edges in the temporal graph.")
        .def(
            "get_node_ids",
            [](const TemporalRandomWalk& tw) {
                const auto ids = tw.get_node_ids();
                py::array_t<int> out(static_cast<py::ssize_t>(ids.size()));
                if (!ids.empty())
                    std::copy(ids.begin(), ids.end(), static_cast<int*>(out.request().ptr));
                return out;
            },
            "Returns a NumPy array containing the IDs of all nodes in the temporal graph.")
        .def(
            "get_node_degrees",
            [](const TemporalRandomWalk& tw,
               const py::array_t<int, py::array::c_style | py::array::forcecast>& nodes,
               const std::string& direction) {
                const py::buffer_info ni = nodes.request();
                if (ni.ndim != 1) throw std::runtime_error("nodes must be a 1D int32 array");
                const WalkDirection d = walk_direction_from_string(direction);
                const auto deg = tw.get_node_degrees(static_cast<const int*>(ni.ptr),
                                                     static_cast<size_t>(ni.shape[0]), d);
                py::array_t<int64_t> out(static_cast<py::ssize_t>(deg.size()));
                if (!deg.empty())
                    std::copy(deg.begin(), deg.end(), static_cast<int64_t*>(out.request().ptr));
                return out;
            },
            "Return the degree of each queried node, in the same order as the input.",
            py::arg("nodes"), py::arg("direction") = "Forward_In_Time")
        .def("clear", &TemporalRandomWalk::clear, "Clears and reinitiates the underlying graph.")
        .def("get_memory_used", &TemporalRandomWalk::get_memory_used,
             "Returns the memory used by the graph arrays in bytes.")
        .def(
            "add_edges_from_networkx",
            [](TemporalRandomWalk& tw, const py::object& nx_graph) {
                const py::object edges = nx_graph.attr("edges")(py::arg("data") = true);
                std::vector<std::tuple<int, int, int64_t>> infos;
                for (const auto& edge : edges) {
                    auto t = edge.cast<py::tuple>();
                    const auto attrs = t[2].cast<py::dict>();
                    infos.emplace_back(py::cast<int>(t[0]), py::cast<int>(t[1]),
                                       py::cast<int64_t>(attrs["timestamp"]));
                }
                tw.add_multiple_edges(infos);
            },
            "Add edges from a NetworkX graph.", py::arg("nx_graph"))
        .def(
            "to_networkx",
            [](TemporalRandomWalk& tw) {
                const auto edges = tw.get_edges();
                const py::module nx = py::module::import("networkx");
                py::object g = tw.get_is_directed() ? nx.attr("DiGraph")() : nx.attr("Graph")();
                for (const auto& [s, d, t] : edges) {
                    py::dict kw;
                    kw["timestamp"] = t;
                    g.attr("add_edge")(s, d, **kw);
                }
                return g;
            },
            "Export graph to NetworkX format.");

    bind_index_picker<LinearRandomPicker>(m, "LinearRandomPicker", "linear time decay");
    bind_index_picker<ExponentialIndexRandomPicker>(m, "ExponentialIndexRandomPicker",
                                                    "index based exponential time decay");
    bind_index_picker<UniformRandomPicker>(m, "UniformRandomPicker", "uniform");

    using Draws = std::optional<py::array_t<double, py::array::c_style | py::array::forcecast>>;
    py::class_<WeightBasedRandomPicker>(m, "WeightBasedRandomPicker")
        .def(py::init([](bool use_gpu) { return WeightBasedRandomPicker(use_gpu); }),
             "Initialize weight-based exponential time decay random picker.\n\nArgs:\n    "
             "use_gpu (bool): accepted for the reference's interface; picks run on the GPU.",
             py::arg("use_gpu") = false)
        .def(
            "pick_random",
            [](const WeightBasedRandomPicker& p, const std::vector<double>& cumulative_weights,
               int group_start, int group_end) {
                return p.pick_random(cumulative_weights, group_start, group_end);
            },
            "Pick random index with exponential weight-based probability using cumulative "
            "weights.\n\nArgs:\n    cumulative_weights (List[float]): List of cumulative "
            "weights\n    group_start (int): Start index inclusive\n    group_end (int): End "
            "index exclusive\n\nReturns:\n    int: Selected index",
            py::arg("cumulative_weights"), py::arg("group_start"), py::arg("group_end"))
        .def(
            "pick_random_batch",
            [](const WeightBasedRandomPicker& p, const std::vector<double>& cumulative_weights,
               const std::vector<uint64_t>& group_starts, const std::vector<uint64_t>& group_ends,
               const Draws& r) {
                return to_numpy(p.pick_random_batch(cumulative_weights, group_starts, group_ends,
                                                    optional_draws(r, group_starts.size())));
            },
            "One pick per [group_starts[i], group_ends[i]) range of one cumulative-weight "
            "array, in one GPU launch; random_numbers as for the index pickers.",
            py::arg("cumulative_weights"), py::arg("group_starts"), py::arg("group_ends"),
            py::arg("random_numbers") = py::none());
}
