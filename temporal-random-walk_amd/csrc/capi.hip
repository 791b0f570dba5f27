// capi.hip -- the extern "C" boundary declared in include/trw_engine.h.
//
// Every entry point: pins the handle's device (restoring the caller's on
// return, like the reference's CudaDeviceGuard, common/error_handlers.cuh:
// 111-139), runs the engine, maps C++ exceptions to trw_status and keeps the
// message in a thread-local buffer for trw_last_error().
#include <stdlib.h>

#include <new>
#include <string>
#include <thread>
#include <type_traits>
#include <vector>

#include "engine.h"

namespace trw {

Engine::Engine(const trw_config& c) : cfg(c), device(c.device_id) {
    init_noalloc_scratch(device);  // the device is current (trw_create)
    check_hip(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
    check_hip(hipStreamCreateWithFlags(&side, hipStreamNonBlocking), "hipStreamCreate");
    check_hip(hipEventCreateWithFlags(&side_done, hipEventDisableTiming), "hipEventCreate");
    check_hip(hipEventCreateWithFlags(&ts_ready, hipEventDisableTiming), "hipEventCreate");
    for (auto& e : ev) check_hip(hipEventCreate(&e), "hipEventCreate");
    check_hip(hipHostMalloc(&host_scalars, 256, hipHostMallocDefault), "hipHostMalloc");
}

Engine::~Engine() {
    (void)join_prefetch();  // no copy may outlive the engine
    if (stream) (void)hipStreamSynchronize(stream);
    if (side) (void)hipStreamSynchronize(side);
    free_retired();
    for (auto& e : ev)
        if (e) (void)hipEventDestroy(e);
    if (side_done) (void)hipEventDestroy(side_done);
    if (ts_ready) (void)hipEventDestroy(ts_ready);
    if (host_scalars) (void)hipHostFree(host_scalars);
    if (side) (void)hipStreamDestroy(side);
    if (stream) (void)hipStreamDestroy(stream);
}

size_t Engine::memory_used() const {
    size_t b = src.bytes() + dst.bytes() + ts.bytes() + feat.bytes() + tsg_off.bytes() +
               uniq_ts.bytes() + erank.bytes() + active.bytes() + fwd_cum.bytes() +
               bwd_cum.bytes() + gwg_fwd.bytes() + gwg_bwd.bytes() + gwt_fwd.bytes() +
               gwt_bwd.bytes() + adj_off.bytes() + adj_nbr.bytes() + adj_hash.bytes();
    for (const DirIndex* d : {&out, &in}) {
        b += d->off.bytes() + d->idx.bytes() + d->rec.bytes() + d->cnt.bytes() + d->grp.bytes() +
             d->first_ts.bytes() + d->pan.bytes() + d->hdr.bytes() + d->tab.bytes() +
             d->w_fwd.bytes() + d->w_bwd.bytes() + d->wrec.bytes() + d->wf.bytes() +
             d->wb.bytes();
    }
    // blocks of grown buffers held until the next clear() (DBuf::ensure)
    return b + retired.bytes;
}

}  // namespace trw

using trw::Engine;

namespace {

thread_local std::string g_last_error;

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        trw::check_hip(hipSetDevice(dev), "hipSetDevice");
    }
    ~DeviceGuard() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

// Points trw::g_retired at an engine's retired-block list for one call.
struct RetireInto {
    trw::RetiredBlocks* prev;
    explicit RetireInto(trw::RetiredBlocks* r) : prev(trw::g_retired) { trw::g_retired = r; }
    ~RetireInto() { trw::g_retired = prev; }
};

template <typename F>
trw_status guarded(void* h, F&& f) {
    try {
        if (!h) throw trw::InvalidArgument("null handle");
        Engine* e = static_cast<Engine*>(h);
        DeviceGuard g(e->device);
        RetireInto r(&e->retired);
        f(*e);
        return TRW_OK;
    } catch (const trw::InvalidArgument& ex) {
        g_last_error = ex.what();
        return TRW_ERR_INVALID_ARGUMENT;
    } catch (const std::bad_alloc& ex) {
        g_last_error = ex.what();
        return TRW_ERR_OUT_OF_MEMORY;
    } catch (const std::exception& ex) {
        g_last_error = ex.what();
        return TRW_ERR_RUNTIME;
    }
}

// A call that needs no engine handle: on device_id (-1: the current device).
template <typename F>
trw_status guarded_device(int32_t device_id, F&& f) {
    try {
        int count = 0;
        if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
            g_last_error = "no HIP device available: this engine runs only on the GPU";
            return TRW_ERR_NO_DEVICE;
        }
        int dev = device_id;
        if (dev < 0) trw::check_hip(hipGetDevice(&dev), "hipGetDevice");
        if (dev >= count) throw trw::InvalidArgument("device_id out of range");
        DeviceGuard g(dev);
        f();
        return TRW_OK;
    } catch (const trw::InvalidArgument& ex) {
        g_last_error = ex.what();
        return TRW_ERR_INVALID_ARGUMENT;
    } catch (const std::bad_alloc& ex) {
        g_last_error = ex.what();
        return TRW_ERR_OUT_OF_MEMORY;
    } catch (const std::exception& ex) {
        g_last_error = ex.what();
        return TRW_ERR_RUNTIME;
    }
}

template <typename T>
T* host_alloc(size_t n) {
    void* p = malloc(n ? n * sizeof(T) : 1);
    if (!p) throw std::bad_alloc();
    return static_cast<T*>(p);
}

template <typename T>
void d2h(T* dst, const T* src, size_t n, hipStream_t s) {
    if (n) trw::check_hip(hipMemcpyAsync(dst, src, n * sizeof(T), hipMemcpyDeviceToHost, s), "D2H");
}

template <typename D, typename S>
void widen_from_device(void* out, const S* dsrc, size_t n, hipStream_t s) {
    std::vector<S> tmp(n);
    d2h(tmp.data(), dsrc, n, s);
    trw::check_hip(hipStreamSynchronize(s), "sync");
    D* o = static_cast<D*>(out);
    for (size_t i = 0; i < n; ++i) o[i] = static_cast<D>(tmp[i]);
}

}  // namespace

extern "C" {

int32_t trw_abi_version(void) { return TRW_ABI_VERSION; }

const char* trw_last_error(void) { return g_last_error.c_str(); }

trw_status trw_create(const trw_config* config, void** out_handle) {
    try {
        if (!config || !out_handle) throw trw::InvalidArgument("null argument");
        int count = 0;
        if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
            g_last_error = "no HIP device available: this engine runs only on the GPU";
            return TRW_ERR_NO_DEVICE;
        }
        if (config->device_id < 0 || config->device_id >= count)
            throw trw::InvalidArgument("device_id out of range");
        if (config->node2vec_p == 0.0 || config->node2vec_q == 0.0)
            throw trw::InvalidArgument("node2vec p and q must be non-zero");
        DeviceGuard g(config->device_id);
        *out_handle = new Engine(*config);
        return TRW_OK;
    } catch (const trw::InvalidArgument& ex) {
        g_last_error = ex.what();
        return TRW_ERR_INVALID_ARGUMENT;
    } catch (const std::exception& ex) {
        g_last_error = ex.what();
        return TRW_ERR_RUNTIME;
    }
}

trw_status trw_destroy(void* handle) {
    if (!handle) return TRW_OK;
    Engine* e = static_cast<Engine*>(handle);
    try {
        DeviceGuard g(e->device);
        delete e;
    } catch (const std::exception& ex) {
        g_last_error = ex.what();
        return TRW_ERR_RUNTIME;
    }
    return TRW_OK;
}

trw_status trw_add_edges(void* handle, const int32_t* sources, const int32_t* targets,
                         const int64_t* timestamps, uint64_t n, const float* edge_features,
                         uint64_t feature_dim) {
    return guarded(handle, [&](Engine& e) {
        if (n == 0) return;  // core/temporal_random_walk.cu:285
        if (!sources || !targets || !timestamps) throw trw::InvalidArgument("null edge arrays");
        trw::validate_batch(e, edge_features, n, feature_dim);
        e.sync();  // the staging buffers may still feed earlier work
        e.stage_src.resize(n);
        e.stage_dst.resize(n);
        e.stage_ts.resize(n);
        std::vector<trw::HostCopy> segs = {{e.stage_src.p, sources, n * 4},
                                           {e.stage_dst.p, targets, n * 4},
                                           {e.stage_ts.p, timestamps, n * 8}};
        const float* df = nullptr;
        if (edge_features && feature_dim) {
            e.stage_feat.resize(n * feature_dim);
            segs.push_back({e.stage_feat.p, edge_features, n * feature_dim * 4});
            df = e.stage_feat.p;
        }
        e.copy_staged(segs.data(), segs.size(), true);
        e.build(e.stage_src.p, e.stage_dst.p, e.stage_ts.p, df, n, feature_dim);
    });
}

trw_status trw_prefetch_edges(void* handle, const int32_t* sources, const int32_t* targets,
                              const int64_t* timestamps, uint64_t n, const float* edge_features,
                              uint64_t feature_dim) {
    return guarded(handle, [&](Engine& e) {
        if (e.pf_pending)
            throw trw::InvalidArgument("a prefetched batch is pending: call trw_add_prefetched_edges first");
        if (n && (!sources || !targets || !timestamps)) throw trw::InvalidArgument("null edge arrays");
        if (edge_features != nullptr && feature_dim == 0)
            throw std::runtime_error("edge_features provided but feature_dim is 0");
        if (edge_features == nullptr && feature_dim != 0)
            throw std::runtime_error("feature_dim must be 0 when edge_features is not provided");
        const bool has_feat = edge_features && feature_dim;
        e.pf_src.resize(n);
        e.pf_dst.resize(n);
        e.pf_ts.resize(n);
        e.pf_feat.resize(has_feat ? n * feature_dim : 0);
        e.pf_n = n;
        e.pf_dim = feature_dim;
        e.pf_has_feat = has_feat;
        std::vector<trw::HostCopy> segs = {{e.pf_src.p, sources, n * 4},
                                           {e.pf_dst.p, targets, n * 4},
                                           {e.pf_ts.p, timestamps, n * 8}};
        if (has_feat) segs.push_back({e.pf_feat.p, edge_features, n * feature_dim * 4});
        e.pf_error.clear();
        Engine* ep = &e;
        e.pf_thread = std::thread([ep, segs]() {
            try {
                trw::check_hip(hipSetDevice(ep->device), "hipSetDevice");
                ep->copy_on_lanes(ep->pf_lanes, segs.data(), segs.size(), true, false);
            } catch (const std::exception& ex) {
                ep->pf_error = std::string("prefetch: ") + ex.what();
            }
        });
        e.pf_pending = true;  // only once the copy is under way
    });
}

trw_status trw_add_prefetched_edges(void* handle) {
    return guarded(handle, [&](Engine& e) {
        if (!e.pf_pending) throw trw::InvalidArgument("no prefetched batch is pending");
        const std::string err = e.join_prefetch();
        if (!err.empty()) throw std::runtime_error(err);
        const size_t n = e.pf_n;
        if (n == 0) return;  // core/temporal_random_walk.cu:285
        const float* df = e.pf_has_feat ? e.pf_feat.p : nullptr;
        trw::validate_batch(e, df, n, e.pf_dim);
        e.build(e.pf_src.p, e.pf_dst.p, e.pf_ts.p, df, n, e.pf_dim);
    });
}

trw_status trw_add_edges_device(void* handle, const int32_t* d_sources, const int32_t* d_targets,
                                const int64_t* d_timestamps, uint64_t n,
                                const float* d_edge_features, uint64_t feature_dim) {
    return guarded(handle, [&](Engine& e) {
        if (n == 0) return;
        if (!d_sources || !d_targets || !d_timestamps) throw trw::InvalidArgument("null edge arrays");
        trw::validate_batch(e, d_edge_features, n, feature_dim);
        e.build(d_sources, d_targets, d_timestamps, d_edge_features, n, feature_dim);
    });
}

trw_status trw_sample_device(void* handle, const trw_sample_params* params, trw_walks* out) {
    return guarded(handle, [&](Engine& e) {
        if (!params || !out) throw trw::InvalidArgument("null argument");
        e.sample(*params);
        out->num_walks = e.w_num;
        out->max_walk_len = e.w_len;
        out->feature_dim = static_cast<int32_t>(e.w_feat.n ? e.feat_dim : 0);
        out->nodes = e.w_nodes.p;
        out->timestamps = e.w_ts.p;
        out->walk_lens = e.w_lens.p;
        out->edge_ids = e.w_eids.p;
        out->edge_features = e.w_feat.n ? e.w_feat.p : nullptr;
    });
}

trw_status trw_sample_device_noalloc(void* handle, const trw_sample_params* params,
                                     uint64_t capacity_walks, trw_walks* out) {
    return guarded(handle, [&](Engine& e) {
        if (!params || !out) throw trw::InvalidArgument("null argument");
        // the device's scratch array is shared by every handle on it: one
        // call at a time (the sample waits for its stream before returning)
        std::lock_guard<std::mutex> scratch_lock(trw::noalloc_scratch_lock(e.device));
        trw::SampleTarget t{};
        t.space.base = static_cast<unsigned char*>(trw::noalloc_scratch(e.device));
        t.space.cap = trw::kNoAllocScratchBytes;
        t.capacity_walks = capacity_walks;
        t.nodes = out->nodes;
        t.ts = out->timestamps;
        t.lens = out->walk_lens;
        t.eids = out->edge_ids;
        t.feat = out->edge_features;
        const bool want_feat = e.feat_dim > 0 && params->max_walk_len > 1;
        if (capacity_walks && (!t.nodes || !t.ts || !t.lens ||
                               (params->max_walk_len > 1 && !t.eids) || (want_feat && !t.feat)))
            throw trw::InvalidArgument("null output buffer");
        // the row writers store 16-byte vectors
        for (const void* p : {static_cast<const void*>(t.nodes), static_cast<const void*>(t.ts),
                              static_cast<const void*>(t.lens), static_cast<const void*>(t.eids),
                              static_cast<const void*>(t.feat)})
            if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
                throw trw::InvalidArgument("output buffers must be 16-byte aligned");
        e.sample(*params, &t);
        out->num_walks = e.w_last_num;
        out->max_walk_len = params->max_walk_len;
        out->feature_dim = static_cast<int32_t>(want_feat ? e.feat_dim : 0);
        if (!want_feat) out->edge_features = nullptr;
    });
}

trw_status trw_sample(void* handle, const trw_sample_params* params, trw_walks* out) {
    return guarded(handle, [&](Engine& e) {
        if (!params || !out) throw trw::InvalidArgument("null argument");
        e.sample(*params);
        const size_t nw = e.w_num, L = static_cast<size_t>(e.w_len);
        const size_t el = L ? L - 1 : 0;
        trw_walks r{};
        r.num_walks = nw;
        r.max_walk_len = e.w_len;
        std::vector<trw::HostCopy> segs;
        // caller-owned (free()); a failure below releases what was taken
        auto take = [&](auto*& field, const auto* dsrc, size_t n) {
            using T = std::remove_pointer_t<std::remove_reference_t<decltype(field)>>;
            field = static_cast<T*>(trw::host_output_alloc(n * sizeof(T)));
            segs.push_back({field, dsrc, n * sizeof(T)});
        };
        try {
            take(r.nodes, e.w_nodes.p, nw * L);
            take(r.timestamps, e.w_ts.p, nw * L);
            take(r.walk_lens, e.w_lens.p, nw);
            take(r.edge_ids, e.w_eids.p, nw * el);
            if (e.w_feat.n) {
                r.feature_dim = static_cast<int32_t>(e.feat_dim);
                take(r.edge_features, e.w_feat.p, e.w_feat.n);
            }
            e.copy_staged(segs.data(), segs.size(), false);
        } catch (...) {
            trw_walks_free(&r);
            throw;
        }
        *out = r;
    });
}

void trw_walks_free(trw_walks* w) {
    if (!w) return;
    free(w->nodes);
    free(w->timestamps);
    free(w->walk_lens);
    free(w->edge_ids);
    free(w->edge_features);
    w->nodes = nullptr;
    w->timestamps = nullptr;
    w->walk_lens = nullptr;
    w->edge_ids = nullptr;
    w->edge_features = nullptr;
}

trw_status trw_get_node_count(void* handle, uint64_t* out) {
    return guarded(handle, [&](Engine& e) {
        std::vector<uint8_t> a(e.active.n);
        d2h(a.data(), e.active.p, a.size(), e.stream);
        e.sync();
        uint64_t c = 0;
        for (uint8_t x : a) c += x;
        *out = c;
    });
}

trw_status trw_get_edge_count(void* handle, uint64_t* out) {
    return guarded(handle, [&](Engine& e) { *out = e.E; });
}

trw_status trw_get_node_ids(void* handle, int32_t* out, uint64_t cap, uint64_t* len) {
    return guarded(handle, [&](Engine& e) {
        std::vector<uint8_t> a(e.active.n);
        d2h(a.data(), e.active.p, a.size(), e.stream);
        e.sync();
        uint64_t c = 0;
        for (size_t i = 0; i < a.size(); ++i) {
            if (a[i]) {
                if (out && c < cap) out[c] = static_cast<int32_t>(i);
                ++c;
            }
        }
        *len = c;
    });
}

trw_status trw_get_node_degrees(void* handle, const int32_t* nodes, uint64_t n,
                                int32_t direction, int64_t* out) {
    return guarded(handle, [&](Engine& e) {
        if (n && (!nodes || !out)) throw trw::InvalidArgument("null argument");
        const bool forward = direction == TRW_FORWARD_IN_TIME;
        const trw::DirIndex& d = (e.cfg.is_directed && !forward) ? e.in : e.out;
        std::vector<uint32_t> off(d.off.n);
        d2h(off.data(), d.off.p, off.size(), e.stream);
        e.sync();
        const int64_t osz = static_cast<int64_t>(off.size());
        for (uint64_t i = 0; i < n; ++i) {
            const int32_t u = nodes[i];
            out[i] = (u < 0 || u >= osz - 1) ? 0 : static_cast<int64_t>(off[u + 1] - off[u]);
        }
    });
}

trw_status trw_get_edges(void* handle, int32_t* sources, int32_t* targets, int64_t* timestamps,
                         uint64_t cap, uint64_t* len) {
    return guarded(handle, [&](Engine& e) {
        *len = e.E;
        if (!sources || !targets || !timestamps) return;
        if (cap < e.E) throw trw::InvalidArgument("output capacity too small");
        d2h(sources, e.src.p, e.E, e.stream);
        d2h(targets, e.dst.p, e.E, e.stream);
        d2h(timestamps, e.ts.p, e.E, e.stream);
        e.sync();
    });
}

trw_status trw_get_is_directed(void* handle, int32_t* out) {
    return guarded(handle, [&](Engine& e) { *out = e.cfg.is_directed ? 1 : 0; });
}

trw_status trw_get_memory_used(void* handle, uint64_t* out) {
    return guarded(handle, [&](Engine& e) { *out = e.memory_used(); });
}

trw_status trw_get_feature_dim(void* handle, uint64_t* out) {
    return guarded(handle, [&](Engine& e) { *out = e.feat_dim; });
}

trw_status trw_get_latest_timestamp(void* handle, int64_t* out) {
    return guarded(handle, [&](Engine& e) { *out = e.latest_ts; });
}

trw_status trw_clear(void* handle) {
    return guarded(handle, [&](Engine& e) {
        e.sync();
        e.clear();
        e.free_retired();
    });
}

trw_status trw_get_array(void* handle, int32_t id, void* dst, uint64_t cap, uint64_t* len,
                         uint32_t* elem_size) {
    return guarded(handle, [&](Engine& e) {
        hipStream_t s = e.stream;
        const bool w = e.weights_ready;
        const bool dir = e.cfg.is_directed != 0;
        size_t n = 0;
        uint32_t es = 8;
        // resolve (pointer, count, source width)
        const void* p = nullptr;
        int kind = 0;  // 0: u32->u64, 1: i32, 2: i64, 3: f64, 4: f32, 5: u8->i32
        switch (id) {
            case TRW_ARR_SOURCES: p = e.src.p; n = e.E; kind = 1; es = 4; break;
            case TRW_ARR_TARGETS: p = e.dst.p; n = e.E; kind = 1; es = 4; break;
            case TRW_ARR_TIMESTAMPS: p = e.ts.p; n = e.E; kind = 2; break;
            case TRW_ARR_TIMESTAMP_GROUP_OFFSETS: p = e.tsg_off.p; n = e.T ? e.T + 1 : 0; break;
            case TRW_ARR_UNIQUE_TIMESTAMPS: p = e.uniq_ts.p; n = e.T; kind = 2; break;
            case TRW_ARR_ACTIVE_NODE_IDS: p = e.active.p; n = e.active.n; kind = 5; es = 4; break;
            case TRW_ARR_NODE_GROUP_OUTBOUND_OFFSETS: p = e.out.off.p; n = e.out.off.n; break;
            case TRW_ARR_NODE_GROUP_INBOUND_OFFSETS: p = e.in.off.p; n = dir ? e.in.off.n : 0; break;
            case TRW_ARR_NODE_TS_SORTED_OUTBOUND_INDICES: p = e.out.idx.p; n = e.out.idx.n; break;
            case TRW_ARR_NODE_TS_SORTED_INBOUND_INDICES: p = e.in.idx.p; n = dir ? e.in.idx.n : 0; break;
            case TRW_ARR_COUNT_TS_GROUP_PER_NODE_OUTBOUND: p = e.out.cnt.p; n = e.out.cnt.n; break;
            case TRW_ARR_COUNT_TS_GROUP_PER_NODE_INBOUND: p = e.in.cnt.p; n = dir ? e.in.cnt.n : 0; break;
            case TRW_ARR_NODE_TS_GROUP_OUTBOUND_OFFSETS: p = e.out.grp.p; n = e.out.n_groups; break;
            case TRW_ARR_NODE_TS_GROUP_INBOUND_OFFSETS: p = e.in.grp.p; n = dir ? e.in.n_groups : 0; break;
            case TRW_ARR_FORWARD_CUMULATIVE_WEIGHTS: p = e.fwd_cum.p; n = w ? e.T : 0; kind = 3; break;
            case TRW_ARR_BACKWARD_CUMULATIVE_WEIGHTS: p = e.bwd_cum.p; n = w ? e.T : 0; kind = 3; break;
            case TRW_ARR_OUTBOUND_FORWARD_CUMULATIVE_WEIGHTS: p = e.out.w_fwd.p; n = w ? e.out.n_groups : 0; kind = 3; break;
            case TRW_ARR_OUTBOUND_BACKWARD_CUMULATIVE_WEIGHTS: p = e.out.w_bwd.p; n = w ? e.out.n_groups : 0; kind = 3; break;
            case TRW_ARR_INBOUND_BACKWARD_CUMULATIVE_WEIGHTS: p = e.in.w_bwd.p; n = (w && dir) ? e.in.n_groups : 0; kind = 3; break;
            case TRW_ARR_NODE_ADJ_OFFSETS:
                e.build_adjacency_lists();
                p = e.adj_off.p;
                n = e.adj_lists_ready ? e.adj_off.n : 0;
                break;
            case TRW_ARR_NODE_ADJ_NEIGHBORS:
                e.build_adjacency_lists();
                p = e.adj_nbr.p;
                n = e.adj_lists_ready ? e.adj_nbr.n : 0;
                kind = 1;
                es = 4;
                break;
            case TRW_ARR_EDGE_FEATURES: p = e.feat.p; n = e.E * e.feat_dim; kind = 4; es = 4; break;
            default: throw trw::InvalidArgument("unknown array id");
        }
        *len = n;
        if (elem_size) *elem_size = es;
        if (!dst || n == 0) return;
        if (cap < n) throw trw::InvalidArgument("output capacity too small");
        switch (kind) {
            case 0: widen_from_device<uint64_t>(dst, static_cast<const uint32_t*>(p), n, s); break;
            case 1: widen_from_device<int32_t>(dst, static_cast<const int32_t*>(p), n, s); break;
            case 2: widen_from_device<int64_t>(dst, static_cast<const int64_t*>(p), n, s); break;
            case 3: widen_from_device<double>(dst, static_cast<const double*>(p), n, s); break;
            case 4: widen_from_device<float>(dst, static_cast<const float*>(p), n, s); break;
            case 5: widen_from_device<int32_t>(dst, static_cast<const uint8_t*>(p), n, s); break;
        }
    });
}

trw_status trw_get_timings(void* handle, trw_timings* out) {
    return guarded(handle, [&](Engine& e) { *out = e.timings; });
}

trw_status trw_get_stream(void* handle, void** out_stream) {
    return guarded(handle, [&](Engine& e) { *out_stream = e.stream; });
}

trw_status trw_get_walk_stats(void* handle, trw_walk_stats* out) {
    return guarded(handle, [&](Engine& e) { trw::walk_stats(e, out); });
}

void trw_debug_fail_allocation(int64_t n) {
    trw::g_alloc_fail_after.store(n < 0 ? -1 : n, std::memory_order_relaxed);
}

void trw_debug_fail_allocation_transient(int64_t n) {
    trw::g_alloc_fail_transient.store(n < 0 ? -1 : n, std::memory_order_relaxed);
}

trw_status trw_pick_index(int32_t device_id, int32_t picker, const int32_t* start,
                          const int32_t* end, uint64_t n, int32_t prioritize_end,
                          const double* draws, uint64_t seed, int32_t* out) {
    return guarded_device(device_id, [&] {
        trw::pick_index_batch(picker, start, end, n, prioritize_end != 0, draws, seed, out);
    });
}

trw_status trw_pick_weights(int32_t device_id, const double* cumulative, uint64_t size,
                            const uint64_t* group_start, const uint64_t* group_end, uint64_t n,
                            const double* draws, uint64_t seed, int32_t* out) {
    return guarded_device(device_id, [&] {
        trw::pick_weights_batch(cumulative, size, group_start, group_end, n, draws, seed, out);
    });
}

}  // extern "C"
