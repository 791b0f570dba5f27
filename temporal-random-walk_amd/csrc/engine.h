// engine.h -- internal state of one engine instance (one device, one stream);
// the HBM layout of its index is described in index_layout.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "../../include/trw_engine.h"
#include "index_layout.h"
#include "primitives.h"

namespace trw {

struct InvalidArgument : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};

// Test hooks: when >= 0, the number of device allocations that still succeed
// before one fails as out of memory -- for good (trw_debug_fail_allocation:
// its retry fails too), or only at its first attempt
// (trw_debug_fail_allocation_transient: the retry after releasing the retired
// blocks succeeds).
inline std::atomic<long long> g_alloc_fail_after{-1};
inline std::atomic<long long> g_alloc_fail_transient{-1};
inline bool alloc_hook_fires(std::atomic<long long>& c) {
    return c.load(std::memory_order_relaxed) >= 0 && c.fetch_sub(1, std::memory_order_relaxed) == 0;
}

// Device blocks whose buffers grew during an engine call (set by the C ABI's
// call guard to the engine's list): they are freed at the engine's next
// clear() or destruction instead of at once.  hipFree synchronises the device
// and unmaps (about 0.3-0.5 ms per block of 100 MB or more), and an ingest
// whose store grows regrows some 40 buffers: freeing them inside the call
// made the ingests where a streaming window fills up 2-3x slower.  nullptr
// (outside engine calls): blocks are freed at once.
struct RetiredBlocks {
    std::vector<void*> blocks;
    size_t bytes = 0;
    // hipFree waits for the device, so no queued kernel still reads a block
    void release() {
        for (void* q : blocks) (void)hipFree(q);
        blocks.clear();
        bytes = 0;
    }
};
inline thread_local RetiredBlocks* g_retired = nullptr;
// Past this many retired bytes a growing buffer frees its old block at once.
constexpr size_t kMaxRetiredBytes = size_t{32} << 30;

// Growth hint of the current engine call (set by an ingest into a windowed
// store, 1 otherwise): a buffer that grows takes at least this many times
// the size asked for, so a store filling its window is sized for the whole
// window at once instead of regrowing batch after batch.
inline thread_local double g_growth_hint = 1.0;
constexpr double kMaxGrowthHint = 4.0;

// Grow-only device buffer; growth discards the contents.  A buffer that grows
// again takes twice its capacity (and at least g_growth_hint times what is
// asked), so a store filling a streaming window regrows its buffers once at
// most rather than at every batch.
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
            const size_t old_cap = cap;
            if (p && g_retired && g_retired->bytes + cap * sizeof(T) <= kMaxRetiredBytes) {
                g_retired->blocks.push_back(p);
                g_retired->bytes += cap * sizeof(T);
                p = nullptr;
                n = cap = 0;
            } else {
                release();
            }
            const size_t hinted = static_cast<size_t>(static_cast<double>(k) * g_growth_hint);
            const size_t c = std::max({k + k / 4, 2 * old_cap, hinted + hinted / 4}) + 64;
            if (alloc_hook_fires(g_alloc_fail_after)) throw std::bad_alloc();
            hipError_t e = alloc_hook_fires(g_alloc_fail_transient) ? hipErrorOutOfMemory
                                                                     : hipMalloc(&p, c * sizeof(T));
            if (e == hipErrorOutOfMemory && g_retired && !g_retired->blocks.empty()) {
                // out of memory while blocks of grown buffers are held: release
                // them and try once more
                (void)hipGetLastError();
                p = nullptr;
                g_retired->release();
                e = hipMalloc(&p, c * sizeof(T));
            }
            if (e == hipErrorOutOfMemory) {
                (void)hipGetLastError();  // clear the sticky error
                p = nullptr;
                throw std::bad_alloc();  // TRW_ERR_OUT_OF_MEMORY / MemoryError
            }
            check_hip(e, "hipMalloc");
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

// Where one sample call's per-call device buffers come from: the engine's
// grow-only buffers, or -- for trw_sample_device_noalloc -- a fixed device
// region handed out front to back (no allocation; a call needing more than
// the region is rejected before any work is queued).
struct SampleSpace {
    unsigned char* base = nullptr;  // nullptr: the engine's buffers
    size_t cap = 0, used = 0;

    // n elements: the engine buffer `own` (grown if needed) or the next
    // 256-byte aligned piece of the region
    template <typename T>
    T* take(DBuf<T>& own, size_t n) {
        if (!base) {
            own.resize(n);
            return own.p;
        }
        const size_t off = (used + 255) & ~static_cast<size_t>(255);
        if (n > (cap - std::min(cap, off)) / sizeof(T))
            throw InvalidArgument("sample needs more device scratch than the " +
                                  std::to_string(cap >> 20) +
                                  " MiB of the no-allocation entry point");
        used = off + n * sizeof(T);
        return reinterpret_cast<T*>(base + off);
    }
};

// Size of the device array trw_sample_device_noalloc takes its per-call
// buffers from (one per device, held for the life of the process).
constexpr size_t kNoAllocScratchBytes = size_t{128} << 20;

// Caller-owned device outputs of trw_sample_device_noalloc, and the fixed
// scratch region its per-call buffers come from.
struct SampleTarget {
    SampleSpace space;
    uint64_t capacity_walks;
    int32_t* nodes;
    int64_t* ts;
    uint64_t* lens;
    int64_t* eids;
    float* feat;
};

// A walk direction's view of its cumulative weights for the weight pickers
// (index_layout.h): node headers with guide parameters, the weighted panel and
// the guide tables.
struct WalkWeights {
    DBuf<WNodeHdr> hdr;   // V_c
    DBuf<WPanelRec> pan;  // g << shift (wide: every record followed by its sum slot)
    DBuf<uint32_t> tab;   // 2 (g + V_c - 1)
    int shift = 0;
    void clear() { hdr.n = pan.n = tab.n = 0; }
    size_t bytes() const { return hdr.bytes() + pan.bytes() + tab.bytes(); }
};

struct DirIndex {
    DBuf<uint32_t> off;      // V_c
    DBuf<uint32_t> idx;      // n entries
    DBuf<EdgeRec> rec;       // n entries, same order as idx
    DBuf<uint32_t> key;      // node of every entry (sorted)
    DBuf<uint32_t> cnt;      // V_c
    DBuf<uint32_t> grp;      // g + 1
    DBuf<int64_t> first_ts;  // g
    DBuf<PanelRec> pan;      // g + 1
    DBuf<NodeHdr> hdr;       // V_c
    DBuf<uint32_t> tab;      // bucket tables
    DBuf<double> w_fwd;      // g (outbound only)
    DBuf<double> w_bwd;      // g
    DBuf<WEdgeRec> wrec;     // n << wrec_shift: entries with next slice bounds (weights only)
    int wrec_shift = 0;      // 1: each record followed by its forward start sum
    // weight pickers' views: of w_fwd for forward walks (out), of w_bwd for
    // backward walks (in; out if undirected)
    WalkWeights wf, wb;
    size_t n_entries = 0;
    size_t n_groups = 0;
    bool present = false;

    void clear() {
        off.n = idx.n = rec.n = key.n = cnt.n = grp.n = first_ts.n = pan.n = hdr.n = tab.n = w_fwd.n =
            w_bwd.n = wrec.n = 0;
        wf.clear();
        wb.clear();
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
    // a second stream for work that overlaps the build (same priority): the
    // batch's endpoint copies and the global weights; the event the build's
    // end waits on, and the one the global weights wait on (the timestamp
    // groups ready)
    hipStream_t side = nullptr;
    hipEvent_t side_done = nullptr;
    hipEvent_t ts_ready = nullptr;

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
    DBuf<uint32_t> erank;
    DBuf<int32_t> neg1_rank;  // rank of timestamp -1 if stored, else -2
    size_t T = 0;

    // node map
    int32_t max_node_id = -1;
    int32_t batch_max_id = -1;  // largest node id of the batch being ingested
    DBuf<uint8_t> active;

    // global weights
    DBuf<double> fwd_cum, bwd_cum;
    DBuf<WGuide> gwg_fwd, gwg_bwd;      // their guides (one segment each)
    DBuf<uint32_t> gwt_fwd, gwt_bwd;
    DBuf<uint32_t> wg_long;  // guide build: long-run count and list
    bool weights_ready = false;

    // node2vec adjacency
    DBuf<uint32_t> adj_off;
    DBuf<int32_t> adj_nbr;
    // membership set of the adjacency's (owner, neighbour) pairs: open
    // addressing over 2^adj_hash_log slots, key owner << adj_bits | neighbour
    DBuf<uint64_t> adj_hash;
    int adj_hash_log = 0;
    int adj_bits = 0;
    size_t adj_nodes = 0;  // node ids the adjacency covers (max_node_id + 1)
    DBuf<uint32_t> adj_rank, adj_ids;  // active ids' ranks and the ids by rank
    bool adj_ready = false;        // the pair set describes the store
    bool adj_lists_ready = false;  // adj_off / adj_nbr do too (built on request)

    DirIndex out, in;

    // the last ingest appended its batch after the store (append_store): the
    // store edges it evicted and the old and batch edges it kept, which the
    // node index update takes its entries from
    bool append_mode = false;
    size_t append_del = 0, append_kept_old = 0, append_kept_new = 0;
    // node index update of an append: evicted prefix and batch offsets per
    // node, entry counts, and the next index arrays (swapped in)
    DBuf<uint32_t> inc_ev, inc_bstart, inc_cnt;
    DBuf<uint32_t> key_next, off_next;
    DBuf<EdgeRec> rec_next;

    // the last ingest merged its batch into the store (merge_store), and the
    // merged store's feature rows' sources (store ids, then e_old + batch row)
    bool merge_mode = false;
    DBuf<uint32_t> merge_perm;

    // last ingested batch (for ..._for_last_batch)
    DBuf<int32_t> last_src, last_dst;
    size_t last_n = 0;

    // scratch
    DBuf<uint64_t> k64a, k64b;
    DBuf<uint64_t> ends64, ends64b;  // packed (src, dst) of the timestamp sort's input
    DBuf<uint32_t> k32a, k32b, v32a, v32b;
    DBuf<uint32_t> hist, flags, scan, scan_scratch;
    DBuf<uint64_t> scan64_scratch;
    DBuf<double> dscratch, fscan_scratch;
    DBuf<double> gsum;         // the global weights' sums (side stream)
    DBuf<uint32_t> wg_long_g;  // their guides' long-run list (side stream)
    DBuf<int64_t> red64;    // reduction results + partials
    DBuf<int32_t> red32;
    DBuf<int32_t> stage_src, stage_dst;
    DBuf<int64_t> stage_ts;
    DBuf<float> stage_feat;
    DBuf<uint32_t> walk_st;  // 16-byte start state per walk (time-ordered sampling)
    DBuf<int32_t> starts;
    DBuf<int64_t> cutoffs;
    DBuf<double> replay;
    // start-array temporaries of a sample (kept between calls: no per-call
    // allocation once they are large enough)
    DBuf<int32_t> s_ids, s_seeds, s_tmp32;
    DBuf<int64_t> s_cuts, s_tmp64;
    // node-grouped processing: walk states between segments, the (node, walk)
    // lists and the live count
    DBuf<uint32_t> ng_carry, ng_keys0, ng_keys1, ng_vals0, ng_vals1, ng_count;
    DBuf<uint64_t> acc64;

    // walks (device): slot-major scratch of 64-bit slot words (node, rank of
    // the slot's time when it fits, 32-bit edge id) where a layout pass writes
    // the rows, then the row-major output [num_walks, L] in the reference's
    // types
    DBuf<uint64_t> sw_packed;
    DBuf<int32_t> w_nodes;
    DBuf<int64_t> w_ts, w_eids;
    DBuf<uint64_t> w_lens;
    DBuf<float> w_feat;
    uint64_t w_num = 0;
    uint64_t w_last_num = 0;  // walks of the last sample, wherever they went
    int w_len = 0;
    int w_dir_forward = 1;
    int w_constrained = 0;  // the last sample started from given nodes
    // what the last sample's walk kernel reads once and how it writes its
    // scratch (the compulsory bytes of trw_get_walk_stats)
    uint64_t w_in_bytes_per_walk = 0;  // start state, processing order, cutoff
    uint64_t w_index_bytes = 0;        // index arrays the launched kernel reads
    int w_rows = 0;  // the walk kernel wrote the output rows itself (no scratch)
    int w_slot_format = 0;  // trw_walk_stats.slot_word_format of the last sample
    int w_replay = 0;

    // pinned host scalars for the few readbacks that size allocations
    void* host_scalars = nullptr;

    // host handoff lanes
    std::vector<std::unique_ptr<HostLane>> lanes;

    // a host batch being staged into HBM beside other calls (trw_prefetch_edges):
    // its own lanes and device buffers, and the thread that copies
    std::vector<std::unique_ptr<HostLane>> pf_lanes;
    std::thread pf_thread;
    bool pf_pending = false;
    std::string pf_error;  // set by the copying thread on failure
    DBuf<int32_t> pf_src, pf_dst;
    DBuf<int64_t> pf_ts;
    DBuf<float> pf_feat;
    size_t pf_n = 0, pf_dim = 0;
    bool pf_has_feat = false;

    // device blocks retired by buffer growth, freed at clear(), after a failed
    // ingest, at destruction, or when an allocation runs out of memory
    RetiredBlocks retired;
    void free_retired() { retired.release(); }

    // timings
    hipEvent_t ev[8] = {};
    trw_timings timings{};

    explicit Engine(const trw_config& c);
    ~Engine();

    void sync() { check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize"); }

    // ingest: batch arrays in device memory.  A failure after the batch is
    // accepted (device out of memory, a HIP error) leaves the engine empty, as
    // after clear(), rather than holding a store its index does not describe.
    void build(const int32_t* d_src, const int32_t* d_dst, const int64_t* d_ts,
               const float* d_feat, size_t n, size_t dim);
    void clear();
    // the sorted adjacency lists adj_off / adj_nbr of the store (for
    // trw_get_array; the walks use the pair set)
    void build_adjacency_lists();
    // the pipeline of build() after the batch's checks
    void build_accepted(const int32_t* d_src, const int32_t* d_dst, const int64_t* d_ts,
                        const float* d_feat, size_t n, size_t dim, int64_t tmin, int64_t tmax);
    // its store update: the sort of the first batch into an empty store, the
    // append of a batch at or after the store's last timestamp (sets
    // append_*), or the merge of any other batch (below)
    void sort_store(const int32_t* d_src, const int32_t* d_dst, const int64_t* d_ts,
                    const float* d_feat, size_t n, int64_t tmin, int64_t tmax);
    void append_store(const int32_t* d_src, const int32_t* d_dst, const int64_t* d_ts,
                      const float* d_feat, size_t n, int64_t btmin, int64_t btmax);
    // any other batch into a non-empty store: the batch sorted alone, then
    // merged with the store (sets merge_*)
    void merge_store(const int32_t* d_src, const int32_t* d_dst, const int64_t* d_ts,
                     const float* d_feat, size_t n, int64_t btmin, int64_t btmax);

    // sampling into w_* buffers
    // sampling: into the engine's w_* buffers, or -- with `into` -- into
    // caller-owned device outputs with every per-call buffer taken from
    // into->space (trw_sample_device_noalloc: no allocation)
    void sample(const trw_sample_params& p, const SampleTarget* into = nullptr);

    size_t memory_used() const;

    // Waits for the engine stream, then copies every span between host and
    // device (pinned staging, several threads); a device -> host copy records
    // timings.handoff_*.  Returns when every byte has landed.
    void copy_staged(const HostCopy* segs, size_t nseg, bool to_device);
    // The same copy on the lanes ls, without waiting for the engine stream
    // (small copies go through the first lane's stream): safe beside other
    // work on the engine as long as no other call uses ls or the spans.
    void copy_on_lanes(std::vector<std::unique_ptr<HostLane>>& ls, const HostCopy* segs, size_t nseg,
                       bool to_device, bool engine_order);
    // Joins a pending prefetch; returns its error text ("" on success).
    std::string join_prefetch();
};

// ---- launchers implemented in build.hip / walk.hip -------------------------
void validate_batch(const Engine& e, const void* feat, size_t n, size_t dim);
void walk_stats(Engine& e, trw_walk_stats* out);

// Standalone pickers (pickers.hip): batches of picks, host arrays in and out.
void pick_index_batch(int picker, const int32_t* start, const int32_t* end, uint64_t n,
                      bool prioritize_end, const double* draws, uint64_t seed, int32_t* out);
void pick_weights_batch(const double* cumulative, uint64_t size, const uint64_t* group_start,
                        const uint64_t* group_end, uint64_t n, const double* draws, uint64_t seed,
                        int32_t* out);
// Rank of timestamp -1 among the stored unique timestamps (-2 if absent) into
// e.neg1_rank (update_neg1_rank) or into out, on the engine stream.
void update_neg1_rank(Engine& e);
void launch_neg1_rank(Engine& e, int32_t* out);
// The no-allocation scratch array of a device: its address is looked up once
// per device, with the device current (init_noalloc_scratch, at the first
// handle's creation); noalloc_scratch returns it.
void init_noalloc_scratch(int device);
void* noalloc_scratch(int device);
// Held for the whole of a no-allocation call: calls on one device (of any
// handles, from any threads) use its scratch array one at a time.
std::mutex& noalloc_scratch_lock(int device);

}  // namespace trw
