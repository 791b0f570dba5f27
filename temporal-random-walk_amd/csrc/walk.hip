// walk.hip -- the walk sampler.
//
// Semantics restate the reference CPU walk loop
// (core/temporal_random_walk_cpu.cuh:19-131) with its selectors
// (graph/edge_selectors.cuh:66-443), pickers (random/pickers.cuh) and the
// node2vec rejection sampler (graph/temporal_node2vec_helpers.cuh:127-199).
// Each walk is one lane; the walk state (current node, time, previous node,
// draws) lives in registers for the whole walk, so there is no per-step
// scheduler and no host round trip between steps.
//
// Per hop the lane reads the node's group range, searches the node's panel of
// 8-byte (timestamp rank, start) group records -- one load per probe instead
// of the reference's three dependent loads ts[idx[grp[p]]] -- applies the
// picker, and takes the picked group's edge range from the panel: pickers
// favour groups next to the boundary the search found, so that range is
// usually on a line the search has just read.  Then it reads the chosen edge
// record (neighbour, edge id).  Ranks (the timestamp's index among the
// graph's unique timestamps) order exactly as the timestamps do, so every
// comparison of the reference is kept; the walk carries the rank of its
// current time, which is the rank of the group it picked, and writes ranks
// and 32-bit edge ids to its scratch; the layout pass turns them into the
// reference's int64 timestamps and edge ids.  The cost is the number of distinct cache lines per
// hop and their dependent latency; hub panels stay resident in L2 / Infinity
// Cache because every walk crossing the hub probes the same keys.
#include <math.h>

#include <algorithm>
#include <mutex>
#include <random>
#include <vector>

#include "engine.h"
#include "trw_device.h"

namespace trw {
namespace {

constexpr int kB = 256;

// Walks per tile of the walk scratch (one wave).
constexpr uint64_t kScratchTile = 64;

// Samples of at least this many walks run sorted by start time (TRW_ORDER_AUTO).
constexpr uint64_t kTimeOrderMinWalks = 1ull << 16;

inline unsigned grid_for(size_t n) {
    const size_t g = (n + kB - 1) / kB;
    return static_cast<unsigned>(g ? g : 1);
}

struct DirView {
    const NodeHdr* hdr;   // V_c node headers
    const uint32_t* tab;  // bucket tables
    const PanelRec* pan;  // g + 1 group records (terminator)
    const EdgeRec* rec;   // walk-order edge records
    uint32_t idx_size;
    // the same records with the walk's next slice bounds (weights only);
    // wrshift 1: each followed by its forward start sum
    const WEdgeRec* wrec;
    uint32_t wrshift;
    // the weight pickers' view of the sampled direction's cumulative weights
    // (read by the weight families' kernels only; nullptr without weights)
    const WNodeHdr* whdr;   // V_c node headers with guide parameters
    const WPanelRec* wpan;  // g << wshift weighted panel records (WPan)
    uint32_t wshift;        // 1: a wide panel (a sum slot after every record)
    const uint32_t* wgt;    // guide tables, node u's at 2 (gb + u)
    uint64_t w_size;        // groups with weights (0: none)
};

// Picker families the walk kernel is specialised for: only index pickers
// (Uniform / Linear / ExponentialIndex / TEST_*) -- no weight or node2vec code,
// so fewer registers and more waves in flight -- or any picker.
constexpr int kFamIndex = 0;
constexpr int kFamAny = 1;
// Index pickers and ExponentialWeight: no node2vec rejection loop.
constexpr int kFamWeight = 2;

struct WalkGraph {
    const int32_t* src;
    const int32_t* dst;
    const int64_t* ts;
    uint32_t E;
    const uint32_t* tsg_off;
    const int64_t* uniq_ts;
    const int32_t* neg1_rank;  // rank of timestamp -1, -2 if no edge has it
    uint32_t T;
    const double* gw;  // global cumulative weights of the sampled direction
    uint64_t gw_size;
    const WGuide* gwg;    // their guide (nullptr: none) and guide table
    const uint32_t* gwt;
    const uint8_t* active;
    int32_t active_size;
    DirView d;
    const uint32_t* adj_off;   // sorted lists (nullptr: not built)
    const int32_t* adj_nbr;
    uint32_t adj_nodes;        // node ids the adjacency covers (0: none)
    const uint64_t* adj_hash;  // pair set (nullptr: search the lists)
    uint64_t adj_mask;
    int adj_shift, adj_bits;
    int tn2v;
    double inv_p, inv_q;
};

// A walk's state after its start edge: the walk's origin (slot 0), the node
// reached over the start edge, the rank of the edge's time and the edge id
// (-1: no start edge, the walk is empty).
struct StartState {
    int32_t first, cur, r, e;
};
static_assert(sizeof(StartState) == 16, "StartState must be 16 bytes");

struct WalkArgs {
    int L;
    int walk_bias;
    int start_bias;
    int pad;
    const int32_t* starts;   // nullptr => all unconstrained
    const int64_t* cutoffs;  // nullptr => none
    uint64_t n;
    DrawSource ds;
    uint64_t* lens;
    // walk scratch, one 64-bit slot word per slot (slot_word below)
    uint64_t* packed;
    int pk_nb, pk_rb;
    // Processing order (nullptr: walk id order).  Position q of the grid runs
    // walk order[q] and writes its scratch column q; outputs indexed by walk
    // (lengths, and the rows the layout pass writes) use the walk id.
    const uint32_t* order;
    const StartState* st;  // start state of every walk (walk_start_kernel)
    int xcd_remap;                // spread the order over the XCDs in contiguous slices
    uint64_t q0, q_end;           // grid positions [q0, q_end) of this launch
    // Row-major outputs written by the walk kernel itself (walk_rows_kernel):
    // nodes [n][L], timestamps [n][L], edge ids [n][L - 1], in the reference's
    // types, with the first slot's timestamp start_ts and the padding.
    int32_t* on;
    int64_t* ot;
    int64_t* oe;
    const int64_t* uniq_ts;
    const int64_t* edge_ts;  // the store's timestamps (slot words without a rank field)
    int64_t start_ts;
};

// A slot of a walk as one 64-bit word: the slot's node in the low nb bits,
// then -- when node id, timestamp rank and edge id fit in 64 bits together
// (rb > 0) -- the rank of the slot's time in rb bits, then the id of the edge
// into the slot.  Otherwise (rb == 0) the word holds node and edge id only,
// which always fit (both below 2^31), and the time is the edge's timestamp in
// the store.  The first slot, which no edge reaches and whose time is the
// direction's sentinel, has every bit above the node set: a rank field of all
// ones (no rank is), or an edge field of all ones (no edge id is).
__device__ __forceinline__ uint64_t first_word(int nb, int32_t node) {
    return static_cast<uint64_t>(static_cast<uint32_t>(node)) | (~0ull << nb);
}
__device__ __forceinline__ uint64_t slot_word(int nb, int rb, int32_t node, uint32_t rank,
                                              uint32_t eid) {
    uint64_t v = static_cast<uint64_t>(static_cast<uint32_t>(node)) |
                 (static_cast<uint64_t>(eid) << (nb + rb));
    if (rb) v |= static_cast<uint64_t>(rank) << nb;
    return v;
}
__device__ __forceinline__ int32_t word_node(uint64_t v, int nb) {
    return static_cast<int32_t>(v & ((1ull << nb) - 1));
}
__device__ __forceinline__ int64_t word_eid(uint64_t v, int nb, int rb) {
    return static_cast<int64_t>(v >> (nb + rb));
}
// The slot's timestamp: the sentinel of the first slot, else uniq_ts of its
// rank or the store's timestamp of its edge.
__device__ __forceinline__ int64_t word_ts(uint64_t v, int nb, int rb, const int64_t* uniq_ts,
                                           const int64_t* edge_ts, int64_t start_ts) {
    if ((v >> nb) == (~0ull >> nb)) return start_ts;
    return rb ? uniq_ts[(v >> nb) & ((1ull << rb) - 1)] : edge_ts[v >> nb];
}

// The walk scratch of one grid position.  Tile-major: grid positions come in
// tiles of 64 (one wave), and slot k of position q lives at
// [(q / 64) * 64 * L + k * 64 + q % 64], so the wave stores 512 B per slot
// contiguously and a tile's whole scratch is one contiguous run for the
// layout pass.
struct SlotWriter {
    uint64_t* wp;
    int nb, rb;
    __device__ __forceinline__ SlotWriter(const WalkArgs& a, uint64_t q) {
        const uint64_t tile = q / 64, lane = q % 64, L = static_cast<uint64_t>(a.L);
        wp = a.packed + tile * 64 * L + lane;
        nb = a.pk_nb;
        rb = a.pk_rb;
    }
    // slot 0: the walk's origin at the direction's sentinel time
    __device__ __forceinline__ void first(int32_t node) {
        __builtin_nontemporal_store(first_word(nb, node), wp);
    }
    // slot k >= 1: its node and rank and the edge that reached it
    __device__ __forceinline__ void slot(int k, int32_t node, uint32_t rank, uint32_t eid) {
        __builtin_nontemporal_store(slot_word(nb, rb, node, rank, eid),
                                    wp + static_cast<uint64_t>(k) * 64);
    }
};

// A start edge: endpoints, edge id (-1 for none) and the rank of its time.
struct Sel {
    int32_t u, v;
    int32_t e;
    int32_t r;
};

// Result of a per-node selection: the node reached, the rank of the edge's
// time and the edge id (-1 for none), and -- for an edge picked over the
// weighted records -- the global bound of the walk's next slice at that node
// (WEdgeRec::nxt read for the walk's direction; kNoNext: search for it) and,
// for a group's first entry, the weight sum that bounds that slice (kNoSum:
// load it).
struct Hop {
    int32_t nbr;
    int32_t r;
    int32_t e;
    uint32_t nx = kNoNext;
    double bs = kNoSum;
};

__device__ __forceinline__ Sel no_edge() { return Sel{-1, -1, -1, -1}; }
__device__ __forceinline__ Hop no_hop() { return Hop{-1, -1, -1}; }
__device__ __forceinline__ Hop hop_of(const EdgeRec& rec, uint32_t rank) {
    return Hop{rec.nbr, static_cast<int32_t>(rank), static_cast<int32_t>(rec.eid)};
}

__device__ __forceinline__ EdgeRec load_rec(const EdgeRec* p) { return *p; }
template <bool Fwd>
__device__ __forceinline__ Hop whop_of(int32_t nbr, uint32_t eid, uint32_t nxt, uint32_t rank,
                                       double bs) {
    return Hop{nbr, static_cast<int32_t>(rank), static_cast<int32_t>(eid), next_bound<Fwd>(nxt),
               bs};
}
// Entry `pick` of the weighted records, or the group's first entry (held in
// the group's weighted panel record: v = {rank, start, end, nxt0}, r0, bs0) or
// second (in a wide panel's slot sl; nullptr for a narrow panel).
template <bool Fwd>
__device__ __forceinline__ Hop weighted_entry(const WalkGraph& g, const u32x4_a8& v,
                                              const EdgeRec& r0, double bs0,
                                              const WPanelSlot* sl, uint32_t pick) {
    if (pick == v.y) return whop_of<Fwd>(r0.nbr, r0.eid, v.w, v.x, bs0);
    if (sl && pick == v.y + 1) return whop_of<Fwd>(sl->rec1.nbr, sl->rec1.eid, sl->nxt1, v.x, sl->bs1);
    const WEdgeRec* p = g.d.wrec + (static_cast<size_t>(pick) << g.d.wrshift);
    const WEdgeRec wr = *p;
    const double bs = g.d.wrshift ? *reinterpret_cast<const double*>(p + 1) : kNoSum;
    return whop_of<Fwd>(wr.nbr, wr.eid, wr.nxt, v.x, bs);
}

// A group's panel record and the next group's start (its end), read as one
// 16-byte load at the record's 8-byte alignment.
struct PanelPair {
    uint32_t rank, start, next_rank, next_start;
};
__device__ __forceinline__ PanelPair load_pair(const PanelRec* p) {
    const u32x4_a8 v = *reinterpret_cast<const u32x4_a8*>(p);
    return PanelPair{v.x, v.y, v.z, v.w};
}

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int64_t i64x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ Sel edge_of(const WalkGraph& g, uint32_t e, long group) {
    return Sel{g.src[e], g.dst[e], static_cast<int32_t>(e), static_cast<int32_t>(group)};
}

// lower_bound over the non-decreasing cumulative weights c(0) .. c(G - 1) of
// one segment, the number of weights below target -- the reference's binary
// search (random/pickers.cuh:84-126) gives the same unique answer.  A
// segment of more than kWGuideMin weights looks the target's key bucket up in
// its guide table (index_layout.h): one 8-byte load brackets the answer in
// [tab[b], tab[b + 1]], usually zero to two weights, which a binary search
// settles.  A target above the segment's total (a rounded-up sum) is above
// every weight.  Decaying: forward weights (the key of 1 - c).
template <bool Decaying, class CAt>
__device__ __forceinline__ uint32_t guided_lower_bound(CAt c, uint32_t G, const uint32_t* gt,
                                                       const WGuide& gd, double target) {
    if (!(target <= gd.total)) return G;
    uint32_t lo = 0, hi = G;
    if (G > kWGuideMin) {
        const u32x2_a4 br =
            *reinterpret_cast<const u32x2_a4*>(gt + wg_bucket(gd.bs, wg_key(target, Decaying)));
        // (the table's entries are local indexes in [0, G]; the clamps keep
        // every probe inside the segment whatever they hold)
        hi = br.y < G ? br.y : G;
        lo = br.x < hi ? br.x : hi;
        // a wide bracket is a run of equal keys (a weight repeated, as a
        // saturated forward sum is): its first weight usually answers
        if (hi - lo > 4 && !(c(lo) < target)) return lo;
    }
    while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        if (c(mid) < target) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}


// A node's weighted panel (or the whole one): record i at p[i << sh]; in a
// wide panel (sh = 1) the slot after each record holds its first entry's
// start sum and its second entry (index_layout.h, WPanelSlot).
struct WPan {
    const WPanelRec* p;
    uint32_t sh;
    __device__ __forceinline__ const WPanelRec& operator[](uint32_t i) const {
        return p[static_cast<size_t>(i) << sh];
    }
    __device__ __forceinline__ const WPanelSlot* slot(uint32_t i) const {
        return sh ? reinterpret_cast<const WPanelSlot*>(p + (static_cast<size_t>(i) << 1) + 1)
                  : nullptr;
    }
    __device__ __forceinline__ double bs0(uint32_t i) const { return sh ? slot(i)->bs0 : kNoSum; }
};

// pick_exponential_weights (random/pickers.cuh:84-126) over the slice
// [vb, ve) of a node's groups (local indexes; f is the node's weighted
// panel), with the slice's sums loaded: the lower_bound over the node's whole
// segment, clamped to the slice, is the slice's lower_bound because the
// segment is non-decreasing.  start_sum >= target puts it before vb (or at
// vb = 0 with start_sum = 0), which the clamp turns into vb: no search.
// Forward weights saturate at their final sum over the late part of a node's
// span, where start_sum == end_sum makes that the common case.
template <bool Fwd>
__device__ __forceinline__ uint32_t node_weight_pick(const WPan& f, uint32_t G,
                                                     const uint32_t* gt, const WGuide& gd,
                                                     uint32_t vb, uint32_t ve, double r,
                                                     double start_sum, double end_sum) {
    const double target = start_sum + r * (end_sum - start_sum);
    if (target <= start_sum) return vb;
    const uint32_t x = guided_lower_bound<Fwd>([&f](uint32_t i) { return f[i].c; }, G, gt, gd, target);
    return x < vb ? vb : (x > ve ? ve : x);
}

// Number of unique timestamps below t: groups at or past this rank have
// timestamps >= t.
__device__ __forceinline__ int32_t rank_lower_bound(const WalkGraph& g, int64_t t) {
    uint32_t lo = 0, hi = g.T;
    while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        if (g.uniq_ts[mid] < t) lo = mid + 1;
        else hi = mid;
    }
    return static_cast<int32_t>(lo);
}

// Unconstrained start (edge_selectors.cuh:177-275 with timestamp == -1).
template <bool Fwd>
__device__ Sel start_edge(const WalkGraph& g, int picker, double rg, double re) {
    if (g.E == 0 || g.T == 0) return no_edge();
    long group;
    if (is_index_picker(picker)) {
        const int idx = pick_index(picker, 0, static_cast<int>(g.T), !Fwd, rg);
        if (idx == -1 || static_cast<uint32_t>(idx) >= g.T) return no_edge();
        group = idx;
    } else {
        if (picker != kExponentialWeight && picker != kTemporalNode2Vec) return no_edge();
        // pick_exponential_weights over [0, T): start_sum 0, end_sum the total
        if (g.T > g.gw_size || g.gwg == nullptr) return no_edge();
        const WGuide gd = *g.gwg;
        const double end_sum = gd.total;
        if (end_sum < 0.0) return no_edge();
        const double target = 0.0 + rg * (end_sum - 0.0);
        const double* gw = g.gw;
        group = target <= 0.0 ? 0
                              : guided_lower_bound<Fwd>([gw](uint32_t i) { return gw[i]; }, g.T,
                                                        g.gwt, gd, target);
        // an index past the last group reads as an empty range in the
        // reference (get_timestamp_group_range_host, edge_selectors.cuh:38-43)
        if (group == -1 || static_cast<uint32_t>(group) >= g.T) return no_edge();
    }
    const uint32_t from = g.tsg_off[group], to = g.tsg_off[group + 1];
    if (from == to) return no_edge();
    const uint32_t e = from + static_cast<uint32_t>(static_cast<int>(re * static_cast<int>(to - from)));
    return edge_of(g, e, group);
}

__device__ __forceinline__ bool adjacent(const WalkGraph& g, int prev, int cand) {
    if (!g.tn2v || g.adj_nodes == 0) return false;
    if (prev < 0 || static_cast<uint32_t>(prev) >= g.adj_nodes) return false;
    if (g.adj_hash) {
        // cand is a stored node id (a record's neighbour), below 2^adj_bits;
        // the set holds each edge's endpoints in increasing order
        if (cand < 0) return false;
        const uint64_t lo = static_cast<uint32_t>(min(prev, cand)),
                       hi = static_cast<uint32_t>(max(prev, cand));
        const uint64_t key = (lo << g.adj_bits) | hi;
        for (uint64_t h = (key * kAdjHashMul) >> g.adj_shift;; h = (h + 1) & g.adj_mask) {
            const uint64_t v = g.adj_hash[h];
            if (v == key) return true;
            if (v == kAdjEmpty) return false;
        }
    }
    if (g.adj_off == nullptr) return false;
    uint32_t lo = g.adj_off[prev];
    const uint32_t end = g.adj_off[prev + 1];
    uint32_t hi = end;
    if (lo >= hi) return false;
    while (lo < hi) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        if (g.adj_nbr[mid] < cand) lo = mid + 1;
        else hi = mid;
    }
    return lo < end && g.adj_nbr[lo] == cand;
}

// The edge of group x of a node's weighted panel f (x < G): a uniform pick re
// within the group's range, (int)(re * size) as edge_selectors.cuh:420-443
// takes it.  The group's record holds its first edge record (and a wide
// panel's slot its second), so a pick of entry 0 (every pick in a group of one
// edge) -- or 1 -- loads no weighted edge record.
template <bool Fwd>
__device__ __forceinline__ Hop weighted_group_hop(const WalkGraph& g, const WPan& f, uint32_t x,
                                                  double re) {
    const u32x4_a8 v = *reinterpret_cast<const u32x4_a8*>(&f[x]);  // rank, start, end, nxt0
    const uint32_t es = v.y, ee = v.z;
    const EdgeRec r0 = f[x].rec0;
    const double bs0 = f.bs0(x);
    if (es >= ee || es >= g.d.idx_size || ee > g.d.idx_size) return no_hop();
    const uint32_t k = static_cast<uint32_t>(static_cast<int>(re * static_cast<int>(ee - es)));
    return weighted_entry<Fwd>(g, v, r0, bs0, f.slot(x), es + k);
}

// graph/temporal_node2vec_helpers.cuh:127-199 over the slice [vb, ve) of a
// node's G groups (local indexes; f is its weighted panel, gt its guide
// table), with the slice's sums loaded.  The candidate node of a proposal is
// its record's neighbour (get_candidate_node, walk_step_helpers.cuh:40-54).
template <bool Fwd>
__device__ Hop tn2v_pick(const WalkGraph& g, int prev, const WPan& f, uint32_t G,
                         const uint32_t* gt, const WGuide& gd, uint32_t vb, uint32_t ve,
                         double start_sum, double end_sum, double rg, double re) {
    if (vb >= ve || prev == -1) return no_hop();
    double bmax = 1.0;
    if (g.inv_p > bmax) bmax = g.inv_p;
    if (g.inv_q > bmax) bmax = g.inv_q;
    const double inv_bmax = 1.0 / bmax;
    // acceptance thresholds beta * inv_bmax of a neighbour of prev (beta = 1)
    // and of another node (beta = 1/q); a draw below both or at or above both
    // is decided without the adjacency lookup
    const double acc_adj = 1.0 * inv_bmax, acc_far = g.inv_q * inv_bmax;
    const double acc_lo = acc_adj < acc_far ? acc_adj : acc_far;
    const double acc_hi = acc_adj < acc_far ? acc_far : acc_adj;
    if (end_sum < start_sum) return no_hop();
    Hop last = no_hop();
    // Retries often repeat the previous one's pick -- a saturated slice
    // (start_sum == end_sum) picks its first group every time -- so the
    // last group's record, edge record and adjacency answer are kept and
    // reused while they still apply: the same values, no reload.
    uint32_t gx = ~0u;
    u32x4_a8 gv{0u, 0u, 0u, 0u};  // the group's rank, start, end, nxt0
    EdgeRec g_r0{0, 0};
    double g_bs0 = 0.0;
    const WPanelSlot* g_sl = nullptr;
    Hop e_hop = no_hop();
    uint32_t e_pick = ~0u;
    int adj_cand = -1;
    bool adj_val = false, adj_known = false;
    for (int retry = 0; retry < kNode2VecMaxRetries; ++retry) {
        const double gr = derive_uniform(rg, re, retry * 3 + 0);
        const double er = derive_uniform(rg, re, retry * 3 + 1);
        const double ar = derive_uniform(rg, re, retry * 3 + 2);
        const uint32_t x = node_weight_pick<Fwd>(f, G, gt, gd, vb, ve, gr, start_sum, end_sum);
        // a pick one past the node's last group is an empty range in the
        // reference (get_node_group_edge_end, walk_step_helpers.cuh:19-38)
        if (x >= G) continue;
        if (x != gx) {
            gv = *reinterpret_cast<const u32x4_a8*>(&f[x]);
            g_r0 = f[x].rec0;
            g_bs0 = f.bs0(x);
            g_sl = f.slot(x);
            gx = x;
        }
        const uint32_t g_es = gv.y, g_ee = gv.z;
        if (g_es >= g_ee || g_es >= g.d.idx_size || g_ee > g.d.idx_size) continue;
        // min((size_t)(er * size), size - 1): temporal_node2vec_helpers.cuh:169-182
        const uint64_t local = static_cast<uint64_t>(er * static_cast<double>(g_ee - g_es));
        const uint32_t pick =
            g_es + static_cast<uint32_t>(local < g_ee - g_es ? local : g_ee - g_es - 1);
        if (pick != e_pick) {
            e_hop = weighted_entry<Fwd>(g, gv, g_r0, g_bs0, g_sl, pick);
            e_pick = pick;
        }
        last = e_hop;
        const int cand = e_hop.nbr;
        bool accept;
        if (cand == prev) {
            accept = ar < g.inv_p * inv_bmax;
        } else if (ar < acc_lo) {
            accept = true;
        } else if (ar >= acc_hi) {
            accept = false;
        } else {
            if (!adj_known || cand != adj_cand) {
                adj_val = adjacent(g, prev, cand);
                adj_cand = cand;
                adj_known = true;
            }
            accept = ar < (adj_val ? acc_adj : acc_far);
        }
        if (accept) return last;
    }
    return last;
}

// ---- node2vec retries decided by the whole wave ------------------------------
// A lane's retries end at its first accepted proposal, 1.7 per hop on average
// at cfg5, but a wave that runs them in step runs as many as its slowest lane
// needs (about 7).  The row-writing kernel instead hands the retries of its
// undecided hops to the whole wave: each round, the lanes whose hops are still
// open are the owners; while more than 32 are, each tries its own next retry;
// with m <= 32 of them, each owner's hop gets 64 / P lanes (P the power of two
// at or above m) that evaluate its next 64 / P retries side by side, and the
// owner takes the first accepted one (or, after the last retry, the last valid
// one) -- the answer of tn2v_pick's loop, which tries the same proposals in
// order.

// What any lane needs to evaluate any retry of one hop (tn2v_pick's state).
struct Tn2vHop {
    const WPanelRec* f;  // the node's weighted panel (WPan's p)
    const uint32_t* gt;  // its guide table
    WGuide gd;
    uint32_t G, vb, ve;
    int prev;
    double start_sum, end_sum, rg, re;
};

// Retry `retry` of hop s (tn2v_pick's loop body): 0 for a proposal that is no
// edge (the loop's `continue`), 1 for an edge it rejects, 2 for an edge it
// accepts; out holds the edge's hop for 1 and 2.
template <bool Fwd>
__device__ __forceinline__ int tn2v_try(const WalkGraph& g, const Tn2vHop& s, int retry,
                                        Hop& out) {
    double bmax = 1.0;
    if (g.inv_p > bmax) bmax = g.inv_p;
    if (g.inv_q > bmax) bmax = g.inv_q;
    const double inv_bmax = 1.0 / bmax;
    const double acc_adj = 1.0 * inv_bmax, acc_far = g.inv_q * inv_bmax;
    const double acc_lo = acc_adj < acc_far ? acc_adj : acc_far;
    const double acc_hi = acc_adj < acc_far ? acc_far : acc_adj;
    const double gr = derive_uniform(s.rg, s.re, retry * 3 + 0);
    const double er = derive_uniform(s.rg, s.re, retry * 3 + 1);
    const double ar = derive_uniform(s.rg, s.re, retry * 3 + 2);
    const WPan f{s.f, g.d.wshift};
    const uint32_t x = node_weight_pick<Fwd>(f, s.G, s.gt, s.gd, s.vb, s.ve, gr, s.start_sum,
                                             s.end_sum);
    if (x >= s.G) return 0;
    const u32x4_a8 v = *reinterpret_cast<const u32x4_a8*>(&f[x]);  // rank, start, end, nxt0
    const uint32_t es = v.y, ee = v.z;
    if (es >= ee || es >= g.d.idx_size || ee > g.d.idx_size) return 0;
    const uint64_t local = static_cast<uint64_t>(er * static_cast<double>(ee - es));
    const uint32_t pick = es + static_cast<uint32_t>(local < ee - es ? local : ee - es - 1);
    out = weighted_entry<Fwd>(g, v, f[x].rec0, f.bs0(x), f.slot(x), pick);
    const int cand = out.nbr;
    bool accept;
    if (cand == s.prev) accept = ar < g.inv_p * inv_bmax;
    else if (ar < acc_lo) accept = true;
    else if (ar >= acc_hi) accept = false;
    else accept = ar < (adjacent(g, s.prev, cand) ? acc_adj : acc_far);
    return accept ? 2 : 1;
}

template <class T>
__device__ __forceinline__ T lane_read(T v, int src) {
    return __shfl(v, src, 64);
}
template <class T>
__device__ __forceinline__ const T* lane_read(const T* v, int src) {
    return reinterpret_cast<const T*>(
        __shfl(static_cast<unsigned long long>(reinterpret_cast<uintptr_t>(v)), src, 64));
}
__device__ __forceinline__ Tn2vHop lane_read(const Tn2vHop& s, int src) {
    Tn2vHop o;
    o.f = lane_read(s.f, src);
    o.gt = lane_read(s.gt, src);
    o.gd.bs = lane_read(static_cast<unsigned long long>(s.gd.bs), src);
    o.gd.total = lane_read(s.gd.total, src);
    o.G = lane_read(s.G, src);
    o.vb = lane_read(s.vb, src);
    o.ve = lane_read(s.ve, src);
    o.prev = lane_read(s.prev, src);
    o.start_sum = lane_read(s.start_sum, src);
    o.end_sum = lane_read(s.end_sum, src);
    o.rg = lane_read(s.rg, src);
    o.re = lane_read(s.re, src);
    return o;
}
__device__ __forceinline__ Hop lane_read(const Hop& h, int src) {
    return Hop{lane_read(h.nbr, src), lane_read(h.r, src), lane_read(h.e, src),
               lane_read(h.nx, src), lane_read(h.bs, src)};
}

// The hops of the lanes with `want` (state s) decided by the whole wave (see
// above); every lane of the (full) wave must call it.  Returns the lane's hop.
template <bool Fwd>
__device__ Hop tn2v_wave(const WalkGraph& g, bool want, const Tn2vHop& s) {
    const int lane = __lane_id();
    Hop res = no_hop(), last = no_hop();
    int base = 0;  // the owner's next retry
    bool open = want;
    for (;;) {
        const uint64_t owners = __ballot(open);
        if (owners == 0) break;
        const int m = __popcll(owners);
        Hop hh = no_hop();
        int st = 0;
        if (m > 32) {
            // as many open hops as lanes to spare: each owner tries its own
            if (open) {
                st = tn2v_try<Fwd>(g, s, base, hh);
                if (st >= 1) last = hh;
                if (st == 2) {
                    res = hh;
                    open = false;
                } else if (++base >= kNode2VecMaxRetries) {
                    res = last;
                    open = false;
                }
            }
            continue;
        }
        // owner i (its rank among the owners) gets the lanes l with
        // l % P == i, P the power of two at or above m: lane l tries its
        // retry base + l / P.  map: lane i holds owner i's lane (each lane
        // pushes its own id, owners to their rank, the rest past m).
        const int lg = 64 - __builtin_clzll(static_cast<unsigned long long>(m - 1) | 1ull) -
                       (m == 1 ? 1 : 0);  // log2 P
        const int h = 64 >> lg;              // lanes per open hop
        const int rank = __popcll(owners & (lane ? ~0ull >> (64 - lane) : 0ull));
        const int map = __builtin_amdgcn_ds_permute((open ? rank : m + lane - rank) << 2, lane);
        const int i = lane & ((1 << lg) - 1), t = lane >> lg;
        const int o = __builtin_amdgcn_ds_bpermute(i << 2, map);
        const Tn2vHop hs = lane_read(s, o);
        const int r = lane_read(base, o) + t;
        if (i < m && r < kNode2VecMaxRetries) st = tn2v_try<Fwd>(g, hs, r, hh);
        const uint64_t acc = __ballot(st == 2), val = __ballot(st >= 1);
        // the owner of rank i reads its tries at lanes i, i + P, ...: the
        // first accepted, else the last valid one
        int src_acc = -1, src_val = -1;
        if (open) {
            for (int k = h - 1; k >= 0; --k) {
                const int b = rank + (k << lg);
                if ((acc >> b) & 1ull) src_acc = b;
                if (src_val < 0 && ((val >> b) & 1ull)) src_val = b;
            }
        }
        const Hop ha = lane_read(hh, src_acc < 0 ? lane : src_acc);
        const Hop hv = lane_read(hh, src_val < 0 ? lane : src_val);
        if (open) {
            if (src_acc >= 0) {
                res = ha;
                open = false;
            } else {
                if (src_val >= 0) last = hv;
                base += h;
                if (base >= kNode2VecMaxRetries) {
                    res = last;
                    open = false;
                }
            }
        }
    }
    return res;
}

// The edge of the picked group gpos of a node whose groups end at ge
// (edge_selectors.cuh:420-443): a uniform pick re within the group's range.
__device__ __forceinline__ Hop hop_from_group(const WalkGraph& g, uint32_t gpos, uint32_t ge,
                                              double re) {
    if (gpos >= ge) return no_hop();
    const PanelPair pp = load_pair(g.d.pan + gpos);
    const uint32_t es = pp.start, ee = pp.next_start;
    if (es >= ee || es >= g.d.idx_size || ee > g.d.idx_size) return no_hop();
    return hop_of(load_rec(g.d.rec + es +
                           static_cast<uint32_t>(static_cast<int>(re * static_cast<int>(ee - es)))),
                  pp.rank);
}

// Per-hop selector (edge_selectors.cuh:277-443).  The reference first checks
// the dense active flag; an inactive node has no entries in either direction,
// so the empty group range below rejects it identically without that load.
// t: rank of the current time, -1 for none (a start, or a current time of
// -1, which the reference also reads as unconstrained); cut: rank bound of
// the walk's cutoff time (groups at or past it are excluded), -1 for none.
//
// The valid slice [vb, ve) of node u's G groups (local indexes), searched in
// its panel f (PanelRec or WPanelRec: the ranks are the same): filter_valid_
// groups_by_timestamp_slice (edge_selectors.cuh:66-120) and the cutoff.  nl:
// the time bound carried from the edge that reached u (the same lower_bound,
// local), searched for when it is not in [0, G].
template <bool Fwd, class Pan>
__device__ __forceinline__ void valid_slice(const uint32_t* tab, const NodeHdr& h, uint32_t u,
                                            int G, const Pan& f, int32_t t, int32_t cut, int& vb,
                                            int& ve, uint32_t nl = kNoNext) {
    vb = 0;
    ve = G;
    if (t != -1) {
        const uint32_t x = static_cast<uint32_t>(t);
        if (nl <= static_cast<uint32_t>(G)) {
            if (Fwd) vb = static_cast<int>(nl);
            else ve = static_cast<int>(nl);
        } else if (Fwd) {
            vb = first_ge(tab, h, u, G, f, x + 1);  // upper_bound
        } else {
            ve = first_ge(tab, h, u, G, f, x);  // lower_bound
        }
    }
    if (cut != -1) {
        // the first group at or past the cutoff, within [vb, ve]
        const int c = first_ge(tab, h, u, G, f, static_cast<uint32_t>(cut));
        ve = c < vb ? vb : (c < ve ? c : ve);
    }
}

// The selection after the header load of node u for the index pickers (the
// index family's kernels): ok is false for a node outside the index (then
// the value of h is ignored).
template <bool Fwd>
__device__ __forceinline__ Hop node_edge_from(const WalkGraph& g, int picker, uint32_t u, bool ok,
                                              const NodeHdr& h, int32_t t, int32_t cut,
                                              double rg, double re, const double* em1) {
    uint32_t Gu = ok ? (h.meta & kHdrGMask) : 0u;
    if (Gu == kHdrGMask) Gu = g.d.hdr[u + 1].gb - h.gb;  // more groups than 24 bits hold
    if (Gu == 0) return no_hop();
    const uint32_t gb = h.gb, ge = gb + Gu;
    const int G = static_cast<int>(Gu);
    int vb, ve;
    valid_slice<Fwd>(g.d.tab, h, u, G, g.d.pan + gb, t, cut, vb, ve);
    if (vb >= ve) return no_hop();
    const int avail = ve - vb;
    const int index = pick_index(picker, 0, avail, !Fwd, rg, em1);
    if (index == -1 || index >= avail) return no_hop();
    return hop_from_group(g, gb + static_cast<uint32_t>(vb + index), ge, re);
}

// The same for any picker, over the weighted view (the weight families'
// kernels): the time search, the slice's sums, the weight search and the
// picked group's range and first edge read the node's weighted panel.
template <bool Fwd, int Fam>
__device__ __forceinline__ Hop wnode_edge_from(const WalkGraph& g, int picker, uint32_t u, bool ok,
                                               const WNodeHdr& wh, int32_t t, int32_t cut,
                                               int prev, double rg, double re,
                                               const double* em1, uint32_t nx, double bs) {
    const NodeHdr& h = wh.h;
    uint32_t Gu = ok ? (h.meta & kHdrGMask) : 0u;
    if (Gu == kHdrGMask) Gu = g.d.whdr[u + 1].h.gb - h.gb;
    if (Gu == 0) return no_hop();
    const uint32_t gb = h.gb;
    const int G = static_cast<int>(Gu);
    const WPan f{g.d.wpan + (static_cast<size_t>(gb) << g.d.wshift), g.d.wshift};
    int vb, ve;
    const uint32_t nl = nx - gb;
    valid_slice<Fwd>(g.d.tab, h, u, G, f, t, cut, vb, ve, nl);
    if (vb >= ve) return no_hop();
    // the slice bound carried from the edge that reached u, and with it (in
    // the ExponentialWeight family's forward kernels, where the build wrote
    // one) the start sum of the slice there (bs)
    const bool csum = Fwd && Fam == kFamWeight && t != -1 && nl <= Gu && !(bs < 0.0);
    uint32_t x;
    if (is_index_picker(picker)) {
        const int avail = ve - vb;
        const int index = pick_index(picker, 0, avail, !Fwd, rg, em1);
        if (index == -1 || index >= avail) return no_hop();
        x = static_cast<uint32_t>(vb + index);
    } else {
        if (picker != kExponentialWeight && picker != kTemporalNode2Vec) return no_hop();
        // the reference's range check: no weights, no pick
        if (gb + Gu > g.d.w_size) return no_hop();
        const uint32_t* gt = g.d.wgt + hdr_tab_base(h, u);
        // the slice's sums: the cumulative weight before vb and at ve - 1
        const double start_sum = !(vb > 0) ? 0.0 : csum ? bs : f[vb - 1].c;
        const double end_sum = ve == G ? wh.g.total : f[ve - 1].c;
        if (Fam != kFamWeight && picker == kTemporalNode2Vec && prev != -1)
            return tn2v_pick<Fwd>(g, prev, f, Gu, gt, wh.g, vb, ve, start_sum, end_sum, rg, re);
        // ExponentialWeight, or node2vec's first hop (no previous node)
        if (end_sum < start_sum) return no_hop();
        x = node_weight_pick<Fwd>(f, Gu, gt, wh.g, static_cast<uint32_t>(vb),
                                  static_cast<uint32_t>(ve), rg, start_sum, end_sum);
        if (x >= Gu) return no_hop();
    }
    return weighted_group_hop<Fwd>(g, f, x, re);
}

// wnode_edge_from in the any-picker row-writing kernel, whose node2vec
// retries the wave decides (tn2v_wave): a node2vec hop from a previous node
// with a non-empty slice returns with `want` set and its retry state in s
// (the checks before tn2v_pick's loop done); any other hop is decided here.
template <bool Fwd>
__device__ __forceinline__ Hop wnode_edge_from_wave(const WalkGraph& g, int picker, uint32_t u,
                                                    bool ok, const WNodeHdr& wh, int32_t t,
                                                    int32_t cut, int prev, double rg, double re,
                                                    const double* em1, uint32_t nx, bool& want,
                                                    Tn2vHop& s) {
    want = false;
    if (picker != kTemporalNode2Vec || prev == -1)
        return wnode_edge_from<Fwd, kFamAny>(g, picker, u, ok, wh, t, cut, prev, rg, re, em1, nx,
                                             kNoSum);
    const NodeHdr& h = wh.h;
    uint32_t Gu = ok ? (h.meta & kHdrGMask) : 0u;
    if (Gu == kHdrGMask) Gu = g.d.whdr[u + 1].h.gb - h.gb;
    if (Gu == 0) return no_hop();
    const uint32_t gb = h.gb;
    const int G = static_cast<int>(Gu);
    const WPan f{g.d.wpan + (static_cast<size_t>(gb) << g.d.wshift), g.d.wshift};
    int vb, ve;
    const uint32_t nl = nx - gb;
    valid_slice<Fwd>(g.d.tab, h, u, G, f, t, cut, vb, ve, nl);
    if (vb >= ve) return no_hop();
    if (gb + Gu > g.d.w_size) return no_hop();
    const double start_sum = vb > 0 ? f[vb - 1].c : 0.0;
    const double end_sum = ve == G ? wh.g.total : f[ve - 1].c;
    if (end_sum < start_sum) return no_hop();
    s = Tn2vHop{f.p, g.d.wgt + hdr_tab_base(h, u), wh.g, Gu, static_cast<uint32_t>(vb),
                static_cast<uint32_t>(ve), prev, start_sum, end_sum, rg, re};
    want = true;
    return no_hop();
}

// The node header a family's kernel loads per hop (issued before the hop's
// draws), and the selection after it.
template <int Fam>
struct HopHdrOf {
    using type = WNodeHdr;
};
template <>
struct HopHdrOf<kFamIndex> {
    using type = NodeHdr;
};
template <int Fam>
using HopHdr = typename HopHdrOf<Fam>::type;

template <int Fam>
__device__ __forceinline__ HopHdr<Fam> load_hop_hdr(const WalkGraph& g, uint32_t u) {
    if constexpr (Fam == kFamIndex) return g.d.hdr[u];
    else return g.d.whdr[u];
}

template <bool Fwd, int Fam>
__device__ __forceinline__ Hop hop_at(const WalkGraph& g, int picker, uint32_t u, bool ok,
                                      const HopHdr<Fam>& hh, int32_t t, int32_t cut, int prev,
                                      double rg, double re, const double* em1,
                                      uint32_t nx = kNoNext, double bs = kNoSum) {
    if constexpr (Fam == kFamIndex) return node_edge_from<Fwd>(g, picker, u, ok, hh, t, cut, rg, re, em1);
    else return wnode_edge_from<Fwd, Fam>(g, picker, u, ok, hh, t, cut, prev, rg, re, em1, nx, bs);
}

template <bool Fwd, int Fam>
__device__ Hop node_edge_at(const WalkGraph& g, int picker, int node, int32_t t, int32_t cut,
                            int prev, double rg, double re, const double* em1 = nullptr) {
    if (!(node >= 0 && node < g.active_size)) return no_hop();
    const uint32_t u = static_cast<uint32_t>(node);
    return hop_at<Fwd, Fam>(g, picker, u, true, load_hop_hdr<Fam>(g, u), t, cut, prev, rg, re, em1);
}

// Rank bound of a walk's cutoff time: groups at or past it are excluded
// (-1: no cutoff).
__device__ __forceinline__ int32_t cutoff_rank(const WalkGraph& g, const WalkArgs& a,
                                               uint64_t w) {
    const int64_t cutoff = a.cutoffs ? a.cutoffs[w] : kNoCutoff;
    return cutoff != kNoCutoff ? rank_lower_bound(g, cutoff) : -1;
}

// Start edge of walk w (temporal_random_walk_cpu.cuh:39-90): the first slot
// holds the walk's origin and `cur` the node reached over the start edge.
template <bool Fwd, bool Dir, int Fam>
__device__ __forceinline__ StartState walk_start(const WalkGraph& g, const WalkArgs& a,
                                                 uint64_t w, int32_t cut) {
    const int start = a.starts ? a.starts[w] : -1;
    const double r0 = draw_slot0(a.ds, w);
    const DrawPair r12 = draw_pair(a.ds, w, 1);
    StartState st{-1, -1, -1, -1};
    if (start == -1) {
        const Sel se = start_edge<Fwd>(g, a.start_bias, r0, r12.a);
        if (se.v != -1) {
            if (Dir) {
                st.first = Fwd ? se.u : se.v;
                st.cur = Fwd ? se.v : se.u;
            } else {
                st.first = r12.b >= 0.5 ? se.u : se.v;
                st.cur = st.first == se.u ? se.v : se.u;
            }
            st.r = se.r;
            st.e = se.e;
        }
    } else {
        // a node's own list: the node is the edge's source (out), target (in)
        // or one endpoint (undirected) -- the record's neighbour is the other
        const Hop h = node_edge_at<Fwd, Fam>(g, a.start_bias, start, -1, cut, -1, r0, r12.a);
        if (h.e != -1) {
            st.first = start;
            st.cur = h.nbr;
            st.r = h.r;
            st.e = h.e;
        }
    }
    return st;
}

// Pre-pass of the walk: every walk's start state, and the key that orders
// walks by the time their first hop starts from (the rank of the start edge's
// time; `none` for walks without a start edge).
template <bool Fwd, bool Dir, int Fam>
__global__ __launch_bounds__(kB) void walk_start_kernel(WalkGraph g, WalkArgs a,
                                                        StartState* __restrict__ st,
                                                        uint32_t* __restrict__ keys,
                                                        uint32_t* __restrict__ vals,
                                                        uint32_t none) {
    const uint64_t w = blockIdx.x * static_cast<uint64_t>(kB) + threadIdx.x;
    if (w >= a.n) return;
    const StartState s0 = walk_start<Fwd, Dir, Fam>(g, a, w, cutoff_rank(g, a, w));
    st[w] = s0;
    keys[w] = s0.e != -1 ? static_cast<uint32_t>(s0.r) : none;
    vals[w] = static_cast<uint32_t>(w);
}

// The same keys for unconstrained starts of an index picker, without the
// start states: start_edge picks timestamp group idx from the walk's first
// draw alone, a group is never empty, and the start edge's time has rank idx.
// The walk kernel then finds the start edge itself (walk_start).
template <bool Fwd>
__global__ __launch_bounds__(kB) void walk_start_keys_kernel(WalkGraph g, WalkArgs a,
                                                             uint32_t* __restrict__ keys,
                                                             uint32_t* __restrict__ vals,
                                                             uint32_t none) {
    const uint64_t w = blockIdx.x * static_cast<uint64_t>(kB) + threadIdx.x;
    if (w >= a.n) return;
    uint32_t key = none;
    if (g.E != 0 && g.T != 0) {
        const int idx = pick_index(a.start_bias, 0, static_cast<int>(g.T), !Fwd, draw_slot0(a.ds, w));
        if (idx != -1 && static_cast<uint32_t>(idx) < g.T) key = static_cast<uint32_t>(idx);
    }
    keys[w] = key;
    vals[w] = static_cast<uint32_t>(w);
}

// Workgroup b runs on XCD b % 8 (round-robin dispatch).  With the remap, XCD
// x runs the x-th contiguous slice of the grid's positions, so the walks
// resident on one XCD -- and sharing its L2 -- are neighbours in the order.
constexpr unsigned kXcds = 8;
__device__ __forceinline__ uint64_t grid_position(int remap) {
    unsigned b = blockIdx.x;
    if (remap) {
        const unsigned nb = gridDim.x, x = b % kXcds, i = b / kXcds;
        const unsigned per = nb / kXcds, extra = nb % kXcds;
        b = x * per + (x < extra ? x : extra) + i;
    }
    return b * static_cast<uint64_t>(kB) + threadIdx.x;
}

// Waves per SIMD: the any-picker instance (node2vec's retry loop) needs
// 146-150 VGPRs, which left it at 3 waves; held to 5 (102 VGPRs) its cfg5
// walks (scratch path) run in 11.1 instead of 13.0 ms per batch (4 waves:
// 11.7 ms; 6: 14.0 ms).  The index family needs 86 (5 waves); held to 6 (80
// VGPRs, 12 bytes of spills) its cfg2 walks run in 9.75 instead of 9.98 ms.
template <bool Fwd, bool Dir, int Fam>
__global__ __launch_bounds__(kB) __attribute__((amdgpu_waves_per_eu(Fam == kFamIndex ? 6 : 5))) void walk_kernel(WalkGraph g, WalkArgs a) {
    // the exponential index picker's thresholds (expm1 of every length it
    // evaluates, exp(-j)), once per workgroup instead of a logarithm per hop
    __shared__ double s_xt[kExpTables];
    const bool use_xt = a.walk_bias == kExponentialIndex;
    if (use_xt) {
        fill_exp_tables(s_xt, threadIdx.x, kB);
        __syncthreads();
    }
    const double* em1 = use_xt ? s_xt : nullptr;
    const uint64_t q = a.q0 + grid_position(a.xcd_remap);
    if (q >= a.q_end) return;
    const uint64_t w = a.order ? a.order[q] : q;
    const int L = a.L;
    if (L == 0) {
        a.lens[w] = 0;
        return;
    }
    // the scratch feeds the layout pass, which produces the row-major output
    // in the reference's types, the padding and the chronological order of
    // backward walks
    SlotWriter out(a, q);
    const int32_t cut = cutoff_rank(g, a, w);
    // the reference's tests of a current time of -1, on ranks
    const int32_t neg1 = *g.neg1_rank;

    // the start state from the pre-pass, or found here
    const StartState s0 = a.st ? a.st[w] : walk_start<Fwd, Dir, Fam>(g, a, w, cut);
    const int first = s0.first;
    int cur = s0.cur;
    int32_t cur_r = s0.r, cur_e = s0.e;
    uint32_t cur_nx = kNoNext;  // the next slice's bound carried by the last edge
    double cur_bs = kNoSum;     // and its bounding sum
    int len = 0;
    if (cur_e != -1) {
        int prev = -1;
        out.first(first);
        len = 1;
        int walk_len = 1;
        while (walk_len < L && cur != a.pad) {
            out.slot(len, cur, static_cast<uint32_t>(cur_r), static_cast<uint32_t>(cur_e));
            ++len;
            // The reference draws and selects once more after the last slot is
            // written; that selection cannot change the output, so it is skipped.
            if (walk_len == L - 1) break;
            // The header load is issued before the hop's Philox draws are
            // computed, in the same basic block, so the rounds run while it
            // is in flight (the empty asm keeps the compiler from sinking them
            // below the load's first use; replay mode computes and discards
            // them).  The walk reached cur over an edge, so the index is not
            // empty and entry 0 is a valid address for a node outside it.
            const bool ok = cur >= 0 && cur < g.active_size;
            const uint32_t u = ok ? static_cast<uint32_t>(cur) : 0u;
            const HopHdr<Fam> hd = load_hop_hdr<Fam>(g, u);
            const uint32_t p = static_cast<uint32_t>(walk_len) + 1;
            DrawPair r = philox_pair(a.ds, w, p);
            asm volatile("" : "+v"(r.a), "+v"(r.b));
            if (a.ds.replay) r = replay_pair(a.ds, w, p);
            const Hop h = hop_at<Fwd, Fam>(g, a.walk_bias, u, ok, hd,
                                                   cur_r == neg1 ? -1 : cur_r, cut, prev, r.a,
                                                   r.b, em1, cur_nx, cur_bs);
            // the reference's failure test is ts == -1: no edge, or an edge at -1
            if (h.e == -1 || h.r == neg1) break;
            prev = cur;
            cur = h.nbr;
            cur_r = h.r;
            cur_e = h.e;
            cur_nx = h.nx;
            cur_bs = h.bs;
            ++walk_len;
        }
    }
    a.lens[w] = static_cast<uint64_t>(len);
}

// ---- walks written as output rows by the walk kernel -----------------------
// Forward walks whose slots pack into 64 bits need no scratch and no layout
// pass: each wave keeps the packed words of its 64 walks' next kRowSlots
// slots in LDS and, every kRowSlots slots, writes them out as segments of the
// walks' output rows in the reference's types (int32 nodes, int64 timestamps
// via uniq_ts, int64 edge ids, padding past a walk's length).  The wave's
// lanes cut those row segments into store units (16 bytes where the rows
// allow), so a store covers whole segments of several rows.  Sixteen slots
// make a timestamp segment one 128-byte line and a node segment half of one
// when L is a multiple of 16; the 8 KB per wave this takes in LDS holds the
// kernel to 4 waves per SIMD.  (8 or 12 slots, with 5 waves per SIMD, left
// partial lines behind every flush and measured slower.)
constexpr int kRowSlots = 16;

// The wave's slot buffer: slot j of lane l at word j * kRowStride + l.  The
// flush reads 4, 8 or 16 consecutive slots of 16, 8 or 4 rows per
// instruction; with a stride of 64 words all slots of a row share a bank (4-,
// 8- and 16-way conflicts), with 68 the 64 lanes' words cover every bank
// twice, the least a 64-bit access needs.  The 4 pad words of each slot row
// hold the row table (RowInfo of lane l at word (l / 4) * kRowStride + 64 +
// l % 4), so the padding costs no LDS.
constexpr int kRowStride = 68;

// A row of the wave's flush: the walk (its output row) and its length, -1
// for a lane without a walk.
struct RowInfo {
    uint32_t w;
    int32_t len;
};
static_assert(sizeof(RowInfo) == sizeof(uint64_t), "a row-table entry is one buffer word");

__device__ __forceinline__ RowInfo* row_info(uint64_t* buf, int l) {
    return reinterpret_cast<RowInfo*>(buf + (l >> 2) * kRowStride + 64 + (l & 3));
}

// Output elements [e0, e0 + ne) of one array (0: nodes, 1: timestamps,
// 2: edge ids) for the 64 rows of the wave, from its slot buffer buf (packed
// words, entry j of lane l holding slot c0 + j of l's walk) and the row table
// in its pad words.  NE > 0 fixes ne at compile time.  Element i of the edge-id row
// is the edge into slot i + 1.  Store units: 16 bytes (4 nodes, 2 timestamps
// or edge ids) when every row's segment is 16-byte aligned, else one element.
// (Aligned 16-byte pairs over the odd-stride edge-id rows, with single
// elements at the ends, measured slower: the pair and single stores of one
// round are separate store instructions.)
template <int Arr, int NE>
__device__ __forceinline__ void rows_out(const WalkArgs& a, uint64_t* buf, int c0, int e0,
                                         int ne_rt, int lane) {
    const int ne = NE > 0 ? NE : ne_rt;
    if (ne <= 0) return;  // uniform
    const int K = Arr == 2 ? a.L - 1 : a.L;
    constexpr int V = Arr == 0 ? 4 : 2;
    const bool vec = K % V == 0 && e0 % V == 0 && ne % V == 0;
    const int S = vec ? V : 1;
    const int U = ne / S;  // store units per row
    const int total = 64 * U;
    const int nb = a.pk_nb, rb = a.pk_rb;
    const int soff = (Arr == 2 ? 1 : 0) - c0;  // buffer entry of element i: i + soff
    // one round at a time: unrolled rounds hold more registers than the 4
    // waves per SIMD the LDS allows (and were not faster unrolled 2, 4 or 8
    // times over the timestamp rounds)
#pragma unroll 1
    for (int t0 = 0; t0 < total; t0 += 64) {
        const int t = t0 + lane;
        const int j = t / U;  // the row: lane j's walk
        const RowInfo ri = *row_info(buf, j);
        if (ri.len < 0) continue;
        const int lj = ri.len;
        const int i0 = e0 + (t - j * U) * S;
        const uint64_t at = static_cast<uint64_t>(ri.w) * static_cast<uint64_t>(K) + i0;
        auto value = [&](int i) -> int64_t {
            const int slot = i + (Arr == 2 ? 1 : 0);
            const uint64_t word = buf[(i + soff) * kRowStride + j];
            if (Arr == 0) return slot < lj ? word_node(word, nb) : a.pad;
            if (Arr == 2) return slot < lj ? word_eid(word, nb, rb) : -1;
            return slot < lj ? word_ts(word, nb, rb, a.uniq_ts, a.edge_ts, a.start_ts) : -1;
        };
        if (vec) {
            if (Arr == 0) {
                const i32x4 o = {static_cast<int32_t>(value(i0)), static_cast<int32_t>(value(i0 + 1)),
                                 static_cast<int32_t>(value(i0 + 2)),
                                 static_cast<int32_t>(value(i0 + 3))};
                __builtin_nontemporal_store(o, reinterpret_cast<i32x4*>(a.on + at));
            } else {
                const i64x2 o = {value(i0), value(i0 + 1)};
                __builtin_nontemporal_store(o, reinterpret_cast<i64x2*>((Arr == 1 ? a.ot : a.oe) + at));
            }
        } else {
            const int64_t y = value(i0);
            if (Arr == 0) __builtin_nontemporal_store(static_cast<int32_t>(y), a.on + at);
            else if (Arr == 1) __builtin_nontemporal_store(y, a.ot + at);
            else __builtin_nontemporal_store(y, a.oe + at);
        }
    }
}

// The timestamp rows of a full chunk (NE slots per row, an even row length,
// 16-byte units of two values) in two phases: rows_ts_fetch looks every value
// up (uniq_ts or edge_ts loads) into tv before the flush stores anything, and
// rows_ts_store writes them last.  One vector-memory counter covers loads and
// stores here, so a lookup issued after a store waits for that store to be
// acknowledged: looked up round by round between the stores, the lookups
// serialised the flush on its stores' acknowledgements.
template <int NE>
__device__ __forceinline__ void rows_ts_fetch(const WalkArgs& a, uint64_t* buf, int c0, int lane,
                                              int64_t (&tv)[NE]) {
    constexpr int U = NE / 2;  // units per row; NE / 2 rounds of 64 units
    const int nb = a.pk_nb, rb = a.pk_rb;
    asm volatile("" : "+v"(lane));
#pragma unroll
    for (int r = 0; r < U; ++r) {
        const int t = r * 64 + lane;
        const int j = t / U;
        const int lj = row_info(buf, j)->len;
        const int s0 = (t - j * U) * 2;  // chunk slot of the unit's first value
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const uint64_t word = buf[(s0 + q) * kRowStride + j];
            tv[2 * r + q] = c0 + s0 + q < lj
                                ? word_ts(word, nb, rb, a.uniq_ts, a.edge_ts, a.start_ts)
                                : -1;
        }
        // round by round: only the values stay live, not every round's words
        // and addresses
        asm volatile("" ::: "memory");
    }
}

template <int NE>
__device__ __forceinline__ void rows_ts_store(const WalkArgs& a, uint64_t* buf, int c0, int lane,
                                              const int64_t (&tv)[NE]) {
    constexpr int U = NE / 2;
    asm volatile("" : "+v"(lane));
#pragma unroll
    for (int r = 0; r < U; ++r) {
        const int t = r * 64 + lane;
        const int j = t / U;
        const RowInfo ri = *row_info(buf, j);
        if (ri.len < 0) continue;
        const uint64_t at = static_cast<uint64_t>(ri.w) * static_cast<uint64_t>(a.L) + c0 +
                            (t - j * U) * 2;
        const i64x2 o = {tv[2 * r], tv[2 * r + 1]};
        __builtin_nontemporal_store(o, reinterpret_cast<i64x2*>(a.ot + at));
    }
}

// Every lane's LDS stores are complete and visible to the whole wave.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Writes slots [c0, c0 + n) of the wave's walks from its slot buffer; n == C
// but for a row's last chunk.
template <int C>
__device__ __forceinline__ void rows_flush(const WalkArgs& a, uint64_t* buf, int c0, int n,
                                           uint32_t w, int len, bool live, int lane) {
    *row_info(buf, lane) = RowInfo{w, live ? len : -1};
    wave_lds_sync();
    const int e0 = c0 > 0 ? c0 - 1 : 0;
    if (n == C && a.L % 2 == 0) {
        int64_t tv[C];
        rows_ts_fetch<C>(a, buf, c0, lane, tv);
        rows_out<0, C>(a, buf, c0, c0, C, lane);
        if (c0 > 0) rows_out<2, C>(a, buf, c0, e0, C, lane);
        else rows_out<2, C - 1>(a, buf, c0, e0, C - 1, lane);
        rows_ts_store<C>(a, buf, c0, lane, tv);
    } else if (n == C) {
        rows_out<0, C>(a, buf, c0, c0, C, lane);
        rows_out<1, C>(a, buf, c0, c0, C, lane);
        if (c0 > 0) rows_out<2, C>(a, buf, c0, e0, C, lane);
        else rows_out<2, C - 1>(a, buf, c0, e0, C - 1, lane);
    } else {
        rows_out<0, 0>(a, buf, c0, c0, n, lane);
        rows_out<1, 0>(a, buf, c0, c0, n, lane);
        rows_out<2, 0>(a, buf, c0, e0, c0 + n - 1 - e0, lane);
    }
    // every lane's reads of the buffer precede the next chunk's stores
    wave_lds_sync();
}

// walk_kernel's walks, forward, written as output rows (above) instead of
// scratch.  The loop runs in chunks of C slots over the whole row for every
// lane (wave-uniform), so every row is written to its end, the padding
// included; a lane whose walk has ended (or that has no walk) only fills.
//
// At least 4 waves per SIMD, as many as the slot buffers' LDS allows: the
// index family needs 109 VGPRs, but the any-picker instance (node2vec's
// retries) took 155 and ran at 3 waves; held to 128 its cfg5 walks ran in
// 12.7 instead of 15.4 ms per batch.  That instance hands node2vec's retries
// to the whole wave (tn2v_wave; 128 VGPRs, 44 bytes of spills).
template <bool Fwd, bool Dir, int Fam, int C>
__global__ __launch_bounds__(kB) __attribute__((amdgpu_waves_per_eu(4))) void walk_rows_kernel(WalkGraph g, WalkArgs a) {
    static_assert(Fwd, "backward walks are reversed by the layout pass");
    __shared__ double s_xt[kExpTables];
    __shared__ uint64_t s_slots[(kB / 64) * C * kRowStride];
    static_assert(C >= 16, "the row table lives in the pad words of 16 slot rows");
    const bool use_xt = a.walk_bias == kExponentialIndex;
    if (use_xt) {
        fill_exp_tables(s_xt, threadIdx.x, kB);
        __syncthreads();
    }
    const double* em1 = use_xt ? s_xt : nullptr;
    const int lane = __lane_id();
    uint64_t* buf = s_slots + (threadIdx.x >> 6) * C * kRowStride;
    const uint64_t q = a.q0 + grid_position(a.xcd_remap);
    const bool live = q < a.q_end;
    const uint64_t w = live ? (a.order ? a.order[q] : q) : 0;
    const int L = a.L;  // >= 1 (the host launches it only then)
    const int32_t cut = live ? cutoff_rank(g, a, w) : -1;
    const int32_t neg1 = *g.neg1_rank;
    // the start state from the pre-pass, or found here
    const StartState s0 = !live ? StartState{-1, -1, -1, -1}
                                : (a.st ? a.st[w] : walk_start<Fwd, Dir, Fam>(g, a, w, cut));
    int cur = s0.cur, prev = -1;
    int32_t cur_r = s0.r, cur_e = s0.e;
    uint32_t cur_nx = kNoNext;  // the next slice's bound carried by the last edge
    double cur_bs = kNoSum;     // and its bounding sum
    bool alive = live && s0.e != -1;  // the walk writes its next slot
    int len = 0;
    const int nb = a.pk_nb, rb = a.pk_rb;
    for (int c0 = 0; c0 < L; c0 += C) {
        const int n = min(C, L - c0);
        if constexpr (Fam == kFamAny) {
            // the same slots; node2vec's retries are decided by the whole
            // wave after every lane has prepared its hop
            for (int j = 0; j < n; ++j) {
                const int k = c0 + j;
                bool stepping = false, want = false;
                Hop h = no_hop();
                Tn2vHop ts{};
                if (alive) {
                    uint64_t word;
                    if (k == 0) {
                        word = first_word(nb, s0.first);
                        len = 1;
                        alive = L > 1 && cur != a.pad;
                    } else {
                        word = slot_word(nb, rb, cur, static_cast<uint32_t>(cur_r),
                                         static_cast<uint32_t>(cur_e));
                        len = k + 1;
                        if (k == L - 1) {
                            alive = false;
                        } else {
                            const bool ok = cur >= 0 && cur < g.active_size;
                            const uint32_t u = ok ? static_cast<uint32_t>(cur) : 0u;
                            const WNodeHdr hd = load_hop_hdr<Fam>(g, u);
                            const uint32_t p = static_cast<uint32_t>(k) + 1;
                            DrawPair r = philox_pair(a.ds, w, p);
                            asm volatile("" : "+v"(r.a), "+v"(r.b));
                            if (a.ds.replay) r = replay_pair(a.ds, w, p);
                            h = wnode_edge_from_wave<Fwd>(g, a.walk_bias, u, ok, hd,
                                                          cur_r == neg1 ? -1 : cur_r, cut, prev,
                                                          r.a, r.b, em1, cur_nx, want, ts);
                            stepping = true;
                        }
                    }
                    buf[j * kRowStride + lane] = word;
                }
                if (__ballot(want)) {
                    const Hop hw = tn2v_wave<Fwd>(g, want, ts);
                    if (want) h = hw;
                }
                if (stepping) {
                    if (h.e == -1 || h.r == neg1) {
                        alive = false;
                    } else {
                        prev = cur;
                        cur = h.nbr;
                        cur_r = h.r;
                        cur_e = h.e;
                        cur_nx = h.nx;
                        cur_bs = h.bs;
                        alive = cur != a.pad;
                    }
                }
            }
            rows_flush<C>(a, buf, c0, n, static_cast<uint32_t>(w), len, live, lane);
            continue;
        }
        for (int j = 0; j < n; ++j) {
            if (!alive) continue;
            const int k = c0 + j;
            uint64_t word;
            if (k == 0) {
                word = first_word(nb, s0.first);
                len = 1;
                alive = L > 1 && cur != a.pad;
            } else {
                word = slot_word(nb, rb, cur, static_cast<uint32_t>(cur_r),
                                 static_cast<uint32_t>(cur_e));
                len = k + 1;
                if (k == L - 1) {
                    alive = false;  // the reference's last selection cannot change the output
                } else {
                    // as in walk_kernel: the header load goes out before the
                    // hop's Philox rounds
                    const bool ok = cur >= 0 && cur < g.active_size;
                    const uint32_t u = ok ? static_cast<uint32_t>(cur) : 0u;
                    const HopHdr<Fam> hd = load_hop_hdr<Fam>(g, u);
                    const uint32_t p = static_cast<uint32_t>(k) + 1;
                    DrawPair r = philox_pair(a.ds, w, p);
                    asm volatile("" : "+v"(r.a), "+v"(r.b));
                    if (a.ds.replay) r = replay_pair(a.ds, w, p);
                    const Hop h = hop_at<Fwd, Fam>(g, a.walk_bias, u, ok, hd,
                                                           cur_r == neg1 ? -1 : cur_r, cut, prev,
                                                           r.a, r.b, em1, cur_nx, cur_bs);
                    if (h.e == -1 || h.r == neg1) {
                        alive = false;
                    } else {
                        prev = cur;
                        cur = h.nbr;
                        cur_r = h.r;
                        cur_e = h.e;
                        cur_nx = h.nx;
                        cur_bs = h.bs;
                        alive = cur != a.pad;
                    }
                }
            }
            buf[j * kRowStride + lane] = word;
        }
        rows_flush<C>(a, buf, c0, n, static_cast<uint32_t>(w), len, live, lane);
    }
    if (live) a.lens[w] = static_cast<uint64_t>(len);
}

// The row-writing walk kernel of a picker family, forward.
void launch_rows(bool directed, int fam, dim3 grid, hipStream_t s, const WalkGraph& g,
                 const WalkArgs& a) {
    constexpr int C = kRowSlots;
#define TRW_ROWS(D, F) hipLaunchKernelGGL((walk_rows_kernel<true, D, F, C>), grid, dim3(kB), 0, s, g, a)
#define TRW_ROWS_FAM(D)                                      \
    do {                                                     \
        if (fam == kFamIndex) TRW_ROWS(D, kFamIndex);        \
        else if (fam == kFamWeight) TRW_ROWS(D, kFamWeight); \
        else TRW_ROWS(D, kFamAny);                           \
    } while (0)
    if (directed) TRW_ROWS_FAM(true);
    else TRW_ROWS_FAM(false);
#undef TRW_ROWS_FAM
#undef TRW_ROWS
}

// ---- node-grouped processing (TRW_ORDER_NODE_GROUPED) ----------------------
// The north star's cooperative alternative to start-time order: every
// kNodeGroupHops hops the live walks are regrouped by their current node (a
// device radix sort of (node, walk)), so the lanes of a wave -- and the
// waves of an XCD -- select their next hops at the same nodes and share the
// header, bucket-table and panel lines.  A walk's state lives in HBM between
// segments; its scratch column is its walk id (its place changes from one
// segment to the next).  Each walk runs exactly the hops of walk_kernel's
// loop with the same draws, so the walks are the same.
constexpr int kNodeGroupHops = 8;

// A walk between segments: at the top of walk_kernel's loop with c slots
// written (c == the loop's walk_len == len).
struct WalkCarry {
    int32_t cur, r, e, prev;
    int32_t c, cut, pad0, pad1;
};
static_assert(sizeof(WalkCarry) == 32, "WalkCarry must be 32 bytes");

// Appends the workgroup's live walks (keep) as (current node, walk) to the
// next segment's list: one atomic per workgroup.  (Keys of node and time rank,
// so that the walks at one node also ran in time order, cut the L1 -> L2
// reads per step from 2.07 to 1.58 but took the walk phase from 44 to 48 ms
// at cfg2: four sort passes per segment instead of two.)
__device__ __forceinline__ void emit_live(bool keep, uint32_t node, uint32_t w,
                                          uint32_t* __restrict__ keys,
                                          uint32_t* __restrict__ vals,
                                          uint32_t* __restrict__ count) {
    __shared__ uint32_t s_wave[kB / 64];
    __shared__ uint32_t s_base;
    const uint64_t m = __ballot(keep);
    const int lane = __lane_id(), wave = threadIdx.x >> 6;
    const uint32_t below = static_cast<uint32_t>(__popcll(m & ((1ull << lane) - 1ull)));
    if (lane == 0) s_wave[wave] = static_cast<uint32_t>(__popcll(m));
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0;
        for (int q = 0; q < kB / 64; ++q) {
            const uint32_t c = s_wave[q];
            s_wave[q] = t;
            t += c;
        }
        s_base = t ? atomicAdd(count, t) : 0u;
    }
    __syncthreads();
    if (keep) {
        const uint32_t pos = s_base + s_wave[wave] + below;
        keys[pos] = node;
        vals[pos] = w;
    }
}

// Segment 0: every walk's first slot from its start state; the walks that go
// on enter the first list.
template <bool Fwd, bool Dir, int Fam>
__global__ __launch_bounds__(kB) void node_group_init_kernel(WalkGraph g, WalkArgs a,
                                                             WalkCarry* __restrict__ carry,
                                                             uint32_t* __restrict__ keys,
                                                             uint32_t* __restrict__ vals,
                                                             uint32_t* __restrict__ count) {
    const uint64_t w = blockIdx.x * static_cast<uint64_t>(kB) + threadIdx.x;
    bool keep = false;
    int32_t cur = 0;
    if (w < a.n) {
        const StartState s0 = a.st[w];
        if (s0.e == -1) {
            a.lens[w] = 0;
        } else {
            SlotWriter out(a, w);
            out.first(s0.first);
            keep = 1 < a.L && s0.cur != a.pad;
            if (keep) {
                cur = s0.cur;
                carry[w] = WalkCarry{s0.cur, s0.r, s0.e, -1, 1, cutoff_rank(g, a, w), 0, 0};
            } else {
                a.lens[w] = 1;
            }
        }
    }
    emit_live(keep, static_cast<uint32_t>(cur), static_cast<uint32_t>(w), keys, vals, count);
}

// One segment: the walks of the list (sorted by current node), up to
// kNodeGroupHops iterations of walk_kernel's loop each; the walks that go on
// enter the next list.  n: the list's length.
template <bool Fwd, bool Dir, int Fam>
__global__ __launch_bounds__(kB) void node_group_segment_kernel(
    WalkGraph g, WalkArgs a, const uint32_t* __restrict__ list, uint32_t n,
    WalkCarry* __restrict__ carry, uint32_t* __restrict__ keys, uint32_t* __restrict__ vals,
    uint32_t* __restrict__ count) {
    __shared__ double s_xt[kExpTables];
    const bool use_xt = a.walk_bias == kExponentialIndex;
    if (use_xt) {
        fill_exp_tables(s_xt, threadIdx.x, kB);
        __syncthreads();
    }
    const double* em1 = use_xt ? s_xt : nullptr;
    const uint32_t i = blockIdx.x * kB + threadIdx.x;
    bool keep = false;
    uint32_t w = 0;
    WalkCarry s{};
    if (i < n) {
        w = list[i];
        s = carry[w];
        const int L = a.L;
        const int32_t neg1 = *g.neg1_rank;
        SlotWriter out(a, w);
        keep = true;
        for (int it = 0; it < kNodeGroupHops; ++it) {
            out.slot(s.c, s.cur, static_cast<uint32_t>(s.r), static_cast<uint32_t>(s.e));
            ++s.c;
            if (s.c == L) {  // the last slot: the reference's final selection is unused
                keep = false;
                break;
            }
            const bool ok = s.cur >= 0 && s.cur < g.active_size;
            const uint32_t u = ok ? static_cast<uint32_t>(s.cur) : 0u;
            const HopHdr<Fam> hd = load_hop_hdr<Fam>(g, u);
            const DrawPair r = draw_pair(a.ds, w, static_cast<uint32_t>(s.c));
            const Hop h = hop_at<Fwd, Fam>(g, a.walk_bias, u, ok, hd,
                                                   s.r == neg1 ? -1 : s.r, s.cut, s.prev, r.a,
                                                   r.b, em1);
            if (h.e == -1 || h.r == neg1) {
                keep = false;
                break;
            }
            s.prev = s.cur;
            s.cur = h.nbr;
            s.r = h.r;
            s.e = h.e;
            if (s.cur == a.pad) {
                keep = false;
                break;
            }
        }
        if (keep) carry[w] = s;
        else a.lens[w] = static_cast<uint64_t>(s.c);
    }
    emit_live(keep, static_cast<uint32_t>(s.cur), w, keys, vals, count);
}

// Layout pass: slot-major scratch [L][n] -> the row-major output arrays the
// reference returns ([n][L] nodes and timestamps, [n][L - 1] edge ids), in
// one pass.  Values become the reference's types on the way: nodes are
// copied, a slot's time becomes its timestamp (word_ts), a 32-bit edge id is
// widened.  `count` of walk w is its number of written slots (len for nodes
// and timestamps, len - 1 for edge ids); slots at or beyond it get the
// padding (data/walk_set/walk_set_host.cu:25-29).  Backward walks come out
// reversed into chronological order (data/walk_set/walk_set_view.cuh:50-80).
//
// A workgroup owns 64 consecutive scratch columns and a chunk of slots -- the
// whole row when L <= kLayoutPackedMaxSlots.  The scratch is read once, in
// 64-column runs of one slot (512 B, coalesced), into an LDS tile of 64-bit
// words from which the three arrays are written.  Each wave then writes whole
// rows, converting as it writes (a walk's ranks increase along its row, so
// the timestamp lookups of one row are close together).  Column q holds walk
// order[q] when the walks ran in another order than their ids; its row goes
// to that walk's place.  In walk-id order the 64 rows are one contiguous span
// of the output, so no cache line is shared with another workgroup.  Scratch
// is read and output written once, with non-temporal hints.
constexpr int kLayoutWalks = 64;
static_assert(kLayoutWalks == kScratchTile, "a layout workgroup owns one scratch tile");
// 64-bit tile <= 64 KB of LDS.  A row split into chunks costs more than the
// occupancy a smaller tile buys: 80-slot rows in two chunks of 40 were
// measured 1.3 ms slower over 10M walks than in one.
constexpr int kLayoutPackedMaxSlots = 120;

struct LayoutArgs {
    const uint64_t* sp;  // scratch slot words
    int pk_nb, pk_rb;    // their node and rank field widths
    int32_t* on;
    int64_t* ot;
    int64_t* oe;
    const uint64_t* lens;
    int L;
    int C;  // slots per chunk
    int reverse;
    int32_t pad;
    const int64_t* uniq_ts;
    const int64_t* edge_ts;
    int64_t start_ts;
    const uint32_t* order;  // walk of each scratch column (nullptr: the column index)
    uint64_t q0, q_end;     // scratch columns [q0, q_end) of this launch (q0 % 64 == 0)
    // edge features of the edge-id slots (fv = feature_dim / 4 vectors per
    // slot; 0: written by a separate gather)
    const float* feat;
    float* of;
    uint32_t fv;
};

// Value of output slot i of a row whose first `cw` slots were written (v: the
// slot word of the slot the value comes from).  Arr 0: nodes, 1: timestamps,
// 2: edge ids.
template <int Arr>
__device__ __forceinline__ int64_t layout_value(const LayoutArgs& a, uint64_t v, int i, int cw) {
    if (Arr == 0) return i < cw ? word_node(v, a.pk_nb) : a.pad;
    if (Arr == 1)
        return i < cw ? word_ts(v, a.pk_nb, a.pk_rb, a.uniq_ts, a.edge_ts, a.start_ts) : -1;
    return i < cw ? word_eid(v, a.pk_nb, a.pk_rb) : -1;
}

// Writes the chunk's output rows of one array: each wave owns whole rows and
// converts values as it writes them.  word_at(wl2, n, cw, i) is the slot word
// output slot i of tile column wl2 comes from, whose walk wrote n node slots
// and has cw slots of this array's chunk below its count.
template <int Arr, class Src>
__device__ __forceinline__ void layout_rows(const LayoutArgs& a, const int* cnt, const uint32_t* row,
                                            uint64_t w0, int k0, Src word_at) {
    const int K = Arr == 2 ? a.L - 1 : a.L;
    const int kc = min(a.C, K - k0);
    if (kc <= 0) return;  // uniform over the workgroup
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    // 16-byte stores (4 nodes or 2 timestamps / edge ids per lane) when every
    // row chunk starts on a 16-byte boundary and holds whole vectors
    constexpr int V = Arr == 0 ? 4 : 2;
    const bool vec = (K % V) == 0 && (k0 % V) == 0 && (kc % V) == 0;
    // The wave's 16 rows (columns wave, wave + 4, ...) are cut into store
    // units (a vector or one value) and the wave's lanes take consecutive
    // units, so a row shorter than 64 units shares a store instruction with
    // the next row instead of leaving lanes idle.
    const int S = vec ? V : 1;
    const int U = kc / S;  // units per row
    constexpr int kRows = kLayoutWalks / 4;
    for (int t = lane; t < kRows * U; t += 64) {
        const int j = t / U;
        const int i = (t - j * U) * S;
        const int wl2 = wave + 4 * j;
        if (w0 + wl2 >= a.q_end) continue;
        const uint64_t base = static_cast<uint64_t>(row[wl2]) * static_cast<uint64_t>(K) + k0;
        const int n = cnt[wl2];
        const int cw = n - (Arr == 2 ? 1 : 0) - k0;  // slots of the row below the count
        auto val = [&](int x) { return layout_value<Arr>(a, word_at(wl2, n, cw, x), x, cw); };
        if (vec) {
            if (Arr == 0) {
                const i32x4 o = {static_cast<int32_t>(val(i)), static_cast<int32_t>(val(i + 1)),
                                 static_cast<int32_t>(val(i + 2)), static_cast<int32_t>(val(i + 3))};
                __builtin_nontemporal_store(o, reinterpret_cast<i32x4*>(a.on + base + i));
            } else {
                const i64x2 o = {val(i), val(i + 1)};
                int64_t* out = Arr == 1 ? a.ot : a.oe;
                __builtin_nontemporal_store(o, reinterpret_cast<i64x2*>(out + base + i));
            }
        } else {
            const int64_t y = val(i);
            if (Arr == 0) __builtin_nontemporal_store(static_cast<int32_t>(y), a.on + base + i);
            else if (Arr == 1) __builtin_nontemporal_store(y, a.ot + base + i);
            else __builtin_nontemporal_store(y, a.oe + base + i);
        }
    }
    if (Arr != 2 || !a.fv) return;
    for (int wl2 = wave; wl2 < kLayoutWalks; wl2 += 4) {
        if (w0 + wl2 >= a.q_end) break;
        const uint64_t base = static_cast<uint64_t>(row[wl2]) * static_cast<uint64_t>(K) + k0;
        const int n = cnt[wl2];
        const int cw = n - 1 - k0;
        // the slots' edge features (finalize_host_walks,
        // walks_with_edge_features_host.cuh:44-62), from the edge ids in
        // the tile: row [slot][dim] of the walk, zeros past the count
        const uint32_t fv = a.fv;
        const f32x4* feat = reinterpret_cast<const f32x4*>(a.feat);
        f32x4* of = reinterpret_cast<f32x4*>(a.of) + base * fv;
        const uint32_t units = static_cast<uint32_t>(kc) * fv;
        for (uint32_t t = lane; t < units; t += 64) {
            const int i = static_cast<int>(t / fv);
            const uint32_t c = t - static_cast<uint32_t>(i) * fv;
            f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
            if (i < cw) {
                const uint64_t e = static_cast<uint64_t>(word_eid(word_at(wl2, n, cw, i), a.pk_nb, a.pk_rb));
                v = __builtin_nontemporal_load(feat + e * fv + c);
            }
            __builtin_nontemporal_store(v, of + t);
        }
    }
}

// Loads the walk count and destination row of the workgroup's 64 columns.
__device__ __forceinline__ void layout_columns(const LayoutArgs& a, uint64_t w0, int* cnt, uint32_t* row) {
    if (threadIdx.x < kLayoutWalks) {
        const uint64_t q = w0 + threadIdx.x;
        const uint64_t w = q < a.q_end ? (a.order ? a.order[q] : q) : 0;
        row[threadIdx.x] = static_cast<uint32_t>(w);
        cnt[threadIdx.x] = q < a.q_end ? static_cast<int>(a.lens[w]) : 0;
    }
    __syncthreads();
}

// The chunk's words are read once into an LDS tile of 64-bit words and all
// three arrays are written from it.  Tile row r holds slot k0 + r (slot
// n - 1 - (k0 + r) for the reversed rows of a walk laid out in several
// chunks), plus, for forward rows, slot k0 + kc: the edge id of output slot i
// is in slot i + 1, the slot the edge reached; reversed rows find it in the
// same word as their node.
__global__ __launch_bounds__(256) void layout_packed_kernel(LayoutArgs a) {
    constexpr int P = kLayoutWalks + 1;
    extern __shared__ uint64_t layout_lds64[];
    uint64_t* tile = layout_lds64;
    int* cnt = reinterpret_cast<int*>(tile + (a.C + 1) * P);
    uint32_t* row = reinterpret_cast<uint32_t*>(cnt + kLayoutWalks);
    const uint64_t w0 = a.q0 + static_cast<uint64_t>(blockIdx.x) * kLayoutWalks;
    const int k0 = blockIdx.y * a.C;
    layout_columns(a, w0, cnt, row);
    const int kc = min(a.C, a.L - k0);
    const bool whole = k0 == 0 && kc == a.L;
    const bool rev_in = a.reverse && !whole;
    const int rows = min(kc + 1, a.L - k0);
    const int wl = threadIdx.x & 63, srow = threadIdx.x >> 6;
    const int c = cnt[wl];
    const bool live = w0 + wl < a.q_end;
    const uint64_t* in = a.sp + w0 * static_cast<uint64_t>(a.L);  // w0 % kScratchTile == 0
    for (int j0 = 0; j0 < rows; j0 += 32) {
        uint64_t v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int r = j0 + srow + 4 * j;
            const int k = k0 + r;
            uint64_t x = 0;
            if (r < rows && live && k < c)
                x = __builtin_nontemporal_load(in + static_cast<uint64_t>(rev_in ? c - 1 - k : k) * kScratchTile + wl);
            v[j] = x;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int r = j0 + srow + 4 * j;
            if (r < rows) tile[r * P + wl] = v[j];
        }
    }
    __syncthreads();
    const bool rev_out = a.reverse && whole;
    // node and timestamp of output slot i: tile row i (reversed whole rows: n - 1 - i)
    auto node_row = [&](int n, int cw, int i) { return rev_out && i < cw ? n - 1 - i : i; };
    layout_rows<0>(a, cnt, row, w0, k0, [&](int wl2, int n, int cw, int i) {
        return tile[node_row(n, cw, i) * P + wl2];
    });
    layout_rows<1>(a, cnt, row, w0, k0, [&](int wl2, int n, int cw, int i) {
        return tile[node_row(n, cw, i) * P + wl2];
    });
    layout_rows<2>(a, cnt, row, w0, k0, [&](int wl2, int n, int cw, int i) {
        const int r = a.reverse ? node_row(n, cw, i) : i + 1;
        return tile[r * P + wl2];
    });
}

// ---- start arrays ----------------------------------------------------------
__global__ void flags_from_u8_kernel(const uint8_t* __restrict__ a, size_t n,
                                     uint32_t* __restrict__ f) {
    const size_t i = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (i < n) f[i] = a[i] ? 1u : 0u;
}

__global__ void compact_ids_kernel(const uint32_t* __restrict__ f, const uint32_t* __restrict__ scan,
                                   size_t n, int32_t* __restrict__ out) {
    const size_t i = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (i < n && f[i]) out[scan[i]] = static_cast<int32_t>(i);
}

__global__ void unique_flags_kernel(const uint32_t* __restrict__ k, size_t n,
                                    uint32_t* __restrict__ f) {
    const size_t i = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (i < n) f[i] = (i == 0 || k[i] != k[i - 1]) ? 1u : 0u;
}

__global__ void compact_keys_kernel(const uint32_t* __restrict__ k, const uint32_t* __restrict__ f,
                                    const uint32_t* __restrict__ scan, size_t n,
                                    int32_t* __restrict__ out) {
    const size_t i = blockIdx.x * static_cast<size_t>(kB) + threadIdx.x;
    if (i < n && f[i]) out[scan[i]] = static_cast<int32_t>(k[i]);
}

template <typename T>
__global__ void repeat_kernel(const T* __restrict__ in, uint64_t n_out, int times,
                              T* __restrict__ out) {
    const uint64_t i = blockIdx.x * static_cast<uint64_t>(kB) + threadIdx.x;
    if (i < n_out) out[i] = in[i / times];
}

__global__ void random_keys_kernel(uint64_t n, uint32_t k0, uint32_t k1, uint32_t* __restrict__ keys,
                                   uint32_t* __restrict__ vals) {
    const uint64_t i = blockIdx.x * static_cast<uint64_t>(kB) + threadIdx.x;
    if (i >= n) return;
    const U4 o = philox4x32_10(U4{static_cast<uint32_t>(i), static_cast<uint32_t>(i >> 32),
                                  0x5348u /* shuffle stream */, 0u},
                               k0, k1);
    keys[i] = o.x;
    vals[i] = static_cast<uint32_t>(i);
}

template <typename T>
__global__ void permute_kernel(const T* __restrict__ in, const uint32_t* __restrict__ perm,
                               uint64_t n, T* __restrict__ out) {
    const uint64_t i = blockIdx.x * static_cast<uint64_t>(kB) + threadIdx.x;
    if (i < n) out[i] = in[perm[i]];
}

__global__ void u32_from_i32_kernel(const int32_t* __restrict__ a, uint64_t n,
                                    uint32_t* __restrict__ out) {
    const uint64_t i = blockIdx.x * static_cast<uint64_t>(kB) + threadIdx.x;
    if (i < n) out[i] = static_cast<uint32_t>(a[i]);
}

// ---- outputs ----------------------------------------------------------------
// Grid-stride: slots * dim reaches 1.6e10 at configs[2], beyond the 32-bit
// work-item count of one dispatch.
__global__ void gather_walk_features_kernel(const int64_t* __restrict__ eids, uint64_t slots,
                                            uint32_t dim, const float* __restrict__ feat,
                                            float* __restrict__ out) {
    const uint64_t total = slots * dim;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kB;
    for (uint64_t x = blockIdx.x * static_cast<uint64_t>(kB) + threadIdx.x; x < total;
         x += stride) {
        const uint64_t slot = x / dim, c = x - slot * dim;
        const int64_t e = eids[slot];
        out[x] = e >= 0 ? feat[static_cast<uint64_t>(e) * dim + c] : 0.0f;
    }
}

// Blocks for a grid-stride launch over n items (at most 2^20 blocks).
inline unsigned grid_capped(uint64_t n) {
    const uint64_t g = (n + kB - 1) / kB;
    return static_cast<unsigned>(g == 0 ? 1 : (g > (1u << 20) ? (1u << 20) : g));
}

// Walk statistics and demand bytes of the walk path (trw_get_walk_stats):
// acc[3] with this engine's 4-byte positions and ranks, acc[4] with the
// reference's element types.  Workgroup b covers the walks [b * wpb,
// (b + 1) * wpb) and its threads take their slots in row order (coalesced
// node loads, independent from one slot to the next); the workgroup's sums
// meet in LDS and leave with one atomic per counter (one per wave contended
// for the same five addresses across all waves and ran the kernel slower than
// the walks themselves).
__global__ __launch_bounds__(kB) void walk_stats_kernel(const int32_t* __restrict__ nodes,
                                                        const uint64_t* __restrict__ lens,
                                                        uint64_t n, int L, uint64_t wpb,
                                                        const uint32_t* __restrict__ cnt,
                                                        int32_t active_size, int constrained,
                                                        unsigned long long* acc) {
    __shared__ unsigned long long red[5][kB / 64];
    unsigned long long v[5] = {0, 0, 0, 0, 0};  // total, trans, nonempty, bytes, ref
    const uint64_t w0 = blockIdx.x * wpb;
    const uint64_t w1 = w0 + wpb < n ? w0 + wpb : n;
    if (w0 < w1) {
        const uint32_t Lu = static_cast<uint32_t>(L);
        const uint32_t slots = static_cast<uint32_t>(w1 - w0) * Lu;  // < 2^32 (host)
        for (uint32_t off = threadIdx.x; off < slots; off += kB) {
            const uint32_t dw = off / Lu, k = off - dw * Lu;
            const uint64_t w = w0 + dw;
            const int len = static_cast<int>(lens[w]);
            if (k == 0) {
                v[0] += len;
                v[1] += len > 0 ? len - 1 : 0;
                v[2] += len > 0;
                v[3] += 24 + (len >= 1 ? 8 : 0) + (len >= 2 ? 12 : 0);
                v[4] += 8 + (constrained ? 52 : 32) + (len >= 1 ? 12 : 0) + (len >= 2 ? 20 : 0);
            }
            // hops are selected at slots 1 .. len - 2
            if (k >= 1 && static_cast<int>(k) + 1 < len) {
                const int u = nodes[w * L + k];
                uint32_t G = 0;
                if (u >= 0 && u < active_size) G = cnt[u + 1] - cnt[u];
                const int probes = G ? 32 - __clz(G) : 0;  // ceil(log2(G + 1))
                v[3] += 36 + 4 * probes;
                v[4] += 72 + 8 * probes;
            }
        }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int c = 0; c < 5; ++c) {
        for (int o = 32; o > 0; o >>= 1) v[c] += __shfl_down(v[c], o, 64);
        if (lane == 0) red[c][wave] = v[c];
    }
    __syncthreads();
    if (threadIdx.x < 5) {
        unsigned long long t = 0;
        for (int q = 0; q < kB / 64; ++q) t += red[threadIdx.x][q];
        atomicAdd(acc + threadIdx.x, t);
    }
}

}  // namespace

// ---- fixed scratch of the no-allocation entry point -------------------------
// trw_sample_device_noalloc takes every per-call buffer of a sample from this
// array instead of allocating.  Each device the library runs on holds its own
// copy for the life of the process.  In host code the array's name is only a
// stand-in: its device address comes from hipGetSymbolAddress, looked up once
// per device (with that device current) when the first handle on it is
// created, and only that address is handed to kernels and copies.  Calls on
// one device share the array, so overlapping calls race.
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;  // per device; nullptr: not looked up yet
// per device: held by a no-allocation call for its whole length, so calls of
// any handles on one device take the device's array in turn
std::vector<std::unique_ptr<std::mutex>> g_scratch_call_mu;
}  // namespace

void init_noalloc_scratch(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device < 0) throw InvalidArgument("device id out of range");
    if (g_scratch_ptr.size() <= static_cast<size_t>(device)) g_scratch_ptr.resize(device + 1, nullptr);
    while (g_scratch_call_mu.size() <= static_cast<size_t>(device))
        g_scratch_call_mu.push_back(std::make_unique<std::mutex>());
    if (g_scratch_ptr[device]) return;
    int cur = -1;
    check_hip(hipGetDevice(&cur), "hipGetDevice");
    if (cur != device) throw std::runtime_error("no-allocation scratch: device is not current");
    void* ptr = nullptr;
    check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!ptr) throw std::runtime_error("no-allocation scratch: null symbol address");
    g_scratch_ptr[device] = ptr;
}

void* noalloc_scratch(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device < 0 || static_cast<size_t>(device) >= g_scratch_ptr.size() || !g_scratch_ptr[device])
        throw std::runtime_error("no-allocation scratch was not set up on this device");
    return g_scratch_ptr[device];
}

std::mutex& noalloc_scratch_lock(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device < 0 || static_cast<size_t>(device) >= g_scratch_call_mu.size())
        throw std::runtime_error("no-allocation scratch was not set up on this device");
    return *g_scratch_call_mu[device];
}

void Engine::sample(const trw_sample_params& p, const SampleTarget* into) {
    hipStream_t s = stream;
    // per-call buffers: the engine's, or the caller's fixed region
    SampleSpace sp = into ? into->space : SampleSpace{};
    int64_t* hs = reinterpret_cast<int64_t*>(host_scalars);
    const int L = p.max_walk_len;
    if (L < 0) throw InvalidArgument("max_walk_len must be >= 0");
    const int walk_bias = p.walk_bias;
    int start_bias = p.initial_edge_bias < 0 ? walk_bias : p.initial_edge_bias;
    if (walk_bias < 0 || walk_bias > kTestLast || start_bias > kTestLast)
        throw InvalidArgument("Invalid picker type");
    if (p.direction != 0 && p.direction != 1) throw InvalidArgument("Invalid walk direction");
    if (p.walk_layout != TRW_LAYOUT_AUTO && p.walk_layout != TRW_LAYOUT_SCRATCH)
        throw InvalidArgument("Invalid walk layout");
    // core/temporal_random_walk_cpu.cuh:168-171
    if (start_bias == kTemporalNode2Vec) start_bias = kExponentialWeight;
    const bool forward = p.direction == 0;
    const bool shuffle = p.shuffle < 0 ? cfg.shuffle_walk_order != 0 : p.shuffle != 0;
    uint64_t seed = cfg.global_seed;
    if (seed == UINT64_MAX) {
        std::random_device rd;
        seed = (static_cast<uint64_t>(rd()) << 32) | rd();
    }

    check_hip(hipEventRecord(ev[4], s), "event");

    // ---- start array (core/temporal_random_walk.cu:394-588)
    uint64_t nw = 0;
    bool have_starts = false, have_cutoffs = false;
    int32_t* a_starts = nullptr;
    int64_t* a_cutoffs = nullptr;
    if (p.num_walks_per_node < 0 && p.mode != TRW_START_TOTAL)
        throw InvalidArgument("num_walks_per_node must be >= 0");
    const int wpn = p.num_walks_per_node;
    switch (p.mode) {
        case TRW_START_TOTAL: {
            if (p.num_walks_total < 0) throw InvalidArgument("num_walks_total must be >= 0");
            nw = static_cast<uint64_t>(p.num_walks_total);
            if (into && nw > into->capacity_walks)
                throw InvalidArgument("the sample has more walks than the outputs' capacity");
            break;
        }
        case TRW_START_ALL_NODES:
        case TRW_START_LAST_BATCH: {
            size_t count = 0;
            int32_t* ids = nullptr;
            if (p.mode == TRW_START_ALL_NODES) {
                const size_t v = active.n;
                uint32_t* fl = sp.take(flags, v + 1);
                uint32_t* sc = sp.take(scan, v + 1);
                uint32_t* ss = sp.take(scan_scratch, scan_scratch_elems(v + 1));
                if (v) {
                    hipLaunchKernelGGL(flags_from_u8_kernel, dim3(grid_for(v)), dim3(kB), 0, s,
                                       active.p, v, fl);
                }
                exclusive_scan_u32(fl, sc, v, ss, s);
                check_hip(hipMemcpyAsync(hs, sc + v, 4, hipMemcpyDeviceToHost, s), "count");
                sync();
                uint32_t c;
                std::memcpy(&c, hs, 4);
                count = c;
                ids = sp.take(s_ids, count);
                if (v) {
                    hipLaunchKernelGGL(compact_ids_kernel, dim3(grid_for(v)), dim3(kB), 0, s,
                                       fl, sc, v, ids);
                }
            } else {
                // unique sources (directed) or unique endpoints (undirected) of the
                // last batch, ascending (core/temporal_random_walk.cu:157-272)
                const size_t m = cfg.is_directed ? last_n : 2 * last_n;
                uint32_t* ka = sp.take(k32a, m);
                uint32_t* kb = sp.take(k32b, m);
                uint32_t* hi = sp.take(hist, radix_hist_elems(m));
                uint32_t* fl = sp.take(flags, m + 1);
                uint32_t* sc = sp.take(scan, m + 1);
                uint32_t* ss = sp.take(scan_scratch, scan_scratch_elems(m + 1));
                if (last_n) {
                    hipLaunchKernelGGL(u32_from_i32_kernel, dim3(grid_for(last_n)), dim3(kB), 0, s,
                                       last_src.p, last_n, ka);
                    if (!cfg.is_directed) {
                        hipLaunchKernelGGL(u32_from_i32_kernel, dim3(grid_for(last_n)), dim3(kB),
                                           0, s, last_dst.p, last_n, ka + last_n);
                    }
                }
                const int w = radix_sort_u32(ka, nullptr, kb, nullptr, m, 0, 32, hi, s);
                uint32_t* keys = w ? kb : ka;
                if (m) {
                    hipLaunchKernelGGL(unique_flags_kernel, dim3(grid_for(m)), dim3(kB), 0, s,
                                       keys, m, fl);
                }
                exclusive_scan_u32(fl, sc, m, ss, s);
                check_hip(hipMemcpyAsync(hs, sc + m, 4, hipMemcpyDeviceToHost, s), "count");
                sync();
                uint32_t c;
                std::memcpy(&c, hs, 4);
                count = c;
                ids = sp.take(s_ids, count);
                if (m) {
                    hipLaunchKernelGGL(compact_keys_kernel, dim3(grid_for(m)), dim3(kB), 0, s,
                                       keys, fl, sc, m, ids);
                }
            }
            nw = static_cast<uint64_t>(count) * static_cast<uint64_t>(wpn);
            if (into && nw > into->capacity_walks)
                throw InvalidArgument("the sample has more walks than the outputs' capacity");
            a_starts = sp.take(starts, nw);
            if (nw) {
                hipLaunchKernelGGL((repeat_kernel<int32_t>), dim3(grid_for(nw)), dim3(kB), 0, s,
                                   ids, nw, wpn, a_starts);
            }
            have_starts = true;
            break;
        }
        case TRW_START_NODES: {
            const size_t ns = p.num_seed_nodes;
            if (ns && !p.seed_nodes) throw InvalidArgument("seed_nodes is null");
            nw = static_cast<uint64_t>(ns) * static_cast<uint64_t>(wpn);
            if (into && nw > into->capacity_walks)
                throw InvalidArgument("the sample has more walks than the outputs' capacity");
            int32_t* seeds = sp.take(s_seeds, ns);
            if (ns) {
                check_hip(hipMemcpyAsync(seeds, p.seed_nodes, ns * 4, hipMemcpyHostToDevice, s),
                          "seeds H2D");
            }
            a_starts = sp.take(starts, nw);
            if (nw) {
                hipLaunchKernelGGL((repeat_kernel<int32_t>), dim3(grid_for(nw)), dim3(kB), 0, s,
                                   seeds, nw, wpn, a_starts);
            }
            if (p.cutoff_times) {
                int64_t* cuts = sp.take(s_cuts, ns);
                if (ns) {
                    check_hip(hipMemcpyAsync(cuts, p.cutoff_times, ns * 8,
                                             hipMemcpyHostToDevice, s),
                              "cutoffs H2D");
                }
                a_cutoffs = sp.take(cutoffs, nw);
                if (nw) {
                    hipLaunchKernelGGL((repeat_kernel<int64_t>), dim3(grid_for(nw)), dim3(kB), 0,
                                       s, cuts, nw, wpn, a_cutoffs);
                }
                have_cutoffs = true;
            }
            // the host arrays may be released once the copies have run
            sync();
            have_starts = true;
            break;
        }
        default:
            throw InvalidArgument("unknown start mode");
    }
    // one lane per walk: a dispatch holds fewer than 2^32 work-items
    if (nw >= (1ull << 32) - kB) throw InvalidArgument("too many walks (limit 2^32 - 256)");

    // ---- optional shuffle of the walk order (same permutation for cutoffs)
    if (have_starts && shuffle && nw > 1) {
        if (nw > 0xffffffffull) throw InvalidArgument("shuffle supports < 2^32 walks");
        uint32_t* ka = sp.take(k32a, nw);
        uint32_t* kb = sp.take(k32b, nw);
        uint32_t* va = sp.take(v32a, nw);
        uint32_t* vb = sp.take(v32b, nw);
        uint32_t* hi = sp.take(hist, radix_hist_elems(nw));
        hipLaunchKernelGGL(random_keys_kernel, dim3(grid_for(nw)), dim3(kB), 0, s, nw,
                           static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32), ka, va);
        const int w = radix_sort_u32(ka, va, kb, vb, nw, 0, 32, hi, s);
        const uint32_t* perm = w ? vb : va;
        int32_t* ps = sp.take(s_tmp32, nw);
        hipLaunchKernelGGL((permute_kernel<int32_t>), dim3(grid_for(nw)), dim3(kB), 0, s,
                           a_starts, perm, nw, ps);
        a_starts = ps;
        if (have_cutoffs) {
            int64_t* pc = sp.take(s_tmp64, nw);
            hipLaunchKernelGGL((permute_kernel<int64_t>), dim3(grid_for(nw)), dim3(kB), 0, s,
                               a_cutoffs, perm, nw, pc);
            a_cutoffs = pc;
        }
    }

    // ---- draws
    DrawSource ds{};
    ds.stride = 1u + 2u * static_cast<uint32_t>(L);
    ds.k0 = static_cast<uint32_t>(seed);
    ds.k1 = static_cast<uint32_t>(seed >> 32);
    ds.replay = nullptr;
    if (p.replay_draws) {
        const uint64_t need = nw * (1ull + 2ull * static_cast<uint64_t>(L));
        if (p.replay_draws_len != need)
            throw InvalidArgument("replay_draws must hold num_walks * (1 + 2 * max_walk_len) values");
        // every draw is turned into an in-range index only if it lies in [0, 1)
        for (uint64_t i = 0; i < need; ++i) {
            const double r = p.replay_draws[i];
            if (!(r >= 0.0 && r < 1.0)) throw InvalidArgument("replay_draws must lie in [0, 1)");
        }
        double* rp = sp.take(replay, need);
        if (need) {
            check_hip(hipMemcpyAsync(rp, p.replay_draws, need * 8, hipMemcpyHostToDevice, s),
                      "replay H2D");
        }
        ds.replay = rp;
    }

    // ---- outputs
    const uint64_t slots = nw * static_cast<uint64_t>(L);
    const uint64_t eslots = nw * static_cast<uint64_t>(L > 0 ? L - 1 : 0);
    // scratch: whole tiles of kScratchTile walks
    const uint64_t padded = (nw + kScratchTile - 1) / kScratchTile * kScratchTile;
    // slot words (slot_word): node id (in [0, max_node_id], as the node index
    // requires), the rank of the slot's time (below T, the all-ones value free
    // for the first slot) and the id of the edge into the slot (below E), or,
    // when the three do not fit in 64 bits, node and edge id alone (rank
    // field width 0; the edge field's all-ones value marks the first slot)
    auto bit_length = [](uint64_t v) { return v ? 64 - __builtin_clzll(v) : 0; };
    const int pk_nb = std::max(1, bit_length(static_cast<uint64_t>(std::max(max_node_id, 0))));
    const int rank_bits = bit_length(T);
    const bool with_rank = T > 0 && pk_nb + rank_bits + (E ? bit_length(E - 1) : 0) <= 64;
    const int pk_rb = with_rank ? rank_bits : 0;
    if (!with_rank && pk_nb + bit_length(E) >= 64)
        throw std::runtime_error("node ids and edge ids do not fit a slot word");
    // no walks until every output buffer is sized: a failed allocation
    // below leaves an empty walk set, not a count over released buffers
    w_num = 0;
    w_len = 0;
    w_feat.n = 0;
    uint64_t* sc_packed = nullptr;
    // forward walks: the walk kernel writes the output rows itself
    // (walk_rows_kernel); backward walks go through scratch and the layout
    // pass, which reverses them
    const bool rows_direct = p.walk_layout == TRW_LAYOUT_AUTO && forward &&
                             L > 0 && nw <= 0xffffffffull &&
                             p.walk_order != TRW_ORDER_NODE_GROUPED;
    if (rows_direct) {
        if (!into) sw_packed.release();
    } else {
        sc_packed = sp.take(sw_packed, padded * L);
    }
    // outputs: the engine's buffers, or the caller's
    int32_t* o_nodes;
    int64_t *o_ts, *o_eids;
    uint64_t* o_lens;
    if (into) {
        o_nodes = into->nodes;
        o_ts = into->ts;
        o_eids = into->eids;
        o_lens = into->lens;
    } else {
        w_nodes.resize(slots);
        w_ts.resize(slots);
        w_eids.resize(eslots);
        w_lens.resize(nw);
        o_nodes = w_nodes.p;
        o_ts = w_ts.p;
        o_eids = w_eids.p;
        o_lens = w_lens.p;
    }
    w_num = into ? 0 : nw;  // the walk statistics describe the engine's buffers
    w_last_num = nw;
    w_len = L;
    w_dir_forward = forward ? 1 : 0;
    w_constrained = have_starts ? 1 : 0;
    w_rows = rows_direct ? 1 : 0;
    w_slot_format = with_rank ? 0 : 1;
    w_replay = p.replay_draws ? 1 : 0;

    // ---- graph view of the sampled direction
    const bool use_in = !forward && cfg.is_directed;
    const DirIndex& d = use_in ? in : out;
    WalkGraph g{};
    g.src = src.p;
    g.dst = dst.p;
    g.ts = ts.p;
    g.E = static_cast<uint32_t>(E);
    g.tsg_off = tsg_off.p;
    g.uniq_ts = uniq_ts.p;
    if (neg1_rank.n == 0) {  // no build since the last clear
        int32_t* nr = sp.take(neg1_rank, 1);
        launch_neg1_rank(*this, nr);
        g.neg1_rank = nr;
    } else {
        g.neg1_rank = neg1_rank.p;
    }
    g.T = static_cast<uint32_t>(T);
    g.gw = forward ? fwd_cum.p : bwd_cum.p;
    g.gw_size = weights_ready ? T : 0;
    {
        const DBuf<WGuide>& gd = forward ? gwg_fwd : gwg_bwd;
        g.gwg = weights_ready && gd.n ? gd.p : nullptr;
        g.gwt = (forward ? gwt_fwd : gwt_bwd).p;
    }
    g.active = active.p;
    g.active_size = static_cast<int32_t>(active.n);
    g.d.hdr = d.hdr.p;
    g.d.tab = d.tab.p;
    g.d.pan = d.pan.p;
    g.d.rec = d.rec.p;
    g.d.idx_size = static_cast<uint32_t>(d.n_entries);
    // the weight pickers' view of the sampled direction's per-node weights
    const WalkWeights& ww = forward ? out.wf : d.wb;
    const bool wview = weights_ready && ww.hdr.n == d.hdr.n &&
                       ww.pan.n == (d.n_groups << ww.shift) &&
                       d.wrec.n == (d.n_entries << d.wrec_shift);
    g.d.wrec = wview ? d.wrec.p : nullptr;
    g.d.wrshift = wview ? static_cast<uint32_t>(d.wrec_shift) : 0u;
    g.d.whdr = wview ? ww.hdr.p : nullptr;
    g.d.wpan = wview ? ww.pan.p : nullptr;
    g.d.wshift = wview ? static_cast<uint32_t>(ww.shift) : 0u;
    g.d.wgt = wview ? ww.tab.p : nullptr;
    g.d.w_size = wview ? d.n_groups : 0;
    g.adj_off = adj_lists_ready ? adj_off.p : nullptr;
    g.adj_nbr = adj_nbr.p;
    g.adj_nodes = adj_ready ? static_cast<uint32_t>(adj_nodes) : 0;
    g.adj_hash = adj_ready && adj_hash.n ? adj_hash.p : nullptr;
    g.adj_mask = adj_hash.n ? adj_hash.n - 1 : 0;
    g.adj_shift = 64 - adj_hash_log;
    g.adj_bits = adj_bits;
    g.tn2v = cfg.enable_temporal_node2vec;
    g.inv_p = 1.0 / cfg.node2vec_p;
    g.inv_q = 1.0 / cfg.node2vec_q;

    WalkArgs a{};
    a.L = L;
    a.walk_bias = walk_bias;
    a.start_bias = start_bias;
    a.pad = cfg.walk_padding_value;
    a.starts = have_starts ? a_starts : nullptr;
    a.cutoffs = have_cutoffs ? a_cutoffs : nullptr;
    a.n = nw;
    a.ds = ds;
    a.lens = o_lens;
    a.packed = sc_packed;
    a.pk_nb = pk_nb;
    a.pk_rb = pk_rb;

    if (nw && E == 0) {
        // empty graph: every start fails; the kernel still writes the padding
        g.T = 0;
        g.active_size = 0;
    }
    // The index family's kernels serve the index pickers; without weights a
    // weight picker picks nothing there, as it does in the reference (its
    // range check against an empty weight array).  The weight families read
    // the weighted view instead of the plain headers and panel.
    const bool index_only = (is_index_picker(walk_bias) && is_index_picker(start_bias)) || !wview;
    const bool no_node2vec = walk_bias != kTemporalNode2Vec;  // start_bias never is (above)
    // the index arrays the launched walk kernel reads (each counted whole):
    // headers (plain or weighted), bucket tables, panel (plain or weighted)
    // and records (plain or weighted) of the sampled direction, the guide
    // tables for the weight families; the adjacency pair set for node2vec
    w_index_bytes = d.tab.bytes() + (index_only ? d.rec.bytes() + d.hdr.bytes() + d.pan.bytes()
                                                : d.wrec.bytes() + ww.bytes());
    if (walk_bias == kTemporalNode2Vec && adj_ready) w_index_bytes += adj_hash.bytes();
#define TRW_LAUNCH_FAMILY(K, F, D, G, ...)                                                     \
    do {                                                                                       \
        if (index_only)                                                                        \
            hipLaunchKernelGGL((K<F, D, kFamIndex>), G, dim3(kB), 0, s, __VA_ARGS__);           \
        else if (no_node2vec)                                                                  \
            hipLaunchKernelGGL((K<F, D, kFamWeight>), G, dim3(kB), 0, s, __VA_ARGS__);          \
        else                                                                                   \
            hipLaunchKernelGGL((K<F, D, kFamAny>), G, dim3(kB), 0, s, __VA_ARGS__);             \
    } while (0)
#define TRW_LAUNCH(K, G, ...)                                                                  \
    do {                                                                                       \
        if (forward && cfg.is_directed) TRW_LAUNCH_FAMILY(K, true, true, G, __VA_ARGS__);      \
        else if (forward) TRW_LAUNCH_FAMILY(K, true, false, G, __VA_ARGS__);                   \
        else if (cfg.is_directed) TRW_LAUNCH_FAMILY(K, false, true, G, __VA_ARGS__);           \
        else TRW_LAUNCH_FAMILY(K, false, false, G, __VA_ARGS__);                               \
    } while (0)

    // ---- processing order: walks sorted by the time rank of their start
    // edge, so the walks of one wave -- and of one XCD -- search the same
    // stretch of a hub's panel and read neighbouring records
    const int order_mode = p.walk_order == TRW_ORDER_AUTO
                               ? (nw >= kTimeOrderMinWalks ? TRW_ORDER_START_TIME : TRW_ORDER_WALK_ID)
                               : p.walk_order;
    if (order_mode != TRW_ORDER_WALK_ID && order_mode != TRW_ORDER_START_TIME &&
        order_mode != TRW_ORDER_NODE_GROUPED)
        throw InvalidArgument("Invalid walk order");
    const bool node_grouped = order_mode == TRW_ORDER_NODE_GROUPED && nw > 1 && L > 1;
    if (nw && L > 0) {
        const uint32_t none = g.T;  // past every rank: walks without a start run last
        const bool sorted = order_mode == TRW_ORDER_START_TIME && nw > 1 && L > 1 && !node_grouped;
        // The start states come from a pre-pass where the order needs them (or
        // its keys need the index); unconstrained starts of an index picker
        // need only keys, and walks in walk-id order no pre-pass: the walk
        // kernel finds their start edges itself.
        const bool keys_only = !have_starts && is_index_picker(start_bias);
        uint32_t* ka = nullptr;
        uint32_t* va = nullptr;
        if (node_grouped || (sorted && !keys_only)) {
            StartState* st = reinterpret_cast<StartState*>(sp.take(walk_st, 4 * nw));
            ka = sp.take(k32a, nw);
            va = sp.take(v32a, nw);
            TRW_LAUNCH(walk_start_kernel, dim3(grid_for(nw)), g, a, st, ka, va, none);
            a.st = st;
        } else if (sorted) {
            ka = sp.take(k32a, nw);
            va = sp.take(v32a, nw);
            if (forward)
                hipLaunchKernelGGL(walk_start_keys_kernel<true>, dim3(grid_for(nw)), dim3(kB), 0, s,
                                   g, a, ka, va, none);
            else
                hipLaunchKernelGGL(walk_start_keys_kernel<false>, dim3(grid_for(nw)), dim3(kB), 0, s,
                                   g, a, ka, va, none);
        }
        if (sorted) {
            uint32_t* kb = sp.take(k32b, nw);
            uint32_t* vb = sp.take(v32b, nw);
            uint32_t* hi = sp.take(hist, radix_hist_elems(nw));
            const int bits = std::max(1, 32 - __builtin_clz(none | 1u));
            const int wsort = radix_sort_u32(ka, va, kb, vb, nw, 0, bits, hi, s);
            a.order = wsort ? vb : va;
            a.xcd_remap = 1;
        }
        check_hip(hipGetLastError(), "walk start launch");
    }

    // a start state read per walk, or (starts found by the walk kernel) the
    // walk's seed node, or the start edge's endpoints and the timestamp
    // groups' offsets
    w_in_bytes_per_walk = (a.st ? sizeof(StartState) : (have_starts ? 4 : 8)) +
                          (a.order ? 4 : 0) + (have_cutoffs ? 8 : 0);
    if (!a.st && !have_starts && nw && L > 0) w_index_bytes += tsg_off.bytes();

    // ---- walk kernel, then the layout pass.  (Running the layout of finished
    // grid chunks on a second stream beside the remaining walks was measured
    // slower: the layout's streaming traffic evicts the hub lines the walks
    // hit in L2.)
    check_hip(hipEventRecord(ev[5], s), "event");
    uint64_t launches = nw ? 1 : 0;
    if (node_grouped) {
        // segments of kNodeGroupHops hops, the live walks regrouped by their
        // current node in between (the count of live walks is read back to
        // size the next sort and launch)
        if (nw > 0xffffffffull) throw InvalidArgument("node-grouped order supports < 2^32 walks");
        WalkCarry* carry = reinterpret_cast<WalkCarry*>(sp.take(ng_carry, 8 * nw));
        uint32_t* kb[2] = {sp.take(ng_keys0, nw), sp.take(ng_keys1, nw)};
        uint32_t* vb[2] = {sp.take(ng_vals0, nw), sp.take(ng_vals1, nw)};
        uint32_t* hi = sp.take(hist, radix_hist_elems(nw));
        uint32_t* cnt = sp.take(ng_count, 1);
        const int nbits = std::max(1, bit_length(static_cast<uint64_t>(std::max(max_node_id, 0))));
        check_hip(hipMemsetAsync(cnt, 0, 4, s), "live count clear");
        int in = 0;  // the pair the next list is emitted into
        TRW_LAUNCH(node_group_init_kernel, dim3(grid_for(nw)), g, a, carry, kb[in], vb[in], cnt);
        check_hip(hipGetLastError(), "node-grouped init launch");
        launches = 1;
        for (;;) {
            check_hip(hipMemcpyAsync(hs, cnt, 4, hipMemcpyDeviceToHost, s), "live count");
            sync();
            uint32_t live;
            std::memcpy(&live, hs, 4);
            if (live == 0) break;
            const int w = radix_sort_u32(kb[in], vb[in], kb[in ^ 1], vb[in ^ 1], live, 0, nbits,
                                         hi, s);
            const int sorted = w ? in ^ 1 : in;  // the pair holding the sorted list
            const uint32_t* list = vb[sorted];
            in = sorted ^ 1;
            check_hip(hipMemsetAsync(cnt, 0, 4, s), "live count clear");
            TRW_LAUNCH(node_group_segment_kernel, dim3(grid_for(live)), g, a, list, live, carry,
                       kb[in], vb[in], cnt);
            check_hip(hipGetLastError(), "node-grouped segment launch");
            ++launches;
        }
    } else if (nw && rows_direct) {
        a.q0 = 0;
        a.q_end = nw;
        a.on = o_nodes;
        a.ot = o_ts;
        a.oe = o_eids;
        a.uniq_ts = uniq_ts.p;
        a.edge_ts = ts.p;
        a.start_ts = INT64_MIN;
        const dim3 grid(grid_for(nw));
        launch_rows(cfg.is_directed, index_only ? kFamIndex : (no_node2vec ? kFamWeight : kFamAny),
                    grid, s, g, a);
        check_hip(hipGetLastError(), "walk kernel launch");
    } else if (nw) {
        a.q0 = 0;
        a.q_end = nw;
        TRW_LAUNCH(walk_kernel, dim3(grid_for(nw)), g, a);
        check_hip(hipGetLastError(), "walk kernel launch");
    }
#undef TRW_LAUNCH
#undef TRW_LAUNCH_FAMILY
    check_hip(hipEventRecord(ev[6], s), "event");
    if (nw && L > 0 && !rows_direct) {
        LayoutArgs la{};
        la.sp = a.packed;
        la.pk_nb = pk_nb;
        la.pk_rb = pk_rb;
        la.on = o_nodes;
        la.ot = o_ts;
        la.oe = o_eids;
        la.lens = o_lens;
        la.L = L;
        const int slot_chunks = (L + kLayoutPackedMaxSlots - 1) / kLayoutPackedMaxSlots;
        la.C = (L + slot_chunks - 1) / slot_chunks;
        la.reverse = forward ? 0 : 1;
        la.pad = static_cast<int32_t>(cfg.walk_padding_value);
        la.uniq_ts = uniq_ts.p;
        la.edge_ts = ts.p;
        la.start_ts = forward ? INT64_MIN : INT64_MAX;
        la.order = a.order;
        la.q0 = 0;
        la.q_end = nw;
        // edge features of dim % 4 == 0 are written by the layout pass, from
        // the edge ids it holds in LDS (device buffers are 256-byte aligned)
        const bool fused_feat = feat_dim > 0 && eslots && feat_dim % 4 == 0;
        if (fused_feat) {
            if (!into) w_feat.resize(eslots * feat_dim);
            la.feat = feat.p;
            la.of = into ? into->feat : w_feat.p;
            la.fv = static_cast<uint32_t>(feat_dim / 4);
        }
        const size_t tile = static_cast<size_t>(la.C + 1) * (kLayoutWalks + 1) * sizeof(uint64_t);
        const size_t lds = tile + kLayoutWalks * (sizeof(int) + sizeof(uint32_t));
        const unsigned gx = static_cast<unsigned>((nw + kLayoutWalks - 1) / kLayoutWalks);
        hipLaunchKernelGGL(layout_packed_kernel, dim3(gx, slot_chunks), dim3(256), lds, s, la);
        check_hip(hipGetLastError(), "layout launch");
    }

    // ---- edge features of every walk slot (finalize_host_walks, on device):
    // other dims than multiples of 4 gather from the laid-out edge ids
    if (feat_dim > 0 && eslots) {
        if (feat_dim % 4 != 0 || rows_direct) {
            if (!into) w_feat.resize(eslots * feat_dim);
            hipLaunchKernelGGL(gather_walk_features_kernel, dim3(grid_capped(eslots * feat_dim)),
                               dim3(kB), 0, s, o_eids, eslots, static_cast<uint32_t>(feat_dim),
                               feat.p, into ? into->feat : w_feat.p);
            check_hip(hipGetLastError(), "feature gather launch");
        }
    } else {
        w_feat.n = 0;
    }
    check_hip(hipEventRecord(ev[7], s), "event");
    sync();
    float ms = 0;
    check_hip(hipEventElapsedTime(&ms, ev[4], ev[7]), "elapsed");
    timings.sample_ms = ms;
    check_hip(hipEventElapsedTime(&ms, ev[5], ev[6]), "elapsed");
    timings.walk_kernel_ms = ms;
    timings.walk_kernel_launches = launches;
}

void walk_stats(Engine& e, trw_walk_stats* out) {
    hipStream_t s = e.stream;
    e.acc64.ensure(5);
    check_hip(hipMemsetAsync(e.acc64.p, 0, 40, s), "memset");
    const bool use_in = !e.w_dir_forward && e.cfg.is_directed;
    const DirIndex& d = use_in ? e.in : e.out;
    if (e.w_num && e.w_len > 0) {
        // about 4096 workgroups, each over a run of walks whose slots number
        // below 2^32
        uint64_t wpb = (e.w_num + 4095) / 4096;
        wpb = std::min<uint64_t>(wpb, 0xffffffffull / static_cast<uint64_t>(e.w_len));
        const uint64_t blocks = (e.w_num + wpb - 1) / wpb;
        hipLaunchKernelGGL(walk_stats_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kB), 0, s,
                           e.w_nodes.p, e.w_lens.p, e.w_num, e.w_len, wpb, d.cnt.p,
                           static_cast<int32_t>(e.active.n), e.w_constrained,
                           reinterpret_cast<unsigned long long*>(e.acc64.p));
        check_hip(hipGetLastError(), "walk stats launch");
    }
    uint64_t h[5];
    check_hip(hipMemcpyAsync(h, e.acc64.p, 40, hipMemcpyDeviceToHost, s), "read stats");
    e.sync();
    out->total_len = h[0];
    out->transitions = h[1];
    out->nonempty_walks = h[2];
    out->algorithmic_bytes = h[3];
    out->reference_bytes = h[4];
    // compulsory bytes of the walk kernel's launch: inputs and the index read
    // once, the scratch slots and lengths written once
    const uint64_t nw = e.w_num;
    out->compulsory_read_bytes =
        nw && e.w_len > 0 ? nw * e.w_in_bytes_per_walk + e.w_index_bytes +
                                (e.w_replay ? 16 * out->transitions : 0)
                          : 0;
    // the kernel's slot writes: scratch slot words, or (rows written by the
    // walk kernel) every output row in full
    const uint64_t L = static_cast<uint64_t>(e.w_len);
    const uint64_t scratch =
        e.w_rows ? nw * (4 * L + 8 * L + 8 * (L > 0 ? L - 1 : 0)) : 8 * out->total_len;
    out->compulsory_write_bytes = nw ? 8 * nw + (e.w_len > 0 ? scratch : 0) : 0;
    out->rows_by_walk_kernel = static_cast<uint64_t>(e.w_rows);
    out->slot_word_format = static_cast<uint64_t>(e.w_slot_format);
}

}  // namespace trw
