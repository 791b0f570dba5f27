/*
 * trw_oracle.c -- CPU restatement of the reference's temporal random walk
 * hot path.  TEST INFRASTRUCTURE ONLY: used by tests/, smoke() and the
 * cpu_baseline leg of bench.py as the parity checker; never linked into the
 * product.  Citations are file:line in the reference (v1.8.6) relative to
 * temporal_random_walk/src/.
 *
 * Parity pins (see tests/test_oracle_*.py):
 *  - edge store order, timestamp groups, eviction: literal expectations of
 *    the reference's test/test_edge_data.cpp and test/test_temporal_graph.cpp,
 *    plus brute-force stable sorts on random inputs;
 *  - node index, per-node weights, walk sampler, pickers, node2vec: the
 *    reference's own code compiled into oracle/_ref (node_edge_index.cu,
 *    buffer.cu and the header-only sampler), compared bit-exactly; picker
 *    closed forms and two-element probabilities of test_random_picker.cpp;
 *  - global weights: closed-form ratios of test_edge_data_weights.cpp, sums
 *    equal to one, monotone cumulative arrays.
 */
#include "trw_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define NODE2VEC_MAX_RETRIES 64 /* common/const.cuh:37 */
#define NO_WALK_CUTOFF (-1)     /* common/const.cuh:24 */

static _Thread_local char g_err[256];
const char* orc_last_error(void) { return g_err; }

struct orc_graph {
    int is_directed;
    int64_t max_time_capacity;
    int enable_weight;
    int enable_tn2v;
    double timescale_bound;
    double inv_p, inv_q;
    int64_t latest_timestamp; /* data/temporal_graph_data.cuh:16 (starts at 0) */

    size_t E;
    int32_t* src;
    int32_t* dst;
    int64_t* ts;
    size_t feat_dim;
    float* feat;

    size_t T;
    uint64_t* ts_group_offsets; /* T + 1 */
    int64_t* unique_ts;         /* T */

    int32_t max_node_id;
    size_t active_size; /* max_node_id + 1 */
    int32_t* active;

    size_t w_size;
    double* fwd_cum;
    double* bwd_cum;

    size_t adj_off_size;
    uint64_t* adj_off;
    size_t adj_nbr_size;
    int32_t* adj_nbr;

    size_t off_size; /* node_index_capacity = active_size + 1 */
    uint64_t* out_off;
    uint64_t* in_off; /* directed only */
    size_t n_out, n_in;
    uint64_t* out_idx;
    uint64_t* in_idx;
    size_t cnt_size; /* active_size + 1 */
    uint64_t* out_cnt;
    uint64_t* in_cnt;
    size_t g_out, g_in;
    uint64_t* out_grp;
    uint64_t* in_grp;
    double* out_fwd_w;
    double* out_bwd_w;
    double* in_bwd_w;

    int threads; /* OpenMP threads of the ingest (orc_set_threads; 1 = serial) */
};

static void* xmalloc(size_t n) {
    void* p = malloc(n ? n : 1);
    if (!p) {
        fprintf(stderr, "oracle: out of memory (%zu bytes)\n", n);
        abort();
    }
    return p;
}

static void set_array(void** slot, void* p) {
    free(*slot);
    *slot = p;
}

orc_graph* orc_create(int is_directed, int64_t max_time_capacity,
                      int enable_weight_computation, int enable_temporal_node2vec,
                      double timescale_bound, double node2vec_p, double node2vec_q) {
    /* core/temporal_random_walk.cu:58-67 */
    orc_graph* g = (orc_graph*)calloc(1, sizeof(orc_graph));
    g->is_directed = is_directed;
    g->max_time_capacity = max_time_capacity;
    g->enable_tn2v = enable_temporal_node2vec;
    g->enable_weight = enable_weight_computation || enable_temporal_node2vec;
    g->timescale_bound = timescale_bound;
    g->inv_p = 1.0 / node2vec_p;
    g->inv_q = 1.0 / node2vec_q;
    g->latest_timestamp = 0;
    g->max_node_id = -1;
    g->threads = 1;
    return g;
}

void orc_set_threads(orc_graph* g, int threads) { g->threads = threads > 0 ? threads : 1; }

void orc_destroy(orc_graph* g) {
    if (!g) return;
    free(g->src); free(g->dst); free(g->ts); free(g->feat);
    free(g->ts_group_offsets); free(g->unique_ts); free(g->active);
    free(g->fwd_cum); free(g->bwd_cum); free(g->adj_off); free(g->adj_nbr);
    free(g->out_off); free(g->in_off); free(g->out_idx); free(g->in_idx);
    free(g->out_cnt); free(g->in_cnt); free(g->out_grp); free(g->in_grp);
    free(g->out_fwd_w); free(g->out_bwd_w); free(g->in_bwd_w);
    free(g);
}

/* ------------------------------------------------------------------ */
/* Parallel building blocks of the ingest.  Every one gives the same     */
/* result for any thread count: the sorts are stable and the scans and   */
/* scatters write each output once.                                      */
/* ------------------------------------------------------------------ */
typedef struct {
    int64_t k;  /* timestamp */
    uint32_t p; /* position in the store */
} orc_kp;

/* [lo, hi) of chunk t of n items split into nt chunks. */
static void chunk_of(size_t n, int nt, int t, size_t* lo, size_t* hi) {
    *lo = n * (size_t)t / (size_t)nt;
    *hi = n * (size_t)(t + 1) / (size_t)nt;
}

/* Bottom-up stable merge sort of (key, position) pairs by key. */
static void sort_kp(orc_kp* a, orc_kp* tmp, size_t n) {
    for (size_t width = 1; width < n; width *= 2) {
        for (size_t lo = 0; lo < n; lo += 2 * width) {
            size_t mid = lo + width < n ? lo + width : n;
            size_t hi = lo + 2 * width < n ? lo + 2 * width : n;
            size_t i = lo, j = mid, k = lo;
            while (i < mid && j < hi) {
                if (a[j].k < a[i].k) tmp[k++] = a[j++];
                else tmp[k++] = a[i++];
            }
            while (i < mid) tmp[k++] = a[i++];
            while (j < hi) tmp[k++] = a[j++];
        }
        memcpy(a, tmp, n * sizeof(orc_kp));
    }
}

/* Number of A's items among the first d outputs of the stable merge of A
 * and B (on equal keys A's item comes first): the merge-path co-rank. */
static size_t merge_corank(const orc_kp* A, size_t na, const orc_kp* B, size_t nb, size_t d) {
    size_t lo = d > nb ? d - nb : 0, hi = d < na ? d : na;
    while (lo < hi) {
        size_t mid = lo + (hi - lo) / 2;
        /* A[mid] precedes B[d - mid - 1]: more than mid items come from A */
        if (A[mid].k <= B[d - mid - 1].k) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

/* Stable merge of A and B into out (std::merge: B's item is taken only when
 * strictly less), cut into nt equal output spans by co-rank. */
static void par_merge(const orc_kp* A, size_t na, const orc_kp* B, size_t nb, orc_kp* out,
                      int nt) {
    size_t n = na + nb;
    if (n < 65536) nt = 1;
#pragma omp parallel for schedule(static, 1) num_threads(nt)
    for (int t = 0; t < nt; t++) {
        size_t d0, d1;
        chunk_of(n, nt, t, &d0, &d1);
        size_t i = merge_corank(A, na, B, nb, d0), i1 = merge_corank(A, na, B, nb, d1);
        size_t j = d0 - i, j1 = d1 - i1, k = d0;
        while (i < i1 && j < j1) {
            if (B[j].k < A[i].k) out[k++] = B[j++];
            else out[k++] = A[i++];
        }
        while (i < i1) out[k++] = A[i++];
        while (j < j1) out[k++] = B[j++];
    }
}

/* Stable LSD radix sort of (key, position) pairs by key - kmin (all keys in
 * [kmin, kmax]), 11-bit digits over the range's bits, per-thread chunk
 * histograms: equal keys keep their input order.  Result in a. */
static void par_radix_kp(orc_kp* a, size_t n, int64_t kmin, int64_t kmax, int nt) {
    enum { RB = 11, RD = 1 << RB };
    if (n < 65536) nt = 1;
    const uint64_t range = (uint64_t)kmax - (uint64_t)kmin;
    int bits = 0;
    while (bits < 64 && (range >> bits) != 0) bits++;
    orc_kp* b = (orc_kp*)xmalloc((n ? n : 1) * sizeof(orc_kp));
    size_t* hist = (size_t*)xmalloc((size_t)nt * RD * sizeof(size_t));
    orc_kp *src = a, *dst = b;
    for (int shift = 0; shift < bits; shift += RB) {
#pragma omp parallel for schedule(static, 1) num_threads(nt)
        for (int t = 0; t < nt; t++) {
            size_t lo, hi;
            chunk_of(n, nt, t, &lo, &hi);
            size_t* h = hist + (size_t)t * RD;
            memset(h, 0, RD * sizeof(size_t));
            for (size_t i = lo; i < hi; i++)
                h[(((uint64_t)src[i].k - (uint64_t)kmin) >> shift) & (RD - 1)]++;
        }
        size_t run = 0;
        for (int d = 0; d < RD; d++) {
            for (int t = 0; t < nt; t++) {
                size_t c = hist[(size_t)t * RD + d];
                hist[(size_t)t * RD + d] = run;
                run += c;
            }
        }
#pragma omp parallel for schedule(static, 1) num_threads(nt)
        for (int t = 0; t < nt; t++) {
            size_t lo, hi;
            chunk_of(n, nt, t, &lo, &hi);
            size_t* h = hist + (size_t)t * RD;
            for (size_t i = lo; i < hi; i++)
                dst[h[(((uint64_t)src[i].k - (uint64_t)kmin) >> shift) & (RD - 1)]++] = src[i];
        }
        orc_kp* t0 = src;
        src = dst;
        dst = t0;
    }
    if (src != a) memcpy(a, src, n * sizeof(orc_kp));
    free(b);
    free(hist);
}

/* Stable sort of n pairs by key: chunks sorted side by side, then merged
 * pairwise, each merge spread over every thread.  Result in a. */
static void par_sort_kp(orc_kp* a, size_t n, int nt) {
    orc_kp* tmp = (orc_kp*)xmalloc(n * sizeof(orc_kp));
    int chunks = 1;
    while (chunks < nt && n / (size_t)(2 * chunks) >= 65536) chunks *= 2;
#pragma omp parallel for schedule(static, 1) num_threads(nt)
    for (int c = 0; c < chunks; c++) {
        size_t lo, hi;
        chunk_of(n, chunks, c, &lo, &hi);
        sort_kp(a + lo, tmp + lo, hi - lo);
    }
    orc_kp* src = a;
    orc_kp* dst = tmp;
    for (int run = 1; run < chunks; run *= 2) {
        for (int c = 0; c < chunks; c += 2 * run) {
            size_t lo, mid, hi, x;
            chunk_of(n, chunks, c, &lo, &x);
            chunk_of(n, chunks, c + run, &mid, &x);
            chunk_of(n, chunks, c + 2 * run - 1, &x, &hi);
            par_merge(src + lo, mid - lo, src + mid, hi - mid, dst + lo, nt);
        }
        orc_kp* t = src;
        src = dst;
        dst = t;
    }
    if (src != a) memcpy(a, src, n * sizeof(orc_kp));
    free(tmp);
}

/* temporal_graph.cu:67-134: sort the new batch positions by timestamp,
 * merge after the old (already sorted) positions, gather src/dst/ts/feat. */
static void sort_and_merge(orc_graph* g, size_t start_idx) {
    size_t total = g->E, n_new = total - start_idx;
    if (n_new == 0) return;
    const int nt = g->threads;
    orc_kp* nw = (orc_kp*)xmalloc(n_new * sizeof(orc_kp));
    orc_kp* old = (orc_kp*)xmalloc((start_idx ? start_idx : 1) * sizeof(orc_kp));
    int64_t kmin = g->ts[start_idx], kmax = g->ts[start_idx];
#pragma omp parallel for schedule(static) reduction(min : kmin) reduction(max : kmax) num_threads(nt)
    for (size_t i = 0; i < n_new; i++) {
        nw[i].k = g->ts[start_idx + i];
        nw[i].p = (uint32_t)(start_idx + i);
        if (nw[i].k < kmin) kmin = nw[i].k;
        if (nw[i].k > kmax) kmax = nw[i].k;
    }
#pragma omp parallel for schedule(static) num_threads(nt)
    for (size_t i = 0; i < start_idx; i++) {
        old[i].k = g->ts[i];
        old[i].p = (uint32_t)i;
    }
    /* a stable sort: the batch's tie order is the reference's input order
     * (its std::sort is not stable; the canonical order is) */
    if (nt > 1) par_radix_kp(nw, n_new, kmin, kmax, nt);
    else par_sort_kp(nw, n_new, 1);
    /* std::merge of the old positions with the sorted batch */
    orc_kp* merged = (orc_kp*)xmalloc(total * sizeof(orc_kp));
    par_merge(old, start_idx, nw, n_new, merged, nt);
    free(nw);
    free(old);

    int32_t* s2 = (int32_t*)xmalloc(total * sizeof(int32_t));
    int32_t* d2 = (int32_t*)xmalloc(total * sizeof(int32_t));
    int64_t* t2 = (int64_t*)xmalloc(total * sizeof(int64_t));
    float* f2 = g->feat_dim ? (float*)xmalloc(total * g->feat_dim * sizeof(float)) : NULL;
#pragma omp parallel for schedule(static) num_threads(nt)
    for (size_t p = 0; p < total; p++) {
        uint32_t id = merged[p].p;
        s2[p] = g->src[id];
        d2[p] = g->dst[id];
        t2[p] = g->ts[id];
        if (f2) memcpy(f2 + p * g->feat_dim, g->feat + (size_t)id * g->feat_dim,
                       g->feat_dim * sizeof(float));
    }
    free(merged);
    set_array((void**)&g->src, s2);
    set_array((void**)&g->dst, d2);
    set_array((void**)&g->ts, t2);
    if (f2) set_array((void**)&g->feat, f2);
}

/* temporal_graph.cu:136-156: drop the prefix with ts <= latest - capacity. */
static void delete_old_edges(orc_graph* g) {
    if (g->max_time_capacity <= 0 || g->E == 0) return;
    int64_t cutoff = g->latest_timestamp - g->max_time_capacity;
    size_t lo = 0, hi = g->E; /* upper_bound */
    while (lo < hi) {
        size_t mid = lo + (hi - lo) / 2;
        if (cutoff < g->ts[mid]) hi = mid; else lo = mid + 1;
    }
    size_t del = lo;
    if (del == 0) return;
    size_t keep = g->E - del;
    memmove(g->src, g->src + del, keep * sizeof(int32_t));
    memmove(g->dst, g->dst + del, keep * sizeof(int32_t));
    memmove(g->ts, g->ts + del, keep * sizeof(int64_t));
    if (g->feat_dim)
        memmove(g->feat, g->feat + del * g->feat_dim, keep * g->feat_dim * sizeof(float));
    g->E = keep;
}

/* edge_data.cu:256-296 */
static void populate_active_nodes(orc_graph* g) {
    if (g->E == 0) {
        g->max_node_id = -1;
        g->active_size = 0;
        set_array((void**)&g->active, NULL);
        return;
    }
    int32_t mx = -1;
    const int nt = g->threads;
#pragma omp parallel for schedule(static) reduction(max : mx) num_threads(nt)
    for (size_t i = 0; i < g->E; i++) {
        if (g->src[i] > mx) mx = g->src[i];
        if (g->dst[i] > mx) mx = g->dst[i];
    }
    g->max_node_id = mx;
    g->active_size = (size_t)mx + 1;
    int32_t* act = (int32_t*)calloc(g->active_size, sizeof(int32_t));
#pragma omp parallel for schedule(static) num_threads(nt)
    for (size_t i = 0; i < g->E; i++) {
        /* a flag already set is left alone (a hub's line is then only read) */
        int32_t a, b;
#pragma omp atomic read
        a = act[g->src[i]];
        if (!a) {
#pragma omp atomic write
            act[g->src[i]] = 1;
        }
#pragma omp atomic read
        b = act[g->dst[i]];
        if (!b) {
#pragma omp atomic write
            act[g->dst[i]] = 1;
        }
    }
    set_array((void**)&g->active, act);
}

/* edge_data.cu:394-438 */
static void update_timestamp_groups(orc_graph* g) {
    size_t n = g->E;
    if (n == 0) {
        g->T = 0;
        set_array((void**)&g->ts_group_offsets, NULL);
        set_array((void**)&g->unique_ts, NULL);
        return;
    }
    /* group starts counted per chunk, chunk bases scanned, then written */
    const int nt = n < 65536 ? 1 : g->threads;
    size_t* base = (size_t*)calloc((size_t)nt + 1, sizeof(size_t));
#pragma omp parallel for schedule(static, 1) num_threads(nt)
    for (int t = 0; t < nt; t++) {
        size_t lo, hi, c = 0;
        chunk_of(n, nt, t, &lo, &hi);
        for (size_t i = lo; i < hi; i++) c += i == 0 || g->ts[i] != g->ts[i - 1];
        base[t + 1] = c;
    }
    for (int t = 0; t < nt; t++) base[t + 1] += base[t];
    size_t T = base[nt];
    uint64_t* off = (uint64_t*)xmalloc((T + 1) * sizeof(uint64_t));
    int64_t* uq = (int64_t*)xmalloc(T * sizeof(int64_t));
#pragma omp parallel for schedule(static, 1) num_threads(nt)
    for (int t = 0; t < nt; t++) {
        size_t lo, hi, k = base[t];
        chunk_of(n, nt, t, &lo, &hi);
        for (size_t i = lo; i < hi; i++) {
            if (i == 0 || g->ts[i] != g->ts[i - 1]) {
                off[k] = i;
                uq[k] = g->ts[i];
                k++;
            }
        }
    }
    free(base);
    off[T] = n;
    g->T = T;
    set_array((void**)&g->ts_group_offsets, off);
    set_array((void**)&g->unique_ts, uq);
}

static int cmp_i32(const void* a, const void* b) {
    int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
    return (x > y) - (x < y);
}

/* edge_data.cu:298-392: symmetric adjacency CSR, duplicates kept, every
 * neighbour list sorted ascending. */
static void build_adjacency(orc_graph* g) {
    size_t n = g->active_size, m = g->E;
    uint64_t* off = (uint64_t*)calloc(n + 1, sizeof(uint64_t));
    g->adj_off_size = n + 1;
    if (n == 0 || m == 0) {
        set_array((void**)&g->adj_off, off);
        set_array((void**)&g->adj_nbr, NULL);
        g->adj_nbr_size = 0;
        return;
    }
    for (size_t i = 0; i < m; i++) {
        off[(size_t)g->src[i] + 1]++;
        off[(size_t)g->dst[i] + 1]++;
    }
    for (size_t i = 0; i < n; i++) off[i + 1] += off[i];
    int32_t* nbr = (int32_t*)xmalloc(2 * m * sizeof(int32_t));
    uint64_t* cur = (uint64_t*)xmalloc(n * sizeof(uint64_t));
    memcpy(cur, off, n * sizeof(uint64_t));
    for (size_t i = 0; i < m; i++) {
        nbr[cur[g->src[i]]++] = g->dst[i];
        nbr[cur[g->dst[i]]++] = g->src[i];
    }
    free(cur);
    for (size_t u = 0; u < n; u++)
        qsort(nbr + off[u], off[u + 1] - off[u], sizeof(int32_t), cmp_i32);
    set_array((void**)&g->adj_off, off);
    set_array((void**)&g->adj_nbr, nbr);
    g->adj_nbr_size = 2 * m;
}

/* Stable LSD radix sort of (key, value) pairs by key (keys < 2^bits), 11-bit
 * digits, per-thread chunk histograms: equal keys keep their input order. */
static void par_radix_kv(uint32_t* key, uint32_t* val, size_t n, int bits, int nt) {
    enum { RB = 11, RD = 1 << RB };
    if (n < 65536) nt = 1;
    uint32_t* k2 = (uint32_t*)xmalloc((n ? n : 1) * sizeof(uint32_t));
    uint32_t* v2 = (uint32_t*)xmalloc((n ? n : 1) * sizeof(uint32_t));
    size_t* hist = (size_t*)xmalloc((size_t)nt * RD * sizeof(size_t));
    uint32_t *ks = key, *vs = val, *kd = k2, *vd = v2;
    for (int shift = 0; shift < bits; shift += RB) {
#pragma omp parallel for schedule(static, 1) num_threads(nt)
        for (int t = 0; t < nt; t++) {
            size_t lo, hi;
            chunk_of(n, nt, t, &lo, &hi);
            size_t* h = hist + (size_t)t * RD;
            memset(h, 0, RD * sizeof(size_t));
            for (size_t i = lo; i < hi; i++) h[(ks[i] >> shift) & (RD - 1)]++;
        }
        /* digit-major, thread-minor exclusive scan */
        size_t run = 0;
        for (int d = 0; d < RD; d++) {
            for (int t = 0; t < nt; t++) {
                size_t c = hist[(size_t)t * RD + d];
                hist[(size_t)t * RD + d] = run;
                run += c;
            }
        }
#pragma omp parallel for schedule(static, 1) num_threads(nt)
        for (int t = 0; t < nt; t++) {
            size_t lo, hi;
            chunk_of(n, nt, t, &lo, &hi);
            size_t* h = hist + (size_t)t * RD;
            for (size_t i = lo; i < hi; i++) {
                size_t p = h[(ks[i] >> shift) & (RD - 1)]++;
                kd[p] = ks[i];
                vd[p] = vs[i];
            }
        }
        uint32_t* t0 = ks; ks = kd; kd = t0;
        uint32_t* t1 = vs; vs = vd; vd = t1;
    }
    if (ks != key) {
        memcpy(key, ks, n * sizeof(uint32_t));
        memcpy(val, vs, n * sizeof(uint32_t));
    }
    free(k2);
    free(v2);
    free(hist);
}

/* out[u] for u in [0, V]: the first position of a sorted array of n node ids
 * whose id is >= u (a lower_bound, i.e. the CSR offsets).  Each out[u] is
 * written once, by the position where the ids reach u. */
static void lower_bound_offsets(const uint32_t* sorted, size_t n, size_t V, uint64_t* out,
                                int nt) {
    if (n == 0) {
        for (size_t u = 0; u <= V; u++) out[u] = 0;
        return;
    }
    if (n < 65536) nt = 1;
    for (size_t u = 0; u <= sorted[0] && u <= V; u++) out[u] = 0;
#pragma omp parallel for schedule(static) num_threads(nt)
    for (size_t i = 1; i < n; i++) {
        for (size_t u = (size_t)sorted[i - 1] + 1; u <= sorted[i] && u <= V; u++) out[u] = i;
    }
    for (size_t u = (size_t)sorted[n - 1] + 1; u <= V; u++) out[u] = n;
}

/* node_edge_index.cu:294-494 for one direction: stable order of entries by
 * node (the radix sort keeps input order within a node), CSR offsets
 * (node_edge_index.cu:254-292), node-timestamp group starts and per-node
 * exclusive group counts. */
static void build_direction(const orc_graph* g, const int32_t* keys, size_t n_entries,
                            int undirected_pairs, uint64_t** off_out,
                            uint64_t** idx_out, uint64_t** cnt_out,
                            uint64_t** grp_out, size_t* n_grp_out) {
    size_t V = g->active_size; /* node_count */
    const int nt = g->threads;
    uint32_t* node = (uint32_t*)xmalloc((n_entries ? n_entries : 1) * sizeof(uint32_t));
    uint32_t* ent = (uint32_t*)xmalloc((n_entries ? n_entries : 1) * sizeof(uint32_t));
#pragma omp parallel for schedule(static) num_threads(nt)
    for (size_t k = 0; k < n_entries; k++) {
        node[k] = (uint32_t)keys[k];
        ent[k] = (uint32_t)k;
    }
    int bits = 1;
    while (bits < 32 && ((size_t)1 << bits) < V) bits++;
    par_radix_kv(node, ent, n_entries, bits, nt);
    uint64_t* off = (uint64_t*)xmalloc((V + 1) * sizeof(uint64_t));
    lower_bound_offsets(node, n_entries, V, off, nt);
    uint64_t* idx = (uint64_t*)xmalloc((n_entries ? n_entries : 1) * sizeof(uint64_t));
#pragma omp parallel for schedule(static) num_threads(nt)
    for (size_t i = 0; i < n_entries; i++)
        idx[i] = undirected_pairs ? (uint64_t)(ent[i] / 2) : (uint64_t)ent[i];
    free(ent);
    /* group starts: a new node or a new timestamp within the node */
    const int gt = n_entries < 65536 ? 1 : nt;
    size_t* base = (size_t*)calloc((size_t)gt + 1, sizeof(size_t));
#pragma omp parallel for schedule(static, 1) num_threads(gt)
    for (int t = 0; t < gt; t++) {
        size_t lo, hi, c = 0;
        chunk_of(n_entries, gt, t, &lo, &hi);
        for (size_t i = lo; i < hi; i++)
            c += i == 0 || node[i] != node[i - 1] || g->ts[idx[i]] != g->ts[idx[i - 1]];
        base[t + 1] = c;
    }
    for (int t = 0; t < gt; t++) base[t + 1] += base[t];
    size_t ng = base[gt];
    uint64_t* grp = (uint64_t*)xmalloc((ng ? ng : 1) * sizeof(uint64_t));
    uint32_t* gnode = (uint32_t*)xmalloc((ng ? ng : 1) * sizeof(uint32_t));
#pragma omp parallel for schedule(static, 1) num_threads(gt)
    for (int t = 0; t < gt; t++) {
        size_t lo, hi, k = base[t];
        chunk_of(n_entries, gt, t, &lo, &hi);
        for (size_t i = lo; i < hi; i++) {
            if (i == 0 || node[i] != node[i - 1] || g->ts[idx[i]] != g->ts[idx[i - 1]]) {
                grp[k] = i;
                gnode[k] = node[i];
                k++;
            }
        }
    }
    free(base);
    /* cnt[u] = number of groups of nodes below u */
    uint64_t* cnt = (uint64_t*)xmalloc((V + 1) * sizeof(uint64_t));
    lower_bound_offsets(gnode, ng, V, cnt, nt);
    free(gnode);
    free(node);
    *off_out = off;
    *idx_out = idx;
    *cnt_out = cnt;
    *grp_out = grp;
    *n_grp_out = ng;
}

/* node_edge_index.cu:1329-1400 */
static void rebuild_node_index(orc_graph* g) {
    size_t E = g->E;
    g->off_size = g->active_size + 1;
    g->cnt_size = g->active_size + 1;
    free(g->out_off); free(g->in_off); free(g->out_idx); free(g->in_idx);
    free(g->out_cnt); free(g->in_cnt); free(g->out_grp); free(g->in_grp);
    g->out_off = g->in_off = g->out_idx = g->in_idx = NULL;
    g->out_cnt = g->in_cnt = g->out_grp = g->in_grp = NULL;
    g->n_out = g->n_in = g->g_out = g->g_in = 0;
    if (g->is_directed) {
        build_direction(g, g->src, E, 0, &g->out_off, &g->out_idx, &g->out_cnt,
                        &g->out_grp, &g->g_out);
        build_direction(g, g->dst, E, 0, &g->in_off, &g->in_idx, &g->in_cnt,
                        &g->in_grp, &g->g_in);
        g->n_out = E;
        g->n_in = E;
    } else {
        /* node_edge_index.cu:306-321: entry 2i = (i, src_i), 2i+1 = (i, dst_i) */
        int32_t* keys = (int32_t*)xmalloc(2 * E * sizeof(int32_t));
        for (size_t i = 0; i < E; i++) {
            keys[2 * i] = g->src[i];
            keys[2 * i + 1] = g->dst[i];
        }
        build_direction(g, keys, 2 * E, 1, &g->out_off, &g->out_idx, &g->out_cnt,
                        &g->out_grp, &g->g_out);
        free(keys);
        g->n_out = 2 * E;
    }
}

/* edge_data.cu:440-514 (global per-timestamp-group weights) */
static void update_global_weights(orc_graph* g) {
    size_t T = g->T;
    free(g->fwd_cum); free(g->bwd_cum);
    g->fwd_cum = g->bwd_cum = NULL;
    g->w_size = 0;
    if (g->E == 0) return;
    int64_t tmin = g->ts[0], tmax = g->ts[g->E - 1];
    double diff = (double)(tmax - tmin);
    double bound = g->timescale_bound;
    double scale = (bound > 0 && diff > 0) ? bound / diff : 1.0;
    double* f = (double*)xmalloc(T * sizeof(double));
    double* b = (double*)xmalloc(T * sizeof(double));
    for (size_t k = 0; k < T; k++) {
        size_t start = g->ts_group_offsets[k];
        double size = (double)(g->ts_group_offsets[k + 1] - start);
        int64_t t = g->ts[start];
        double tf = (double)(tmin - t), tb = (double)(t - tmax);
        double fs = bound > 0 ? tf * scale : tf;
        double bs = bound > 0 ? tb * scale : tb;
        f[k] = size * exp(fs);
        b[k] = size * exp(bs);
    }
    double fsum = 0, bsum = 0;
    for (size_t k = 0; k < T; k++) { fsum += f[k]; bsum += b[k]; }
    for (size_t k = 0; k < T; k++) { f[k] /= fsum; b[k] /= bsum; }
    for (size_t k = 1; k < T; k++) { f[k] += f[k - 1]; b[k] += b[k - 1]; }
    g->fwd_cum = f;
    g->bwd_cum = b;
    g->w_size = T;
}

/* node_edge_index.cu:500-640 for one direction. */
static void per_node_weights(const orc_graph* g, const uint64_t* cnt, const uint64_t* grp,
                             const uint64_t* idx, const uint64_t* off, size_t n_groups,
                             size_t node_cap, int compute_forward, double* fwd_out,
                             double* bwd_out) {
    if (n_groups == 0 || node_cap == 0) return;
    double bound = g->timescale_bound;
    for (size_t u = 0; u < node_cap; u++) {
        size_t s = cnt[u], e = cnt[u + 1];
        if (s >= e) continue;
        int64_t mn = g->ts[idx[grp[s]]];
        int64_t mx = g->ts[idx[grp[e - 1]]];
        double diff = (double)(mx - mn);
        double scale = (bound > 0 && diff > 0) ? bound / diff : 1.0;
        double fsum = 0, bsum = 0;
        for (size_t p = s; p < e; p++) {
            size_t es = grp[p];
            size_t ee = (p + 1 < e) ? grp[p + 1] : off[u + 1];
            double sz = (double)(ee - es);
            int64_t t = g->ts[idx[es]];
            double bsc = bound > 0 ? (double)(t - mx) * scale : (double)(t - mx);
            bwd_out[p] = sz * exp(bsc);
            bsum += bwd_out[p];
            if (compute_forward) {
                double fsc = bound > 0 ? (double)(mn - t) * scale : (double)(mn - t);
                fwd_out[p] = sz * exp(fsc);
                fsum += fwd_out[p];
            }
        }
        double fc = 0, bc = 0;
        for (size_t p = s; p < e; p++) {
            bc += bwd_out[p] / bsum;
            bwd_out[p] = bc;
            if (compute_forward) {
                fc += fwd_out[p] / fsum;
                fwd_out[p] = fc;
            }
        }
    }
}

/* node_edge_index.cu:644-684 */
static void update_node_weights(orc_graph* g) {
    free(g->out_fwd_w); free(g->out_bwd_w); free(g->in_bwd_w);
    g->out_fwd_w = (double*)xmalloc(g->g_out * sizeof(double));
    g->out_bwd_w = (double*)xmalloc(g->g_out * sizeof(double));
    g->in_bwd_w = NULL;
    size_t cap = g->off_size - 1;
    per_node_weights(g, g->out_cnt, g->out_grp, g->out_idx, g->out_off, g->g_out, cap, 1,
                     g->out_fwd_w, g->out_bwd_w);
    if (g->is_directed) {
        g->in_bwd_w = (double*)xmalloc(g->g_in * sizeof(double));
        per_node_weights(g, g->in_cnt, g->in_grp, g->in_idx, g->in_off, g->g_in, cap, 0,
                         NULL, g->in_bwd_w);
    }
}

/* temporal_graph.cu:158-220 with the validation of edge_data.cu:71-89.
 * Validation runs before any state changes. */
int orc_add_edges(orc_graph* g, const int32_t* src, const int32_t* dst,
                  const int64_t* ts, size_t n, const float* features,
                  size_t feature_dim) {
    g_err[0] = 0;
    if (n == 0) return 0; /* core/temporal_random_walk.cu:285 */
    if (features != NULL && feature_dim == 0) {
        snprintf(g_err, sizeof g_err, "edge_features provided but feature_dim is 0");
        return 1;
    }
    if (g->E != 0 && feature_dim != g->feat_dim) {
        snprintf(g_err, sizeof g_err, "feature_dim mismatch with existing data.feature_dim");
        return 1;
    }
    size_t eff_dim = g->E == 0 ? feature_dim : g->feat_dim;
    if (features == NULL && feature_dim != 0) {
        snprintf(g_err, sizeof g_err, "feature_dim must be 0 when edge_features is not provided");
        return 1;
    }
    if (eff_dim > 0 && features == NULL) {
        snprintf(g_err, sizeof g_err,
                 "edge features enabled; non-empty ingestion must provide edge_features");
        return 1;
    }
    int64_t mx = g->latest_timestamp;
    for (size_t i = 0; i < n; i++) if (ts[i] > mx) mx = ts[i];
    g->latest_timestamp = mx;

    size_t start = g->E, total = g->E + n;
    g->src = (int32_t*)realloc(g->src, total * sizeof(int32_t));
    g->dst = (int32_t*)realloc(g->dst, total * sizeof(int32_t));
    g->ts = (int64_t*)realloc(g->ts, total * sizeof(int64_t));
    memcpy(g->src + start, src, n * sizeof(int32_t));
    memcpy(g->dst + start, dst, n * sizeof(int32_t));
    memcpy(g->ts + start, ts, n * sizeof(int64_t));
    if (g->E == 0) g->feat_dim = feature_dim;
    if (g->feat_dim > 0) {
        g->feat = (float*)realloc(g->feat, total * g->feat_dim * sizeof(float));
        memcpy(g->feat + start * g->feat_dim, features, n * g->feat_dim * sizeof(float));
    }
    g->E = total;

    sort_and_merge(g, start);
    if (g->max_time_capacity > 0) delete_old_edges(g);
    populate_active_nodes(g);
    update_timestamp_groups(g);
    if (g->enable_tn2v) build_adjacency(g);
    rebuild_node_index(g);
    if (g->enable_weight) {
        update_global_weights(g);
        update_node_weights(g);
    }
    return 0;
}

/* Overwrite one cumulative-weight array (same length required).  fp64
 * weights are only reproducible to ~1e-15 across summation orders and libm
 * exp implementations, and picks on the flat tail of a cumulative array turn
 * ulp differences into different groups; tests therefore compare the weight
 * arrays within 1e-12 and then check the sampler bit-exactly on identical
 * weights by injecting the engine's arrays here. */
int orc_set_weights(orc_graph* g, const char* name, const double* data, size_t len) {
    double* dst = NULL;
    size_t n = 0;
    if (strcmp(name, "forward_cumulative_weights_exponential") == 0) { dst = g->fwd_cum; n = g->w_size; }
    else if (strcmp(name, "backward_cumulative_weights_exponential") == 0) { dst = g->bwd_cum; n = g->w_size; }
    else if (strcmp(name, "outbound_forward_cumulative_weights_exponential") == 0) { dst = g->out_fwd_w; n = g->g_out; }
    else if (strcmp(name, "outbound_backward_cumulative_weights_exponential") == 0) { dst = g->out_bwd_w; n = g->g_out; }
    else if (strcmp(name, "inbound_backward_cumulative_weights_exponential") == 0) { dst = g->in_bwd_w; n = g->g_in; }
    if (dst == NULL || n != len) return 1;
    memcpy(dst, data, len * sizeof(double));
    return 0;
}

int64_t orc_latest_timestamp(const orc_graph* g) { return g->latest_timestamp; }
int32_t orc_max_node_id(const orc_graph* g) { return g->max_node_id; }
size_t orc_feature_dim(const orc_graph* g) { return g->feat_dim; }

const void* orc_array(const orc_graph* g, const char* name, size_t* len, size_t* es) {
#define ARR(nm, ptr, n, sz)            \
    if (strcmp(name, nm) == 0) {       \
        *len = (ptr) ? (n) : 0;        \
        *es = (sz);                    \
        return (ptr);                  \
    }
    int w = g->enable_weight;
    ARR("sources", g->src, g->E, 4)
    ARR("targets", g->dst, g->E, 4)
    ARR("timestamps", g->ts, g->E, 8)
    ARR("edge_features", g->feat, g->E * g->feat_dim, 4)
    ARR("timestamp_group_offsets", g->ts_group_offsets, g->T + 1, 8)
    ARR("unique_timestamps", g->unique_ts, g->T, 8)
    ARR("active_node_ids", g->active, g->active_size, 4)
    ARR("node_group_outbound_offsets", g->out_off, g->off_size, 8)
    ARR("node_group_inbound_offsets", g->in_off, g->off_size, 8)
    ARR("node_ts_sorted_outbound_indices", g->out_idx, g->n_out, 8)
    ARR("node_ts_sorted_inbound_indices", g->in_idx, g->n_in, 8)
    ARR("count_ts_group_per_node_outbound", g->out_cnt, g->cnt_size, 8)
    ARR("count_ts_group_per_node_inbound", g->in_cnt, g->cnt_size, 8)
    ARR("node_ts_group_outbound_offsets", g->out_grp, g->g_out, 8)
    ARR("node_ts_group_inbound_offsets", g->in_grp, g->g_in, 8)
    ARR("forward_cumulative_weights_exponential", w ? g->fwd_cum : NULL, g->w_size, 8)
    ARR("backward_cumulative_weights_exponential", w ? g->bwd_cum : NULL, g->w_size, 8)
    ARR("outbound_forward_cumulative_weights_exponential", w ? g->out_fwd_w : NULL, g->g_out, 8)
    ARR("outbound_backward_cumulative_weights_exponential", w ? g->out_bwd_w : NULL, g->g_out, 8)
    ARR("inbound_backward_cumulative_weights_exponential", w ? g->in_bwd_w : NULL, g->g_in, 8)
    ARR("node_adj_offsets", g->adj_off, g->adj_off_size, 8)
    ARR("node_adj_neighbors", g->adj_nbr, g->adj_nbr_size, 4)
#undef ARR
    *len = 0;
    *es = 0;
    return NULL;
}

/* ------------------------------------------------------------------ */
/* Pickers: random/pickers.cuh:15-126                                  */
/* ------------------------------------------------------------------ */
int orc_pick_linear(int start, int end, int prioritize_end, double r) {
    if (start >= end) return -1;
    int len = end - start;
    double total = (double)len * ((double)len + 1.0) / 2.0;
    double scaled = total * r;
    double disc = 1.0 + 8.0 * scaled;
    double root = (-1.0 + sqrt(disc)) / 2.0;
    int index = (int)floor(root);
    if (prioritize_end) return start + (index < len - 1 ? index : len - 1);
    int rev = len - 1 - index;
    return start + (rev > 0 ? rev : 0);
}

int orc_pick_exponential_index(int start, int end, int prioritize_end, double r) {
    if (start >= end) return -1;
    int len = end - start;
    double k;
    if (len < 710) k = log1p(r * expm1((double)len)) - 1;
    else k = len + log(r) - 1;
    int ki = (int)(k + 1);
    int ri = ki < len - 1 ? ki : len - 1;
    if (ri < 0) ri = 0;
    return prioritize_end ? start + ri : start + (len - 1 - ri);
}

int orc_pick_uniform(int start, int end, double r) {
    if (start >= end) return -1;
    return start + (int)(r * (end - start));
}

int orc_pick_exponential_weights(const double* w, size_t wsize, size_t gs, size_t ge,
                                 double r, size_t slice_start) {
    if (gs >= ge || ge > wsize) return -1;
    double start_sum = gs > slice_start ? w[gs - 1] : 0.0;
    double end_sum = w[ge - 1];
    if (end_sum < start_sum) return -1;
    double target = start_sum + r * (end_sum - start_sum);
    size_t lo = gs, hi = ge;
    while (lo < hi) {
        size_t mid = lo + ((hi - lo) >> 1);
        if (w[mid] < target) lo = mid + 1; else hi = mid;
    }
    return (int)lo;
}

static int is_index_picker(int p) {
    return p == ORC_LINEAR || p == ORC_UNIFORM || p == ORC_EXPONENTIAL_INDEX ||
           p == ORC_TEST_FIRST || p == ORC_TEST_LAST;
}

static int pick_index(int picker, int start, int end, int prioritize_end, double r) {
    switch (picker) {
        case ORC_LINEAR: return orc_pick_linear(start, end, prioritize_end, r);
        case ORC_EXPONENTIAL_INDEX: return orc_pick_exponential_index(start, end, prioritize_end, r);
        case ORC_UNIFORM: return orc_pick_uniform(start, end, r);
        case ORC_TEST_FIRST: return start;
        case ORC_TEST_LAST: return end - 1;
        default: return -1;
    }
}

static int pick_weight(int picker, const double* w, size_t wsize, size_t gs, size_t ge,
                       double r, size_t slice_start) {
    if (picker != ORC_EXPONENTIAL_WEIGHT && picker != ORC_TEMPORAL_NODE2VEC) return -1;
    return orc_pick_exponential_weights(w, wsize, gs, ge, r, slice_start);
}

/* graph/temporal_node2vec_helpers.cuh:46-70 */
double orc_derive_uniform(double a, double b, int counter) {
    uint64_t ua, ub;
    memcpy(&ua, &a, 8);
    memcpy(&ub, &b, 8);
    uint64_t s = ua * 0x9E3779B97F4A7C15ULL;
    s ^= ub + 0xBF58476D1CE4E5B9ULL;
    s += (uint64_t)counter * 0x94D049BB133111EBULL;
    s ^= s >> 30;
    s *= 0xBF58476D1CE4E5B9ULL;
    s ^= s >> 27;
    s *= 0x94D049BB133111EBULL;
    s ^= s >> 31;
    return (double)(s >> 11) * (1.0 / 9007199254740992.0);
}

/* ------------------------------------------------------------------ */
/* Selectors: graph/edge_selectors.cuh                                 */
/* ------------------------------------------------------------------ */
typedef struct { int u, i; int64_t ts; int64_t eid; } orc_edge;
static const orc_edge NO_EDGE = {-1, -1, -1, -1};

/* edge_selectors.cuh:177-275 with timestamp == -1 (the only call made by
 * the walk loop). */
static orc_edge edge_at(const orc_graph* g, int forward, int picker, double rg, double re) {
    if (g->E == 0 || g->T == 0) return NO_EDGE;
    long group;
    if (is_index_picker(picker)) {
        int idx = pick_index(picker, 0, (int)g->T, !forward, rg);
        if (idx == -1 || (size_t)idx >= g->T) return NO_EDGE;
        group = idx;
    } else {
        const double* w = forward ? g->fwd_cum : g->bwd_cum;
        size_t ws = g->enable_weight ? g->w_size : 0;
        group = pick_weight(picker, w, ws, 0, g->T, rg, 0);
        if (group == -1) return NO_EDGE;
        /* edge_selectors.cuh:38-43: a group index past the end is an empty range */
        if ((size_t)group >= g->T) return NO_EDGE;
    }
    size_t from = g->ts_group_offsets[group], to = g->ts_group_offsets[group + 1];
    if (from == to) return NO_EDGE;
    size_t e = from + (size_t)(int)(re * (int)(to - from));
    orc_edge out = {g->src[e], g->dst[e], g->ts[e], (int64_t)e};
    return out;
}

typedef struct {
    const uint64_t* cnt;
    const uint64_t* grp;
    const uint64_t* idx;
    size_t idx_size;
    const uint64_t* off;
    const double* w;
    size_t w_size;
} orc_dir_view;

static orc_dir_view dir_view(const orc_graph* g, int forward) {
    orc_dir_view v;
    int use_in = !forward && g->is_directed;
    v.cnt = use_in ? g->in_cnt : g->out_cnt;
    v.grp = use_in ? g->in_grp : g->out_grp;
    v.idx = use_in ? g->in_idx : g->out_idx;
    v.idx_size = use_in ? g->n_in : g->n_out;
    v.off = use_in ? g->in_off : g->out_off;
    if (forward) {
        v.w = g->out_fwd_w;
        v.w_size = g->enable_weight ? g->g_out : 0;
    } else if (g->is_directed) {
        v.w = g->in_bwd_w;
        v.w_size = g->enable_weight ? g->g_in : 0;
    } else {
        v.w = g->out_bwd_w;
        v.w_size = g->enable_weight ? g->g_out : 0;
    }
    return v;
}

/* edge_selectors.cuh:66-120 (first_ts == nullptr: double-indirect probe) */
static void filter_valid_groups(const orc_graph* g, const uint64_t* grp_base, const uint64_t* idx,
                                int G, int64_t t, int64_t cutoff, int forward, int* vb, int* ve) {
    *vb = 0;
    *ve = G;
    if (t == -1 && cutoff == NO_WALK_CUTOFF) return;
#define TS_OF(p) (g->ts[idx[grp_base[(p)]]])
    if (t != -1) {
        int lo = 0, hi = G;
        if (forward) {
            while (lo < hi) {
                int mid = lo + ((hi - lo) >> 1);
                if (t < TS_OF(mid)) hi = mid; else lo = mid + 1;
            }
            *vb = lo;
        } else {
            while (lo < hi) {
                int mid = lo + ((hi - lo) >> 1);
                if (TS_OF(mid) < t) lo = mid + 1; else hi = mid;
            }
            *ve = lo;
        }
    }
    if (cutoff != NO_WALK_CUTOFF) {
        int lo = *vb, hi = *ve;
        while (lo < hi) {
            int mid = lo + ((hi - lo) >> 1);
            if (TS_OF(mid) < cutoff) lo = mid + 1; else hi = mid;
        }
        *ve = lo;
    }
#undef TS_OF
}

static int adjacent(const orc_graph* g, int prev, int cand) {
    /* temporal_node2vec_helpers.cuh:81-107 */
    if (!g->enable_tn2v || g->adj_off == NULL) return 0;
    if (prev < 0 || (size_t)prev + 1 >= g->adj_off_size) return 0;
    size_t s = g->adj_off[prev], e = g->adj_off[prev + 1];
    if (s >= e) return 0;
    size_t lo = s, hi = e;
    while (lo < hi) {
        size_t mid = lo + ((hi - lo) >> 1);
        if (g->adj_nbr[mid] < cand) lo = mid + 1; else hi = mid;
    }
    return lo < e && g->adj_nbr[lo] == cand;
}

/* temporal_node2vec_helpers.cuh:127-199 */
static long tn2v_pick(const orc_graph* g, const orc_dir_view* v, int forward, int node, int prev,
                      size_t vb, size_t ve, size_t gb, size_t ge, double rg, double re) {
    if (vb >= ve || prev == -1) return -1;
    double bmax = 1.0;
    if (g->inv_p > bmax) bmax = g->inv_p;
    if (g->inv_q > bmax) bmax = g->inv_q;
    double inv_bmax = 1.0 / bmax;
    long last = -1;
    for (int retry = 0; retry < NODE2VEC_MAX_RETRIES; ++retry) {
        double gr = orc_derive_uniform(rg, re, retry * 3 + 0);
        double er = orc_derive_uniform(rg, re, retry * 3 + 1);
        double ar = orc_derive_uniform(rg, re, retry * 3 + 2);
        long gp = orc_pick_exponential_weights(v->w, v->w_size, vb, ve, gr, gb);
        if (gp == -1) return -1;
        /* one past the node's last group: the reference reads an empty range
         * (walk_step_helpers.cuh:19-38) -- except for the globally last group,
         * where it reads past the array */
        if ((size_t)gp >= ge) continue;
        size_t es = v->grp[gp];
        size_t ee = ((size_t)gp + 1 < ge) ? v->grp[gp + 1] : v->off[node + 1];
        if (es >= ee) continue;
        size_t local = (size_t)(er * (double)(ee - es));
        size_t pick = es + (local < ee - es ? local : ee - es - 1);
        long eid = (long)v->idx[pick];
        int cand;
        if (g->is_directed) cand = forward ? g->dst[eid] : g->src[eid];
        else cand = g->src[eid] == node ? g->dst[eid] : g->src[eid];
        double beta = (cand == prev) ? g->inv_p : (adjacent(g, prev, cand) ? 1.0 : g->inv_q);
        last = eid;
        if (ar < beta * inv_bmax) return eid;
    }
    return last;
}

/* edge_selectors.cuh:277-443 */
static orc_edge node_edge_at(const orc_graph* g, int forward, int picker, int node, int64_t t,
                             int64_t cutoff, int prev, double rg, double re) {
    if (!(node >= 0 && (size_t)node < g->active_size && g->active[node] == 1)) return NO_EDGE;
    orc_dir_view v = dir_view(g, forward);
    size_t gb = v.cnt[node], ge = v.cnt[node + 1];
    if (gb == ge) return NO_EDGE;
    int G = (int)(ge - gb);
    long gpos;
    if (picker == ORC_TEMPORAL_NODE2VEC) {
        int lb, le;
        filter_valid_groups(g, v.grp + gb, v.idx, G, t, cutoff, forward, &lb, &le);
        if (lb >= le) return NO_EDGE;
        size_t vb = gb + (size_t)lb, ve = gb + (size_t)le;
        if (prev == -1) {
            gpos = orc_pick_exponential_weights(v.w, v.w_size, vb, ve, rg, gb);
            if (gpos == -1) return NO_EDGE;
        } else {
            long eid = tn2v_pick(g, &v, forward, node, prev, vb, ve, gb, ge, rg, re);
            if (eid == -1) return NO_EDGE;
            orc_edge out = {g->src[eid], g->dst[eid], g->ts[eid], eid};
            return out;
        }
    } else {
        int vb, ve;
        filter_valid_groups(g, v.grp + gb, v.idx, G, t, cutoff, forward, &vb, &ve);
        if (vb >= ve) return NO_EDGE;
        long local;
        if (is_index_picker(picker)) {
            int avail = ve - vb;
            int index = pick_index(picker, 0, avail, !forward, rg);
            if (index == -1 || index >= avail) return NO_EDGE;
            local = forward ? (long)(vb + index) : (long)(ve - 1 - (avail - index - 1));
        } else {
            int p = pick_weight(picker, v.w, v.w_size, gb + vb, gb + ve, rg, gb);
            if (p == -1) return NO_EDGE;
            local = (long)p - (long)gb;
        }
        gpos = local + (long)gb;
    }
    /* one past the node's last group reads as an empty range in the reference
     * (edge_selectors.cuh:416-426), except past the globally last group */
    if ((size_t)gpos >= ge) return NO_EDGE;
    size_t es = v.grp[gpos];
    size_t ee = ((size_t)gpos + 1 < ge) ? v.grp[gpos + 1] : v.off[node + 1];
    if (es >= ee || es >= v.idx_size || ee > v.idx_size) return NO_EDGE;
    long eid = (long)v.idx[es + (size_t)(int)(re * (int)(ee - es))];
    orc_edge out = {g->src[eid], g->dst[eid], g->ts[eid], eid};
    return out;
}

/* Selector entry points for tests (the reference's test shims
 * test/test_temporal_graph_utils.h:56-213 call the selectors with given
 * draws).  out = {u, i, ts, edge_id}. */
void orc_node_edge_at(const orc_graph* g, int forward, int picker, int node, int64_t t,
                      int64_t cutoff, int prev, double rg, double re, int64_t* out) {
    orc_edge e = node_edge_at(g, forward, picker, node, t, cutoff, prev, rg, re);
    out[0] = e.u; out[1] = e.i; out[2] = e.ts; out[3] = e.eid;
}

void orc_edge_at(const orc_graph* g, int forward, int picker, double rg, double re,
                 int64_t* out) {
    orc_edge e = edge_at(g, forward, picker, rg, re);
    out[0] = e.u; out[1] = e.i; out[2] = e.ts; out[3] = e.eid;
}

/* core/temporal_random_walk_cpu.cuh:19-131 plus WalkSetView::add_hop /
 * reverse_walk (data/walk_set/walk_set_view.cuh:27-80). */
static void one_walk(const orc_graph* g, size_t w, int L, int walk_bias, int start_bias,
                     int forward, const int32_t* starts, const int64_t* cutoffs,
                     const double* draws, int pad, int32_t* nodes, int64_t* tss,
                     uint64_t* lens, int64_t* eids) {
    int32_t* wn = nodes + w * (size_t)L;
    int64_t* wt = tss + w * (size_t)L;
    int64_t* we = eids + w * (size_t)(L > 0 ? L - 1 : 0);
    for (int k = 0; k < L; k++) { wn[k] = pad; wt[k] = -1; }
    for (int k = 0; k + 1 < L; k++) we[k] = -1;
    lens[w] = 0;
    if (L == 0) return;
    const double* r = draws + w + w * (size_t)L * 2;
    int64_t cutoff = cutoffs ? cutoffs[w] : NO_WALK_CUTOFF;
    int start = starts[w];
    orc_edge se;
    if (start == -1) se = edge_at(g, forward, start_bias, r[0], r[1]);
    else se = node_edge_at(g, forward, start_bias, start, -1, cutoff, -1, r[0], r[1]);
    if (se.i == -1) return;
    size_t len = 0;
#define ADD_HOP(node, t, e)                                   \
    do {                                                      \
        wn[len] = (node);                                     \
        wt[len] = (t);                                        \
        if ((e) != -1 && len > 0) we[len - 1] = (e);          \
        len++;                                                \
    } while (0)
    int cur, prev = -1;
    int64_t cur_t = forward ? INT64_MIN : INT64_MAX;
    if (g->is_directed) {
        ADD_HOP(forward ? se.u : se.i, cur_t, (int64_t)-1);
        cur = forward ? se.i : se.u;
    } else {
        int picked = start != -1 ? start : (r[2] >= 0.5 ? se.u : se.i);
        ADD_HOP(picked, cur_t, (int64_t)-1);
        cur = picked == se.u ? se.i : se.u;
    }
    cur_t = se.ts;
    int64_t cur_e = se.eid;
    int walk_len = 1;
    while (walk_len < L && cur != pad) {
        size_t s = (size_t)walk_len * 2 + 1;
        ADD_HOP(cur, cur_t, cur_e);
        orc_edge ne = node_edge_at(g, forward, walk_bias, cur, cur_t, cutoff, prev, r[s], r[s + 1]);
        if (ne.ts == -1) {
            cur = pad;
            continue;
        }
        prev = cur;
        if (g->is_directed) cur = forward ? ne.i : ne.u;
        else cur = (cur == ne.u) ? ne.i : ne.u;
        cur_t = ne.ts;
        cur_e = ne.eid;
        walk_len++;
    }
#undef ADD_HOP
    lens[w] = len;
    if (!forward && len > 1) {
        for (size_t i = 0; i < len / 2; i++) {
            int32_t tn = wn[i]; wn[i] = wn[len - 1 - i]; wn[len - 1 - i] = tn;
            int64_t tt = wt[i]; wt[i] = wt[len - 1 - i]; wt[len - 1 - i] = tt;
        }
        size_t ec = len - 1;
        for (size_t i = 0; i < ec / 2; i++) {
            int64_t te = we[i]; we[i] = we[ec - 1 - i]; we[ec - 1 - i] = te;
        }
    }
}

void orc_walks(const orc_graph* g, int L, int walk_bias, int start_bias, int forward,
               const int32_t* starts, const int64_t* cutoffs, size_t n, const double* draws,
               int pad, int32_t* nodes, int64_t* tss, uint64_t* lens, int64_t* eids,
               int num_threads) {
    /* core/temporal_random_walk_cpu.cuh:168-171 */
    if (start_bias == ORC_TEMPORAL_NODE2VEC) start_bias = ORC_EXPONENTIAL_WEIGHT;
#ifdef _OPENMP
    if (num_threads <= 0) num_threads = omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 256) num_threads(num_threads)
#endif
    for (long w = 0; w < (long)n; w++)
        one_walk(g, (size_t)w, L, walk_bias, start_bias, forward, starts, cutoffs, draws, pad,
                 nodes, tss, lens, eids);
}

/* ---- the engine's normal-mode draw stream (see trw_oracle.h) ------------- */

void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; r++) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n1 = (uint32_t)p1;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        const uint32_t n3 = (uint32_t)p0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

static double unit_from_bits(uint32_t lo, uint32_t hi) {
    const uint64_t m = (((uint64_t)hi << 32) | lo) >> 12;
    return ((double)m + 0.5) * 0x1p-52;
}

void orc_philox_draws(uint64_t seed, uint64_t walk0, uint64_t n, int L, double* out) {
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    const size_t stride = 1 + 2 * (size_t)L;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (long i = 0; i < (long)n; i++) {
        const uint64_t w = walk0 + (uint64_t)i;
        double* d = out + (size_t)i * stride;
        uint32_t ctr[4] = {0u, (uint32_t)w, (uint32_t)(w >> 32), 0u}, o[4];
        orc_philox4x32_10(ctr, key, o);
        d[0] = unit_from_bits(o[0], o[1]);
        for (int p = 1; p <= L; p++) {
            ctr[0] = (uint32_t)p;
            orc_philox4x32_10(ctr, key, o);
            d[2 * p - 1] = unit_from_bits(o[0], o[1]);
            d[2 * p] = unit_from_bits(o[2], o[3]);
        }
    }
}

void orc_philox_shuffle_keys(uint64_t seed, uint64_t n, uint32_t* out) {
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    for (uint64_t i = 0; i < n; i++) {
        const uint32_t ctr[4] = {(uint32_t)i, (uint32_t)(i >> 32), 0x5348u, 0u};
        uint32_t o[4];
        orc_philox4x32_10(ctr, key, o);
        out[i] = o[0];
    }
}
