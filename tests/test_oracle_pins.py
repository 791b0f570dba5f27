"""Pins of the oracle (CPU only).

Each check is chosen so that a plausible mistake in the restatement (a wrong
tie order, an off-by-one in a group offset, a reversed picker, a dropped term
in a weight) fails it:

* literal expectations of the reference's own tests (test/test_temporal_graph.cpp,
  test/test_edge_data.cpp, test/test_node_edge_index.cpp,
  test/test_edge_data_weights.cpp, test/test_temporal_node2vec.cpp,
  test/test_random_picker.cpp), restated as values;
* brute force on random inputs (numpy stable sorts);
* closed forms of the pickers (inverse CDFs) on fine deterministic grids;
* the reference's own CPU code compiled into oracle/_ref (node index, per-node
  weights, the walk loop with its selectors, pickers and node2vec sampler).
"""
import math

import numpy as np
import pytest

from oracle import pyoracle as po
from tests import graphs


def _graph(edges_batches, directed=True, cap=-1, weights=False, tn2v=False, bound=-1.0, p=1.0,
           q=1.0):
    g = po.OracleGraph(directed, cap, weights, tn2v, bound, p, q)
    for batch in edges_batches:
        a = np.asarray(batch, dtype=np.int64).reshape(-1, 3)
        g.add_edges(a[:, 0].astype(np.int32), a[:, 1].astype(np.int32), a[:, 2])
    return g


# ---- edge store (test_temporal_graph.cpp:56-149) ------------------------------

def test_maintain_sorted_order():
    g = _graph([[(10, 20, 200), (20, 30, 100)]])
    assert list(g.array("timestamps")) == [100, 200]
    g.add_edges(np.array([30, 40], np.int32), np.array([40, 50], np.int32),
                np.array([150, 250], np.int64))
    assert list(g.array("timestamps")) == [100, 150, 200, 250]
    g.add_edges(np.array([50, 60, 70], np.int32), np.array([60, 70, 80], np.int32),
                np.array([150, 200, 175], np.int64))
    assert list(g.array("timestamps")) == [100, 150, 150, 175, 200, 200, 250]
    # ties keep insertion order: the old 150 (30->40) precedes the new one (50->60)
    assert list(g.array("sources")) == [20, 30, 50, 70, 10, 60, 40]


def test_time_window():
    g = _graph([[(1, 2, 100), (2, 3, 150), (3, 4, 249)]], cap=100)
    assert list(g.array("timestamps")) == [150, 249]


def test_edge_addition_edge_cases():
    g = _graph([])
    assert g.array("timestamps").size == 0
    g.add_edges(np.array([1], np.int32), np.array([2], np.int32), np.array([100], np.int64))
    g.add_edges(np.array([1, 2, 3], np.int32), np.array([2, 3, 4], np.int32),
                np.array([100, 100, 100], np.int64))
    assert g.array("timestamps").size == 4
    g.add_edges(np.array([1], np.int32), np.array([2], np.int32),
                np.array([np.iinfo(np.int64).max], np.int64))
    assert g.array("timestamps").size == 5


def test_node_deletion():
    g = _graph([[(1, 2, 100), (2, 3, 100), (3, 1, 100)]], cap=100)
    assert np.count_nonzero(g.array("active_node_ids")) == 3
    g.add_edges(np.array([4], np.int32), np.array([5], np.int32), np.array([250], np.int64))
    ids = np.nonzero(g.array("active_node_ids"))[0]
    assert list(ids) == [4, 5]


# ---- timestamp groups (test_edge_data.cpp:64-172) -------------------------------

def test_timestamp_groups_literals():
    g = _graph([[(100, 200, 100)]])
    assert list(g.array("timestamp_group_offsets")) == [0, 1]
    assert g.max_node_id == 200
    g = _graph([[(100, 200, 100), (200, 300, 100), (300, 400, 100)]])
    assert list(g.array("timestamp_group_offsets")) == [0, 3]
    g = _graph([[(1, 2, 100), (2, 3, 200), (3, 4, 300)]])
    assert list(g.array("timestamp_group_offsets")) == [0, 1, 2, 3]
    assert g.max_node_id == 4
    g = _graph([[(100, 200, 100), (200, 300, 100), (300, 400, 200), (400, 500, 300),
                 (500, 600, 300)]])
    assert list(g.array("timestamp_group_offsets")) == [0, 2, 3, 5]
    assert list(g.array("unique_timestamps")) == [100, 200, 300]


# ---- node index (test_node_edge_index.cpp:85-197) -------------------------------

def test_node_index_directed_literals():
    g = _graph([[(10, 20, 100), (10, 30, 100), (10, 20, 200), (20, 30, 300), (20, 10, 300)]])
    src, dst, ts = g.array("sources"), g.array("targets"), g.array("timestamps")
    off = g.array("node_group_outbound_offsets")
    out_idx = g.array("node_ts_sorted_outbound_indices")
    assert off[11] - off[10] == 3 and all(src[out_idx[i]] == 10 for i in range(off[10], off[11]))
    ioff = g.array("node_group_inbound_offsets")
    in_idx = g.array("node_ts_sorted_inbound_indices")
    assert ioff[21] - ioff[20] == 2 and all(dst[in_idx[i]] == 20 for i in range(ioff[20], ioff[21]))
    cnt = g.array("count_ts_group_per_node_outbound")
    grp = g.array("node_ts_group_outbound_offsets")
    gs, ge = cnt[10], cnt[11]
    assert ge - gs == 2
    g0s, g0e = grp[gs], grp[gs + 1]
    assert g0e - g0s == 2 and all(ts[out_idx[i]] == 100 for i in range(g0s, g0e))
    g1s, g1e = grp[gs + 1], off[11]
    assert g1e - g1s == 1 and ts[out_idx[g1s]] == 200 and dst[out_idx[g1s]] == 20


def test_node_index_undirected_literals():
    g = _graph([[(100, 200, 1000), (100, 300, 1000), (100, 200, 2000), (200, 300, 3000)]],
               directed=False)
    off = g.array("node_group_outbound_offsets")
    assert off[101] - off[100] == 3 and off[201] - off[200] == 3
    assert g.array("node_group_inbound_offsets").size == 0
    cnt = g.array("count_ts_group_per_node_outbound")
    grp = g.array("node_ts_group_outbound_offsets")
    idx = g.array("node_ts_sorted_outbound_indices")
    ts = g.array("timestamps")
    gs, ge = cnt[100], cnt[101]
    assert ge - gs == 2
    assert grp[gs + 1] - grp[gs] == 2 and ts[idx[grp[gs]]] == 1000
    assert off[101] - grp[gs + 1] == 1 and ts[idx[grp[gs + 1]]] == 2000


# ---- brute force ------------------------------------------------------------------

@pytest.mark.parametrize("directed", [True, False])
def test_store_and_index_brute_force(directed):
    rng = np.random.default_rng(21)
    batches = []
    for k in range(4):
        n = 3000
        batches.append((rng.integers(0, 300, n).astype(np.int32),
                        rng.integers(0, 300, n).astype(np.int32),
                        rng.integers(k * 100, k * 100 + 250, n).astype(np.int64)))
    cap = 200
    g = po.OracleGraph(directed, cap)
    all_s, all_d, all_t = [np.zeros(0, np.int32)] * 2 + [np.zeros(0, np.int64)]
    latest = 0
    for s, d, t in batches:
        g.add_edges(s, d, t)
        latest = max(latest, int(t.max()))
        cs, cd, ct = np.concatenate([all_s, s]), np.concatenate([all_d, d]), np.concatenate([all_t, t])
        order = np.argsort(ct, kind="stable")
        cs, cd, ct = cs[order], cd[order], ct[order]
        keep = ct > latest - cap
        all_s, all_d, all_t = cs[keep], cd[keep], ct[keep]
        assert np.array_equal(g.array("sources"), all_s)
        assert np.array_equal(g.array("targets"), all_d)
        assert np.array_equal(g.array("timestamps"), all_t)
    # node index by brute force
    E = len(all_t)
    if directed:
        keys, vals = all_s, np.arange(E)
    else:
        keys = np.empty(2 * E, np.int32)
        keys[0::2], keys[1::2] = all_s, all_d
        vals = np.repeat(np.arange(E), 2)
    order = np.argsort(keys, kind="stable")
    assert np.array_equal(g.array("node_ts_sorted_outbound_indices"), vals[order])
    V = max(all_s.max(), all_d.max()) + 1
    off = np.searchsorted(keys[order], np.arange(V + 1), side="left")
    assert np.array_equal(g.array("node_group_outbound_offsets"), off)
    sk, st = keys[order], all_t[vals[order]]
    flags = np.ones(len(sk), bool)
    flags[1:] = (sk[1:] != sk[:-1]) | (st[1:] != st[:-1])
    assert np.array_equal(g.array("node_ts_group_outbound_offsets"), np.nonzero(flags)[0])
    cnt = np.concatenate([[0], np.cumsum(np.bincount(sk[flags], minlength=V))])
    assert np.array_equal(g.array("count_ts_group_per_node_outbound"), cnt)


# ---- global weights (test_edge_data_weights.cpp:144-173, 374-406) ------------------

def _individual(cum):
    return np.diff(np.concatenate([[0.0], cum]))


def test_global_weight_decay_and_sums():
    g = _graph([[(1, 2, 10), (2, 3, 20), (3, 4, 30)]], weights=True)
    f = _individual(g.array("forward_cumulative_weights_exponential"))
    b = _individual(g.array("backward_cumulative_weights_exponential"))
    u = g.array("unique_timestamps")
    for i in range(len(u) - 1):
        dt = u[i + 1] - u[i]
        assert math.isclose(math.log(f[i + 1] / f[i]), -dt, abs_tol=1e-6)
        assert math.isclose(math.log(b[i + 1] / b[i]), dt, abs_tol=1e-6)
    assert math.isclose(g.array("forward_cumulative_weights_exponential")[-1], 1.0, abs_tol=1e-12)


def test_global_weight_timescale():
    g = _graph([[(1, 2, 100), (2, 3, 300), (3, 4, 700)]], weights=True, bound=2.0)
    f = _individual(g.array("forward_cumulative_weights_exponential"))
    b = _individual(g.array("backward_cumulative_weights_exponential"))
    u = g.array("unique_timestamps")
    scale = 2.0 / 600.0
    for i in range(len(u) - 1):
        dt = float(u[i + 1] - u[i])
        assert math.isclose(f[i + 1] / f[i], math.exp(-dt * scale), abs_tol=1e-6)
        assert math.isclose(b[i + 1] / b[i], math.exp(dt * scale), abs_tol=1e-6)


def test_global_weights_group_size_term():
    # two edges in the first group: its weight carries the factor 2
    g = _graph([[(1, 2, 10), (3, 4, 10), (2, 3, 11)]], weights=True)
    f = _individual(g.array("forward_cumulative_weights_exponential"))
    assert math.isclose(f[0] / f[1], 2.0 * math.e, rel_tol=1e-12)


# ---- pickers: closed forms on deterministic grids ---------------------------------

GRID = (np.arange(200_000) + 0.5) / 200_000


def _hist(pick, n, prioritize_end):
    L = po.lib()
    c = np.zeros(n)
    for r in GRID[::20]:
        c[pick(0, n, prioritize_end, float(r))] += 1
    return c / c.sum()


def test_linear_picker_closed_form():
    L = po.lib()
    for n in (1, 2, 7):
        h = _hist(L.orc_pick_linear, n, 1)
        w = np.arange(1, n + 1, dtype=float)
        np.testing.assert_allclose(h, w / w.sum(), atol=2e-3)
        h = _hist(L.orc_pick_linear, n, 0)
        np.testing.assert_allclose(h, (w / w.sum())[::-1], atol=2e-3)


def test_exponential_index_picker_closed_form():
    L = po.lib()
    e = math.e
    h = _hist(L.orc_pick_exponential_index, 2, 1)
    assert abs(h[1] - (e - 1) * e / (e * e - 1)) < 2e-3  # test_random_picker.cpp:188-191
    for n in (3, 6):
        h = _hist(L.orc_pick_exponential_index, n, 1)
        w = np.exp(np.arange(n, dtype=float))
        np.testing.assert_allclose(h, w / w.sum(), atol=2e-3)
        h = _hist(L.orc_pick_exponential_index, n, 0)
        np.testing.assert_allclose(h, (w / w.sum())[::-1], atol=2e-3)
    # large ranges use the n + log(r) - 1 branch: still the last index for r -> 1
    assert L.orc_pick_exponential_index(0, 1000, 1, 0.999999) == 999
    assert L.orc_pick_exponential_index(0, 1000, 0, 0.999999) == 0


def test_uniform_and_weight_pickers():
    L = po.lib()
    assert L.orc_pick_uniform(3, 7, 0.0) == 3 and L.orc_pick_uniform(3, 7, 0.999) == 6
    assert L.orc_pick_uniform(5, 5, 0.3) == -1
    cum = np.array([0.1, 0.3, 0.6, 1.0])
    c = np.zeros(4)
    for r in GRID[::20]:
        c[L.orc_pick_exponential_weights(cum.ctypes.data, 4, 0, 4, float(r), 0)] += 1
    np.testing.assert_allclose(c / c.sum(), [0.1, 0.2, 0.3, 0.4], atol=2e-3)
    # a slice starting inside the CDF renormalises to its own mass
    c = np.zeros(4)
    for r in GRID[::20]:
        c[L.orc_pick_exponential_weights(cum.ctypes.data, 4, 2, 4, float(r), 0)] += 1
    np.testing.assert_allclose(c[2:] / c.sum(), [3 / 7, 4 / 7], atol=2e-3)


# ---- node2vec (test_temporal_node2vec.cpp:74-80, 150-203) ---------------------------

def test_node2vec_pq_distribution():
    V, P, N, F = 0, 1, 2, 3
    g = _graph([[(V, P, 100), (V, N, 100), (V, F, 100), (P, N, 50)]], weights=True, tn2v=True,
               p=2.0, q=0.5)
    rng = np.random.default_rng(5)
    counts = {P: 0, N: 0, F: 0}
    n = 20_000
    for rg, re in rng.random((n, 2)):
        u, i, t, e = g.node_edge_at(V, "TemporalNode2Vec", prev=P, rg=rg, re=re)
        assert u == V
        counts[i] += 1
    assert abs(counts[P] / n - 1 / 7) < 0.015
    assert abs(counts[N] / n - 2 / 7) < 0.015
    assert abs(counts[F] / n - 4 / 7) < 0.015


def test_node2vec_adjacency_csr():
    g = _graph([[(0, 1, 10), (0, 2, 10), (3, 0, 20), (1, 2, 30), (0, 1, 40)]], tn2v=True)
    off = g.array("node_adj_offsets")
    nbr = g.array("node_adj_neighbors")
    lists = [list(nbr[off[u]:off[u + 1]]) for u in range(len(off) - 1)]
    assert lists == [[1, 1, 2, 3], [0, 0, 2], [0, 1], [0]]


# ---- the reference's own code (oracle/_ref) -----------------------------------------

@pytest.mark.skipif(not po.ref_available(), reason="oracle/_ref not built (reference absent)")
@pytest.mark.parametrize("directed", [True, False])
def test_oracle_matches_compiled_reference(directed):
    rng = np.random.default_rng(17 if directed else 18)
    n, V = 12_000, 400
    src = rng.integers(0, V, n).astype(np.int32)
    dst = rng.integers(0, V, n).astype(np.int32)
    ts = rng.integers(0, 2_000, n).astype(np.int64)
    og = po.OracleGraph(directed, -1, True, True, 20.0, 0.5, 2.0)
    og.add_edges(src[:7000], dst[:7000], ts[:7000])
    og.add_edges(src[7000:], dst[7000:], ts[7000:])
    rg = po.RefGraph(og)
    for name in po.NODE_INDEX_ARRAYS:
        assert np.array_equal(og.array(name), rg.array(name)), name
    for name in po.NODE_WEIGHT_ARRAYS:
        a, b = og.array(name), rg.array(name)
        assert a.shape == b.shape
        np.testing.assert_allclose(a, b, rtol=1e-12, atol=0, err_msg=name)
        rg_w = b
        if a.size:
            og.set_weights(name, rg_w)  # identical weights -> walks must agree bit-exactly
    L = 14
    for picker in ["Uniform", "Linear", "ExponentialIndex", "ExponentialWeight", "TemporalNode2Vec"]:
        for forward in (True, False):
            for constrained in (False, True):
                nw = 1500
                starts = (rng.integers(0, V, nw) if constrained else -np.ones(nw)).astype(np.int32)
                cut = None
                if constrained:
                    cut = rng.integers(0, 2_500, nw).astype(np.int64)
                    cut[::3] = -1
                dr = rng.random(nw * (1 + 2 * L))
                a = og.walks(L, picker, picker, forward, starts, dr, cutoffs=cut)
                b = rg.walks(L, picker, picker, forward, starts, dr, cutoffs=cut)
                for k in ("nodes", "timestamps", "lens", "edge_ids"):
                    assert np.array_equal(getattr(a, k), getattr(b, k)), (picker, forward, k)


def test_philox_known_answers():
    """Philox4x32-10 against the known-answer vectors published with
    Random123 (kat_vectors: philox4x32 10 rounds)."""
    kat = [
        ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
        ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
        ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
         [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
    ]
    for ctr, key, want in kat:
        assert list(po.philox4x32_10(ctr, key)) == want


def test_philox_draw_layout():
    """Slot layout of the normal-mode draws: slot 0 from pair 0's (x, y),
    slots 2p-1 / 2p from pair p's (x, y) / (z, w); counter (pair, walk_lo,
    walk_hi, 0), key = the seed's halves; (m + 0.5) * 2^-52 with m the top 52
    of the 64 bits."""
    seed, L = 0x0123456789ABCDEF, 5
    walks = [0, 1, 7, (1 << 32) + 3]
    key = [seed & 0xFFFFFFFF, seed >> 32]

    def unit(lo, hi):
        m = ((int(hi) << 32) | int(lo)) >> 12
        return (m + 0.5) / 2.0 ** 52

    for w in walks:
        d = po.philox_draws(seed, 1, L, walk0=w)
        ctr = [0, w & 0xFFFFFFFF, w >> 32, 0]
        o = po.philox4x32_10(ctr, key)
        assert d[0] == unit(o[0], o[1])
        for p in range(1, L + 1):
            o = po.philox4x32_10([p] + ctr[1:], key)
            assert d[2 * p - 1] == unit(o[0], o[1]) and d[2 * p] == unit(o[2], o[3])
    # many draws: strictly inside (0, 1), mean 1/2, no two equal
    d = po.philox_draws(seed, 20_000, 8)
    assert d.min() > 0.0 and d.max() < 1.0
    assert abs(d.mean() - 0.5) < 5 * math.sqrt(1 / 12 / d.size)
    assert np.unique(d).size == d.size
    # the unit map's extremes: m = 0 and m = 2^52 - 1 stay inside (0, 1)
    assert unit(0, 0) == 2.0 ** -53 and unit(0xFFFFFFFF, 0xFFFFFFFF) == 1 - 2.0 ** -53


def test_philox_shuffle_order_is_a_permutation():
    order = po.philox_shuffle_order(99, 10_000)
    assert np.array_equal(np.sort(order), np.arange(10_000))
    assert not np.array_equal(order, np.arange(10_000))
    assert np.array_equal(order, po.philox_shuffle_order(99, 10_000))


@pytest.mark.parametrize("directed", [True, False])
def test_parallel_oracle_ingest_equals_serial(directed):
    """The oracle's OpenMP ingest (parallel stable sort and merge, radix node
    sort, chunked group scans) gives the serial ingest's arrays for any
    thread count: multi-batch, ties, eviction and weights included."""
    rng = np.random.default_rng(17)
    batches = []
    for k in range(3):
        n = 150_000
        s = graphs.zipf_ids(rng, n, 40_000, 1.6)
        d = rng.integers(0, 40_000, n).astype(np.int32)
        t = rng.integers(k * 300, k * 300 + 1_000, n).astype(np.int64)  # heavy ties
        batches.append((s, d, t))
    names = list(po.ARRAY_DTYPES)
    names.remove("edge_features")
    results = []
    for threads in (1, 3, 8):
        og = po.OracleGraph(directed, max_time_capacity=1_500, enable_weight_computation=True,
                            enable_temporal_node2vec=True, timescale_bound=20.0)
        for b in batches:
            og.add_edges(*b, num_threads=threads)
        results.append({n: og.array(n) for n in names})
    for r in results[1:]:
        for n in names:
            assert np.array_equal(results[0][n], r[n]), n
