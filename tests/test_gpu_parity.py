"""GPU parity: the HIP engine (through the C ABI) against the oracle.

Index arrays must be bit-exact; cumulative weights within 1e-12 relative;
replay-mode walks (injected uniform draws in the reference layout) bit-exact.
"""
import numpy as np
import pytest

from oracle import pyoracle as po
from tests import graphs

pytestmark = pytest.mark.gpu

INDEX_ARRAYS = [
    "sources", "targets", "timestamps", "timestamp_group_offsets", "unique_timestamps",
    "active_node_ids", "node_group_outbound_offsets", "node_group_inbound_offsets",
    "node_ts_sorted_outbound_indices", "node_ts_sorted_inbound_indices",
    "count_ts_group_per_node_outbound", "count_ts_group_per_node_inbound",
    "node_ts_group_outbound_offsets", "node_ts_group_inbound_offsets",
]
WEIGHT_ARRAYS = [
    "forward_cumulative_weights_exponential", "backward_cumulative_weights_exponential",
    "outbound_forward_cumulative_weights_exponential",
    "outbound_backward_cumulative_weights_exponential",
    "inbound_backward_cumulative_weights_exponential",
]
ADJ_ARRAYS = ["node_adj_offsets", "node_adj_neighbors"]


def _engine(**kw):
    from temporal_random_walk import capi
    return capi.Engine(**kw)


def _pair(is_directed, batches, max_time_capacity=-1, weights=False, tn2v=False,
          timescale_bound=-1.0, p=1.0, q=1.0, features=None):
    og = po.OracleGraph(is_directed, max_time_capacity, weights, tn2v, timescale_bound, p, q)
    eng = _engine(is_directed=is_directed, max_time_capacity=max_time_capacity,
                  enable_weight_computation=weights, enable_temporal_node2vec=tn2v,
                  timescale_bound=timescale_bound, node2vec_p=p, node2vec_q=q,
                  shuffle_walk_order=False, global_seed=1234)
    for k, (s, d, t) in enumerate(batches):
        f = None if features is None else features[k]
        og.add_edges(s, d, t, f)
        eng.add_edges(s, d, t, f)
    return og, eng


def _assert_index_equal(og, eng, weights=False, tn2v=False):
    for name in INDEX_ARRAYS:
        a, b = og.array(name), eng.array(name)
        assert a.dtype == b.dtype, name
        assert np.array_equal(a, b), f"{name}: oracle {a[:8]} engine {b[:8]} sizes {a.size} {b.size}"
    if weights:
        for name in WEIGHT_ARRAYS:
            a, b = og.array(name), eng.array(name)
            assert a.shape == b.shape, name
            # 1e-12 relative; unscaled exponentials over long time spans
            # (timescale_bound <= 0) end in subnormals, where the libms'
            # exp may differ by one subnormal ulp (5e-324): values below
            # 1e-300 compare absolutely
            np.testing.assert_allclose(b, a, rtol=1e-12, atol=1e-300, err_msg=name)
        # per-node cumulative arrays must be non-decreasing inside every node
        for name, cnt_name in [
                ("outbound_forward_cumulative_weights_exponential", "count_ts_group_per_node_outbound"),
                ("outbound_backward_cumulative_weights_exponential", "count_ts_group_per_node_outbound"),
                ("inbound_backward_cumulative_weights_exponential", "count_ts_group_per_node_inbound")]:
            w, cnt = eng.array(name), eng.array(cnt_name)
            if w.size == 0:
                continue
            same_node = np.ones(w.size, bool)
            same_node[cnt[(cnt > 0) & (cnt < w.size)].astype(np.int64)] = False
            same_node[0] = False
            assert np.all(np.diff(w)[same_node[1:]] >= 0), name
    if tn2v:
        for name in ADJ_ARRAYS:
            assert np.array_equal(og.array(name), eng.array(name)), name


def test_index_sample_data_directed():
    s, d, t = graphs.sample_data()
    og, eng = _pair(True, [(s, d, t)])
    _assert_index_equal(og, eng)


def test_index_cfg1_directed_and_undirected():
    s, d, t = graphs.cfg1()
    for directed in (True, False):
        og, eng = _pair(directed, [(s, d, t)])
        _assert_index_equal(og, eng)


def test_index_powerlaw_ties_multibatch():
    s, d, t = graphs.powerlaw(20_000, 200_000, s=1.8, n_ts=2_000, seed=3)
    batches = [(s[i:i + 50_000], d[i:i + 50_000], t[i:i + 50_000]) for i in range(0, 200_000, 50_000)]
    og, eng = _pair(True, batches)
    _assert_index_equal(og, eng)


def test_index_streaming_window_eviction():
    rng = np.random.default_rng(11)
    batches = []
    for k in range(5):
        n = 30_000
        s = graphs.zipf_ids(rng, n, 5_000, 1.6)
        d = graphs.zipf_ids(rng, n, 5_000, 1.6)
        t = rng.integers(k * 1000, (k + 1) * 1000, n).astype(np.int64)
        batches.append((s, d, t))
    og, eng = _pair(True, batches, max_time_capacity=2500)
    _assert_index_equal(og, eng)
    assert eng.latest_timestamp() == og.latest_timestamp


def _append_batches(seed, n_batches, n, span, overlap=0, n_ids=5_000, dims=0):
    """Batches whose timestamps start where the previous batch's end (ties at
    the boundary: a batch's first timestamp equals the previous one's last),
    each shifted back by `overlap` to make batches that interleave with the
    store instead."""
    rng = np.random.default_rng(seed)
    out, feats = [], []
    t0 = 0
    for k in range(n_batches):
        s = graphs.zipf_ids(rng, n, n_ids, 1.6)
        d = graphs.zipf_ids(rng, n, n_ids, 1.6)
        t = rng.integers(t0, t0 + span, n).astype(np.int64)
        t[rng.integers(0, n)] = t0  # the boundary tie
        t0 = int(t.max()) - overlap
        out.append((s, d, t))
        feats.append(rng.standard_normal((n, dims)).astype(np.float32) if dims else None)
    return out, (feats if dims else None)


@pytest.mark.parametrize("directed", [True, False])
@pytest.mark.parametrize("cap", [-1, 2_500, 700, 150])
def test_index_append_batches(directed, cap):
    """Streaming batches whose timestamps start at the store's last one take
    the append path (the batch sorted alone, old entries moved by a scatter);
    the window cuts inside the store (2500), empties it and cuts into the
    batch (700, 150: narrower than a batch), or not at all.  Every index array
    equals the oracle's after every batch; weights, the adjacency and replay
    walks after the last."""
    batches, _ = _append_batches(21, 6, 20_000, 1_000)
    og = po.OracleGraph(directed, cap, True, True, 30.0, 0.5, 2.0)
    eng = _engine(is_directed=directed, max_time_capacity=cap, enable_weight_computation=True,
                  enable_temporal_node2vec=True, timescale_bound=30.0, node2vec_p=0.5,
                  node2vec_q=2.0, shuffle_walk_order=False, global_seed=77)
    for b in batches:
        og.add_edges(*b)
        eng.add_edges(*b)
        _assert_index_equal(og, eng)
    _assert_index_equal(og, eng, weights=True, tn2v=True)
    assert eng.edge_count() == len(og.array("timestamps"))
    for forward in (True, False):
        _walk_case(og, eng, "Linear", "Uniform", forward, "total", 16, 3_000, seed=31)


@pytest.mark.parametrize("directed", [True, False])
@pytest.mark.parametrize("cap", [-1, 2_500, 700, 150])
def test_index_merge_batches(directed, cap):
    """Batches reaching back before the store's last timestamp take the merge
    path (the batch sorted alone, then merged into the store by binary search;
    the node index rebuilt): batches overlapping the store's end, one lying
    wholly before the store, one spanning all of it, ties at equal timestamps
    throughout, edge features carried along.  The window cuts inside the store
    (2500), into the batch (700, 150) or not at all.  Every index array and the
    features equal the oracle's after every batch; weights, the adjacency and
    replay walks after the last."""
    batches, feats = _append_batches(25, 5, 20_000, 1_000, overlap=400, dims=4)
    rng = np.random.default_rng(26)
    t_hi = int(batches[-1][2].max())
    s = graphs.zipf_ids(rng, 20_000, 5_000, 1.6)
    d = graphs.zipf_ids(rng, 20_000, 5_000, 1.6)
    batches.append((s, d, rng.integers(0, t_hi + 1, 20_000).astype(np.int64)))  # spans all
    feats.append(rng.standard_normal((20_000, 4)).astype(np.float32))
    batches.append((d, s, rng.integers(t_hi - 3_000, t_hi - 2_000, 20_000).astype(np.int64)))
    feats.append(rng.standard_normal((20_000, 4)).astype(np.float32))
    og = po.OracleGraph(directed, cap, True, True, 30.0, 0.5, 2.0)
    eng = _engine(is_directed=directed, max_time_capacity=cap, enable_weight_computation=True,
                  enable_temporal_node2vec=True, timescale_bound=30.0, node2vec_p=0.5,
                  node2vec_q=2.0, shuffle_walk_order=False, global_seed=78)
    for b, f in zip(batches, feats):
        og.add_edges(*b, f)
        eng.add_edges(*b, f)
        _assert_index_equal(og, eng)
        assert np.array_equal(og.array("edge_features"), eng.array("edge_features"))
    _assert_index_equal(og, eng, weights=True, tn2v=True)
    assert eng.edge_count() == len(og.array("timestamps"))
    for forward in (True, False):
        _walk_case(og, eng, "Linear", "Uniform", forward, "total", 16, 3_000, seed=32)


def test_index_cfg5_shaped_stream():
    """configs[4]'s stream at a tenth of its batch size: the same 1M-id
    Zipf(1.8) graph, 10 batches of 300k edges in consecutive time ranges,
    window 3e6, node2vec p=0.5 q=2.  Every batch takes the append path; after
    each one every index array equals the oracle's, after the last also the
    weights and the adjacency, and node2vec replay walks (on the engine's
    weights) are bit-exact."""
    from tests import configs
    cap = 3_000_000
    og = po.OracleGraph(True, cap, False, True, -1.0, 0.5, 2.0)
    eng = _engine(is_directed=True, max_time_capacity=cap, enable_temporal_node2vec=True,
                  node2vec_p=0.5, node2vec_q=2.0, shuffle_walk_order=False, global_seed=3)
    for b in configs.cfg5_batches(batch=300_000):
        og.add_edges(*b, num_threads=8)
        eng.add_edges(*b)
        _assert_index_equal(og, eng)
    # the window keeps the last three batches' time ranges
    assert abs(eng.edge_count() - 900_000) < 100
    _assert_index_equal(og, eng, weights=True, tn2v=True)
    for name in WEIGHT_ARRAYS:
        w = eng.array(name)
        if w.size:
            og.set_weights(name, w)
    _walk_case(og, eng, "TemporalNode2Vec", "Uniform", True, "total", 20, 20_000, seed=6)


def test_index_append_then_interleaved_batches():
    """Append batches, then batches reaching back before the store's last
    timestamp (the general sort of store and batch), then append again, with
    edge features carried along: identical to the oracle throughout."""
    a, fa = _append_batches(22, 3, 15_000, 1_000, dims=4)
    b, fb = _append_batches(23, 2, 15_000, 1_000, overlap=600, dims=4)
    b = [(s, d, t + int(a[-1][2].max()) - 300) for s, d, t in b]  # reach into the store
    c, fc = _append_batches(24, 2, 15_000, 1_000, dims=4)
    c = [(s, d, t + int(b[-1][2].max())) for s, d, t in c]
    og, eng = _pair(True, [], max_time_capacity=2_000)
    for (s, d, t), f in zip(a + b + c, fa + fb + fc):
        og.add_edges(s, d, t, f)
        eng.add_edges(s, d, t, f)
        _assert_index_equal(og, eng)
        assert np.array_equal(og.array("edge_features"), eng.array("edge_features"))


def test_index_weights_and_adjacency():
    s, d, t = graphs.powerlaw(5_000, 60_000, s=1.6, seed=5, ts_hi=10_000_000)
    for directed in (True, False):
        og, eng = _pair(directed, [(s, d, t)], weights=True, tn2v=True, timescale_bound=50.0)
        _assert_index_equal(og, eng, weights=True, tn2v=True)


def _node_segments(cnt):
    """(start, end) of every node's groups from count_ts_group_per_node_*."""
    return [(int(cnt[u]), int(cnt[u + 1])) for u in range(cnt.size - 1) if cnt[u] < cnt[u + 1]]


@pytest.mark.parametrize("bound", [-1.0, 0.0, 10.0, 50.0])
def test_reference_weight_edge_cases(bound):
    """The reference's small weight cases (test/test_edge_data_weights.cpp:
    TimescaleBoundZero, SingleTimestampWithBounds, TimescaleBoundPositive;
    test/test_node_edge_index_weights.cpp: EmptyGraph,
    SingleTimestampGroupPerNode, TimescaleBoundZero,
    TimescaleBoundWithSingleTimestamp, WeightBiasPerNode) on the device
    engine: the same arrays as the oracle, and the reference's own assertions
    (cumulative arrays non-decreasing to 1 within 1e-6 per segment, one group
    of weight 1 for a single timestamp, forward weights falling and backward
    rising in time when the bound scales them)."""
    def arr(*x):
        return np.array(x, np.int32)

    # an engine without edges has empty weight arrays
    og, eng = _pair(True, [], weights=True, timescale_bound=bound)
    for name in WEIGHT_ARRAYS:
        assert eng.array(name).size == 0, name
    eng.close()

    cases = [
        (arr(1, 1, 2, 2, 3, 4), arr(2, 3, 3, 4, 4, 1), np.array([10, 10, 20, 20, 30, 40])),
        (arr(1, 2, 3), arr(2, 3, 4), np.array([100, 100, 100])),  # one timestamp
        (arr(1, 1, 2), arr(2, 3, 3), np.array([10, 10, 10])),     # one group per node
        (arr(1, 1, 1), arr(2, 3, 4), np.array([10, 20, 30])),     # one node, three groups
    ]
    for k, (s, d, t) in enumerate(cases):
        og, eng = _pair(True, [(s, d, t.astype(np.int64))], weights=True, timescale_bound=bound)
        _assert_index_equal(og, eng, weights=True)
        T = np.unique(t).size
        for name in ("forward_cumulative_weights_exponential",
                     "backward_cumulative_weights_exponential"):
            w = eng.array(name)
            assert w.size == T and np.all(w >= 0) and np.all(np.diff(w) >= 0), name
            assert abs(w[-1] - 1.0) <= 1e-6, name
        for name, cnt_name in (
                ("outbound_forward_cumulative_weights_exponential", "count_ts_group_per_node_outbound"),
                ("outbound_backward_cumulative_weights_exponential", "count_ts_group_per_node_outbound"),
                ("inbound_backward_cumulative_weights_exponential", "count_ts_group_per_node_inbound")):
            w = eng.array(name)
            for a, b in _node_segments(eng.array(cnt_name)):
                seg = w[a:b]
                assert np.all(seg >= 0) and np.all(np.diff(seg) >= 0), name
                assert abs(seg[-1] - 1.0) <= 1e-6, name
                if T == 1 or k == 2:
                    assert b - a == 1, name
        if k == 0 and bound > 0:
            # scaled by the bound: earlier groups weigh more forward, later
            # ones backward (TimescaleBoundPositive)
            f = np.diff(eng.array("forward_cumulative_weights_exponential"), prepend=0.0)
            b_ = np.diff(eng.array("backward_cumulative_weights_exponential"), prepend=0.0)
            assert np.all(np.diff(f) < 0) and np.all(np.diff(b_) > 0)
        if k == 3:
            # node 1 with groups at 10, 20, 30 (WeightBiasPerNode): forward
            # weights fall in time, backward ones rise
            cnt = eng.array("count_ts_group_per_node_outbound")
            a, b = int(cnt[1]), int(cnt[2])
            fw = np.diff(eng.array("outbound_forward_cumulative_weights_exponential")[a:b],
                         prepend=0.0)
            bw = np.diff(eng.array("outbound_backward_cumulative_weights_exponential")[a:b],
                         prepend=0.0)
            assert np.all(np.diff(fw) < 0) and np.all(np.diff(bw) > 0)
        eng.close()


def test_reference_cutoff_selector_cases():
    """test/test_walk_cutoff_times.cpp:163-252 (ForwardCutoffUpperBound,
    BackwardCutoffUpperBound, CutoffBoundaryIsExclusive): get_node_edge_at
    with the TEST_FIRST / TEST_LAST pickers, no time bound and a cutoff, read
    as the start edge of a two-slot walk from the node (its start selection is
    that call); an invalid edge is a walk of length 0."""
    I64 = np.int64

    def start_edge(eng, node, picker, forward, cutoff):
        got = eng.sample("nodes", 2, picker, 1, initial_edge_bias=picker,
                         direction="Forward_In_Time" if forward else "Backward_In_Time",
                         seed_nodes=np.array([node], np.int32),
                         cutoff_times=np.array([cutoff], I64), shuffle=False)
        n = int(got.lens[0])
        if n == 0:
            return None
        assert n == 2
        nd, ts = got.nodes[0], got.timestamps[0]
        return (int(nd[0]), int(nd[1]), int(ts[1] if forward else ts[0]))

    def engine(edges):
        e = _engine(is_directed=True, global_seed=5, shuffle_walk_order=False)
        s, d, t = (np.array(x) for x in zip(*edges))
        e.add_edges(s.astype(np.int32), d.astype(np.int32), t.astype(I64))
        return e

    F, L_, NONE = "TEST_FIRST", "TEST_LAST", -1
    fwd = engine([(10, 20, 100), (10, 30, 101), (10, 40, 102), (10, 50, 103), (10, 60, 104)])
    for picker, cut, want in [(F, NONE, (10, 20, 100)), (L_, NONE, (10, 60, 104)),
                              (L_, 104, (10, 50, 103)), (L_, 103, (10, 40, 102)),
                              (F, 101, (10, 20, 100)), (F, 100, None), (F, 50, None),
                              (L_, 1000, (10, 60, 104))]:
        assert start_edge(fwd, 10, picker, True, cut) == want, (picker, cut)
    fwd.close()
    bwd = engine([(20, 10, 100), (30, 10, 101), (40, 10, 102), (50, 10, 103), (60, 10, 104)])
    for picker, cut, want in [(F, NONE, (20, 10, 100)), (L_, NONE, (60, 10, 104)),
                              (L_, 104, (50, 10, 103)), (L_, 102, (30, 10, 101)),
                              (F, 101, (20, 10, 100)), (F, 100, None),
                              (L_, 1000, (60, 10, 104))]:
        assert start_edge(bwd, 10, picker, False, cut) == want, (picker, cut)
    bwd.close()
    both = engine([(10, 20, 100), (10, 30, 110), (10, 40, 120),
                   (50, 70, 100), (60, 70, 110), (80, 70, 120)])
    assert start_edge(both, 10, L_, True, 110) == (10, 20, 100)
    assert start_edge(both, 70, L_, False, 110) == (50, 70, 100)
    both.close()


@pytest.mark.parametrize("forward", [True, False])
def test_reference_node2vec_rejection_cases(forward):
    """test/test_temporal_node2vec_rejection.cpp:171-260 on the device's
    in-kernel draws: at V with previous node P, the candidates P (beta 1/p),
    N (a neighbour of P, beta 1) and F (beta 1/q) are taken in the analytic
    proportions within 0.025 over 10,000 hops, across the reference's (p, q)
    sweep, and under the degenerate p = 0.1, q = 10 every hop still returns
    one of them.  The previous node is set only after a walk's first loop hop
    (temporal_random_walk_cpu.cuh:65, 116-120), so the hop is the last of a
    four-slot walk seeded at S: S -> P (start edge), P -> V (the only edge
    on), then V's pick with P behind it (forward: S->P at 5, P->V at 10, P->N
    at 2; backward: P->S at 300, V->P at 200, P->N at 50)."""
    V, P, N, F, S = 0, 1, 2, 3, 4
    if forward:
        edges = [(V, P, 100), (V, N, 100), (V, F, 100), (P, N, 2), (S, P, 5), (P, V, 10)]
    else:
        edges = [(P, V, 100), (N, V, 100), (F, V, 100), (P, N, 50), (V, P, 200), (P, S, 300)]
    s, d, t = (np.array(x) for x in zip(*edges))
    n = 10_000
    for p, q in [(1.0, 1.0), (1.0, 2.0), (0.5, 2.0), (2.0, 0.5), (0.25, 4.0), (0.1, 10.0)]:
        eng = _engine(is_directed=True, enable_weight_computation=True,
                      enable_temporal_node2vec=True, timescale_bound=-1.0, node2vec_p=p,
                      node2vec_q=q, global_seed=31, shuffle_walk_order=False)
        eng.add_edges(s.astype(np.int32), d.astype(np.int32), t.astype(np.int64))
        w = eng.sample("nodes", 4, "TemporalNode2Vec", n, initial_edge_bias="TEST_FIRST",
                       direction="Forward_In_Time" if forward else "Backward_In_Time",
                       seed_nodes=np.array([S], np.int32), shuffle=False)
        assert np.all(w.lens == 4), (p, q)
        path = w.nodes[:, :3] if forward else w.nodes[:, 1:][:, ::-1]
        assert np.all(path == [S, P, V])
        cand = w.nodes[:, 3] if forward else w.nodes[:, 0]
        assert np.all(np.isin(cand, [P, N, F])), (p, q)
        wts = np.array([1.0 / p, 1.0, 1.0 / q])
        want = wts / wts.sum()
        got = np.array([(cand == c).mean() for c in (P, N, F)])
        assert np.all(np.abs(got - want) <= 0.025), (p, q, got, want)
        eng.close()


def _walk_case(og, eng, picker, start_picker, forward, mode, L, n_or_wpn, seed_nodes=None,
               cutoffs=None, seed=0):
    direction = "Forward_In_Time" if forward else "Backward_In_Time"
    if mode == "total":
        starts = -np.ones(n_or_wpn, dtype=np.int32)
        cut = None
    elif mode == "all_nodes":
        ids = np.nonzero(og.array("active_node_ids"))[0].astype(np.int32)
        starts = np.repeat(ids, n_or_wpn)
        cut = None
    else:
        starts = np.repeat(np.asarray(seed_nodes, dtype=np.int32), n_or_wpn)
        cut = None if cutoffs is None else np.repeat(np.asarray(cutoffs, dtype=np.int64), n_or_wpn)
    dr = graphs.draws(len(starts), L, seed=seed)
    ref = og.walks(L, picker, start_picker, forward, starts, dr, cutoffs=cut)
    # every device processing order gives the reference's walks, row for row,
    # and so do both ways to the output rows (written by the walk kernel, or
    # scratch and the layout pass)
    for order, layout in (("walk_id", "auto"), ("start_time", "auto"),
                          ("start_time", "scratch"), ("node_grouped", "auto")):
        got = eng.sample(mode, L, picker, n_or_wpn, initial_edge_bias=start_picker,
                         direction=direction, seed_nodes=seed_nodes, cutoff_times=cutoffs,
                         replay=dr, shuffle=False, walk_order=order, walk_layout=layout)
        for k in ("nodes", "timestamps", "lens", "edge_ids"):
            a = getattr(ref, k)
            b = getattr(got, k)
            assert a.shape == b.shape, k
            bad = np.nonzero((a != b).reshape(len(starts), -1).any(axis=1))[0] if a.ndim > 1 \
                else np.nonzero(a != b)[0]
            assert bad.size == 0, (f"{picker}/{start_picker} fwd={forward} {mode} {order} "
                                   f"{layout}: {k} differs in {bad.size} walks, first {bad[:5]}")
    return got


@pytest.mark.parametrize("directed", [True, False])
@pytest.mark.parametrize("forward", [True, False])
@pytest.mark.parametrize("picker", ["Uniform", "Linear", "ExponentialIndex"])
def test_replay_walks_index_pickers(directed, forward, picker):
    s, d, t = graphs.cfg1(n_nodes=2_000, n_edges=40_000, seed=42)
    t = t // 50  # many tied timestamps
    og, eng = _pair(directed, [(s, d, t)])
    _walk_case(og, eng, picker, "Uniform", forward, "total", 20, 4_000, seed=1)
    _walk_case(og, eng, picker, picker, forward, "all_nodes", 20, 2, seed=2)
    seeds = np.arange(0, 2_000, 3, dtype=np.int32)
    cuts = np.where(np.arange(seeds.size) % 3 == 0, -1,
                    np.random.default_rng(3).integers(0, 20_000, seeds.size)).astype(np.int64)
    _walk_case(og, eng, picker, picker, forward, "nodes", 16, 3, seed_nodes=seeds, cutoffs=cuts,
               seed=3)


@pytest.mark.parametrize("p,q", [(2.0, 0.5), (1.0, 1.0), (0.25, 4.0), (4.0, 1.0), (0.5, 50.0)])
def test_replay_walks_node2vec_return_in_out(p, q):
    """TemporalNode2Vec's acceptance (temporal_node2vec_helpers.cuh:127-199)
    with the in-out bias on either side of 1 and a return bias above and
    below the others: a draw below both non-return thresholds, at or above
    both, or between them (the only case that asks whether the candidate
    neighbours the previous node) decides as the reference does.  q = 50
    accepts a far candidate with probability 0.01, so most hops run all 64
    retries and take the last valid proposal (the row-writing kernel's
    wave-decided retries, with few open hops and many lanes each)."""
    s, d, t = graphs.powerlaw(2_000, 40_000, s=1.4, seed=19, ts_hi=500_000)
    og, eng = _pair(True, [(s, d, t)], weights=True, tn2v=True, timescale_bound=20.0, p=p, q=q)
    for name in WEIGHT_ARRAYS:
        w = eng.array(name)
        if w.size:
            og.set_weights(name, w)
    _walk_case(og, eng, "TemporalNode2Vec", "Uniform", True, "total", 24, 3_000, seed=8)
    _walk_case(og, eng, "TemporalNode2Vec", "ExponentialWeight", False, "total", 16, 2_000,
               seed=9)


@pytest.mark.parametrize("directed", [True, False])
@pytest.mark.parametrize("forward", [True, False])
@pytest.mark.parametrize("picker", ["ExponentialWeight", "TemporalNode2Vec"])
def test_replay_walks_weight_pickers(directed, forward, picker):
    s, d, t = graphs.powerlaw(3_000, 50_000, s=1.6, seed=9, ts_hi=1_000_000)
    og, eng = _pair(directed, [(s, d, t)], weights=True, tn2v=picker == "TemporalNode2Vec",
                    timescale_bound=50.0, p=0.5, q=2.0)
    # the weights agree to 1e-12; the sampler is then checked bit-exactly on
    # identical weights (picks on a flat cumulative tail amplify ulp noise)
    _assert_index_equal(og, eng, weights=True)
    for name in WEIGHT_ARRAYS:
        w = eng.array(name)
        if w.size:
            og.set_weights(name, w)
    _walk_case(og, eng, picker, picker, forward, "total", 24, 4_000, seed=4)
    _walk_case(og, eng, picker, picker, forward, "all_nodes", 12, 1, seed=5)
    # per-walk cutoffs: the slice's cutoff end moves off the time search's
    # bound (the hubs' tables hold several groups in some buckets)
    seeds = np.unique(s[:600]).astype(np.int32)
    cuts = np.where(np.arange(seeds.size) % 3 == 0, -1,
                    np.random.default_rng(6).integers(0, 1_000_000, seeds.size)).astype(np.int64)
    _walk_case(og, eng, picker, picker, forward, "nodes", 16, 3, seed_nodes=seeds, cutoffs=cuts,
               seed=6)


@pytest.mark.parametrize("directed", [True, False])
@pytest.mark.parametrize("forward", [True, False])
@pytest.mark.parametrize("picker", ["ExponentialWeight", "TemporalNode2Vec"])
def test_replay_walks_weight_pickers_multi_entry_groups(directed, forward, picker):
    """The weight pickers on a graph whose node-timestamp groups hold many
    entries (60k edges over 400 timestamps): picks of a group's first, second
    and later entries read the group's panel record, its wide slot and the
    weighted edge records, each with the next slice's bound and start sum
    they carry (forward walks over the ExponentialWeight weights' wide
    panel), so every one of those sources feeds the next hop."""
    s, d, t = graphs.powerlaw(2_000, 60_000, s=1.6, seed=19, ts_hi=400)
    og, eng = _pair(directed, [(s, d, t)], weights=True, tn2v=picker == "TemporalNode2Vec",
                    timescale_bound=20.0, p=0.5, q=2.0)
    _assert_index_equal(og, eng, weights=True)
    for name in WEIGHT_ARRAYS:
        w = eng.array(name)
        if w.size:
            og.set_weights(name, w)
    # groups of several entries: the test means what it says only if they occur
    # (and a walk picks past their first entry)
    counts = np.diff(eng.array("node_ts_group_outbound_offsets"))
    assert counts.size and (counts >= 3).mean() > 0.15, np.bincount(counts)[:8]
    _walk_case(og, eng, picker, picker, forward, "total", 24, 4_000, seed=21)
    _walk_case(og, eng, picker, "Uniform", forward, "total", 16, 2_000, seed=22)


@pytest.mark.parametrize("directed,g", [(True, 300_000), (False, 300_000), (True, 1_200_000)])
def test_replay_walks_exponential_weight_deep_search_index(directed, g):
    """ExponentialWeight walks through a hub of 300k (1.2M) timestamp groups,
    whose picks go through its guide table (and, for a wide bracket, its
    weight search index of five or six levels).  Walks of every length end
    at different hops.  Walk-picker index families mixed with weight starts
    go through the same kernels."""
    rng = np.random.default_rng(71)
    hub_t = rng.permutation(g).astype(np.int64) * 3
    hub_d = rng.integers(1, 3_000, g).astype(np.int32)
    n_o = 150_000
    s_o = rng.integers(1, 3_000, n_o).astype(np.int32)
    d_o = np.where(rng.random(n_o) < 0.4, 0, rng.integers(1, 3_000, n_o)).astype(np.int32)
    t_o = rng.integers(0, 3 * g, n_o).astype(np.int64)
    s = np.concatenate([np.zeros(g, np.int32), s_o])
    d = np.concatenate([hub_d, d_o])
    t = np.concatenate([hub_t, t_o])
    og, eng = _pair(directed, [(s, d, t)], weights=True, timescale_bound=30.0)
    if g < 1_000_000:
        _assert_index_equal(og, eng, weights=True)
    else:
        # over 1.3M timestamp groups the oracle's sequential fp64 prefix sum
        # (the reference's order) carries ~3e-12 relative roundoff: the global
        # weights are held to 1e-12 against the closed form in extended
        # precision instead (x86 80-bit long double)
        _assert_index_equal(og, eng)
        LD = np.longdouble
        ts_all = eng.array("timestamps")
        u, c = np.unique(ts_all, return_counts=True)
        scale = 30.0 / float(ts_all[-1] - ts_all[0])
        fw = c.astype(LD) * np.exp((ts_all[0] - u).astype(np.float64).astype(LD) * LD(scale))
        np.testing.assert_allclose(eng.array("forward_cumulative_weights_exponential"),
                                   np.cumsum(fw / fw.sum()).astype(np.float64), rtol=1e-12,
                                   atol=0)
    for name in WEIGHT_ARRAYS:
        w = eng.array(name)
        if w.size:
            og.set_weights(name, w)
    for forward in (True, False):
        _walk_case(og, eng, "ExponentialWeight", "ExponentialWeight", forward, "total", 30,
                   6_000, seed=72)
        _walk_case(og, eng, "ExponentialWeight", "Uniform", forward, "nodes", 20, 400,
                   seed_nodes=np.array([0, 7, 11], np.int32), seed=73)
        _walk_case(og, eng, "Linear", "ExponentialWeight", forward, "total", 12, 3_000, seed=74)
        # the hub's single-rank buckets give the time bound and its weight
        # sum; cutoffs inside its span move the slice's other end
        _walk_case(og, eng, "ExponentialWeight", "ExponentialWeight", forward, "nodes", 20, 300,
                   seed_nodes=np.array([0, 0, 0, 7], np.int32),
                   cutoffs=np.array([g, 2 * g, -1, 3 * g // 2], np.int64), seed=75)


@pytest.mark.parametrize("bound", [-1.0, 1e-4, 5.0, 200.0])
def test_replay_walks_weight_guide_profiles(bound):
    """Weight picks look their group up in a per-node guide table keyed by
    the bit pattern of the cumulative weight (1 - c for forward weights, c
    for backward ones), then settle the bracket.  Profiles that stress it,
    bit-exact against the oracle on the engine's weights: unscaled weights
    (bound -1) over gaps of 1 to 10^6, which fall by hundreds of orders of
    magnitude between groups (runs of thousands of empty buckets, filled by
    workgroups) and sit at exactly 0 or 1 over long stretches; nearly flat
    weights (bound 1e-4: many groups per bucket where the key is linear in
    c); the cfg4-like exponential (bound 5); and a steep one (200, weights
    exhausted within a few percent of the span).  Most other edges reuse the
    hubs' timestamps, so the hubs hold most ranks of their span and take the
    rank-table path (single-rank time buckets).  The hubs are picked from by
    ExponentialWeight and TemporalNode2Vec walks in both directions, from
    weight-picked starts (the global guides) and from seeds with cutoffs."""
    rng = np.random.default_rng(401)
    n_hub = 40_000
    gaps = rng.choice(np.array([1, 2, 3, 40, 5_000, 1_000_000]), n_hub,
                      p=[0.5, 0.2, 0.15, 0.1, 0.045, 0.005])
    hub_t = np.cumsum(gaps).astype(np.int64)
    span = int(hub_t[-1])
    # hub 0: one edge per group; hub 1: the same times with 1-6 edges each
    reps = rng.integers(1, 7, n_hub)
    s = [np.zeros(n_hub, np.int32), np.ones(int(reps.sum()), np.int32)]
    d = [rng.integers(2, 2_000, n_hub).astype(np.int32),
         rng.integers(2, 2_000, int(reps.sum())).astype(np.int32)]
    t = [hub_t, np.repeat(hub_t, reps)]
    n_o = 60_000
    s.append(rng.integers(2, 2_000, n_o).astype(np.int32))
    d.append(np.where(rng.random(n_o) < 0.5, rng.integers(0, 2, n_o),
                      rng.integers(2, 2_000, n_o)).astype(np.int32))
    t.append(np.where(rng.random(n_o) < 0.8, rng.choice(hub_t, n_o),
                      rng.integers(0, span, n_o)).astype(np.int64))
    s, d, t = np.concatenate(s), np.concatenate(d), np.concatenate(t)
    og, eng = _pair(True, [(s, d, t)], weights=True, tn2v=True, timescale_bound=bound, p=0.5,
                    q=2.0)
    for name in WEIGHT_ARRAYS:
        w = eng.array(name)
        if w.size:
            og.set_weights(name, w)
    seeds = np.array([0, 1, 0, 1, 5, 0, 1], np.int32)
    cuts = np.array([-1, -1, span // 2, span // 3, -1, int(hub_t[100]), int(hub_t[-50])], np.int64)
    for forward in (True, False):
        _walk_case(og, eng, "ExponentialWeight", "ExponentialWeight", forward, "total", 24,
                   8_000, seed=402)
        _walk_case(og, eng, "ExponentialWeight", "Uniform", forward, "nodes", 16, 300,
                   seed_nodes=seeds, cutoffs=cuts, seed=403)
        _walk_case(og, eng, "TemporalNode2Vec", "ExponentialWeight", forward, "total", 16,
                   4_000, seed=404)
        _walk_case(og, eng, "TemporalNode2Vec", "Uniform", forward, "nodes", 12, 200,
                   seed_nodes=seeds, cutoffs=cuts, seed=405)
    eng.close()


def test_replay_walks_powerlaw_exponential_index():
    s, d, t = graphs.powerlaw(100_000, 400_000, s=1.8, n_ts=5_000, seed=44)
    og, eng = _pair(True, [(s, d, t)])
    _walk_case(og, eng, "ExponentialIndex", "Uniform", True, "total", 80, 20_000, seed=6)


def test_normal_mode_invariants_and_features():
    s, d, t = graphs.cfg1(n_nodes=3_000, n_edges=30_000, seed=8)
    rng = np.random.default_rng(8)
    feat = rng.standard_normal((len(s), 4)).astype(np.float32)
    og, eng = _pair(True, [(s, d, t)], features=[feat])
    L = 20
    w = eng.sample("total", L, "Linear", 5_000, initial_edge_bias="Uniform")
    store_s, store_d, store_t = eng.array("sources"), eng.array("targets"), eng.array("timestamps")
    store_f = eng.array("edge_features").reshape(-1, 4)
    lens = w.lens.astype(np.int64)
    assert np.all((lens == 0) | ((lens >= 2) & (lens <= L)))
    for i in range(0, 5_000, 7):
        n = lens[i]
        if n == 0:
            continue
        e = w.edge_ids[i, :n - 1]
        assert np.all(e >= 0)
        assert np.array_equal(store_s[e], w.nodes[i, :n - 1])
        assert np.array_equal(store_d[e], w.nodes[i, 1:n])
        assert np.array_equal(store_t[e], w.timestamps[i, 1:n])
        assert np.all(np.diff(w.timestamps[i, 1:n]) > 0)
        assert np.all(w.nodes[i, n:] == -1) and np.all(w.edge_ids[i, n - 1:] == -1)
        np.testing.assert_array_equal(w.edge_features[i, :n - 1], store_f[e])
        assert np.all(w.edge_features[i, n - 1:] == 0)


@pytest.mark.parametrize("dim", [8, 6])
@pytest.mark.parametrize("forward", [True, False])
def test_walk_features_through_every_layout_path(dim, forward):
    """Edge features of every walk slot: dims that are multiples of 4 are
    written by the layout pass from the edge ids it holds (packed scratch
    here), others -- and those of rows the walk kernel wrote itself -- by a
    gather over the laid-out edge ids.  Rows of one chunk (L = 20) and of
    several (L = 150), reversed for backward walks, in both processing orders
    and both ways to the rows: each row's features are the store's rows of
    its edge ids, zeros past its length."""
    s, d, t = graphs.cfg1(n_nodes=200, n_edges=100_000, seed=18)
    rng = np.random.default_rng(18)
    feat = rng.standard_normal((len(s), dim)).astype(np.float32)
    og, eng = _pair(True, [(s, d, t)], features=[feat])
    store_f = eng.array("edge_features").reshape(-1, dim)
    direction = "Forward_In_Time" if forward else "Backward_In_Time"
    for L in (20, 150):
        for order, layout in (("walk_id", "auto"), ("start_time", "auto"),
                              ("start_time", "scratch")):
            w = eng.sample("total", L, "ExponentialIndex", 3_000, initial_edge_bias="Uniform",
                           direction=direction, walk_order=order, walk_layout=layout)
            lens = w.lens.astype(np.int64)
            assert w.edge_features.shape == (3_000, L - 1, dim)
            assert lens.max() > 100 or L == 20
            for i in range(0, 3_000, 5):
                n = int(lens[i])
                e = w.edge_ids[i, :max(n - 1, 0)]
                np.testing.assert_array_equal(w.edge_features[i, :len(e)], store_f[e])
                assert np.all(w.edge_features[i, len(e):] == 0)


def test_host_handoff_matches_device_buffers():
    """trw_sample's staged, multi-threaded host delivery (used above 32 MiB)
    returns exactly the bytes trw_sample_device leaves in HBM; a fixed
    global seed makes the two calls sample the same walks."""
    from temporal_random_walk import capi

    s, d, t = graphs.cfg1(n_nodes=10_000, n_edges=100_000, seed=9)
    rng = np.random.default_rng(9)
    feat = rng.standard_normal((len(s), 3)).astype(np.float32)
    eng = capi.Engine(is_directed=True, global_seed=77, shuffle_walk_order=False)
    eng.add_edges(s, d, t, feat)
    L, n = 40, 100_000
    host = eng.sample("total", L, "ExponentialIndex", n, initial_edge_bias="Uniform")
    tm = eng.timings()
    expect_bytes = n * L * (4 + 8) + n * 8 + n * (L - 1) * (8 + 3 * 4)
    assert tm["handoff_bytes"] == expect_bytes > (32 << 20)
    dev = eng.sample_device("total", L, "ExponentialIndex", n, initial_edge_bias="Uniform")
    assert int(dev.num_walks) == n and int(dev.feature_dim) == 3
    np.testing.assert_array_equal(capi.device_to_host(dev.nodes, n * L, np.int32),
                                  host.nodes.ravel())
    np.testing.assert_array_equal(capi.device_to_host(dev.timestamps, n * L, np.int64),
                                  host.timestamps.ravel())
    np.testing.assert_array_equal(capi.device_to_host(dev.walk_lens, n, np.uint64), host.lens)
    np.testing.assert_array_equal(capi.device_to_host(dev.edge_ids, n * (L - 1), np.int64),
                                  host.edge_ids.ravel())
    np.testing.assert_array_equal(
        capi.device_to_host(dev.edge_features, n * (L - 1) * 3, np.float32),
        host.edge_features.ravel())
    assert host.lens.sum() > n  # non-trivial walks
    eng.close()


@pytest.mark.parametrize("forward", [True, False])
@pytest.mark.parametrize("picker", ["Uniform", "ExponentialIndex"])
def test_replay_walks_bursty_hubs_with_cutoffs(forward, picker):
    """Hubs whose timestamps come in bursts (uneven bucket tables: most
    buckets empty, a few crowded) with per-walk cutoffs."""
    rng = np.random.default_rng(21)
    s, d, _ = graphs.powerlaw(20_000, 300_000, s=1.7, seed=21)
    centers = rng.integers(0, 10_000_000, 40)
    t = (centers[rng.integers(0, 40, s.size)] +
         rng.exponential(2_000.0, s.size).astype(np.int64)).astype(np.int64)
    og, eng = _pair(True, [(s, d, t)])
    _walk_case(og, eng, picker, "Uniform", forward, "total", 30, 6_000, seed=11)
    seeds = np.unique(s[:5_000]).astype(np.int32)
    cuts = np.where(np.arange(seeds.size) % 4 == 0, -1,
                    rng.integers(0, 10_000_000, seeds.size)).astype(np.int64)
    _walk_case(og, eng, picker, picker, forward, "nodes", 30, 2, seed_nodes=seeds, cutoffs=cuts,
               seed=12)


@pytest.mark.parametrize("forward", [True, False])
@pytest.mark.parametrize("picker", ["ExponentialIndex", "Uniform"])
def test_replay_walks_dense_hubs_with_cutoffs(forward, picker):
    """Hubs with a group at every timestamp rank of their span (their time
    search answers from the rank, with no table) inside a graph whose other
    edges reach before and after those spans, so the searched rank falls
    before, inside and past a dense span; per-walk cutoffs bound it again."""
    rng = np.random.default_rng(23)
    T = 4_000
    hubs = []
    for hub, (lo, hi) in enumerate([(1_000, 3_000), (0, 2_500), (1_800, 4_000)]):
        span = np.arange(lo, hi, dtype=np.int64)
        extra = rng.integers(lo, hi, (hi - lo) // 2)  # repeated ranks: groups of 2+
        ts = np.concatenate([span, extra])
        hubs.append((np.full(ts.size, hub, np.int32), rng.integers(3, 600, ts.size).astype(np.int32), ts))
    n_o = 40_000
    s_o = rng.integers(3, 600, n_o).astype(np.int32)
    d_o = np.where(rng.random(n_o) < 0.5, rng.integers(0, 3, n_o),
                   rng.integers(3, 600, n_o)).astype(np.int32)
    t_o = rng.integers(0, T, n_o).astype(np.int64)
    s = np.concatenate([h[0] for h in hubs] + [s_o])
    d = np.concatenate([h[1] for h in hubs] + [d_o])
    t = np.concatenate([h[2] for h in hubs] + [t_o]) * 7  # distinct timestamps, not ranks
    og, eng = _pair(True, [(s, d, t)])
    _walk_case(og, eng, picker, "Uniform", forward, "total", 24, 8_000, seed=24)
    seeds = np.array([0, 1, 2, 3, 4, 5], np.int32)
    cuts = np.array([-1, 7 * 2_000, 7 * 500, 7 * 3_500, -1, 7 * 1_000], np.int64)
    _walk_case(og, eng, picker, picker, forward, "nodes", 24, 300, seed_nodes=seeds,
               cutoffs=cuts, seed=25)


@pytest.mark.parametrize("directed", [True, False])
@pytest.mark.parametrize("forward", [True, False])
def test_replay_walks_negative_and_minus_one_timestamps(directed, forward):
    """Edges at timestamp -1 end a walk where the reference tests `ts == -1`
    (and a start at -1 leaves the next hop unconstrained); other negative
    timestamps are ordinary."""
    s, d, t = graphs.cfg1(n_nodes=500, n_edges=20_000, seed=31)
    t = (t % 40) - 20  # ts in [-20, 20): many ties, -1 among them
    assert np.any(t == -1)
    og, eng = _pair(directed, [(s, d, t)])
    for picker in ("Uniform", "ExponentialIndex", "Linear"):
        _walk_case(og, eng, picker, "Uniform", forward, "total", 16, 3_000, seed=13)
        _walk_case(og, eng, picker, picker, forward, "all_nodes", 16, 2, seed=14)


@pytest.mark.parametrize("forward", [True, False])
def test_replay_long_walks_span_layout_chunks(forward):
    """Walks longer than one layout chunk (rows of more than 96 slots are
    laid out in several chunks), padded and reversed like short ones."""
    s, d, t = graphs.cfg1(n_nodes=200, n_edges=100_000, seed=41)
    og, eng = _pair(True, [(s, d, t)])
    got = _walk_case(og, eng, "ExponentialIndex", "Uniform", forward, "total", 150, 2_000, seed=15)
    lens = got.lens.astype(np.int64)
    assert lens.max() == 150 and (lens > 96).mean() > 0.5


@pytest.mark.parametrize("forward", [True, False])
def test_replay_walks_stop_at_the_padding_node(forward):
    """The reference's walk loop runs while the current node differs from the
    padding value (temporal_random_walk_cpu.cuh:93): a walk that reaches a
    node whose id is the padding value ends there, without writing it.  Here
    the padding value is the id of the node with the sixth most in-edges: it
    cuts about 40 % of the walks short (against the same walks with padding
    -1), and about a third still run to L; every order and both ways to the
    rows."""
    s, d, t = graphs.powerlaw(3_000, 60_000, s=1.7, n_ts=4_000, seed=61)
    hub = int(np.argsort(-np.bincount(d), kind="stable")[5])
    og = po.OracleGraph(True)
    og.add_edges(s, d, t)
    eng = _engine(is_directed=True, shuffle_walk_order=False, global_seed=1234,
                  walk_padding_value=hub)
    eng.add_edges(s, d, t)
    L, n = 24, 70_000  # >= 2^16 walks: start-time order in the automatic choice
    dr = graphs.draws(n, L, seed=62)
    direction = "Forward_In_Time" if forward else "Backward_In_Time"
    ref = og.walks(L, "ExponentialIndex", "Uniform", forward, -np.ones(n, np.int32), dr, pad=hub)
    unpadded = og.walks(L, "ExponentialIndex", "Uniform", forward, -np.ones(n, np.int32), dr)
    lens = ref.lens.astype(np.int64)
    assert (lens < unpadded.lens.astype(np.int64)).mean() > 0.3 and (lens == L).mean() > 0.2
    for order, layout in (("walk_id", "auto"), ("start_time", "auto"), ("start_time", "scratch"),
                          ("node_grouped", "auto")):
        got = eng.sample("total", L, "ExponentialIndex", n, initial_edge_bias="Uniform",
                         direction=direction, replay=dr, shuffle=False, walk_order=order,
                         walk_layout=layout)
        for k in ("nodes", "timestamps", "lens", "edge_ids"):
            np.testing.assert_array_equal(getattr(got, k), getattr(ref, k), err_msg=f"{order} {layout} {k}")
    eng.close()


def test_replay_walks_million_scale():
    """2^20 + a ragged remainder of walks (time-ordered by default at this
    size) against the oracle, forward and backward."""
    s, d, t = graphs.powerlaw(20_000, 300_000, s=1.7, n_ts=30_000, seed=81)
    og, eng = _pair(True, [(s, d, t)])
    n = (1 << 20) + 4_321
    _walk_case(og, eng, "ExponentialIndex", "Uniform", True, "total", 12, n, seed=82)
    _walk_case(og, eng, "Linear", "Uniform", False, "total", 9, n, seed=83)


def test_replay_walks_hub_with_more_groups_than_the_header_holds():
    """A node with 2^24 + 100 timestamp groups: more than the 24 bits the walk's
    node header keeps for the group count, so the count comes from the next
    header.  Walks from it and through it, forward and backward."""
    rng = np.random.default_rng(91)
    g = (1 << 24) + 100
    hub_t = rng.permutation(g).astype(np.int64)
    hub_d = rng.integers(1, 2_000, g).astype(np.int32)
    s_o = rng.integers(1, 2_000, 200_000).astype(np.int32)
    d_o = np.where(rng.random(200_000) < 0.3, 0, rng.integers(1, 2_000, 200_000)).astype(np.int32)
    t_o = rng.integers(0, g, 200_000).astype(np.int64)
    s = np.concatenate([np.zeros(g, np.int32), s_o])
    d = np.concatenate([hub_d, d_o])
    t = np.concatenate([hub_t, t_o])
    og, eng = _pair(True, [(s, d, t)])
    assert int(eng.array("count_ts_group_per_node_outbound")[1]) == g
    for forward in (True, False):
        for picker in ("ExponentialIndex", "Uniform"):
            _walk_case(og, eng, picker, "Uniform", forward, "nodes", 12, 500,
                       seed_nodes=np.array([0, 5], np.int32), seed=92)
            _walk_case(og, eng, picker, "Uniform", forward, "total", 12, 3_000, seed=93)


@pytest.mark.parametrize("forward", [True, False])
@pytest.mark.parametrize("e,n_ts,fmt", [((1 << 21) + 60_000, (1 << 21) + 60_000, 1),
                                        (1 << 21, (1 << 21) - 1, 0)],
                         ids=["66_bits", "64_bits"])
def test_replay_walks_at_the_scratch_packing_limit(forward, e, n_ts, fmt):
    """Node ids up to 2^22 - 1 with E edges and n_ts distinct timestamps.
    66 bits: a node id, a rank and an edge id need 22 + 22 + 22 bits, more than
    one 64-bit slot word holds, so the slot words hold node and edge id only
    and a slot's timestamp is its edge's (every smaller graph here fits the
    rank).  64 bits: 22 + 21 + 21 bits exactly fill the slot word -- the edge
    id in its top bits and the largest rank one below the all-ones start
    sentinel.  Both through rows written by the walk kernel (forward) and
    through scratch and the layout pass."""
    rng = np.random.default_rng(95)
    ids = np.concatenate([[0, (1 << 22) - 1],
                          rng.choice(np.arange(1, (1 << 22) - 1), 6_000, replace=False)])
    perm = rng.permutation(ids.size)
    s = ids[graphs.zipf_ids(rng, e, ids.size, 1.5, perm)].astype(np.int32)
    d = ids[graphs.zipf_ids(rng, e, ids.size, 1.5, perm)].astype(np.int32)
    t = np.concatenate([rng.permutation(n_ts), rng.integers(0, n_ts, e - n_ts)]).astype(np.int64)
    og, eng = _pair(True, [(s, d, t)])
    assert int(eng.array("active_node_ids").size) == 1 << 22
    assert int(eng.array("unique_timestamps").size) == n_ts
    _walk_case(og, eng, "ExponentialIndex", "Uniform", forward, "total", 20, 20_000, seed=96)
    assert eng.walk_stats()["slot_word_format"] == fmt
    _walk_case(og, eng, "Uniform", "Linear", forward, "nodes", 20, 4,
               seed_nodes=ids[:500].astype(np.int32), seed=97)


@pytest.mark.parametrize("forward", [True, False])
def test_replay_walks_from_seeds_outside_the_graph(forward):
    """Seeds that are no node of the graph (negative other than -1, past the
    largest id, or an id without edges) start no walk; -1 is an unconstrained
    start; the other seeds walk as usual."""
    s, d, t = graphs.cfg1(n_nodes=300, n_edges=10_000, seed=61)
    s = np.where(s == 7, 8, s).astype(np.int32)
    d = np.where(d == 7, 8, d).astype(np.int32)
    og, eng = _pair(True, [(s, d, t)])
    seeds = np.array([-3, 3, 10**7, -1, 7, 299, -2**31, 2**31 - 1, 0], np.int32)
    got = _walk_case(og, eng, "ExponentialIndex", "Uniform", forward, "nodes", 12, 3,
                     seed_nodes=seeds, seed=62)
    lens = got.lens.reshape(seeds.size, 3)
    assert np.all(lens[[0, 2, 4, 6, 7]] == 0)
    assert np.all(lens[[1, 3, 8]] >= 1)


# ---- normal mode: the in-kernel Philox stream -----------------------------

GLOBAL_SEED = 1234  # the seed _pair gives the engine


def _starts(og, mode, n_or_wpn, seed_nodes=None):
    if mode == "total":
        return -np.ones(n_or_wpn, dtype=np.int32)
    if mode == "all_nodes":
        ids = np.nonzero(og.array("active_node_ids"))[0].astype(np.int32)
        return np.repeat(ids, n_or_wpn)
    return np.repeat(np.asarray(seed_nodes, dtype=np.int32), n_or_wpn)


def _normal_case(og, eng, picker, start_picker, forward, mode, L, n_or_wpn, seed_nodes=None,
                 cutoffs=None, shuffle=False):
    """Normal-mode walks (no injected draws) must equal the oracle's replay
    of the engine's Philox draws, in the shuffled start order if shuffled."""
    direction = "Forward_In_Time" if forward else "Backward_In_Time"
    starts = _starts(og, mode, n_or_wpn, seed_nodes)
    cut = None if cutoffs is None else np.repeat(np.asarray(cutoffs, dtype=np.int64), n_or_wpn)
    if shuffle and mode != "total":
        order = po.philox_shuffle_order(GLOBAL_SEED, starts.size)
        starts = starts[order]
        cut = None if cut is None else cut[order]
    dr = po.philox_draws(GLOBAL_SEED, starts.size, L)
    ref = og.walks(L, picker, start_picker, forward, starts, dr, cutoffs=cut)
    for order in ("walk_id", "start_time", "node_grouped"):
        got = eng.sample(mode, L, picker, n_or_wpn, initial_edge_bias=start_picker,
                         direction=direction, seed_nodes=seed_nodes, cutoff_times=cutoffs,
                         shuffle=shuffle, walk_order=order)
        for k in ("nodes", "timestamps", "lens", "edge_ids"):
            a, b = getattr(ref, k), getattr(got, k)
            assert a.shape == b.shape, k
            assert np.array_equal(a, b), (f"{picker}/{start_picker} fwd={forward} {mode} "
                                          f"shuffle={shuffle} {order}: {k} differs")
    return got


@pytest.mark.parametrize("directed", [True, False])
@pytest.mark.parametrize("forward", [True, False])
def test_normal_mode_walks_are_the_philox_replay(directed, forward):
    s, d, t = graphs.powerlaw(5_000, 80_000, s=1.7, n_ts=20_000, seed=51)
    og, eng = _pair(directed, [(s, d, t)])
    _normal_case(og, eng, "ExponentialIndex", "Uniform", forward, "total", 40, 20_000)
    _normal_case(og, eng, "Linear", "Linear", forward, "all_nodes", 20, 2)
    _normal_case(og, eng, "Uniform", "ExponentialIndex", forward, "all_nodes", 20, 2,
                 shuffle=True)
    seeds = np.unique(s[:2_000]).astype(np.int32)
    cuts = np.where(np.arange(seeds.size) % 3 == 0, -1,
                    np.random.default_rng(52).integers(0, 100_000_000, seeds.size)).astype(np.int64)
    _normal_case(og, eng, "ExponentialIndex", "ExponentialIndex", forward, "nodes", 30, 3,
                 seed_nodes=seeds, cutoffs=cuts, shuffle=True)


@pytest.mark.parametrize("forward", [True, False])
@pytest.mark.parametrize("picker", ["ExponentialWeight", "TemporalNode2Vec"])
def test_normal_mode_weight_pickers_are_the_philox_replay(forward, picker):
    s, d, t = graphs.powerlaw(3_000, 50_000, s=1.6, seed=53, ts_hi=1_000_000)
    og, eng = _pair(True, [(s, d, t)], weights=True, tn2v=picker == "TemporalNode2Vec",
                    timescale_bound=50.0, p=0.5, q=2.0)
    for name in WEIGHT_ARRAYS:
        w = eng.array(name)
        if w.size:
            og.set_weights(name, w)
    _normal_case(og, eng, picker, picker, forward, "total", 24, 8_000)
    _normal_case(og, eng, picker, picker, forward, "all_nodes", 12, 1, shuffle=True)


def _chi2_two_sample(a, b, min_expected=5.0):
    """Two-sample chi-square on category samples a, b (equal sizes): categories
    with small expected counts are pooled into one bin.  Returns the p-value."""
    from scipy.stats import chi2_contingency
    cats, inv = np.unique(np.concatenate([a, b]), return_inverse=True)
    ca = np.bincount(inv[:a.size], minlength=cats.size)
    cb = np.bincount(inv[a.size:], minlength=cats.size)
    small = (ca + cb) / 2.0 < min_expected
    table = np.stack([ca[~small], cb[~small]])
    if small.any():
        table = np.concatenate([table, [[ca[small].sum()], [cb[small].sum()]]], axis=1)
    return chi2_contingency(table)[1]


@pytest.mark.parametrize("picker", ["Uniform", "Linear", "ExponentialIndex", "ExponentialWeight",
                                    "TemporalNode2Vec"])
def test_normal_mode_chi_square_against_independent_draws(picker):
    """The distribution of normal-mode walks matches the oracle's walks under
    independent numpy uniforms (two-sample chi-square, p > 0.01) on the start
    edge, the first hop's edge, the fifth slot's node and the walk length."""
    s, d, t = graphs.cfg1(n_nodes=60, n_edges=1_500, seed=61)
    weights = picker in ("ExponentialWeight", "TemporalNode2Vec")
    og, eng = _pair(True, [(s, d, t)], weights=weights, tn2v=picker == "TemporalNode2Vec",
                    timescale_bound=20.0, p=0.5, q=2.0)
    if weights:
        for name in WEIGHT_ARRAYS:
            w = eng.array(name)
            if w.size:
                og.set_weights(name, w)
    n, L = 200_000, 8
    got = eng.sample("total", L, picker, n, initial_edge_bias=picker)
    ref = og.walks(L, picker, picker, True, -np.ones(n, np.int32), graphs.draws(n, L, seed=62))
    for name, a, b in [("start edge", ref.edge_ids[:, 0], got.edge_ids[:, 0]),
                       ("hop-1 edge", ref.edge_ids[:, 1], got.edge_ids[:, 1]),
                       ("slot-4 node", ref.nodes[:, 4], got.nodes[:, 4]),
                       ("length", ref.lens.astype(np.int64), got.lens.astype(np.int64))]:
        pv = _chi2_two_sample(np.asarray(a), np.asarray(b))
        assert pv > 0.01, f"{picker}: {name} p = {pv:.3g}"


def test_staged_host_ingest_matches_device_ingest():
    """trw_add_edges copies batches above 32 MiB through the staged lanes
    (pinned buffers, several threads); the store and index must equal those
    of the same batch handed over in HBM (trw_add_edges_device)."""
    import torch

    from temporal_random_walk import capi

    s, d, t = graphs.powerlaw(200_000, 5_000_000, s=1.7, n_ts=50_000, seed=71)
    feat = np.random.default_rng(71).standard_normal((s.size, 3)).astype(np.float32)
    a = capi.Engine(is_directed=True, global_seed=5, shuffle_walk_order=False)
    a.add_edges(s, d, t, feat)
    b = capi.Engine(is_directed=True, global_seed=5, shuffle_walk_order=False)
    dv = [torch.from_numpy(x).cuda() for x in (s, d, t, feat)]
    torch.cuda.synchronize()
    b.add_edges_device(dv[0].data_ptr(), dv[1].data_ptr(), dv[2].data_ptr(), s.size,
                       dv[3].data_ptr(), 3)
    for name in ("sources", "targets", "timestamps", "edge_features", *INDEX_ARRAYS):
        assert np.array_equal(a.array(name), b.array(name)), name
    a.close()
    b.close()
