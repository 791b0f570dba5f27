"""The drop-in Python surface on the GPU: the reference's own Python tests
(py_tests/test_edge_features.py) restated, plus its C++ tests' behaviours for
cutoffs, padding, last-batch starts, queries and errors
(test/test_walk_cutoff_times.cpp, test_walk_padding_value.cpp,
test_temporal_random_walk.cpp)."""
import numpy as np
import pytest

from tests import graphs

pytestmark = pytest.mark.gpu


def _trw(**kw):
    from temporal_random_walk import TemporalRandomWalk
    kw.setdefault("use_gpu", True)
    return TemporalRandomWalk(**kw)


def _features_graph():
    tw = _trw(is_directed=True)
    tw.add_multiple_edges(np.array([0, 1, 2], np.int32), np.array([1, 2, 3], np.int32),
                          np.array([10, 20, 30], np.int64),
                          np.array([[1.0, 1.5], [2.0, 2.5], [3.0, 3.5]], np.float32))
    feat = {(0, 1, 10): [1.0, 1.5], (1, 2, 20): [2.0, 2.5], (2, 3, 30): [3.0, 3.5]}
    return tw, feat


def test_walks_include_edge_features_and_zero_unused_slots():
    tw, feat = _features_graph()
    L = 4
    nodes, ts, lens, wf = tw.get_random_walks_and_times_for_all_nodes(
        max_walk_len=L, walk_bias="Uniform", num_walks_per_node=1,
        walk_direction="Forward_In_Time")
    assert wf is not None and wf.shape == (len(lens), L - 1, 2)
    for w, n in enumerate(lens):
        n = int(n)
        for j in range(max(0, n - 1)):
            key = (int(nodes[w, j]), int(nodes[w, j + 1]), int(ts[w, j + 1]))
            np.testing.assert_allclose(wf[w, j], feat[key])
        for j in range(max(0, n - 1), L - 1):
            np.testing.assert_allclose(wf[w, j], [0.0, 0.0])


def test_walks_return_none_without_features():
    tw = _trw(is_directed=True)
    tw.add_multiple_edges(np.array([0, 1], np.int32), np.array([1, 2], np.int32),
                          np.array([10, 20], np.int64))
    _, _, _, wf = tw.get_random_walks_and_times(max_walk_len=3, walk_bias="Uniform",
                                                 num_walks_total=2)
    assert wf is None


def test_feature_validation_errors():
    tw, _ = _features_graph()
    with pytest.raises(RuntimeError, match="feature_dim mismatch"):
        tw.add_multiple_edges(np.array([4], np.int32), np.array([5], np.int32),
                              np.array([40], np.int64), np.array([[9.0, 9.1, 9.2]], np.float32))
    # edge_data.cu:75-89 checks the dimension before the missing features, so a
    # featureless batch on a featured store reports the dimension mismatch
    with pytest.raises(RuntimeError, match="feature_dim mismatch"):
        tw.add_multiple_edges(np.array([4], np.int32), np.array([5], np.int32),
                              np.array([40], np.int64))
    with pytest.raises(RuntimeError, match="same length"):
        tw.add_multiple_edges(np.array([4, 5], np.int32), np.array([5], np.int32),
                              np.array([40], np.int64))


def test_negative_node_ids_are_rejected_before_the_store_changes():
    """The node index is keyed by ids in [0, max_node_id]: a batch holding a
    negative id raises ValueError and leaves the store and the last batch as
    they were."""
    tw = _trw(is_directed=True, global_seed=5)
    tw.add_multiple_edges(np.array([0, 1, 2], np.int32), np.array([1, 2, 3], np.int32),
                          np.array([10, 20, 30], np.int64))
    for s, d in (([4, -1], [5, 6]), ([4, 5], [6, -7]), ([-2**31], [0])):
        with pytest.raises(ValueError, match="non-negative"):
            tw.add_multiple_edges(np.array(s, np.int32), np.array(d, np.int32),
                                  np.arange(40, 40 + len(s), dtype=np.int64))
    assert tw.get_edge_count() == 3
    assert np.array_equal(tw.get_node_ids(), [0, 1, 2, 3])
    nodes, _, lens, _ = tw.get_random_walks_and_times_for_last_batch(
        max_walk_len=4, walk_bias="Uniform", num_walks_per_node=2)
    assert nodes.shape == (3 * 2, 4) and set(int(x) for x in nodes[:, 0]) <= {0, 1, 2}
    tw.add_multiple_edges(np.array([3], np.int32), np.array([4], np.int32),
                          np.array([40], np.int64))
    assert tw.get_edge_count() == 4


def test_invalid_strings_raise_value_error():
    tw = _trw(is_directed=True)
    tw.add_multiple_edges(np.array([0], np.int32), np.array([1], np.int32),
                          np.array([1], np.int64))
    with pytest.raises(ValueError, match="Invalid picker type"):
        tw.get_random_walks_and_times(max_walk_len=3, walk_bias="Bogus", num_walks_total=1)
    with pytest.raises(ValueError, match="Invalid walk direction"):
        tw.get_random_walks_and_times(max_walk_len=3, walk_bias="Uniform", num_walks_total=1,
                                      walk_direction="Sideways")
    with pytest.raises(ValueError, match="kernel_launch_type"):
        tw.get_random_walks_and_times(max_walk_len=3, walk_bias="Uniform", num_walks_total=1,
                                      kernel_launch_type="WARP")


def test_device_allocation_failure_raises_memory_error_and_engine_recovers():
    """A sample whose walk buffers exceed HBM (2^31 - 1 walks of 2,000 slots, about
    17 TB of scratch) fails its allocation: MemoryError, as the reference's
    std::bad_alloc maps, and the instance keeps working."""
    tw = _trw(is_directed=True, global_seed=3)
    tw.add_multiple_edges(np.array([0, 1, 2], np.int32), np.array([1, 2, 3], np.int32),
                          np.arange(3, dtype=np.int64))
    with pytest.raises(MemoryError):
        tw.get_random_walks_and_times(max_walk_len=2_000, walk_bias="Uniform",
                                      num_walks_total=(1 << 31) - 1)
    nodes, ts, lens, _ = tw.get_random_walks_and_times(max_walk_len=4, walk_bias="Uniform",
                                                       num_walks_total=100)
    assert nodes.shape == (100, 4) and int(lens.max()) >= 2


def test_queries_match_store():
    s, d, t = graphs.sample_data()
    tw = _trw(is_directed=True)
    tw.add_multiple_edges(s, d, t)
    assert tw.get_edge_count() == len(s)
    ids = tw.get_node_ids()
    assert np.array_equal(ids, np.unique(np.concatenate([s, d])))
    assert tw.get_node_count() == len(ids)
    deg_out = tw.get_node_degrees(ids, "Forward_In_Time")
    deg_in = tw.get_node_degrees(ids, "Backward_In_Time")
    assert np.array_equal(deg_out, np.bincount(s, minlength=ids.max() + 1)[ids])
    assert np.array_equal(deg_in, np.bincount(d, minlength=ids.max() + 1)[ids])
    assert list(tw.get_node_degrees(np.array([-1, 10**6], np.int32), "Forward_In_Time")) == [0, 0]
    assert tw.get_memory_used() > 0
    tw.clear()
    assert tw.get_edge_count() == 0 and tw.get_node_count() == 0
    nodes, _, lens, _ = tw.get_random_walks_and_times(max_walk_len=5, walk_bias="Uniform",
                                                      num_walks_total=4)
    assert np.all(lens == 0) and np.all(nodes == -1)


def test_padding_value_and_short_lengths():
    tw = _trw(is_directed=True, walk_padding_value=-7)
    tw.add_multiple_edges(np.array([1, 2], np.int32), np.array([2, 3], np.int32),
                          np.array([10, 20], np.int64))
    nodes, ts, lens, _ = tw.get_random_walks_and_times_for_all_nodes(
        max_walk_len=6, walk_bias="Linear", num_walks_per_node=3)
    for w, n in enumerate(lens):
        assert np.all(nodes[w, int(n):] == -7) and np.all(ts[w, int(n):] == -1)
    nodes, ts, lens, _ = tw.get_random_walks_and_times(max_walk_len=1, walk_bias="Uniform",
                                                       num_walks_total=5)
    assert nodes.shape == (5, 1) and np.all(lens == 1)
    nodes, ts, lens, _ = tw.get_random_walks_and_times(max_walk_len=0, walk_bias="Uniform",
                                                       num_walks_total=5)
    assert nodes.shape == (5, 0) and np.all(lens == 0)


def test_cutoff_times_bound_every_hop():
    # test_walk_cutoff_times.cpp: a cutoff is an exclusive upper bound on the
    # time of every edge of the walk, in both directions; -1 is unbounded
    s, d, t = graphs.cfg1(n_nodes=500, n_edges=20_000, seed=3)
    tw = _trw(is_directed=True, global_seed=11, shuffle_walk_order=False)
    tw.add_multiple_edges(s, d, t)
    seeds = np.arange(0, 500, 2, dtype=np.int32)
    cut = np.full(seeds.size, 400_000, np.int64)
    cut[::4] = -1
    wpn = 4
    for direction in ("Forward_In_Time", "Backward_In_Time"):
        nodes, ts, lens, _ = tw.get_random_walks_and_times_for_nodes(
            seeds, max_walk_len=12, walk_bias="Uniform", num_walks_per_node=wpn,
            walk_direction=direction, cutoff_times=cut)
        assert nodes.shape == (seeds.size * wpn, 12)
        bounded_hops = 0
        late_hops_unbounded = 0
        for w, n in enumerate(lens):
            n = int(n)
            if n < 2:
                continue
            c = int(cut[w // wpn])
            origin = nodes[w, 0] if direction == "Forward_In_Time" else nodes[w, n - 1]
            assert origin == seeds[w // wpn]
            if c != -1:
                assert np.all(ts[w, 1:n] < c) if direction == "Forward_In_Time" else \
                    np.all(ts[w, :n - 1] < c)
                bounded_hops += n - 1
            else:
                late_hops_unbounded += int(np.sum(ts[w] >= 400_000))
        assert bounded_hops > 0 and late_hops_unbounded > 0


def _every_edge_before_cutoff(ts, lens, cutoffs, wpn):
    """expect_every_edge_before_cutoff of test/test_walk_cutoff_times.cpp:63-83:
    every real edge time of walk w is below its seed slot's cutoff (-1: none)."""
    sentinel = (np.iinfo(np.int64).min, np.iinfo(np.int64).max)
    for w, n in enumerate(lens):
        c = int(cutoffs[w // wpn])
        if c == -1:
            continue
        row = ts[w, :int(n)]
        row = row[(row != sentinel[0]) & (row != sentinel[1])]
        assert np.all(row < c), (w, row, c)


def test_cutoff_reference_cases():
    """test/test_walk_cutoff_times.cpp:301-415 on the reference's
    sample_data.csv (walks of up to 20 slots, 8 per seed, seed-major): a
    cutoff at the earliest timestamp admits no hop; one past the latest leaves
    every walk as it is without a cutoff (same engine, same global seed);
    cutoffs at the midpoint bound every edge, forward and backward; per-seed
    cutoffs over repeated seeds with one unbounded position bound backward
    ExponentialWeight walks, directed and undirected."""
    s, d, t = graphs.sample_data()
    lo, hi = int(t.min()), int(t.max())
    L, wpn = 20, 8

    def walks(tw, seeds, bias, direction, cut):
        return tw.get_random_walks_and_times_for_nodes(
            np.asarray(seeds, np.int32), max_walk_len=L, walk_bias=bias,
            num_walks_per_node=wpn, walk_direction=direction,
            cutoff_times=None if cut is None else np.asarray(cut, np.int64))

    tw = _trw(is_directed=True, global_seed=0xC0FFEE, shuffle_walk_order=False,
              enable_weight_computation=True)
    tw.add_multiple_edges(s, d, t)
    # CutoffBelowAllProducesEmptyWalks
    _, _, lens, _ = walks(tw, [109, 41, 15], "Uniform", "Backward_In_Time", [lo] * 3)
    assert int(lens.sum()) == 0
    # CutoffAboveAllEqualsUnbounded
    for direction in ("Backward_In_Time", "Forward_In_Time"):
        bounded = walks(tw, [109, 41, 15, 7], "ExponentialIndex", direction, [hi + 1] * 4)
        unbounded = walks(tw, [109, 41, 15, 7], "ExponentialIndex", direction, None)
        for a, b in zip(bounded[:3], unbounded[:3]):
            np.testing.assert_array_equal(a, b)
        assert int(bounded[2].sum()) > 4
    # Backward/ForwardEveryEdgeBeforeCutoff
    mid = lo + (hi - lo) // 2
    seeds = [109, 41, 15, 7, 88]
    for direction in ("Backward_In_Time", "Forward_In_Time"):
        _, ts, lens, _ = walks(tw, seeds, "ExponentialIndex", direction, [mid] * 5)
        _every_edge_before_cutoff(ts, lens, [mid] * 5, wpn)
        if direction == "Backward_In_Time":
            assert int(lens.sum()) > len(seeds)
    # HeterogeneousPerSeedCutoffs
    q1, q2, q3 = lo + (hi - lo) // 4, mid, lo + 3 * (hi - lo) // 4
    cuts = [q1, q2, -1, q3, q2]
    _, ts, lens, _ = walks(tw, [109, 109, 109, 41, 15], "ExponentialWeight", "Backward_In_Time",
                           cuts)
    _every_edge_before_cutoff(ts, lens, cuts, wpn)
    # UndirectedBackwardRespectsCutoff
    tu = _trw(is_directed=False, global_seed=0xC0FFEE, shuffle_walk_order=False,
              enable_weight_computation=True)
    tu.add_multiple_edges(s, d, t)
    _, ts, lens, _ = walks(tu, [109, 41, 15], "ExponentialWeight", "Backward_In_Time", [mid] * 3)
    _every_edge_before_cutoff(ts, lens, [mid] * 3, wpn)
    assert int(lens.sum()) > 3


@pytest.mark.parametrize("picker,wpn,bound,directed", [
    ("Linear", 10, -1.0, True), ("ExponentialWeight", 100, -1.0, True),
    ("ExponentialWeight", 20, 10.0, True), ("Linear", 10, -1.0, False)])
def test_walks_end_only_where_no_edge_continues(picker, wpn, bound, directed):
    """test/test_temporal_random_walk.cpp:246-570 (WalkCountAndLens,
    WalkIncreasingTimestamp, WalkValidEdges, WalkTerminalEdges and their
    ExponentialWeight forms) on the reference's sample_data.csv, directed,
    walks of up to 20 slots from every node: lengths are 0 or in [2, 20];
    every step is an edge of the graph at the step's time, times rise along
    the walk; a forward walk shorter than 20 ends at a node with no edge after
    its last time, a backward one starts at a node with no edge into it
    before its first time.  Timescale bound 10: TimescaleBoundedTemporalRandomWalkTest
    (ValidEdgesWithScaling, TerminalEdgeValidation).  Undirected
    (FilledUndirectedTemporalRandomWalkTest): an edge serves both ways."""
    s, d, t = graphs.sample_data()
    L = 20
    tw = _trw(is_directed=directed, enable_weight_computation=True, global_seed=17,
              timescale_bound=bound)
    tw.add_multiple_edges(s, d, t)
    if not directed:
        s, d, t = np.concatenate([s, d]), np.concatenate([d, s]), np.concatenate([t, t])
    n_id = int(max(s.max(), d.max())) + 1
    uniq = np.unique(t)
    edge_keys = np.unique((s.astype(np.int64) * n_id + d) * (uniq.size + 1) +
                          np.searchsorted(uniq, t))
    max_out = np.full(n_id, np.iinfo(np.int64).min)
    np.maximum.at(max_out, s, t)
    min_in = np.full(n_id, np.iinfo(np.int64).max)
    np.minimum.at(min_in, d, t)

    def are_edges(a, b, ts):
        r = np.searchsorted(uniq, ts)
        ok = (r < uniq.size) & (uniq[np.minimum(r, uniq.size - 1)] == ts)
        keys = (a.astype(np.int64) * n_id + b) * (uniq.size + 1) + r
        return ok & np.isin(keys, edge_keys)

    for direction in ("Forward_In_Time", "Backward_In_Time"):
        nodes, ts, lens, _ = tw.get_random_walks_and_times_for_all_nodes(
            max_walk_len=L, walk_bias=picker, num_walks_per_node=wpn, walk_direction=direction)
        lens = lens.astype(np.int64)
        assert np.all((lens == 0) | ((lens >= 2) & (lens <= L)))
        assert lens[lens > 0].mean() > 2
        fwd = direction == "Forward_In_Time"
        for n in range(2, L + 1):
            rows = np.nonzero(lens == n)[0]
            if rows.size == 0:
                continue
            nd, tt = nodes[rows, :n], ts[rows, :n]
            # edge times: slots 1.. forward, slots ..n-2 backward (the other
            # end holds the direction's sentinel)
            et = tt[:, 1:] if fwd else tt[:, :-1]
            assert np.all(np.diff(et, axis=1) > 0)
            assert np.all(are_edges(nd[:, :-1], nd[:, 1:], et)), (direction, n)
            if n < L:
                if fwd:
                    assert np.all(max_out[nd[:, -1]] <= et[:, -1]), (direction, n)
                else:
                    assert np.all(min_in[nd[:, 0]] >= et[:, 0]), (direction, n)


def test_reference_node_and_edge_counts():
    """test/test_temporal_random_walk.cpp:116-168 (ConstructorTest,
    AddEdgeTest, WhenMaxTimeCapacityExceedsEdgesAreDeletedAutomatically with
    max_time_capacity 5): node and edge counts of the engine, through the
    window's evictions."""
    def add(tw, edges):
        s, d, t = (np.array(x) for x in zip(*edges))
        tw.add_multiple_edges(s.astype(np.int32), d.astype(np.int32), t.astype(np.int64))

    tw = _trw(is_directed=True)
    assert tw.get_node_count() == 0
    add(tw, [(1, 2, 100), (2, 3, 101), (7, 8, 102), (1, 7, 103), (3, 2, 103), (10, 11, 104)])
    assert tw.get_edge_count() == 6 and tw.get_node_count() == 7

    tw = _trw(is_directed=True, max_time_capacity=5, enable_weight_computation=True,
              timescale_bound=-1.0)
    steps = [
        ([(0, 2, 1), (2, 3, 3), (1, 9, 2), (2, 4, 3), (2, 4, 1), (1, 5, 4)], 7, 6),
        ([(5, 6, 4), (2, 5, 4), (4, 3, 5)], 8, 9),
        ([(1, 7, 6)], 8, 8),
        ([(1, 5, 7), (4, 7, 8)], 7, 7),
    ]
    for edges, nodes, n_edges in steps:
        add(tw, edges)
        assert tw.get_node_count() == nodes and tw.get_edge_count() == n_edges, edges


def test_last_batch_starts_only_from_batch_sources():
    tw = _trw(is_directed=True, global_seed=3)
    tw.add_multiple_edges(np.array([1, 2], np.int32), np.array([2, 3], np.int32),
                          np.array([10, 20], np.int64))
    tw.add_multiple_edges(np.array([7, 7, 8], np.int32), np.array([1, 2, 9], np.int32),
                          np.array([30, 40, 50], np.int64))
    nodes, _, lens, _ = tw.get_random_walks_and_times_for_last_batch(
        max_walk_len=4, walk_bias="Uniform", num_walks_per_node=5)
    assert nodes.shape == (2 * 5, 4)
    assert set(int(x) for x in nodes[:, 0] if x != -1) <= {7, 8}


def test_seed_reproducibility_and_shuffle():
    s, d, t = graphs.cfg1(n_nodes=1_000, n_edges=20_000, seed=5)
    out = []
    for _ in range(2):
        tw = _trw(is_directed=True, global_seed=99)
        tw.add_multiple_edges(s, d, t)
        out.append(tw.get_random_walks_and_times_for_all_nodes(
            max_walk_len=10, walk_bias="ExponentialIndex", num_walks_per_node=2))
    for a, b in zip(out[0][:3], out[1][:3]):
        assert np.array_equal(a, b)
    starts = out[0][0][:, 0]
    assert not np.all(np.diff(starts[starts >= 0]) >= 0), "walk order should be shuffled"


def test_networkx_round_trip():
    nx = pytest.importorskip("networkx")
    g = nx.DiGraph()
    g.add_edge(1, 2, timestamp=5)
    g.add_edge(2, 3, timestamp=7)
    tw = _trw(is_directed=True)
    tw.add_edges_from_networkx(g)
    h = tw.to_networkx()
    assert sorted(h.edges(data="timestamp")) == [(1, 2, 5), (2, 3, 7)]


def _stream_batches(n_batches, n_edges, seed):
    rng = np.random.default_rng(seed)
    out = []
    for k in range(n_batches):
        s = graphs.zipf_ids(rng, n_edges, 200_000, 1.8)
        d = graphs.zipf_ids(rng, n_edges, 200_000, 1.8)
        t = rng.integers(k * 1_000_000, (k + 1) * 1_000_000, n_edges).astype(np.int64)
        out.append((s, d, t))
    return out


def test_prefetched_batches_overlap_sampling_and_match_direct_ingest():
    """trw_prefetch_edges copies the next host batch while a sample runs;
    trw_add_prefetched_edges then ingests it.  Store, index and walks equal
    those of plain trw_add_edges of the same batches, through the staged lanes
    (batches above 32 MiB) and the direct copy (a small batch), with a rolling
    window evicting old edges."""
    from temporal_random_walk import capi
    from tests.test_gpu_parity import INDEX_ARRAYS

    batches = _stream_batches(3, 3_000_000, 41) + _stream_batches(1, 50_000, 42)
    kw = dict(is_directed=True, global_seed=9, shuffle_walk_order=False,
              max_time_capacity=2_000_000)
    a, b = capi.Engine(**kw), capi.Engine(**kw)
    a.add_edges(*batches[0])
    b.add_edges(*batches[0])
    for s, d, t in batches[1:]:
        a.prefetch_edges(s, d, t)
        # the copy runs beside this sample; the store is not yet touched
        a.sample_device("total", 20, "ExponentialIndex", 500_000, initial_edge_bias="Uniform")
        a.add_prefetched_edges()
        b.add_edges(s, d, t)
        for name in ("sources", "targets", "timestamps", *INDEX_ARRAYS):
            assert np.array_equal(a.array(name), b.array(name)), name
    dr = graphs.draws(20_000, 16, seed=43)
    wa = a.sample("total", 16, "ExponentialIndex", 20_000, replay=dr, shuffle=False)
    wb = b.sample("total", 16, "ExponentialIndex", 20_000, replay=dr, shuffle=False)
    for k in ("nodes", "timestamps", "lens", "edge_ids"):
        assert np.array_equal(getattr(wa, k), getattr(wb, k)), k
    a.close()
    b.close()


def test_prefetch_errors_and_validation():
    from temporal_random_walk import capi

    e = capi.Engine(is_directed=True, global_seed=1)
    e.add_edges(np.array([0, 1], np.int32), np.array([1, 2], np.int32), np.array([1, 2], np.int64))
    with pytest.raises(ValueError, match="no prefetched batch"):
        e.add_prefetched_edges()
    e.prefetch_edges(np.array([2], np.int32), np.array([3], np.int32), np.array([3], np.int64))
    with pytest.raises(ValueError, match="pending"):
        e.prefetch_edges(np.array([3], np.int32), np.array([4], np.int32), np.array([4], np.int64))
    e.add_prefetched_edges()
    assert e.edge_count() == 3
    # validated when ingested, against the store as it is then
    e.prefetch_edges(np.array([4, -1], np.int32), np.array([5, 6], np.int32),
                     np.array([5, 6], np.int64))
    with pytest.raises(ValueError, match="non-negative"):
        e.add_prefetched_edges()
    assert e.edge_count() == 3
    e.prefetch_edges(np.array([4], np.int32), np.array([5], np.int32), np.array([5], np.int64),
                     np.array([[1.0, 2.0]], np.float32))
    with pytest.raises(Exception, match="feature_dim mismatch"):
        e.add_prefetched_edges()
    # a pending copy is waited for when the engine goes away
    big = _stream_batches(1, 3_000_000, 44)[0]
    e.prefetch_edges(*big)
    e.close()


def test_python_class_prefetch_matches_add_multiple_edges():
    batches = _stream_batches(2, 3_000_000, 45)
    tw_a = _trw(is_directed=True, global_seed=17, shuffle_walk_order=False)
    tw_b = _trw(is_directed=True, global_seed=17, shuffle_walk_order=False)
    tw_a.add_multiple_edges(*batches[0])
    tw_b.add_multiple_edges(*batches[0])
    # int64 ids are converted for the copy; the converted arrays are held
    s, d, t = batches[1]
    tw_a.prefetch_edges(s.astype(np.int64), d, t)
    tw_a.get_random_walks_and_times(max_walk_len=10, walk_bias="Uniform", num_walks_total=100_000)
    tw_a.add_prefetched_edges()
    tw_b.add_multiple_edges(s, d, t)
    assert tw_a.get_edge_count() == tw_b.get_edge_count()
    out = [tw.get_random_walks_and_times_for_last_batch(max_walk_len=12, walk_bias="Linear",
                                                         num_walks_per_node=1)
           for tw in (tw_a, tw_b)]
    for x, y in zip(out[0][:3], out[1][:3]):
        assert np.array_equal(x, y)


def _last_batch_graph(seed):
    """Two undirected batches; the second batch's targets (ids 50..79) are
    nodes the first batch never had."""
    rng = np.random.default_rng(seed)
    s1 = rng.integers(0, 50, 400).astype(np.int32)
    d1 = ((s1 + rng.integers(1, 50, 400)) % 50).astype(np.int32)  # no self-loops
    t1 = rng.integers(0, 1_000, 400).astype(np.int64)
    s2 = rng.integers(0, 50, 300).astype(np.int32)
    d2 = rng.integers(50, 80, 300).astype(np.int32)
    t2 = rng.integers(500, 2_000, 300).astype(np.int64)
    return (s1, d1, t1), (s2, d2, t2)


@pytest.mark.parametrize("forward", [True, False])
def test_last_batch_undirected_starts_are_the_batch_endpoints(forward):
    """..._for_last_batch on an undirected graph starts from the sorted unique
    union of the last batch's sources and targets, each repeated
    num_walks_per_node times (core/temporal_random_walk.cu:248-272; pinned by
    test/test_temporal_random_walk.cpp:669-685).  With shuffling off and
    injected draws the walks equal the oracle's walks from exactly those
    starts, row for row."""
    from oracle import pyoracle as po
    from temporal_random_walk import capi
    b1, b2 = _last_batch_graph(11)
    og = po.OracleGraph(False)
    eng = capi.Engine(is_directed=False, shuffle_walk_order=False, global_seed=5)
    for b in (b1, b2):
        og.add_edges(*b)
        eng.add_edges(*b)
    wpn, L = 3, 12
    uniq = np.unique(np.concatenate([b2[0], b2[1]])).astype(np.int32)
    assert uniq.size > np.unique(b2[0]).size  # the targets add starts
    starts = np.repeat(uniq, wpn)
    direction = "Forward_In_Time" if forward else "Backward_In_Time"
    for picker in ("Linear", "ExponentialIndex"):
        dr = graphs.draws(len(starts), L, seed=21)
        ref = og.walks(L, picker, "Uniform", forward, starts, dr)
        got = eng.sample("last_batch", L, picker, wpn, initial_edge_bias="Uniform",
                         direction=direction, replay=dr, shuffle=False)
        for k in ("nodes", "timestamps", "lens", "edge_ids"):
            assert np.array_equal(getattr(ref, k), getattr(got, k)), (picker, k)
        # every walk that found a start edge begins at its start node
        lens = got.lens.astype(np.int64)
        rows = np.nonzero(lens > 0)[0]
        assert rows.size > len(starts) // 2
        origin = got.nodes[rows, 0] if forward else got.nodes[rows, lens[rows] - 1]
        assert np.array_equal(origin, starts[rows])
    eng.close()


def test_last_batch_undirected_through_the_class():
    """The drop-in class: unshuffled last-batch walks of an undirected graph
    come in the order of the batch's sorted unique endpoints."""
    b1, b2 = _last_batch_graph(12)
    tw = _trw(is_directed=False, global_seed=8, shuffle_walk_order=False)
    tw.add_multiple_edges(*b1)
    tw.add_multiple_edges(*b2)
    wpn = 2
    nodes, _, lens, _ = tw.get_random_walks_and_times_for_last_batch(
        max_walk_len=6, walk_bias="Uniform", num_walks_per_node=wpn)
    starts = np.repeat(np.unique(np.concatenate([b2[0], b2[1]])), wpn)
    assert nodes.shape == (starts.size, 6)
    rows = np.nonzero(lens > 0)[0]
    assert np.array_equal(nodes[rows, 0], starts[rows])


def test_node_features_grow_and_keep_old_rows():
    """graph/node_features.cu:7-66, restating test/test_node_features.cpp:32-75:
    setting features sizes the dense store to max_node_id + 1 rows (zeros
    where unset), a later call after the graph grows keeps the old rows, and
    rows can be set through arbitrary id lists."""
    tw = _trw(is_directed=True)
    tw.add_multiple_edges(np.array([0, 2], np.int32), np.array([1, 3], np.int32),
                          np.array([1, 2], np.int64))  # max_node_id 3
    tw.set_node_features(np.array([1, 3], np.int32),
                         np.array([[1.0, 2.0], [3.0, 4.0]], np.float32))
    f = tw.get_node_features()
    assert f.shape == (4, 2)
    np.testing.assert_array_equal(f[1], [1.0, 2.0])
    np.testing.assert_array_equal(f[3], [3.0, 4.0])
    np.testing.assert_array_equal(f[[0, 2]], 0.0)
    tw.add_multiple_edges(np.array([4], np.int32), np.array([5], np.int32),
                          np.array([3], np.int64))  # max_node_id 5
    tw.set_node_features(np.array([5], np.int32), np.array([[9.0, 10.0]], np.float32))
    f = tw.get_node_features()
    assert f.shape == (6, 2)
    np.testing.assert_array_equal(f[1], [1.0, 2.0])  # kept on grow
    np.testing.assert_array_equal(f[3], [3.0, 4.0])
    np.testing.assert_array_equal(f[5], [9.0, 10.0])
    np.testing.assert_array_equal(f[[0, 2, 4]], 0.0)
    with pytest.raises(RuntimeError, match="feature_dim mismatch"):
        tw.set_node_features(np.array([1], np.int32), np.array([[1.0, 2.0, 3.0]], np.float32))

    # SetNodeFeaturesWithPointers: ids {0, 2}, dim 3
    tw2 = _trw(is_directed=True)
    tw2.add_multiple_edges(np.array([0], np.int32), np.array([2], np.int32),
                           np.array([5], np.int64))  # max_node_id 2
    tw2.set_node_features(np.array([0, 2], np.int32),
                          np.array([[7.0, 8.0, 9.0], [1.0, 2.0, 3.0]], np.float32))
    flat = tw2.get_node_features().ravel()
    assert flat[2] == 9.0 and flat[2 * 3] == 1.0
    assert tw2.get_node_features().shape == (3, 3)
    with pytest.raises(RuntimeError, match="row count"):
        tw2.set_node_features(np.array([0, 1], np.int32), np.array([[1.0, 2.0, 3.0]], np.float32))


@pytest.mark.parametrize("shift", [0, 2_000_000])
def test_failed_ingest_leaves_an_empty_usable_engine(shift):
    """A device allocation failing at any point of an ingest (forced by the
    test hook) raises MemoryError and leaves the engine empty, as after
    clear(); the engine then samples (no walks start) and a new ingest gives
    the oracle's index and replay walks.  shift puts the second batch after
    the first in time (the append path) or among it (the merge path)."""
    from oracle import pyoracle as po
    from temporal_random_walk import capi
    s1, d1, t1 = graphs.cfg1(n_nodes=300, n_edges=2_000, seed=3)
    s2, d2, t2 = graphs.cfg1(n_nodes=3_000, n_edges=40_000, seed=4)
    t2 = t2 + shift
    og1 = po.OracleGraph(True, enable_weight_computation=True, enable_temporal_node2vec=True)
    og1.add_edges(s1, d1, t1)
    og = po.OracleGraph(True, enable_weight_computation=True, enable_temporal_node2vec=True)
    og.add_edges(s2, d2, t2)
    L = 8
    starts = -np.ones(500, np.int32)
    dr = graphs.draws(500, L, seed=2)
    ref = og.walks(L, "ExponentialIndex", "Uniform", True, starts, dr)
    failures = 0
    for k in range(200):
        eng = capi.Engine(is_directed=True, enable_weight_computation=True,
                          enable_temporal_node2vec=True, shuffle_walk_order=False, global_seed=1)
        eng.add_edges(s1, d1, t1)
        capi.debug_fail_allocation(k)
        try:
            eng.add_edges(s2, d2, t2)  # larger: grows the buffers
            done = True
        except MemoryError:
            done = False
        finally:
            capi.debug_fail_allocation(-1)
        if done:
            eng.close()
            break
        failures += 1
        # a failure before the batch was accepted (staging) keeps the store;
        # one after it leaves the engine empty
        if eng.edge_count() == len(s1):
            for name in ("timestamps", "node_ts_sorted_outbound_indices"):
                assert np.array_equal(og1.array(name), eng.array(name)), (k, name)
        else:
            assert eng.edge_count() == 0
            w = eng.sample("total", L, "Uniform", 50, shuffle=False)
            assert int(w.lens.sum()) == 0 and np.all(w.nodes == -1)
        eng.clear()
        eng.add_edges(s2, d2, t2)
        for name in ("timestamps", "node_ts_sorted_outbound_indices",
                     "node_ts_group_inbound_offsets", "node_adj_neighbors"):
            assert np.array_equal(og.array(name), eng.array(name)), (k, name)
        got = eng.sample("total", L, "ExponentialIndex", 500, initial_edge_bias="Uniform",
                         replay=dr, shuffle=False)
        for name in ("nodes", "timestamps", "lens", "edge_ids"):
            assert np.array_equal(getattr(ref, name), getattr(got, name)), (k, name)
        eng.close()
    assert failures >= 10  # the ingest allocates at many points


def test_out_of_memory_with_held_blocks_releases_them_and_retries():
    """A device allocation that runs out of memory while the engine holds the
    blocks of buffers that grew (kept until clear(), a failed ingest or
    destruction, and counted by get_memory_used) releases them and tries once
    more (the transient test hook fails only the first attempt): the ingest
    completes with the oracle's index.  A fresh engine holds no such blocks,
    so the same failure ends its first ingest with MemoryError and leaves it
    empty and usable."""
    from oracle import pyoracle as po
    from temporal_random_walk import capi
    s1, d1, t1 = graphs.cfg1(n_nodes=300, n_edges=2_000, seed=3)
    s2, d2, t2 = graphs.cfg1(n_nodes=3_000, n_edges=40_000, seed=4)
    t2 = t2 + 4_000_000
    og = po.OracleGraph(True, enable_weight_computation=True)
    for b in ((s1, d1, t1), (s1, d1, t1 + 2_000_000), (s2, d2, t2)):
        og.add_edges(*b)
    # a fresh engine: nothing held, the failure stands
    eng = capi.Engine(is_directed=True, enable_weight_computation=True, global_seed=1)
    capi.debug_fail_allocation_transient(0)
    try:
        with pytest.raises(MemoryError):
            eng.add_edges(s1, d1, t1)
    finally:
        capi.debug_fail_allocation_transient(-1)
    assert eng.edge_count() == 0
    eng.close()
    retried = 0
    for k in (0, 1, 5, 20, 60):
        eng = capi.Engine(is_directed=True, enable_weight_computation=True, global_seed=1)
        eng.add_edges(s1, d1, t1)
        eng.add_edges(s1, d1, t1 + 2_000_000)  # the store doubles: blocks are held
        capi.debug_fail_allocation_transient(k)
        try:
            eng.add_edges(s2, d2, t2)  # larger: grows the buffers, retiring their blocks
        finally:
            capi.debug_fail_allocation_transient(-1)
        for name in ("timestamps", "node_ts_sorted_outbound_indices",
                     "node_ts_group_inbound_offsets", "count_ts_group_per_node_outbound"):
            assert np.array_equal(og.array(name), eng.array(name)), (k, name)
        np.testing.assert_allclose(eng.array("outbound_forward_cumulative_weights_exponential"),
                                   og.array("outbound_forward_cumulative_weights_exponential"),
                                   rtol=1e-12, atol=1e-300)
        retried += 1
        eng.close()
    assert retried == 5


def test_walk_stats_byte_accounting():
    """trw_get_walk_stats against numpy: steps, the per-hop demand bytes
    (72 + 8 ceil(log2(G_u + 1)) B with the reference's types) and the
    compulsory bytes of the walk kernel (processing order and the sampled
    direction's index read once, and per walk its start edge's endpoints --
    the kernel finds unconstrained starts of an index picker itself -- with
    the timestamp groups' offsets, or the start state a pre-pass found;
    lengths written once, and either scratch slot words or -- rows written by
    the walk kernel -- every output row in full)."""
    from temporal_random_walk import capi
    s, d, t = graphs.powerlaw(5_000, 60_000, n_ts=2_000, seed=9)
    eng = capi.Engine(is_directed=True, shuffle_walk_order=False, global_seed=3)
    eng.add_edges(s, d, t)
    L, n = 16, 70_000  # >= 2^16 walks: start-time order
    w = eng.sample("total", L, "ExponentialIndex", n, initial_edge_bias="Uniform",
                   walk_layout="scratch")
    st = eng.walk_stats()
    lens = w.lens.astype(np.int64)
    assert st["total_len"] == lens.sum()
    assert st["transitions"] == np.maximum(lens - 1, 0).sum()
    assert st["nonempty_walks"] == (lens > 0).sum()
    cnt = eng.array("count_ts_group_per_node_outbound").astype(np.int64)
    G = np.diff(cnt)
    ref = 40 * n + 12 * (lens >= 1).sum() + 20 * (lens >= 2).sum()
    for k in range(1, L - 1):
        rows = lens > k + 1
        g = G[w.nodes[rows, k]]
        probes = np.where(g > 0, np.ceil(np.log2(g + 1)), 0).astype(np.int64)
        ref += int((72 + 8 * probes).sum())
    assert st["reference_bytes"] == ref
    vc = eng.array("node_group_outbound_offsets").size
    g_o = eng.array("node_ts_group_outbound_offsets").size
    n_ent = eng.array("node_ts_sorted_outbound_indices").size
    index = 16 * vc + 4 * 2 * (g_o + vc) + 8 * (g_o + 1) + 8 * n_ent
    tsg = 4 * eng.array("timestamp_group_offsets").size
    assert st["compulsory_read_bytes"] == (8 + 4) * n + index + tsg
    assert st["compulsory_write_bytes"] == 8 * n + 8 * lens.sum()
    # the same sample with the rows written by the walk kernel
    w2 = eng.sample("total", L, "ExponentialIndex", n, initial_edge_bias="Uniform")
    np.testing.assert_array_equal(w2.nodes, w.nodes)
    st2 = eng.walk_stats()
    assert st2["compulsory_read_bytes"] == st["compulsory_read_bytes"]
    assert st2["compulsory_write_bytes"] == 8 * n + n * (4 * L + 8 * L + 8 * (L - 1))
    assert st2["reference_bytes"] == st["reference_bytes"]
    eng.close()

