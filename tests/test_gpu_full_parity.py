"""Full-size parity of BASELINE configs[2..4] (cfg3, cfg4, cfg5) with the
oracle.

The oracle ingests each whole workload on the host's cores (OpenMP; its
result is the same for any thread count), then:
- every index array is compared bit for bit, and the per-node and global
  cumulative weights within 1e-12 relative where a sequential fp64 sum is
  that accurate (nodes of fewer than 10^5 groups; the hubs and the global
  arrays, whose sequential sums carry more roundoff than that, are held to
  their extended-precision closed forms in test_gpu_configs.py);
- 100,000 replay walks of each workload's own call are compared bit for bit
  -- the weight pickers on the engine's weights injected into the oracle,
  since picks on a flat cumulative tail turn ulp differences of summation
  order into different groups.
cfg3: undirected, backward Linear/Linear from seed nodes with dim-16 edge
features (slot words of node and edge id: 23 + 27 bits leave no room for a
rank); cfg4: ExponentialWeight starts and hops through hubs of millions of
timestamp groups; cfg5: the streaming window after batches 3 and 10 with
TemporalNode2Vec walks.
"""
import os

import numpy as np
import pytest

from oracle import pyoracle as po
from tests import configs, graphs

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)))

INDEX_ARRAYS = [
    "sources", "targets", "timestamps", "timestamp_group_offsets", "unique_timestamps",
    "active_node_ids", "node_group_outbound_offsets", "node_group_inbound_offsets",
    "node_ts_sorted_outbound_indices", "node_ts_sorted_inbound_indices",
    "count_ts_group_per_node_outbound", "count_ts_group_per_node_inbound",
    "node_ts_group_outbound_offsets", "node_ts_group_inbound_offsets",
]
NODE_WEIGHTS = [
    ("outbound_forward_cumulative_weights_exponential", "count_ts_group_per_node_outbound"),
    ("outbound_backward_cumulative_weights_exponential", "count_ts_group_per_node_outbound"),
    ("inbound_backward_cumulative_weights_exponential", "count_ts_group_per_node_inbound"),
]
GLOBAL_WEIGHTS = ["forward_cumulative_weights_exponential",
                  "backward_cumulative_weights_exponential"]
N_WALKS = 100_000


def _engine(**kw):
    from temporal_random_walk import capi
    kw.setdefault("global_seed", 2024)
    kw.setdefault("shuffle_walk_order", False)
    return capi.Engine(**kw)


def _cmp_index(og, eng, label):
    for name in INDEX_ARRAYS:
        a, b = og.array(name), eng.array(name)
        assert a.dtype == b.dtype and a.shape == b.shape, (label, name, a.shape, b.shape)
        assert np.array_equal(a, b), (label, name)


def _cmp_weights(og, eng, label, small=100_000):
    """Per-node weights of nodes with fewer than `small` groups within 1e-12
    relative (values below 1e-300 absolutely: unscaled exponentials end in
    subnormals, where two libms' exp may differ by one ulp), the rest and the
    global arrays within 1e-9."""
    for name, cnt_name in NODE_WEIGHTS:
        a, b = og.array(name), eng.array(name)
        assert a.shape == b.shape, (label, name)
        if a.size == 0:
            continue
        cnt = eng.array(cnt_name).astype(np.int64)
        G = np.diff(cnt)
        light = np.repeat(G < small, G)
        np.testing.assert_allclose(b[light], a[light], rtol=1e-12, atol=1e-300,
                                   err_msg=f"{label} {name}")
        np.testing.assert_allclose(b, a, rtol=1e-9, atol=1e-300, err_msg=f"{label} {name}")
    for name in GLOBAL_WEIGHTS:
        np.testing.assert_allclose(eng.array(name), og.array(name), rtol=1e-9, atol=1e-300,
                                   err_msg=f"{label} {name}")


def _inject_weights(og, eng):
    for name, _ in NODE_WEIGHTS:
        w = eng.array(name)
        if w.size:
            og.set_weights(name, w)
    for name in GLOBAL_WEIGHTS:
        og.set_weights(name, eng.array(name))


def _cmp_walks(ref, got, label):
    for k in ("nodes", "timestamps", "lens", "edge_ids"):
        a, b = getattr(ref, k), getattr(got, k)
        assert a.shape == b.shape, (label, k)
        bad = np.nonzero((a != b).reshape(a.shape[0], -1).any(axis=1))[0]
        assert bad.size == 0, f"{label}: {k} differs in {bad.size} walks, first {bad[:5]}"


def test_cfg3_full_oracle_parity():
    """undirected 5M ids / 100M edges with dim-16 features."""
    src, dst, ts, feats = configs.cfg3()
    og = po.OracleGraph(False)
    og.add_edges(src, dst, ts, feats, num_threads=THREADS)
    eng = _engine(is_directed=False)
    eng.add_edges(src, dst, ts, feats)
    del src, dst, ts, feats
    _cmp_index(og, eng, "cfg3")
    # the cfg3 call (for_all_nodes wpn=5, L=40, Linear/Linear, backward) on
    # 20,000 active nodes spread over the id range
    ids = np.nonzero(og.array("active_node_ids"))[0].astype(np.int32)
    seeds = ids[:: ids.size // 20_000][:20_000]
    L, wpn = 40, 5
    starts = np.repeat(seeds, wpn)
    dr = graphs.draws(len(starts), L, seed=45)
    ref = og.walks(L, "Linear", "Linear", False, starts, dr, num_threads=THREADS)
    got = eng.sample("nodes", L, "Linear", wpn, initial_edge_bias="Linear",
                     direction="Backward_In_Time", seed_nodes=seeds, replay=dr, shuffle=False)
    assert len(starts) == N_WALKS
    _cmp_walks(ref, got, "cfg3")
    assert eng.walk_stats()["slot_word_format"] == 1
    assert int(got.lens.sum()) > 5 * N_WALKS
    # every edge-id slot carries its edge's feature row, zeros past the length
    store_f = og.array("edge_features").reshape(-1, 16)
    e = got.edge_ids
    exp = np.zeros(e.shape + (16,), np.float32)
    exp[e >= 0] = store_f[e[e >= 0]]
    assert np.array_equal(got.edge_features, exp)
    eng.close()


def test_cfg4_full_oracle_parity():
    """directed 2M ids / 50M edges, weights with timescale_bound
    50; ExponentialWeight walks (L=80) from ExponentialWeight starts."""
    src, dst, ts = configs.cfg4()
    og = po.OracleGraph(True, enable_weight_computation=True, timescale_bound=50.0)
    og.add_edges(src, dst, ts, num_threads=THREADS)
    eng = _engine(is_directed=True, enable_weight_computation=True, timescale_bound=50.0)
    eng.add_edges(src, dst, ts)
    del src, dst, ts
    _cmp_index(og, eng, "cfg4")
    _cmp_weights(og, eng, "cfg4")
    G = np.diff(eng.array("count_ts_group_per_node_outbound").astype(np.int64))
    assert G.max() > 8_000_000  # the walks cross hubs of millions of groups
    _inject_weights(og, eng)
    L = 80
    dr = graphs.draws(N_WALKS, L, seed=46)
    starts = -np.ones(N_WALKS, np.int32)
    ref = og.walks(L, "ExponentialWeight", "ExponentialWeight", True, starts, dr,
                   num_threads=THREADS)
    got = eng.sample("total", L, "ExponentialWeight", N_WALKS,
                     initial_edge_bias="ExponentialWeight", replay=dr, shuffle=False)
    _cmp_walks(ref, got, "cfg4")
    assert int(got.lens.sum()) > 50 * N_WALKS
    eng.close()


def test_cfg5_full_oracle_parity():
    """10 batches of 3M edges through a window of 3e6 time units
    with TemporalNode2Vec (p=0.5, q=2); after batches 3 and 10 the index,
    weights and adjacency, then TemporalNode2Vec/Uniform walks (L=40)."""
    cap = 3_000_000
    og = po.OracleGraph(True, cap, enable_temporal_node2vec=True, p=0.5, q=2.0)
    eng = _engine(is_directed=True, max_time_capacity=cap, enable_temporal_node2vec=True,
                  node2vec_p=0.5, node2vec_q=2.0)
    checked = 0
    for k, (s_b, d_b, t_b) in enumerate(configs.cfg5_batches()):
        og.add_edges(s_b, d_b, t_b, num_threads=THREADS)
        eng.add_edges(s_b, d_b, t_b)
        if k not in (2, 9):
            continue
        label = f"cfg5 batch {k + 1}"
        _cmp_index(og, eng, label)
        _cmp_weights(og, eng, label)
        for name in ("node_adj_offsets", "node_adj_neighbors"):
            assert np.array_equal(og.array(name), eng.array(name)), (label, name)
        _inject_weights(og, eng)
        L = 40
        dr = graphs.draws(N_WALKS, L, seed=47 + k)
        ref = og.walks(L, "TemporalNode2Vec", "Uniform", True, -np.ones(N_WALKS, np.int32), dr,
                       num_threads=THREADS)
        got = eng.sample("total", L, "TemporalNode2Vec", N_WALKS, initial_edge_bias="Uniform",
                         replay=dr, shuffle=False)
        _cmp_walks(ref, got, label)
        assert int(got.lens.sum()) > 10 * N_WALKS
        checked += 1
    assert checked == 2
    eng.close()
