"""Normal-mode walks at BASELINE scale against the reference sampler's law.

The reference's CPU sampler draws from a std::mt19937 seeded by
random_device and cannot be replayed, so normal mode (in-kernel Philox) is
checked statistically: the engine's walks and the oracle's walks under
independent numpy uniforms are two samples of the same process, and their
per-node transition distributions -- the next node at each of the 20 nodes
that take the most hops -- and their walk-length distributions must pass a
two-sample chi-square test.  The 21 tests of a workload share a family-wise
level of 0.01 (Bonferroni: each p > 0.01 / 21).  Both samples come from fixed
seeds, so the outcome is deterministic.

cfg2: the full 20M-edge graph, 1M walks of L = 80 (ExponentialIndex,
Uniform starts).  cfg5: the window after its third batch, 1M TemporalNode2Vec
walks of L = 40 (p = 0.5, q = 2), the oracle on the engine's weights.
"""
import os

import numpy as np
import pytest

from oracle import pyoracle as po
from tests import configs, graphs
from tests.laws import law_tests

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)))


def _engine(**kw):
    from temporal_random_walk import capi
    kw.setdefault("shuffle_walk_order", False)
    return capi.Engine(**kw)


def test_cfg2_transition_and_length_laws():
    src, dst, ts = configs.cfg2()
    og = po.OracleGraph(True)
    og.add_edges(src, dst, ts, num_threads=THREADS)
    eng = _engine(is_directed=True, global_seed=4402)
    eng.add_edges(src, dst, ts)
    del src, dst, ts
    n, L = 1_000_000, 80
    got = eng.sample("total", L, "ExponentialIndex", n, initial_edge_bias="Uniform")
    ref = og.walks(L, "ExponentialIndex", "Uniform", True, -np.ones(n, np.int32),
                   graphs.draws(n, L, seed=4403), num_threads=THREADS)
    _, covered = law_tests(ref, got, "cfg2")
    assert covered > 0.5  # the busiest nodes take most of the hops
    eng.close()


def test_cfg5_node2vec_transition_and_length_laws():
    cap = 3_000_000
    og = po.OracleGraph(True, cap, enable_temporal_node2vec=True, p=0.5, q=2.0)
    eng = _engine(is_directed=True, max_time_capacity=cap, enable_temporal_node2vec=True,
                  node2vec_p=0.5, node2vec_q=2.0, global_seed=4702)
    for k, (s_b, d_b, t_b) in enumerate(configs.cfg5_batches()):
        og.add_edges(s_b, d_b, t_b, num_threads=THREADS)
        eng.add_edges(s_b, d_b, t_b)
        if k == 2:
            break
    for name in ("outbound_forward_cumulative_weights_exponential",
                 "outbound_backward_cumulative_weights_exponential",
                 "inbound_backward_cumulative_weights_exponential",
                 "forward_cumulative_weights_exponential",
                 "backward_cumulative_weights_exponential"):
        og.set_weights(name, eng.array(name))
    n, L = 1_000_000, 40
    got = eng.sample("total", L, "TemporalNode2Vec", n, initial_edge_bias="Uniform")
    ref = og.walks(L, "TemporalNode2Vec", "Uniform", True, -np.ones(n, np.int32),
                   graphs.draws(n, L, seed=4703), num_threads=THREADS)
    law_tests(ref, got, "cfg5 node2vec")
    eng.close()
