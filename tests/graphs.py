"""Seeded synthetic graphs and draw buffers shared by the tests."""
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def sample_data():
    """The reference's own fixture data/sample_data.csv (20,818 directed edges)."""
    a = np.loadtxt(os.path.join(GOLDEN, "sample_data.csv"), delimiter=",", skiprows=1,
                   dtype=np.int64)
    return a[:, 0].astype(np.int32), a[:, 1].astype(np.int32), a[:, 2].astype(np.int64)


def cfg1(n_nodes=10_000, n_edges=100_000, seed=42):
    """uniform src/dst without self-loops, ts uniform [0, 1e6)."""
    rng = np.random.default_rng(seed)
    src = rng.integers(0, n_nodes, n_edges).astype(np.int32)
    dst = rng.integers(0, n_nodes, n_edges).astype(np.int32)
    loops = src == dst
    while loops.any():
        dst[loops] = rng.integers(0, n_nodes, int(loops.sum()))
        loops = src == dst
    ts = rng.integers(0, 1_000_000, n_edges).astype(np.int64)
    return src, dst, ts


def zipf_ids(rng, n, n_ids, s, perm=None):
    """Bounded Zipf(s) ranks over n_ids ids (inverse CDF), mapped rank -> id
    through `perm` (a fresh seeded permutation when None)."""
    ranks = np.arange(1, n_ids + 1, dtype=np.float64)
    p = ranks ** (-s)
    cdf = np.cumsum(p)
    cdf /= cdf[-1]
    r = np.searchsorted(cdf, rng.random(n), side="right")
    if perm is None:
        perm = rng.permutation(n_ids)
    return perm[np.minimum(r, n_ids - 1)].astype(np.int32)


def powerlaw(n_nodes, n_edges, s=1.8, n_ts=None, ts_hi=100_000_000, seed=44):
    """configs[1]-shaped graph, any size: src and dst Zipf(s) ranks mapped to ids
    through ONE shared permutation (so the src hub is the dst hub), self-loops
    redrawn, timestamps uniform in [0, ts_hi) quantised to n_ts values."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(n_nodes)
    src = zipf_ids(rng, n_edges, n_nodes, s, perm)
    dst = zipf_ids(rng, n_edges, n_nodes, s, perm)
    loops = src == dst
    while loops.any():
        dst[loops] = zipf_ids(rng, int(loops.sum()), n_nodes, s, perm)
        loops = src == dst
    if n_ts:
        ts = (rng.integers(0, n_ts, n_edges) * (ts_hi // n_ts)).astype(np.int64)
    else:
        ts = rng.integers(0, ts_hi, n_edges).astype(np.int64)
    return src, dst, ts


def draws(n_walks, max_walk_len, seed=7):
    return np.random.default_rng(seed).random(n_walks * (1 + 2 * max_walk_len))
