"""The five BASELINE.json workloads as seeded synthetic inputs (numpy PCG64,
seed 42 for configs[0], 42 + K for configs[K])."""
import numpy as np

from tests import graphs


def _zipf_ranks(rng, n, n_ids, s):
    """Bounded Zipf(s) over ranks 1..n_ids (rejection of the unbounded draw:
    conditioning on rank <= n_ids gives P(k) proportional to k^-s)."""
    out = rng.zipf(s, n)
    bad = out > n_ids
    while bad.any():
        out[bad] = rng.zipf(s, int(bad.sum()))
        bad = out > n_ids
    return out - 1


def _no_self_loops(rng, src, dst, redraw):
    loops = src == dst
    while loops.any():
        dst[loops] = redraw(int(loops.sum()))
        loops = src == dst
    return dst


def cfg1():
    """directed, 10k nodes, 100k uniform edges, ts uniform [0, 1e6)."""
    return graphs.cfg1(10_000, 100_000, seed=42)


def cfg2():
    """directed, 1M ids, 20M Zipf(1.8) edges, 1e5 distinct ts."""
    return graphs.powerlaw(1_000_000, 20_000_000, s=1.8, n_ts=100_000, ts_hi=100_000_000, seed=44)


def cfg3(n_nodes=5_000_000, n_edges=100_000_000, dim=16, seed=45):
    """undirected; src Zipf(1.5), dst uniform; piecewise-Poisson
    timestamps over 1,000 segments of [0, 1e9) with log-uniform rates [1, 100];
    fp32 N(0,1) edge features of dim 16."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(n_nodes).astype(np.int32)
    src = perm[_zipf_ranks(rng, n_edges, n_nodes, 1.5)]
    dst = rng.integers(0, n_nodes, n_edges).astype(np.int32)
    dst = _no_self_loops(rng, src, dst,
                         lambda k: rng.integers(0, n_nodes, k).astype(np.int32))
    segs = 1000
    rates = np.exp(rng.uniform(np.log(1.0), np.log(100.0), segs))
    counts = rng.multinomial(n_edges, rates / rates.sum())
    seg_len = 1_000_000_000 // segs
    base = np.repeat(np.arange(segs, dtype=np.int64) * seg_len, counts)
    ts = base + rng.integers(0, seg_len, n_edges)
    order = rng.permutation(n_edges)  # edges arrive unsorted
    ts = ts[order]
    feats = rng.standard_normal((n_edges, dim), dtype=np.float32)
    return src, dst, ts, feats


def cfg4(n_nodes=2_000_000, n_edges=50_000_000, seed=46):
    """directed, Zipf(1.6) both ends, ts uniform [0, 1e7)."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(n_nodes).astype(np.int32)
    src = perm[_zipf_ranks(rng, n_edges, n_nodes, 1.6)]
    dst = perm[_zipf_ranks(rng, n_edges, n_nodes, 1.6)]
    dst = _no_self_loops(rng, src, dst,
                         lambda k: perm[_zipf_ranks(rng, k, n_nodes, 1.6)])
    ts = rng.integers(0, 10_000_000, n_edges).astype(np.int64)
    return src, dst, ts


def cfg5_batches(n_nodes=1_000_000, batch=3_000_000, n_batches=10, seed=47):
    """directed Zipf(1.8) streaming; batch k has ts uniform in
    [k*1e6, (k+1)*1e6)."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(n_nodes).astype(np.int32)
    for k in range(n_batches):
        src = perm[_zipf_ranks(rng, batch, n_nodes, 1.8)]
        dst = perm[_zipf_ranks(rng, batch, n_nodes, 1.8)]
        dst = _no_self_loops(rng, src, dst,
                             lambda m: perm[_zipf_ranks(rng, m, n_nodes, 1.8)])
        ts = rng.integers(k * 1_000_000, (k + 1) * 1_000_000, batch).astype(np.int64)
        yield src, dst, ts
