"""trw_sample_device_noalloc, the entry point that allocates nothing: its
walks, written into caller-owned device buffers with every per-call buffer
taken from the library's fixed per-device scratch array, equal those of
trw_sample_device for the same call -- on consecutive calls, the second
smaller than the first, across start modes, processing orders, shuffles,
cutoffs, replay draws and edge features.  Through the C ABI."""
import numpy as np
import pytest

from tests import graphs

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _torch_device_first():
    """torch's HIP runtime starts before the engine's: the test's output
    buffers are torch tensors, and torch brings its own copy of the runtime
    library, which must be the first one loaded in the process."""
    import torch
    torch.zeros(1, device="cuda")
    torch.cuda.synchronize()


def _engine(dim, seed=9):
    from temporal_random_walk import capi
    s, d, t = graphs.powerlaw(20_000, 300_000, n_ts=5_000, seed=5)
    f = np.random.default_rng(2).standard_normal((len(s), dim)).astype(np.float32) if dim else None
    eng = capi.Engine(is_directed=True, global_seed=seed, shuffle_walk_order=True)
    eng.add_edges(s, d, t, f)
    return eng


def _rows(w, L, dim, n=None):
    """Device copies (torch) of the first n walks of a device sample."""
    import torch
    from temporal_random_walk import capi
    n = int(w.num_walks) if n is None else n
    out = []
    specs = [(w.nodes, n * L, torch.int32), (w.timestamps, n * L, torch.int64),
             (w.walk_lens, n, torch.int64), (w.edge_ids, n * (L - 1), torch.int64)]
    if dim:
        specs.append((w.edge_features, n * (L - 1) * dim, torch.float32))
    for ptr, count, dt in specs:
        t = torch.empty(count, dtype=dt, device="cuda")
        if count:
            capi.device_copy(t.data_ptr(), ptr, t.numel() * t.element_size())
        out.append(t)
    torch.cuda.synchronize()
    return out


def _noalloc(eng, cap, L, dim, mode, bias, n, **kw):
    import torch
    bufs = {
        "nodes": torch.full((cap * L,), -7, dtype=torch.int32, device="cuda"),
        "ts": torch.full((cap * L,), -7, dtype=torch.int64, device="cuda"),
        "lens": torch.full((cap,), 7, dtype=torch.int64, device="cuda"),
        "eids": torch.full((cap * (L - 1),), -7, dtype=torch.int64, device="cuda"),
        "feat": torch.full((cap * (L - 1) * max(dim, 1),), -7.0, dtype=torch.float32,
                           device="cuda"),
    }
    torch.cuda.synchronize()
    w = eng.sample_device_noalloc(mode, L, bias, n, capacity_walks=cap,
                                  nodes_ptr=bufs["nodes"].data_ptr(),
                                  timestamps_ptr=bufs["ts"].data_ptr(),
                                  lens_ptr=bufs["lens"].data_ptr(),
                                  edge_ids_ptr=bufs["eids"].data_ptr(),
                                  features_ptr=bufs["feat"].data_ptr() if dim else None, **kw)
    assert w.max_walk_len == L and w.feature_dim == dim
    return w, bufs


def _same(eng, cap, L, dim, mode, bias, n, **kw):
    import torch
    ref = _rows(eng.sample_device(mode, L, bias, n, **kw), L, dim)
    w, bufs = _noalloc(eng, cap, L, dim, mode, bias, n, **kw)
    got = _rows(w, L, dim)
    assert int(w.num_walks) == ref[2].numel()
    for name, x, y in zip(("nodes", "timestamps", "lens", "edge_ids", "features"), ref, got):
        assert torch.equal(x, y), (mode, bias, n, name)
    # rows past the sample's walks are left as they were
    nw = int(w.num_walks)
    assert bool((bufs["lens"][nw:] == 7).all())
    return nw


@pytest.mark.parametrize("dim", [8, 6])
def test_noalloc_sample_equals_sample_device(dim):
    eng = _engine(dim)
    cap = 100_000
    L = 24
    # >= 2^16 walks: start-time order; then a smaller call in a row
    assert _same(eng, cap, L, dim, "total", "ExponentialIndex", 80_000,
                 initial_edge_bias="Uniform") == 80_000
    assert _same(eng, cap, L, dim, "total", "Linear", 5_000) == 5_000
    # the scratch and layout pass, in place of rows written by the walk kernel
    _same(eng, cap, L, dim, "total", "ExponentialIndex", 60_000, initial_edge_bias="Uniform",
          walk_layout="scratch")
    # start arrays built in the scratch: all nodes (shuffled), seeds with
    # cutoffs (shuffled together), replay draws, backward walks
    nodes = eng.node_count()
    _same(eng, cap, L, dim, "all_nodes", "Uniform", 2)
    assert 2 * nodes <= cap
    seeds = np.arange(0, 3_000, 3, dtype=np.int32)
    cut = np.full(seeds.size, 60_000_000, dtype=np.int64)
    _same(eng, cap, L, dim, "nodes", "ExponentialIndex", 4, seed_nodes=seeds, cutoff_times=cut,
          direction="Backward_In_Time")
    dr = graphs.draws(3_000, L, seed=4)
    _same(eng, cap, L, dim, "total", "Uniform", 3_000, replay=dr, shuffle=False,
          walk_order="start_time")
    eng.close()


def test_noalloc_sample_rejects_what_does_not_fit():
    eng = _engine(0)
    L = 80
    # more walks than the outputs hold
    with pytest.raises(ValueError, match="capacity"):
        _noalloc(eng, 1_000, L, 0, "total", "Uniform", 2_000)
    # more scratch than the fixed array holds (walk scratch of 640 B per walk
    # at L = 80)
    with pytest.raises(ValueError, match="no-allocation"):
        _noalloc(eng, 400_000, L, 0, "total", "Uniform", 400_000, walk_layout="scratch")
    # outputs the 16-byte row stores cannot take
    import torch
    ts = torch.empty(1_000 * L + 1, dtype=torch.int64, device="cuda")
    with pytest.raises(ValueError, match="aligned"):
        eng.sample_device_noalloc("total", L, "Uniform", 1_000, capacity_walks=1_000,
                                  nodes_ptr=torch.empty(1_000 * L, dtype=torch.int32,
                                                        device="cuda").data_ptr(),
                                  timestamps_ptr=ts.data_ptr() + 8,
                                  lens_ptr=torch.empty(1_000, dtype=torch.int64,
                                                       device="cuda").data_ptr(),
                                  edge_ids_ptr=torch.empty(1_000 * (L - 1), dtype=torch.int64,
                                                           device="cuda").data_ptr())
    # the handle and the array stay usable
    _same(eng, 20_000, L, 0, "total", "ExponentialIndex", 20_000)
    # rows written by the walk kernel need no walk scratch: the same sample fits
    _same(eng, 400_000, L, 0, "total", "Uniform", 400_000)
    eng.close()
