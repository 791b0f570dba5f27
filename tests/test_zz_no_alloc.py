"""trw_sample_device_noalloc, the entry point that allocates nothing: its
walks, written into caller-owned device buffers with every per-call buffer
taken from the library's fixed per-device scratch array, equal those of
trw_sample_device for the same call -- on consecutive calls, the second
smaller than the first, across start modes, processing orders, shuffles,
cutoffs, replay draws, edge features and the weight pickers -- and every
call runs with the engine's allocation hook armed, so any device allocation
inside it would fail the call.  Calls of two handles from two threads take
the device's array in turn.  Through the C ABI."""
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


def _engine(dim, seed=9, weights=False):
    from temporal_random_walk import capi
    s, d, t = graphs.powerlaw(20_000, 300_000, n_ts=5_000, seed=5)
    f = np.random.default_rng(2).standard_normal((len(s), dim)).astype(np.float32) if dim else None
    eng = capi.Engine(is_directed=True, global_seed=seed, shuffle_walk_order=True,
                      enable_weight_computation=weights, enable_temporal_node2vec=weights,
                      timescale_bound=20.0 if weights else -1.0, node2vec_p=0.5, node2vec_q=2.0)
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
    w = _call_noalloc(eng, cap, L, dim, mode, bias, n, bufs, **kw)
    assert w.max_walk_len == L and w.feature_dim == dim
    return w, bufs


def _call_noalloc(eng, cap, L, dim, mode, bias, n, bufs, **kw):
    """The call with the engine's allocation hook armed: the first device
    allocation of any handle would fail it (MemoryError)."""
    from temporal_random_walk import capi
    capi.debug_fail_allocation(0)
    try:
        return eng.sample_device_noalloc(mode, L, bias, n, capacity_walks=cap,
                                         nodes_ptr=bufs["nodes"].data_ptr(),
                                         timestamps_ptr=bufs["ts"].data_ptr(),
                                         lens_ptr=bufs["lens"].data_ptr(),
                                         edge_ids_ptr=bufs["eids"].data_ptr(),
                                         features_ptr=bufs["feat"].data_ptr() if dim else None,
                                         **kw)
    finally:
        capi.debug_fail_allocation(-1)


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


def test_noalloc_sample_weight_pickers():
    """The weight families' kernels (guide tables, weighted panel) through the
    entry point that allocates nothing: ExponentialWeight walks from weight-
    picked starts, then a smaller node2vec sample, then backward walks."""
    eng = _engine(0, weights=True)
    cap = 70_000
    L = 20
    _same(eng, cap, L, 0, "total", "ExponentialWeight", 70_000,
          initial_edge_bias="ExponentialWeight")
    _same(eng, cap, L, 0, "total", "TemporalNode2Vec", 30_000, initial_edge_bias="Uniform")
    _same(eng, cap, L, 0, "total", "ExponentialWeight", 20_000, initial_edge_bias="Uniform",
          direction="Backward_In_Time")
    eng.close()


def test_noalloc_calls_of_two_handles_from_two_threads():
    """Two handles on one device, each sampling from its own thread: the
    device's scratch array is taken in turn, so both threads' walks equal
    their handles' trw_sample_device walks on every round."""
    import threading

    import torch
    L, n = 24, 70_000
    engs = [_engine(0, seed=11), _engine(0, seed=12)]
    kw = dict(initial_edge_bias="Uniform")
    refs = [_rows(e.sample_device("total", L, "ExponentialIndex", n, **kw), L, 0) for e in engs]
    bufs = []
    for _ in engs:
        bufs.append({
            "nodes": torch.empty(n * L, dtype=torch.int32, device="cuda"),
            "ts": torch.empty(n * L, dtype=torch.int64, device="cuda"),
            "lens": torch.empty(n, dtype=torch.int64, device="cuda"),
            "eids": torch.empty(n * (L - 1), dtype=torch.int64, device="cuda"),
            "feat": torch.empty(1, dtype=torch.float32, device="cuda"),
        })
    torch.cuda.synchronize()
    from temporal_random_walk import capi
    for rnd in range(3):
        errors, walks = [], [None, None]
        start = threading.Barrier(2)

        def run(k):
            try:
                start.wait()
                walks[k] = engs[k].sample_device_noalloc(
                    "total", L, "ExponentialIndex", n, capacity_walks=n,
                    nodes_ptr=bufs[k]["nodes"].data_ptr(),
                    timestamps_ptr=bufs[k]["ts"].data_ptr(),
                    lens_ptr=bufs[k]["lens"].data_ptr(),
                    edge_ids_ptr=bufs[k]["eids"].data_ptr(), **kw)
            except Exception as ex:  # reported on the main thread
                errors.append(ex)

        threads = [threading.Thread(target=run, args=(k,)) for k in range(2)]
        for t in threads:
            t.start()
        for t in threads:
            t.join()
        assert not errors, errors
        for k in range(2):
            got = _rows(walks[k], L, 0)
            for name, x, y in zip(("nodes", "timestamps", "lens", "edge_ids"), refs[k], got):
                assert torch.equal(x, y), (rnd, k, name)
    capi.debug_fail_allocation(-1)
    for e in engs:
        e.close()
