"""CPU checks of the drop-in boundary: the C-ABI library loads and exports
every symbol include/trw_engine.h declares; the Python module imports and,
without a GPU, fails loudly instead of falling back to a CPU path."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "trw_engine.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(trw_[a-z_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = _declared_functions()
    for required in ("trw_create", "trw_destroy", "trw_add_edges", "trw_add_edges_device",
                     "trw_sample", "trw_sample_device", "trw_get_array", "trw_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from temporal_random_walk import capi

    lib = ctypes.CDLL(capi.LIB_PATH)
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    assert sorted(capi.EXPORTS) == _declared_functions()
    header = open(HEADER).read()
    declared = int(re.search(r"#define TRW_ABI_VERSION (\d+)", header).group(1))
    assert capi.lib().trw_abi_version() == capi.ABI_VERSION == declared


def test_library_carries_gfx950_code():
    from temporal_random_walk import capi

    blob = open(capi.LIB_PATH, "rb").read()
    assert b"gfx950" in blob


def test_python_surface_matches_reference_names():
    import temporal_random_walk as trw

    cls = trw.TemporalRandomWalk
    for m in ("add_multiple_edges", "get_random_walks_and_times_for_all_nodes",
              "get_random_walks_and_times_for_last_batch", "get_random_walks_and_times_for_nodes",
              "get_random_walks_and_times", "get_node_count", "get_edge_count", "get_node_ids",
              "get_node_degrees", "clear", "get_memory_used", "set_node_features",
              "get_node_features", "add_edges_from_networkx", "to_networkx"):
        assert hasattr(cls, m), m
    # the standalone pickers (py_interface/_temporal_random_walk.cu:904-1016)
    for name in ("LinearRandomPicker", "ExponentialIndexRandomPicker", "UniformRandomPicker",
                 "WeightBasedRandomPicker"):
        picker = getattr(trw, name)(use_gpu=False)
        assert hasattr(picker, "pick_random") and hasattr(picker, "pick_random_batch"), name
    doc = trw.LinearRandomPicker.pick_random.__doc__
    assert "start" in doc and "end" in doc and "prioritize_end" in doc
    assert "cumulative_weights" in trw.WeightBasedRandomPicker.pick_random.__doc__


def test_pickers_fail_loudly_without_gpu():
    import temporal_random_walk as trw

    if _has_gpu():
        pytest.skip("a GPU is present")
    with pytest.raises(RuntimeError, match="only on the GPU"):
        trw.ExponentialIndexRandomPicker(use_gpu=True).pick_random(0, 10)
    with pytest.raises(RuntimeError, match="only on the GPU"):
        trw.WeightBasedRandomPicker().pick_random([0.2, 0.5, 1.0], 0, 3)


def _has_gpu():
    import torch

    return torch.cuda.device_count() > 0


@pytest.mark.skipif(_has_gpu(), reason="checks the no-GPU behaviour")
def test_no_gpu_fails_loudly():
    import temporal_random_walk as trw
    from temporal_random_walk import capi

    with pytest.raises(RuntimeError, match="no HIP device"):
        trw.TemporalRandomWalk(is_directed=True, use_gpu=False)
    with pytest.raises(capi.EngineError, match="no HIP device"):
        capi.Engine(is_directed=True)


def test_host_results_are_adopted_and_freed():
    """trw_sample's arrays are malloc'd and caller-owned: the Python binding
    wraps them without a copy and free()s each when its last view dies."""
    import gc

    import numpy as np

    from temporal_random_walk import capi

    libc = ctypes.CDLL(None)
    libc.malloc.restype = ctypes.c_void_p
    libc.malloc.argtypes = [ctypes.c_size_t]
    ptr = libc.malloc(6 * 8)
    ctypes.memmove(ptr, np.arange(6, dtype=np.int64).ctypes.data, 48)
    a = capi._adopt(ptr, (2, 3), np.int64)
    assert a.ctypes.data == ptr and a.shape == (2, 3)
    np.testing.assert_array_equal(a, np.arange(6).reshape(2, 3))
    view = a[1]
    del a
    gc.collect()
    np.testing.assert_array_equal(view, [3, 4, 5])  # still owned through the view
    del view
    gc.collect()
    empty = capi._adopt(None, (0, 4), np.int32)
    assert empty.shape == (0, 4)
