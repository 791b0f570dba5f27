"""ctypes view of the engine's C ABI (``include/trw_engine.h``).

This is what a maintainer of the reference would add to bind the engine from
Python without the pybind11 module; the test-suite and ``bench.py`` use it to
reach the device-resident entry points (``trw_add_edges_device``,
``trw_sample_device``) and the index snapshots.

Loading fails loudly when ``libtrw_engine.so`` has not been built: there is no
CPU fallback behind this API.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtrw_engine.so")

PICKERS = {
    "Uniform": 0,
    "Linear": 1,
    "ExponentialIndex": 2,
    "ExponentialWeight": 3,
    "TemporalNode2Vec": 4,
    "TEST_FIRST": 5,
    "TEST_LAST": 6,
}
DIRECTIONS = {"Forward_In_Time": 0, "Backward_In_Time": 1}
# trw_walk_order: the order walks run in on the device (the output is the same)
WALK_ORDERS = {"auto": 0, "walk_id": 1, "start_time": 2, "node_grouped": 3}
# trw_walk_layout: rows written by the walk kernel where it applies, or always
# scratch and the layout pass (the output is the same)
WALK_LAYOUTS = {"auto": 0, "scratch": 1}
MODES = {"total": 0, "all_nodes": 1, "last_batch": 2, "nodes": 3}

# (id, numpy dtype) in the order of trw_array_id
ARRAYS = {
    "sources": (0, np.int32),
    "targets": (1, np.int32),
    "timestamps": (2, np.int64),
    "timestamp_group_offsets": (3, np.uint64),
    "unique_timestamps": (4, np.int64),
    "active_node_ids": (5, np.int32),
    "node_group_outbound_offsets": (6, np.uint64),
    "node_group_inbound_offsets": (7, np.uint64),
    "node_ts_sorted_outbound_indices": (8, np.uint64),
    "node_ts_sorted_inbound_indices": (9, np.uint64),
    "count_ts_group_per_node_outbound": (10, np.uint64),
    "count_ts_group_per_node_inbound": (11, np.uint64),
    "node_ts_group_outbound_offsets": (12, np.uint64),
    "node_ts_group_inbound_offsets": (13, np.uint64),
    "forward_cumulative_weights_exponential": (14, np.float64),
    "backward_cumulative_weights_exponential": (15, np.float64),
    "outbound_forward_cumulative_weights_exponential": (16, np.float64),
    "outbound_backward_cumulative_weights_exponential": (17, np.float64),
    "inbound_backward_cumulative_weights_exponential": (18, np.float64),
    "node_adj_offsets": (19, np.uint64),
    "node_adj_neighbors": (20, np.int32),
    "edge_features": (21, np.float32),
}

# every symbol include/trw_engine.h declares
EXPORTS = [
    "trw_create", "trw_destroy", "trw_last_error", "trw_abi_version", "trw_add_edges",
    "trw_add_edges_device", "trw_prefetch_edges", "trw_add_prefetched_edges", "trw_sample",
    "trw_sample_device", "trw_sample_device_noalloc", "trw_walks_free",
    "trw_get_node_count", "trw_get_edge_count", "trw_get_node_ids", "trw_get_node_degrees",
    "trw_get_edges", "trw_get_is_directed", "trw_get_memory_used", "trw_get_feature_dim",
    "trw_get_latest_timestamp", "trw_clear", "trw_get_array", "trw_get_timings",
    "trw_get_stream", "trw_get_walk_stats", "trw_debug_fail_allocation",
    "trw_debug_fail_allocation_transient", "trw_pick_index", "trw_pick_weights",
]


class TrwConfig(C.Structure):
    _fields_ = [
        ("is_directed", C.c_int32),
        ("enable_weight_computation", C.c_int32),
        ("enable_temporal_node2vec", C.c_int32),
        ("walk_padding_value", C.c_int32),
        ("max_time_capacity", C.c_int64),
        ("timescale_bound", C.c_double),
        ("node2vec_p", C.c_double),
        ("node2vec_q", C.c_double),
        ("global_seed", C.c_uint64),
        ("shuffle_walk_order", C.c_int32),
        ("device_id", C.c_int32),
    ]


class TrwSampleParams(C.Structure):
    _fields_ = [
        ("mode", C.c_int32),
        ("max_walk_len", C.c_int32),
        ("walk_bias", C.c_int32),
        ("initial_edge_bias", C.c_int32),
        ("direction", C.c_int32),
        ("num_walks_per_node", C.c_int32),
        ("num_walks_total", C.c_int64),
        ("seed_nodes", C.c_void_p),
        ("cutoff_times", C.c_void_p),
        ("num_seed_nodes", C.c_uint64),
        ("replay_draws", C.c_void_p),
        ("replay_draws_len", C.c_uint64),
        ("shuffle", C.c_int32),
        ("walk_order", C.c_int32),
        ("walk_layout", C.c_int32),
    ]


class TrwWalks(C.Structure):
    _fields_ = [
        ("num_walks", C.c_uint64),
        ("max_walk_len", C.c_int32),
        ("feature_dim", C.c_int32),
        ("nodes", C.c_void_p),
        ("timestamps", C.c_void_p),
        ("walk_lens", C.c_void_p),
        ("edge_ids", C.c_void_p),
        ("edge_features", C.c_void_p),
    ]


class TrwTimings(C.Structure):
    _fields_ = [
        ("build_ms", C.c_double),
        ("sort_ms", C.c_double),
        ("index_ms", C.c_double),
        ("sample_ms", C.c_double),
        ("walk_kernel_ms", C.c_double),
        ("walk_kernel_launches", C.c_uint64),
        ("handoff_ms", C.c_double),
        ("handoff_bytes", C.c_uint64),
    ]


class TrwWalkStats(C.Structure):
    _fields_ = [
        ("total_len", C.c_uint64),
        ("transitions", C.c_uint64),
        ("nonempty_walks", C.c_uint64),
        ("algorithmic_bytes", C.c_uint64),
        ("reference_bytes", C.c_uint64),
        ("compulsory_read_bytes", C.c_uint64),
        ("compulsory_write_bytes", C.c_uint64),
        ("rows_by_walk_kernel", C.c_uint64),
        ("slot_word_format", C.c_uint64),
    ]


ABI_VERSION = 7  # TRW_ABI_VERSION of include/trw_engine.h
_lib = None


class EngineError(RuntimeError):
    pass


def lib():
    """Load libtrw_engine.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build the HIP engine first "
                "(python temporal-random-walk_amd/build.py)")
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        L.trw_create.argtypes = [C.POINTER(TrwConfig), C.POINTER(C.c_void_p)]
        L.trw_destroy.argtypes = [P]
        L.trw_last_error.restype = C.c_char_p
        L.trw_abi_version.restype = C.c_int32
        L.trw_add_edges.argtypes = [P, P, P, P, C.c_uint64, P, C.c_uint64]
        L.trw_add_edges_device.argtypes = [P, P, P, P, C.c_uint64, P, C.c_uint64]
        L.trw_prefetch_edges.argtypes = [P, P, P, P, C.c_uint64, P, C.c_uint64]
        L.trw_add_prefetched_edges.argtypes = [P]
        L.trw_sample.argtypes = [P, C.POINTER(TrwSampleParams), C.POINTER(TrwWalks)]
        L.trw_sample_device.argtypes = [P, C.POINTER(TrwSampleParams), C.POINTER(TrwWalks)]
        L.trw_sample_device_noalloc.argtypes = [P, C.POINTER(TrwSampleParams), C.c_uint64,
                                                C.POINTER(TrwWalks)]
        L.trw_walks_free.argtypes = [C.POINTER(TrwWalks)]
        L.trw_walks_free.restype = None
        L.trw_get_node_count.argtypes = [P, C.POINTER(C.c_uint64)]
        L.trw_get_edge_count.argtypes = [P, C.POINTER(C.c_uint64)]
        L.trw_get_node_ids.argtypes = [P, P, C.c_uint64, C.POINTER(C.c_uint64)]
        L.trw_get_node_degrees.argtypes = [P, P, C.c_uint64, C.c_int32, P]
        L.trw_get_edges.argtypes = [P, P, P, P, C.c_uint64, C.POINTER(C.c_uint64)]
        L.trw_get_is_directed.argtypes = [P, C.POINTER(C.c_int32)]
        L.trw_get_memory_used.argtypes = [P, C.POINTER(C.c_uint64)]
        L.trw_get_feature_dim.argtypes = [P, C.POINTER(C.c_uint64)]
        L.trw_get_latest_timestamp.argtypes = [P, C.POINTER(C.c_int64)]
        L.trw_clear.argtypes = [P]
        L.trw_get_array.argtypes = [P, C.c_int32, P, C.c_uint64, C.POINTER(C.c_uint64),
                                    C.POINTER(C.c_uint32)]
        L.trw_get_timings.argtypes = [P, C.POINTER(TrwTimings)]
        L.trw_get_stream.argtypes = [P, C.POINTER(C.c_void_p)]
        L.trw_get_walk_stats.argtypes = [P, C.POINTER(TrwWalkStats)]
        L.trw_debug_fail_allocation.argtypes = [C.c_int64]
        L.trw_debug_fail_allocation.restype = None
        L.trw_debug_fail_allocation_transient.argtypes = [C.c_int64]
        L.trw_debug_fail_allocation_transient.restype = None
        L.trw_pick_index.argtypes = [C.c_int32, C.c_int32, P, P, C.c_uint64, C.c_int32, P,
                                     C.c_uint64, P]
        L.trw_pick_weights.argtypes = [C.c_int32, P, C.c_uint64, P, P, C.c_uint64, P,
                                       C.c_uint64, P]
        if L.trw_abi_version() != ABI_VERSION:
            raise ImportError(f"{LIB_PATH} has ABI {L.trw_abi_version()}, these bindings "
                              f"expect {ABI_VERSION}: rebuild the HIP engine")
        _lib = L
    return _lib


_free = None


class _HostBuffer:
    """Owner of one malloc'd host result array (caller-owned per the C ABI)."""

    def __init__(self, ptr, shape, dtype):
        self.ptr = ptr
        self.__array_interface__ = {"shape": tuple(int(x) for x in shape),
                                    "typestr": np.dtype(dtype).str,
                                    "data": (int(ptr or 0), False), "version": 3}

    def __del__(self):
        if self.ptr:
            _free(self.ptr)
            self.ptr = None


def _adopt(ptr, shape, dtype):
    global _free
    if _free is None:
        f = C.CDLL(None).free
        f.argtypes = [C.c_void_p]
        f.restype = None
        _free = f
    if not ptr:
        return np.zeros(shape, dtype=dtype)
    return np.asarray(_HostBuffer(ptr, shape, dtype))


_hip = None


def device_to_host(dptr, count, dtype, offset_elems=0):
    """Copy `count` elements of `dtype` starting `offset_elems` into a device
    buffer returned by trw_sample_device (hipMemcpy, device -> host)."""
    global _hip
    if _hip is None:
        lib()  # the engine pulls in the HIP runtime
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        _hip.hipMemcpy.restype = C.c_int
    out = np.empty(int(count), dtype=dtype)
    if count:
        src = int(dptr) + int(offset_elems) * out.itemsize
        rc = _hip.hipMemcpy(out.ctypes.data, src, out.nbytes, 2)  # hipMemcpyDeviceToHost
        if rc != 0:
            raise EngineError(f"hipMemcpy failed ({rc})")
    return out


def device_copy(dst_ptr, src_ptr, nbytes):
    """hipMemcpy of nbytes between two device buffers (e.g. a buffer returned
    by trw_sample_device into a torch tensor)."""
    global _hip
    if _hip is None:
        device_to_host(0, 0, np.uint8)  # loads the HIP runtime
    if nbytes:
        rc = _hip.hipMemcpy(int(dst_ptr), int(src_ptr), int(nbytes), 3)  # hipMemcpyDeviceToDevice
        if rc != 0:
            raise EngineError(f"hipMemcpy failed ({rc})")


def _fresh_seed():
    return int.from_bytes(os.urandom(8), "little")


def pick_index(picker, starts, ends, prioritize_end=True, draws=None, seed=None, device_id=-1):
    """trw_pick_index: one pick per (start, end) range with the named index
    picker; draws (uniforms in [0, 1)) or in-kernel Philox keyed by seed (a
    fresh one if None).  Returns int32 picks, -1 for an empty range."""
    s = np.ascontiguousarray(starts, dtype=np.int32).ravel()
    e = np.ascontiguousarray(ends, dtype=np.int32).ravel()
    if s.size != e.size:
        raise ValueError("starts and ends must have the same length")
    d = None if draws is None else np.ascontiguousarray(draws, dtype=np.float64).ravel()
    if d is not None and d.size != s.size:
        raise ValueError("one random number per pick is required")
    out = np.empty(s.size, dtype=np.int32)
    _check(lib().trw_pick_index(int(device_id), PICKERS[picker], s.ctypes.data, e.ctypes.data,
                                s.size, int(bool(prioritize_end)),
                                None if d is None else d.ctypes.data,
                                _fresh_seed() if seed is None else int(seed), out.ctypes.data))
    return out


def pick_weights(cumulative, group_starts, group_ends, draws=None, seed=None, device_id=-1):
    """trw_pick_weights: one weight-based pick per [group_start, group_end)
    range of one cumulative-weight array; draws as for pick_index."""
    w = np.ascontiguousarray(cumulative, dtype=np.float64).ravel()
    gs = np.ascontiguousarray(group_starts, dtype=np.uint64).ravel()
    ge = np.ascontiguousarray(group_ends, dtype=np.uint64).ravel()
    if gs.size != ge.size:
        raise ValueError("group_starts and group_ends must have the same length")
    d = None if draws is None else np.ascontiguousarray(draws, dtype=np.float64).ravel()
    if d is not None and d.size != gs.size:
        raise ValueError("one random number per pick is required")
    out = np.empty(gs.size, dtype=np.int32)
    _check(lib().trw_pick_weights(int(device_id), w.ctypes.data if w.size else None, w.size,
                                  gs.ctypes.data, ge.ctypes.data, gs.size,
                                  None if d is None else d.ctypes.data,
                                  _fresh_seed() if seed is None else int(seed), out.ctypes.data))
    return out


def _check(rc):
    if rc != 0:
        msg = lib().trw_last_error().decode()
        if rc == 1:
            raise ValueError(msg)
        if rc == 3:
            raise MemoryError(msg)
        raise EngineError(msg)


def _ptr(a):
    return None if a is None else a.ctypes.data


def debug_fail_allocation(n):
    """Test hook: the next n device allocations succeed, the one after them
    fails as out of memory (MemoryError), its retry included; n < 0 disarms."""
    lib().trw_debug_fail_allocation(int(n))


def debug_fail_allocation_transient(n):
    """Test hook: the next n device allocations succeed and the first attempt
    of the one after them fails as out of memory; the retry after releasing
    the blocks of grown buffers the engine holds succeeds (with none held the
    allocation fails: MemoryError).  n < 0 disarms."""
    lib().trw_debug_fail_allocation_transient(int(n))


class Walks:
    """Host copy of one sampling call (numpy arrays)."""

    def __init__(self, nodes, timestamps, lens, edge_ids, edge_features):
        self.nodes = nodes
        self.timestamps = timestamps
        self.lens = lens
        self.edge_ids = edge_ids
        self.edge_features = edge_features


class Engine:
    def __init__(self, is_directed, max_time_capacity=-1, enable_weight_computation=False,
                 enable_temporal_node2vec=False, timescale_bound=-1.0, node2vec_p=1.0,
                 node2vec_q=1.0, walk_padding_value=-1, global_seed=None,
                 shuffle_walk_order=True, device_id=0):
        self._L = lib()
        cfg = TrwConfig(
            is_directed=int(bool(is_directed)),
            enable_weight_computation=int(bool(enable_weight_computation)),
            enable_temporal_node2vec=int(bool(enable_temporal_node2vec)),
            walk_padding_value=int(walk_padding_value),
            max_time_capacity=int(max_time_capacity),
            timescale_bound=float(timescale_bound),
            node2vec_p=float(node2vec_p),
            node2vec_q=float(node2vec_q),
            global_seed=(2**64 - 1) if global_seed is None else int(global_seed),
            shuffle_walk_order=int(bool(shuffle_walk_order)),
            device_id=int(device_id),
        )
        h = C.c_void_p()
        _check(self._L.trw_create(C.byref(cfg), C.byref(h)))
        self.h = h
        self.is_directed = bool(is_directed)

    def close(self):
        if getattr(self, "h", None):
            self._L.trw_destroy(self.h)  # waits for a pending prefetch
            self.h = None
        self._prefetch_keep = None

    def __del__(self):
        self.close()

    # ---- ingest
    def add_edges(self, src, dst, ts, features=None):
        src = np.ascontiguousarray(src, dtype=np.int32)
        dst = np.ascontiguousarray(dst, dtype=np.int32)
        ts = np.ascontiguousarray(ts, dtype=np.int64)
        dim = 0
        f = None
        if features is not None:
            f = np.ascontiguousarray(features, dtype=np.float32)
            dim = f.size // max(len(src), 1)
        _check(self._L.trw_add_edges(self.h, _ptr(src), _ptr(dst), _ptr(ts), len(src), _ptr(f),
                                     dim))

    def prefetch_edges(self, src, dst, ts, features=None):
        """Starts copying a host batch to the device beside later calls; the
        arrays are held until add_prefetched_edges."""
        src = np.ascontiguousarray(src, dtype=np.int32)
        dst = np.ascontiguousarray(dst, dtype=np.int32)
        ts = np.ascontiguousarray(ts, dtype=np.int64)
        dim = 0
        f = None
        if features is not None:
            f = np.ascontiguousarray(features, dtype=np.float32)
            dim = f.size // max(len(src), 1)
        _check(self._L.trw_prefetch_edges(self.h, _ptr(src), _ptr(dst), _ptr(ts), len(src),
                                          _ptr(f), dim))
        self._prefetch_keep = (src, dst, ts, f)

    def add_prefetched_edges(self):
        # the call joins the copy (or finds none pending) before it returns,
        # so the held arrays may go either way
        try:
            _check(self._L.trw_add_prefetched_edges(self.h))
        finally:
            self._prefetch_keep = None

    def add_edges_device(self, src_ptr, dst_ptr, ts_ptr, n, feat_ptr=None, dim=0):
        _check(self._L.trw_add_edges_device(self.h, src_ptr, dst_ptr, ts_ptr, int(n), feat_ptr,
                                            int(dim)))

    # ---- sampling
    def _params(self, mode, max_walk_len, walk_bias, num_walks=0, initial_edge_bias=None,
                direction="Forward_In_Time", seed_nodes=None, cutoff_times=None, replay=None,
                shuffle=None, walk_order="auto", walk_layout="auto"):
        keep = []
        p = TrwSampleParams()
        p.mode = MODES[mode]
        p.max_walk_len = int(max_walk_len)
        p.walk_bias = PICKERS[walk_bias]
        p.initial_edge_bias = -1 if initial_edge_bias is None else PICKERS[initial_edge_bias]
        p.direction = DIRECTIONS[direction]
        if mode == "total":
            p.num_walks_total = int(num_walks)
        else:
            p.num_walks_per_node = int(num_walks)
        if seed_nodes is not None:
            s = np.ascontiguousarray(seed_nodes, dtype=np.int32)
            keep.append(s)
            p.seed_nodes = s.ctypes.data
            p.num_seed_nodes = len(s)
        if cutoff_times is not None:
            c = np.ascontiguousarray(cutoff_times, dtype=np.int64)
            keep.append(c)
            p.cutoff_times = c.ctypes.data
        if replay is not None:
            r = np.ascontiguousarray(replay, dtype=np.float64)
            keep.append(r)
            p.replay_draws = r.ctypes.data
            p.replay_draws_len = r.size
        p.shuffle = -1 if shuffle is None else int(bool(shuffle))
        p.walk_order = WALK_ORDERS[walk_order]
        p.walk_layout = WALK_LAYOUTS[walk_layout]
        return p, keep

    def sample(self, mode, max_walk_len, walk_bias, num_walks=0, **kw):
        p, keep = self._params(mode, max_walk_len, walk_bias, num_walks, **kw)
        w = TrwWalks()
        _check(self._L.trw_sample(self.h, C.byref(p), C.byref(w)))
        n, L = int(w.num_walks), int(w.max_walk_len)
        el = max(L - 1, 0)
        d = int(w.feature_dim) if w.edge_features else 0
        # each array adopts its malloc'd buffer (no copy); free() runs when
        # the last view of it goes away
        nodes = _adopt(w.nodes, (n, L), np.int32)
        ts = _adopt(w.timestamps, (n, L), np.int64)
        lens = _adopt(w.walk_lens, (n,), np.uint64)
        eids = _adopt(w.edge_ids, (n, el), np.int64)
        feats = _adopt(w.edge_features, (n, el, d), np.float32) if d else None
        return Walks(nodes, ts, lens, eids, feats)

    def sample_device(self, mode, max_walk_len, walk_bias, num_walks=0, **kw):
        """Walks stay in HBM; returns the TrwWalks with device pointers."""
        p, keep = self._params(mode, max_walk_len, walk_bias, num_walks, **kw)
        w = TrwWalks()
        _check(self._L.trw_sample_device(self.h, C.byref(p), C.byref(w)))
        return w

    def sample_device_noalloc(self, mode, max_walk_len, walk_bias, num_walks=0, *,
                              capacity_walks, nodes_ptr, timestamps_ptr, lens_ptr,
                              edge_ids_ptr, features_ptr=None, **kw):
        """trw_sample_device_noalloc: walks into the caller's device buffers
        (room for capacity_walks walks), nothing allocated.  Returns the
        TrwWalks filled in by the call."""
        p, keep = self._params(mode, max_walk_len, walk_bias, num_walks, **kw)
        w = TrwWalks()
        w.nodes = nodes_ptr
        w.timestamps = timestamps_ptr
        w.walk_lens = lens_ptr
        w.edge_ids = edge_ids_ptr
        w.edge_features = features_ptr
        _check(self._L.trw_sample_device_noalloc(self.h, C.byref(p), int(capacity_walks),
                                                 C.byref(w)))
        return w

    # ---- queries
    def array(self, name):
        aid, dt = ARRAYS[name]
        n = C.c_uint64()
        es = C.c_uint32()
        _check(self._L.trw_get_array(self.h, aid, None, 0, C.byref(n), C.byref(es)))
        out = np.zeros(n.value, dtype=dt)
        if n.value:
            _check(self._L.trw_get_array(self.h, aid, out.ctypes.data, n.value, C.byref(n),
                                         C.byref(es)))
        return out

    def node_count(self):
        v = C.c_uint64()
        _check(self._L.trw_get_node_count(self.h, C.byref(v)))
        return v.value

    def edge_count(self):
        v = C.c_uint64()
        _check(self._L.trw_get_edge_count(self.h, C.byref(v)))
        return v.value

    def latest_timestamp(self):
        v = C.c_int64()
        _check(self._L.trw_get_latest_timestamp(self.h, C.byref(v)))
        return v.value

    def timings(self):
        t = TrwTimings()
        _check(self._L.trw_get_timings(self.h, C.byref(t)))
        return {k: getattr(t, k) for k, _ in TrwTimings._fields_}

    def stream(self):
        s = C.c_void_p()
        _check(self._L.trw_get_stream(self.h, C.byref(s)))
        return s.value

    def walk_stats(self):
        s = TrwWalkStats()
        _check(self._L.trw_get_walk_stats(self.h, C.byref(s)))
        return {k: getattr(s, k) for k, _ in TrwWalkStats._fields_}

    def clear(self):
        _check(self._L.trw_clear(self.h))
