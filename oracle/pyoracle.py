"""ctypes bindings for the parity checkers (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this module.  It loads

* ``oracle/_build/libtrw_oracle.so`` -- the C restatement of the reference's
  CPU path (oracle/trw_oracle.c), and
* ``oracle/_ref/libtrw_ref.so`` -- the reference's own node-index rebuild,
  per-node weights and walk sampler compiled from its sources (only where the
  reference tree was present at build time).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "_build", "libtrw_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libtrw_ref.so")
REF_SRC_ROOT = "/root/reference/temporal_random_walk/src"

PICKERS = {
    "Uniform": 0,
    "Linear": 1,
    "ExponentialIndex": 2,
    "ExponentialWeight": 3,
    "TemporalNode2Vec": 4,
    "TEST_FIRST": 5,
    "TEST_LAST": 6,
}

# name -> numpy dtype of the reference's element type
ARRAY_DTYPES = {
    "sources": np.int32,
    "targets": np.int32,
    "timestamps": np.int64,
    "edge_features": np.float32,
    "timestamp_group_offsets": np.uint64,
    "unique_timestamps": np.int64,
    "active_node_ids": np.int32,
    "node_group_outbound_offsets": np.uint64,
    "node_group_inbound_offsets": np.uint64,
    "node_ts_sorted_outbound_indices": np.uint64,
    "node_ts_sorted_inbound_indices": np.uint64,
    "count_ts_group_per_node_outbound": np.uint64,
    "count_ts_group_per_node_inbound": np.uint64,
    "node_ts_group_outbound_offsets": np.uint64,
    "node_ts_group_inbound_offsets": np.uint64,
    "forward_cumulative_weights_exponential": np.float64,
    "backward_cumulative_weights_exponential": np.float64,
    "outbound_forward_cumulative_weights_exponential": np.float64,
    "outbound_backward_cumulative_weights_exponential": np.float64,
    "inbound_backward_cumulative_weights_exponential": np.float64,
    "node_adj_offsets": np.uint64,
    "node_adj_neighbors": np.int32,
}

NODE_INDEX_ARRAYS = [
    "node_group_outbound_offsets",
    "node_group_inbound_offsets",
    "node_ts_sorted_outbound_indices",
    "node_ts_sorted_inbound_indices",
    "count_ts_group_per_node_outbound",
    "count_ts_group_per_node_inbound",
    "node_ts_group_outbound_offsets",
    "node_ts_group_inbound_offsets",
]
NODE_WEIGHT_ARRAYS = [
    "outbound_forward_cumulative_weights_exponential",
    "outbound_backward_cumulative_weights_exponential",
    "inbound_backward_cumulative_weights_exponential",
]

_P = C.c_void_p


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_P)


def build(ref: bool = True) -> None:
    """Compile the oracle (and the reference driver where the reference is
    mounted).  Called from ``__graft_entry__.build()``."""
    subprocess.check_call(["make", "-s", "-C", HERE, "all"])
    if ref and os.path.isdir(REF_SRC_ROOT):
        subprocess.check_call(["make", "-s", "-C", HERE, "ref"])


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            build(ref=False)
        L = C.CDLL(ORACLE_SO)
        L.orc_create.restype = _P
        L.orc_create.argtypes = [C.c_int, C.c_int64, C.c_int, C.c_int, C.c_double,
                                 C.c_double, C.c_double]
        L.orc_destroy.argtypes = [_P]
        L.orc_set_threads.restype = None
        L.orc_set_threads.argtypes = [_P, C.c_int]
        L.orc_add_edges.restype = C.c_int
        L.orc_add_edges.argtypes = [_P, _P, _P, _P, C.c_size_t, _P, C.c_size_t]
        L.orc_last_error.restype = C.c_char_p
        L.orc_array.restype = _P
        L.orc_array.argtypes = [_P, C.c_char_p, C.POINTER(C.c_size_t),
                                C.POINTER(C.c_size_t)]
        L.orc_set_weights.restype = C.c_int
        L.orc_set_weights.argtypes = [_P, C.c_char_p, _P, C.c_size_t]
        L.orc_latest_timestamp.restype = C.c_int64
        L.orc_latest_timestamp.argtypes = [_P]
        L.orc_max_node_id.restype = C.c_int32
        L.orc_max_node_id.argtypes = [_P]
        L.orc_feature_dim.restype = C.c_size_t
        L.orc_feature_dim.argtypes = [_P]
        L.orc_walks.argtypes = [_P, C.c_int, C.c_int, C.c_int, C.c_int, _P, _P,
                                C.c_size_t, _P, C.c_int, _P, _P, _P, _P, C.c_int]
        L.orc_node_edge_at.argtypes = [_P, C.c_int, C.c_int, C.c_int, C.c_int64, C.c_int64,
                                       C.c_int, C.c_double, C.c_double, _P]
        L.orc_edge_at.argtypes = [_P, C.c_int, C.c_int, C.c_double, C.c_double, _P]
        L.orc_pick_linear.restype = C.c_int
        L.orc_pick_linear.argtypes = [C.c_int, C.c_int, C.c_int, C.c_double]
        L.orc_pick_exponential_index.restype = C.c_int
        L.orc_pick_exponential_index.argtypes = [C.c_int, C.c_int, C.c_int, C.c_double]
        L.orc_pick_uniform.restype = C.c_int
        L.orc_pick_uniform.argtypes = [C.c_int, C.c_int, C.c_double]
        L.orc_pick_exponential_weights.restype = C.c_int
        L.orc_pick_exponential_weights.argtypes = [_P, C.c_size_t, C.c_size_t, C.c_size_t,
                                                   C.c_double, C.c_size_t]
        L.orc_derive_uniform.restype = C.c_double
        L.orc_derive_uniform.argtypes = [C.c_double, C.c_double, C.c_int]
        L.orc_philox4x32_10.restype = None
        L.orc_philox4x32_10.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p]
        L.orc_philox_draws.restype = None
        L.orc_philox_draws.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_int, C.c_void_p]
        L.orc_philox_shuffle_keys.restype = None
        L.orc_philox_shuffle_keys.argtypes = [C.c_uint64, C.c_uint64, C.c_void_p]
        _lib = L
    return _lib


def philox4x32_10(ctr, key):
    """One Philox4x32-10 block (the engine's draw generator)."""
    c = np.ascontiguousarray(ctr, dtype=np.uint32)
    k = np.ascontiguousarray(key, dtype=np.uint32)
    out = np.zeros(4, dtype=np.uint32)
    lib().orc_philox4x32_10(c.ctypes.data, k.ctypes.data, out.ctypes.data)
    return out


def philox_draws(seed, n_walks, max_walk_len, walk0=0):
    """The engine's normal-mode draws of walks [walk0, walk0 + n) in the
    replay layout, n * (1 + 2L) doubles."""
    out = np.empty(int(n_walks) * (1 + 2 * int(max_walk_len)), dtype=np.float64)
    lib().orc_philox_draws(int(seed), int(walk0), int(n_walks), int(max_walk_len),
                           out.ctypes.data)
    return out


def philox_shuffle_order(seed, n):
    """The engine's walk-order shuffle: position i of the shuffled start
    array holds the unshuffled entry order[i]."""
    keys = np.empty(int(n), dtype=np.uint32)
    lib().orc_philox_shuffle_keys(int(seed), int(n), keys.ctypes.data)
    return np.argsort(keys, kind="stable")


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref_lib():
    global _ref
    if _ref is None:
        R = C.CDLL(REF_SO)
        R.ref_create.restype = _P
        R.ref_create.argtypes = [C.c_int, C.c_int, C.c_int, C.c_double, C.c_double,
                                 C.c_double]
        R.ref_destroy.argtypes = [_P]
        R.ref_set_edge_store.argtypes = [_P, _P, _P, _P, C.c_size_t, _P, _P, C.c_size_t,
                                         _P, C.c_size_t, C.c_int, _P, _P, C.c_size_t, _P,
                                         C.c_size_t, _P, C.c_size_t]
        R.ref_rebuild.argtypes = [_P]
        R.ref_array.restype = _P
        R.ref_array.argtypes = [_P, C.c_char_p, C.POINTER(C.c_size_t),
                                C.POINTER(C.c_size_t)]
        R.ref_walks.argtypes = [_P, C.c_int, C.c_int, C.c_int, C.c_int, _P, _P,
                                C.c_size_t, _P, C.c_int, _P, _P, _P, _P]
        _ref = R
    return _ref


def _copy_array(getter, handle, name):
    n = C.c_size_t()
    es = C.c_size_t()
    p = getter(handle, name.encode(), C.byref(n), C.byref(es))
    dt = ARRAY_DTYPES[name]
    if not p or n.value == 0:
        return np.zeros(0, dtype=dt)
    buf = (C.c_char * (n.value * es.value)).from_address(p)
    return np.frombuffer(bytes(buf), dtype=dt).copy()


class WalkResult:
    def __init__(self, nodes, timestamps, lens, edge_ids):
        self.nodes = nodes
        self.timestamps = timestamps
        self.lens = lens
        self.edge_ids = edge_ids


def _alloc_walks(n, L):
    nodes = np.empty(n * L, dtype=np.int32)
    ts = np.empty(n * L, dtype=np.int64)
    lens = np.empty(n, dtype=np.uint64)
    eids = np.empty(n * max(L - 1, 0), dtype=np.int64)
    return nodes, ts, lens, eids


class OracleGraph:
    """The C restatement of the reference's CPU path."""

    def __init__(self, is_directed, max_time_capacity=-1, enable_weight_computation=False,
                 enable_temporal_node2vec=False, timescale_bound=-1.0, p=1.0, q=1.0):
        self._L = lib()
        self.is_directed = bool(is_directed)
        self.enable_weight = bool(enable_weight_computation or enable_temporal_node2vec)
        self.enable_tn2v = bool(enable_temporal_node2vec)
        self.timescale_bound = float(timescale_bound)
        self.p, self.q = float(p), float(q)
        self.h = self._L.orc_create(int(is_directed), int(max_time_capacity),
                                    int(enable_weight_computation),
                                    int(enable_temporal_node2vec), float(timescale_bound),
                                    float(p), float(q))

    def __del__(self):
        if getattr(self, "h", None):
            self._L.orc_destroy(self.h)
            self.h = None

    def add_edges(self, src, dst, ts, features=None, num_threads=1):
        """Ingest one batch; num_threads OpenMP threads (same result for any
        count)."""
        self._L.orc_set_threads(self.h, int(num_threads))
        src = np.ascontiguousarray(src, dtype=np.int32)
        dst = np.ascontiguousarray(dst, dtype=np.int32)
        ts = np.ascontiguousarray(ts, dtype=np.int64)
        dim = 0
        fp = None
        if features is not None:
            features = np.ascontiguousarray(features, dtype=np.float32)
            dim = features.size // max(len(src), 1)
            fp = features
        rc = self._L.orc_add_edges(self.h, _ptr(src), _ptr(dst), _ptr(ts), len(src),
                                   _ptr(fp), dim)
        if rc != 0:
            raise RuntimeError(self._L.orc_last_error().decode())

    def array(self, name):
        return _copy_array(self._L.orc_array, self.h, name)

    def set_weights(self, name, values):
        v = np.ascontiguousarray(values, dtype=np.float64)
        if self._L.orc_set_weights(self.h, name.encode(), _ptr(v), v.size) != 0:
            raise ValueError(f"cannot set {name} ({v.size} values)")

    def node_edge_at(self, node, picker, timestamp=-1, cutoff=-1, prev=-1, forward=True,
                     rg=0.5, re=0.5):
        out = np.zeros(4, dtype=np.int64)
        self._L.orc_node_edge_at(self.h, int(forward), PICKERS[picker], int(node),
                                 int(timestamp), int(cutoff), int(prev), float(rg), float(re),
                                 _ptr(out))
        return tuple(int(x) for x in out)

    def edge_at(self, picker, forward=True, rg=0.5, re=0.5):
        out = np.zeros(4, dtype=np.int64)
        self._L.orc_edge_at(self.h, int(forward), PICKERS[picker], float(rg), float(re),
                            _ptr(out))
        return tuple(int(x) for x in out)

    @property
    def max_node_id(self):
        return self._L.orc_max_node_id(self.h)

    @property
    def latest_timestamp(self):
        return self._L.orc_latest_timestamp(self.h)

    @property
    def feature_dim(self):
        return self._L.orc_feature_dim(self.h)

    def walks(self, max_walk_len, walk_bias, start_bias, forward, start_nodes, draws,
              cutoffs=None, pad=-1, num_threads=0):
        n = len(start_nodes)
        L = int(max_walk_len)
        starts = np.ascontiguousarray(start_nodes, dtype=np.int32)
        draws = np.ascontiguousarray(draws, dtype=np.float64)
        assert draws.size == n * (1 + 2 * L), "draw buffer must hold n*(1+2L) uniforms"
        cut = None if cutoffs is None else np.ascontiguousarray(cutoffs, dtype=np.int64)
        nodes, ts, lens, eids = _alloc_walks(n, L)
        self._L.orc_walks(self.h, L, PICKERS[walk_bias], PICKERS[start_bias], int(forward),
                          _ptr(starts), _ptr(cut), n, _ptr(draws), int(pad), _ptr(nodes),
                          _ptr(ts), _ptr(lens), _ptr(eids), int(num_threads))
        return WalkResult(nodes.reshape(n, L), ts.reshape(n, L), lens,
                          eids.reshape(n, max(L - 1, 0)))


class RefGraph:
    """The reference's own node-index rebuild, per-node weights and CPU walk
    loop, fed with an OracleGraph's edge store."""

    def __init__(self, og: OracleGraph):
        self._R = ref_lib()
        self.og = og
        self.h = self._R.ref_create(int(og.is_directed), int(og.enable_weight),
                                    int(og.enable_tn2v), og.timescale_bound, og.p, og.q)
        a = {k: og.array(k) for k in [
            "sources", "targets", "timestamps", "timestamp_group_offsets",
            "unique_timestamps", "active_node_ids", "forward_cumulative_weights_exponential",
            "backward_cumulative_weights_exponential", "node_adj_offsets",
            "node_adj_neighbors"]}
        self._keep = a
        self._R.ref_set_edge_store(
            self.h, _ptr(a["sources"]), _ptr(a["targets"]), _ptr(a["timestamps"]),
            len(a["timestamps"]), _ptr(a["timestamp_group_offsets"]),
            _ptr(a["unique_timestamps"]), len(a["unique_timestamps"]),
            _ptr(a["active_node_ids"]), len(a["active_node_ids"]), og.max_node_id,
            _ptr(a["forward_cumulative_weights_exponential"]),
            _ptr(a["backward_cumulative_weights_exponential"]),
            len(a["forward_cumulative_weights_exponential"]), _ptr(a["node_adj_offsets"]),
            len(a["node_adj_offsets"]), _ptr(a["node_adj_neighbors"]),
            len(a["node_adj_neighbors"]))
        self._R.ref_rebuild(self.h)

    def __del__(self):
        if getattr(self, "h", None):
            self._R.ref_destroy(self.h)
            self.h = None

    def array(self, name):
        return _copy_array(self._R.ref_array, self.h, name)

    def walks(self, max_walk_len, walk_bias, start_bias, forward, start_nodes, draws,
              cutoffs=None, pad=-1):
        n = len(start_nodes)
        L = int(max_walk_len)
        starts = np.ascontiguousarray(start_nodes, dtype=np.int32)
        draws = np.ascontiguousarray(draws, dtype=np.float64)
        assert draws.size == n * (1 + 2 * L)
        cut = None if cutoffs is None else np.ascontiguousarray(cutoffs, dtype=np.int64)
        nodes, ts, lens, eids = _alloc_walks(n, L)
        self._R.ref_walks(self.h, L, PICKERS[walk_bias], PICKERS[start_bias], int(forward),
                          _ptr(starts), _ptr(cut), n, _ptr(draws), int(pad), _ptr(nodes),
                          _ptr(ts), _ptr(lens), _ptr(eids))
        return WalkResult(nodes.reshape(n, L), ts.reshape(n, L), lens,
                          eids.reshape(n, max(L - 1, 0)))
