"""bench.py's random-gather probe (libtrw_probe.so, built from probe.hip beside
this file by build.py): a measurement aid, not part of the engine."""
from __future__ import annotations

import ctypes as C
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtrw_probe.so")
_L = None


def _lib():
    global _L
    if _L is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run temporal-random-walk_amd/build.py")
        L = C.CDLL(LIB_PATH)
        L.trwp_gather.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.c_int32, C.c_int32,
                                  C.POINTER(C.c_double)]
        L.trwp_gather.restype = C.c_int
        L.trwp_last_error.restype = C.c_char_p
        _L = L
    return _L


def gather(table_bytes, lanes=256 * 2048, rounds=256, chained=False, reps=3):
    """Random 8-byte gathers from a table of table_bytes (a power of two) on
    the current device: lanes * rounds per launch, independent or chained
    (each address follows from the previous load's value).  Returns {"ms",
    "gathers_per_s", "gathers"} of one launch (mean over reps after a
    warm-up).  The rate bounds the walk kernels' L1 -> L2 read rate."""
    out = (C.c_double * 3)()
    rc = _lib().trwp_gather(int(table_bytes), int(lanes), int(rounds), 1 if chained else 0,
                            int(reps), out)
    if rc == 1:
        raise ValueError(_lib().trwp_last_error().decode())
    if rc == 3:
        raise MemoryError(_lib().trwp_last_error().decode())
    if rc != 0:
        raise RuntimeError(_lib().trwp_last_error().decode())
    return {"ms": out[0], "gathers_per_s": out[1], "gathers": int(out[2])}
