"""MI355X temporal random walk engine -- drop-in for ``temporal_random_walk``.

``from temporal_random_walk import TemporalRandomWalk`` (and the standalone
``*RandomPicker`` classes) gives the same classes, methods, keyword arguments
and return shapes as the reference's pybind11 module.  Every call runs on the
GPU through the HIP engine (``libtrw_engine.so``); importing fails loudly if it
has not been built.
"""
import os as _os

_here = _os.path.dirname(_os.path.abspath(__file__))
if not _os.path.exists(_os.path.join(_here, "libtrw_engine.so")):
    raise ImportError(
        "temporal_random_walk: libtrw_engine.so is not built; run "
        "`python temporal-random-walk_amd/build.py` (there is no CPU fallback)")

from ._temporal_random_walk import (  # noqa: E402
    ExponentialIndexRandomPicker,
    LinearRandomPicker,
    TemporalRandomWalk,
    UniformRandomPicker,
    WeightBasedRandomPicker,
)

__all__ = [
    "TemporalRandomWalk",
    "LinearRandomPicker",
    "ExponentialIndexRandomPicker",
    "UniformRandomPicker",
    "WeightBasedRandomPicker",
]
