"""The walk-law tests of test_gpu_scale_statistics.py (tests/laws.py) on the
CPU, between oracle samples: two samples of one process under independent
uniforms pass, and a planted mistake -- the oracle's hops drawn with another
index picker -- is rejected, so the tests have power against a wrong picker
law.  A cfg2-shaped power-law graph of 2M edges."""
import os

import numpy as np
import pytest

from oracle import pyoracle as po
from tests import graphs
from tests.laws import law_tests

THREADS = max(1, min(8, os.cpu_count() or 1))


@pytest.fixture(scope="module")
def oracle_graph():
    s, d, t = graphs.powerlaw(100_000, 2_000_000, s=1.8, n_ts=20_000, seed=71)
    og = po.OracleGraph(True)
    og.add_edges(s, d, t, num_threads=THREADS)
    return og


def _walks(og, picker, seed, n=150_000, L=40):
    return og.walks(L, picker, "Uniform", True, -np.ones(n, np.int32), graphs.draws(n, L, seed),
                    num_threads=THREADS)


def test_one_process_passes(oracle_graph):
    law_tests(_walks(oracle_graph, "ExponentialIndex", 1),
              _walks(oracle_graph, "ExponentialIndex", 2), "same law")


@pytest.mark.parametrize("planted", ["Linear", "Uniform"])
def test_a_wrong_picker_law_is_rejected(oracle_graph, planted):
    with pytest.raises(AssertionError):
        law_tests(_walks(oracle_graph, "ExponentialIndex", 1),
                  _walks(oracle_graph, planted, 3), f"planted {planted}")
