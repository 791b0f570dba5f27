"""bench.py's random-gather probe (temporal-random-walk_amd/probe, a
measurement aid outside the engine): it counts its gathers and checks its
arguments."""
import pytest

pytestmark = pytest.mark.gpu


def test_gather_probe_counts_its_gathers_and_checks_arguments():
    """lanes * rounds gathers per launch, a positive rate in both modes, and
    its argument checks."""
    import probe
    for chained in (False, True):
        r = probe.gather(1 << 20, lanes=512, rounds=16, chained=chained, reps=2)
        assert r["gathers"] == 512 * 16
        assert r["ms"] > 0 and r["gathers_per_s"] > 0
    for bad in (dict(table_bytes=3 << 20), dict(table_bytes=1024), dict(lanes=100),
                dict(rounds=0), dict(reps=0), dict(lanes=1 << 20, rounds=1 << 17)):
        kw = dict(table_bytes=1 << 20, lanes=256, rounds=4, reps=1)
        kw.update(bad)
        with pytest.raises(ValueError):
            probe.gather(**kw)
