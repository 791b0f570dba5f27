"""The standalone pickers (trw_pick_index / trw_pick_weights, the classes of
proxies/RandomPicker.cu:11-313) on the GPU.

Bit-exact against the oracle's picker functions for provided numbers; the
reference's own picker tests (test/test_random_picker.cpp,
test/test_weight_based_random_picker.cpp) restated through the drop-in
classes; and a chi-square check of the in-kernel draws (pick_random)."""
import numpy as np
import pytest

from oracle import pyoracle as po

pytestmark = pytest.mark.gpu


def _oracle():
    return po.lib()


def test_index_pickers_bit_exact_against_oracle():
    from temporal_random_walk import capi

    L = _oracle()
    rng = np.random.default_rng(5)
    n = 200_000
    starts = rng.integers(-50, 1_000, n).astype(np.int32)
    lens = np.concatenate([rng.integers(0, 40, n // 2), rng.integers(600, 2_000, n - n // 2)])
    rng.shuffle(lens)
    ends = (starts + lens).astype(np.int32)
    draws = rng.random(n)
    draws[:1000] = np.linspace(0.0, 1.0, 1000, endpoint=False)  # a grid including 0
    for picker, ref in (("Uniform", lambda s, e, p, r: L.orc_pick_uniform(s, e, r)),
                        ("Linear", L.orc_pick_linear),
                        ("ExponentialIndex", L.orc_pick_exponential_index)):
        for pe in (True, False):
            got = capi.pick_index(picker, starts, ends, prioritize_end=pe, draws=draws)
            want = np.array([ref(int(s), int(e), int(pe), float(r))
                             for s, e, r in zip(starts[:20_000], ends[:20_000], draws[:20_000])],
                            dtype=np.int32)
            np.testing.assert_array_equal(got[:20_000], want, err_msg=f"{picker} pe={pe}")
            valid = ends > starts
            assert np.all((got[valid] >= starts[valid]) & (got[valid] < ends[valid]))
            assert np.all(got[~valid] == -1)
    # the test pickers
    np.testing.assert_array_equal(capi.pick_index("TEST_FIRST", starts[:10], ends[:10] + 1,
                                                  draws=draws[:10]), starts[:10])
    np.testing.assert_array_equal(capi.pick_index("TEST_LAST", starts[:10], ends[:10] + 1,
                                                  draws=draws[:10]), ends[:10])


def test_exponential_index_draws_at_thresholds_match_oracle():
    """The device evaluates the exponential index picker from threshold tables
    and falls back to the logarithm only near a threshold (expm1(i) /
    expm1(len) below 710 groups, exp(-j) above).  Draws 1e-11 to 1e-5 away
    from every threshold give the oracle's index bit-exactly.  Draws within
    four ulps of one are decided by how log1p / log round a value that close
    to an integer, where the device's libm and the C library's can differ by
    an ulp (as the reference's CPU and GPU paths do): there the index may
    differ by one, and only rarely."""
    from temporal_random_walk import capi

    L = _oracle()
    far, near = [], []
    for n in (1, 2, 3, 7, 50, 300, 708, 709):
        i = np.arange(1, n + 1)
        r0 = np.expm1(i.astype(np.float64)) / np.expm1(float(n))
        for k in (-4, -1, 0, 1, 4):
            near.append((r0 * (1.0 + k * 2.0 ** -52), np.full(i.size, n)))
        for rel in (-1e-9, -1e-11, 1e-11, 1e-9):
            far.append((r0 * (1.0 + rel), np.full(i.size, n)))
    j = np.arange(0, 38, dtype=np.float64)
    for n in (710, 5_000, 1 << 20, (1 << 31) - 1):
        for rel in (-1e-5, -1e-9, 1e-9, 1e-5):
            far.append((np.exp(-j) * (1.0 + rel), np.full(j.size, n)))
        for rel in (-2.0 ** -50, 0.0, 2.0 ** -50):
            near.append((np.exp(-j) * (1.0 + rel), np.full(j.size, n)))

    def run(cases):
        r = np.concatenate([c[0] for c in cases])
        ends = np.concatenate([c[1] for c in cases]).astype(np.int32)
        keep = (r >= 0.0) & (r < 1.0)
        r, ends = r[keep], ends[keep]
        starts = np.zeros(r.size, np.int32)
        out = []
        for pe in (True, False):
            got = capi.pick_index("ExponentialIndex", starts, ends, prioritize_end=pe, draws=r)
            want = np.array([L.orc_pick_exponential_index(0, int(e), int(pe), float(x))
                             for e, x in zip(ends, r)], dtype=np.int32)
            out.append((got, want, ends, r))
        return out

    for got, want, ends, r in run(far):
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, [(int(ends[b]), float(r[b]), int(got[b]), int(want[b]))
                               for b in bad[:10]]
    for got, want, ends, r in run(near):
        assert np.all(np.abs(got.astype(np.int64) - want) <= 1)
        assert np.count_nonzero(got != want) <= got.size // 100


def test_weight_picker_bit_exact_against_oracle():
    from temporal_random_walk import capi

    L = _oracle()
    rng = np.random.default_rng(6)
    w = np.cumsum(rng.random(5_000) ** 3)
    w /= w[-1]
    n = 50_000
    gs = rng.integers(0, 5_100, n).astype(np.uint64)
    ge = (gs + rng.integers(-3, 400, n).astype(np.int64).clip(0).astype(np.uint64))
    draws = rng.random(n)
    got = capi.pick_weights(w, gs, ge, draws=draws)
    wp = w.ctypes.data
    want = np.array([L.orc_pick_exponential_weights(wp, w.size, int(a), int(b), float(r), 0)
                     for a, b, r in zip(gs[:10_000], ge[:10_000], draws[:10_000])], dtype=np.int32)
    np.testing.assert_array_equal(got[:10_000], want)


def _avg(picker, pe, rng):
    r = rng.random(100_000)
    return picker.pick_random_batch([0] * r.size, [10_000] * r.size, pe, r).mean()


def test_reference_random_picker_cases():
    """test/test_random_picker.cpp:48-199 through the drop-in classes."""
    import temporal_random_walk as trw

    lin = trw.LinearRandomPicker(use_gpu=True)
    exp = trw.ExponentialIndexRandomPicker(use_gpu=True)
    rng = np.random.default_rng(7)
    lin_end, lin_start = _avg(lin, True, rng), _avg(lin, False, rng)
    exp_end, exp_start = _avg(exp, True, rng), _avg(exp, False, rng)
    assert lin_end > lin_start and exp_end > exp_start      # PrioritizeEndGivesHigherAverage
    assert exp_end > lin_end                                # ExponentialMoreExtremeForEnd
    assert exp_start < lin_start                            # ExponentialMoreExtremeForStart
    for p in (lin, exp):                                    # BoundsTest
        for pe in (True, False):
            got = p.pick_random_batch([5] * 1000, [10] * 1000, pe, rng.random(1000))
            assert got.min() >= 5 and got.max() < 10
    for pe in (True, False):                                # SingleElementRangeTest
        assert lin.pick_random(5, 6, pe) == 5 and exp.pick_random(5, 6, pe) == 5
    n = 100_000                                             # TwoElementRange* tests
    e = np.e
    for p, want_end, want_start in ((lin, 2 / 3, 1 / 3),
                                    (exp, (e - 1) * e / (e * e - 1), (e - 1) / (e * e - 1))):
        ones_end = (p.pick_random_batch([0] * n, [2] * n, True, rng.random(n)) == 1).mean()
        ones_start = (p.pick_random_batch([0] * n, [2] * n, False, rng.random(n)) == 1).mean()
        assert abs(ones_end - want_end) < 0.02 and abs(ones_start - want_start) < 0.02
    assert trw.UniformRandomPicker().pick_random(3, 3) == -1


def test_reference_weight_picker_cases():
    """test/test_weight_based_random_picker.cpp:57-128 through the drop-in class."""
    import temporal_random_walk as trw

    p = trw.WeightBasedRandomPicker(use_gpu=True)
    w = [0.2, 0.5, 0.7, 1.0]
    assert p.pick_random(w, -1, 2) == -1                    # ValidationChecks
    assert p.pick_random(w, 2, 2) == -1
    assert p.pick_random(w, 2, 1) == -1
    assert p.pick_random(w, 0, 5) == -1
    rng = np.random.default_rng(8)
    for a, b in ((0, 4), (1, 3), (0, 2), (2, 4)):           # Full/SubrangeSampling
        got = p.pick_random_batch(w, [a] * 1000, [b] * 1000, rng.random(1000))
        assert got.min() >= a and got.max() < b
        assert set(got.tolist()) == set(range(a, b))
    got = p.pick_random_batch(w, [1] * 100, [2] * 100, rng.random(100))   # SingleElementRange
    assert np.all(got == 1)
    got = p.pick_random_batch([0.25, 0.5, 0.75, 1.0], [0] * 100_000, [4] * 100_000,
                              rng.random(100_000))                       # WeightDistributionTest
    assert np.all(np.abs(np.bincount(got, minlength=4) / 100_000 - 0.25) < 0.01)
    assert p.pick_random([0.1, 0.100001, 0.100002, 0.100003], 0, 4) != -1  # EdgeCaseWeights
    assert p.pick_random([0.1, 0.5, 0.9, 1000.0], 0, 4) != -1


def test_in_kernel_draws_follow_the_picker_distributions():
    """pick_random (no provided numbers): two independent calls of the batch
    path differ, and the picks follow the closed-form distributions
    (chi-square p > 0.01)."""
    from scipy.stats import chisquare
    from temporal_random_walk import capi

    n, m = 400_000, 8
    s, e = np.zeros(n, np.int32), np.full(n, m, np.int32)
    a = capi.pick_index("Linear", s, e, prioritize_end=True, seed=11)
    b = capi.pick_index("Linear", s, e, prioritize_end=True, seed=12)
    assert not np.array_equal(a, b)
    np.testing.assert_array_equal(a, capi.pick_index("Linear", s, e, True, seed=11))
    want = np.arange(1, m + 1) / (m * (m + 1) / 2)            # Linear, prioritize_end
    assert chisquare(np.bincount(a, minlength=m), want * n).pvalue > 0.01
    u = capi.pick_index("Uniform", s, e, seed=13)
    assert chisquare(np.bincount(u, minlength=m), np.full(m, n / m)).pvalue > 0.01
    x = capi.pick_index("ExponentialIndex", s, e, prioritize_end=True, seed=14)
    # P(index >= j) from the inverse CDF k = log1p(r * expm1(m)) - 1, index = clamp(int(k + 1))
    cdf = np.concatenate([[0.0], np.expm1(np.arange(1, m)) / np.expm1(m), [1.0]])
    assert chisquare(np.bincount(x, minlength=m), np.diff(cdf) * n).pvalue > 0.01
    wts = np.cumsum(np.arange(1.0, 6.0))
    wp = capi.pick_weights(wts, np.zeros(n, np.uint64), np.full(n, 5, np.uint64), seed=15)
    assert chisquare(np.bincount(wp, minlength=5), np.arange(1.0, 6.0) / 15 * n).pvalue > 0.01


def test_provided_numbers_outside_unit_interval_are_rejected():
    import temporal_random_walk as trw

    p = trw.LinearRandomPicker()
    with pytest.raises(ValueError, match=r"\[0, 1\)"):
        p.pick_random_batch([0], [5], True, [1.0])
    with pytest.raises(ValueError, match="one value per pick"):
        p.pick_random_batch([0, 0], [5, 5], True, [0.5])
