"""Two-sample tests of walk laws (test helpers): the next-node law at the
busiest nodes and the walk-length law of two walk samples."""
import numpy as np

N_NODES_TESTED = 20
ALPHA = 0.01


def _chi2_two_sample(a, b, min_expected=5.0):
    """Two-sample chi-square on category samples a and b (sizes may differ):
    categories whose expected count in either sample is below min_expected
    are pooled into one bin.  Returns the p-value."""
    from scipy.stats import chi2_contingency
    cats, inv = np.unique(np.concatenate([a, b]), return_inverse=True)
    ca = np.bincount(inv[:a.size], minlength=cats.size)
    cb = np.bincount(inv[a.size:], minlength=cats.size)
    tot = ca + cb
    small = np.minimum(tot * a.size, tot * b.size) / (a.size + b.size) < min_expected
    table = np.stack([ca[~small], cb[~small]])
    if small.any():
        table = np.concatenate([table, [[ca[small].sum()], [cb[small].sum()]]], axis=1)
    if table.shape[1] < 2:
        return 1.0
    return chi2_contingency(table)[1]


def _transitions(nodes, lens):
    """Every (node, next node) pair of every walk, within its length."""
    L = nodes.shape[1]
    lens = lens.astype(np.int64)
    valid = np.arange(L - 1)[None, :] < (lens[:, None] - 1)
    return nodes[:, :-1][valid], nodes[:, 1:][valid]


def law_tests(ref, got, label):
    """Two-sample chi-square of the next-node law at each of the N_NODES_TESTED
    nodes that take the most hops in ref, and of the walk-length law, at a
    family-wise level of ALPHA (Bonferroni).  Raises AssertionError on a
    rejection; returns the smallest transition p-value and the share of
    ref's hops the tested nodes take."""
    ru, rv = _transitions(ref.nodes, ref.lens)
    gu, gv = _transitions(got.nodes, got.lens)
    ids, cnt = np.unique(ru, return_counts=True)
    busiest = ids[np.argsort(cnt)[::-1][:N_NODES_TESTED]]
    level = ALPHA / (N_NODES_TESTED + 1)
    order_r, order_g = np.argsort(ru, kind="stable"), np.argsort(gu, kind="stable")
    sr, sg = ru[order_r], gu[order_g]
    pvals = []
    for u in busiest:
        a = rv[order_r[np.searchsorted(sr, u):np.searchsorted(sr, u, side="right")]]
        b = gv[order_g[np.searchsorted(sg, u):np.searchsorted(sg, u, side="right")]]
        assert a.size > 1_000 and b.size > 1_000, (label, int(u), a.size, b.size)
        p = _chi2_two_sample(a, b)
        pvals.append(p)
        assert p > level, f"{label}: next-node law at node {int(u)}: p = {p:.3g} ({a.size} hops)"
    p = _chi2_two_sample(ref.lens.astype(np.int64), got.lens.astype(np.int64))
    assert p > level, f"{label}: walk-length law: p = {p:.3g}"
    # the hops the tests cover
    covered = np.isin(ru, busiest).mean()
    return min(pvals), covered
