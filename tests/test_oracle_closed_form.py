"""The oracle against what the mathematics fixes (closed forms, brute force, invariants) and
the known-answer tests the reference itself holds:

  * tests/test_des.py:10-217 (reference): the DES fixture — 6 rows, 2 eras, 4 bins — whose
    expected scores the reference computes in-test with a two-pass float64 NumPy loop;
    restated here as data (hess == 1, the only loss this path supports) with the same
    closed form, tolerance 1e-6 like the reference's test;
  * tests/test_des.py:220-226 (reference): era weights [0, 5.5, 7.5] for counts [0, 3, 5]
    and alpha 2.5, checked through the weighted era mean they produce;
  * tests/test_execution_modes.py:84-132 (reference): prefix/total/reverse-cumsum identities
    of the histogram;
  * brute force over every candidate of tiny problems in float64;
  * closed-form even K-cut positions (frontier_cpu.cpp:35-60).

Each check is chosen so that a dropped term, a wrong sign or index, or swapped operands
fails it: test_planted_mistakes_are_caught builds the restatement with such mistakes
planted (frontier_ref.c, ORACLE_MUTANT) and requires these checks to fail on each.
"""

from __future__ import annotations

import numpy as np
import pytest


def des_closed_form(counts, grads, lam, dro, dirw, weights, msl):
    """Two-pass float64 DES of one feature: counts/grads [E, nb] per-bin (not prefix)."""
    E, nb = counts.shape
    T = nb - 1
    gain = np.zeros((E, T))
    lv = np.zeros((E, T))
    rv = np.zeros((E, T))
    valid = np.zeros((E, T), bool)
    for e in range(E):
        for t in range(T):
            L, R = counts[e, : t + 1].sum(), counts[e, t + 1:].sum()
            if L <= 0 or R <= 0:
                continue
            valid[e, t] = True
            GL, GR = grads[e, : t + 1].sum(), grads[e, t + 1:].sum()
            G = grads[e].sum()
            gain[e, t] = 0.5 * GL**2 / (L + lam) + 0.5 * GR**2 / (R + lam) - 0.5 * G**2 / (L + R + lam)
            lv[e, t], rv[e, t] = -GL / (L + lam), -GR / (R + lam)
    score = np.full(T, -np.inf)
    left_total = np.cumsum(counts.sum(0))[:-1]
    for t in range(T):
        w = weights * valid[:, t]
        ws = w.sum()
        if ws <= 0:
            continue
        m = float(np.dot(gain[:, t], w) / ws)
        var = float(np.dot(w, (gain[:, t] - m) ** 2) / ws)
        d = float(np.dot(np.where(lv[:, t] > rv[:, t], 1.0, -1.0), w) / ws)
        s = m - dro * np.sqrt(max(var, 0.0)) + dirw * d
        ok = left_total[t] >= msl and counts.sum() - left_total[t] >= msl
        score[t] = s if ok else -np.inf
    return score, left_total


def per_bin(bins_col, grad, rows_per_era, nb):
    E = len(rows_per_era)
    c = np.zeros((E, nb), np.int64)
    g = np.zeros((E, nb), np.float64)
    for e, rows in enumerate(rows_per_era):
        np.add.at(c[e], bins_col[rows], 1)
        np.add.at(g[e], bins_col[rows], grad[rows].astype(np.float64))
    return c, g


@pytest.mark.parametrize("era_alpha", [0.0, 1.5])
def test_reference_des_fixture(oracle_mod, era_alpha):
    grad = np.array([0.5, -0.2, 0.1, -0.3, 0.4, -0.1], np.float32)
    bins = np.array([[0], [1], [1], [2], [2], [3]], np.uint8)
    eras = [np.array([0, 1]), np.array([2, 3, 4, 5])]
    lam, dro, dirw, nb, msl = 0.5, 0.1, 0.2, 4, 1
    res = oracle_mod.split_batch(bins, grad, [eras], np.array([0], np.int32), nb, lambda_l2=lam,
                                 lambda_dro=dro, direction_weight=dirw, era_alpha=era_alpha,
                                 min_samples_leaf=msl, want_cands=True)
    c, g = per_bin(bins[:, 0], grad, eras, nb)
    sizes = np.array([r.size for r in eras], np.float64)
    w = np.where(sizes > 0, sizes + era_alpha if era_alpha > 0 else 1.0, 0.0)
    want, left_total = des_closed_form(c, g, lam, dro, dirw, w, msl)
    got = res.cands[0][0, 0].astype(np.float64)
    ok = np.isfinite(want)
    np.testing.assert_array_equal(res.cands[3][0, 0].astype(bool), ok)
    np.testing.assert_allclose(got[ok], want[ok], rtol=1e-6, atol=1e-6)
    best = int(np.argmax(want))
    assert (res.feature[0], res.threshold[0]) == (0, best)
    assert res.left_count[0] == left_total[best]
    assert np.isclose(res.score[0], want[best], rtol=1e-6, atol=1e-6)


def test_era_alpha_weights_golden(oracle_mod):
    """Counts [0, 3, 5], alpha 2.5 -> weights [0, 5.5, 7.5] (reference test_des.py:220-226):
    with lambda_dro = dir = 0 the score is the weighted era mean of the gains."""
    rows = [np.zeros(0, np.int64), np.arange(0, 3), np.arange(3, 8)]
    bins = np.array([[0], [1], [1], [0], [0], [1], [1], [1]], np.uint8)
    grad = np.array([0.3, -0.5, 0.2, 0.7, -0.1, 0.4, -0.9, 0.25], np.float32)
    res = oracle_mod.split_batch(bins, grad, [rows], np.array([0], np.int32), 2, lambda_l2=0.25,
                                 era_alpha=2.5, min_samples_leaf=1, want_cands=True)
    c, g = per_bin(bins[:, 0], grad, rows, 2)
    want, _ = des_closed_form(c, g, 0.25, 0.0, 0.0, np.array([0.0, 5.5, 7.5]), 1)
    assert np.isclose(res.cands[0][0, 0, 0], want[0], rtol=1e-6, atol=1e-7)
    # the unweighted mean (alpha = 0) differs, so the weights are what the check sees
    unweighted, _ = des_closed_form(c, g, 0.25, 0.0, 0.0, np.array([0.0, 1.0, 1.0]), 1)
    assert not np.isclose(unweighted[0], want[0], rtol=1e-4)


def _tiny_problem(seed):
    rng = np.random.default_rng(seed)
    N, F, E, nb = 60, 3, 3, int(rng.integers(2, 6))
    bins = rng.integers(0, nb, size=(N, F)).astype(np.uint8)
    grad = rng.standard_normal(N).astype(np.float32)
    era = rng.integers(0, E, size=N)
    rows = [np.nonzero(era == e)[0] for e in range(E)]
    return bins, grad, rows, nb


@pytest.mark.parametrize("seed", range(12))
def test_brute_force_best_split(oracle_mod, seed):
    bins, grad, rows, nb = _tiny_problem(seed)
    lam, dro, dirw, alpha, msl = 0.3, 0.4, 0.1 * (seed % 2), 1.0 * (seed % 3 == 0), 4
    feats = np.arange(bins.shape[1], dtype=np.int32)
    res = oracle_mod.split_batch(bins, grad, [rows], feats, nb, lambda_l2=lam, lambda_dro=dro,
                                 direction_weight=dirw, era_alpha=alpha, min_samples_leaf=msl,
                                 want_cands=True)
    sizes = np.array([r.size for r in rows], np.float64)
    w = np.where(sizes > 0, sizes + alpha if alpha > 0 else 1.0, 0.0)
    allsc = []
    for k in range(bins.shape[1]):
        c, g = per_bin(bins[:, k], grad, rows, nb)
        sc, _ = des_closed_form(c, g, lam, dro, dirw, w, msl)
        ok = np.isfinite(sc)
        np.testing.assert_array_equal(res.cands[3][0, k].astype(bool), ok)
        np.testing.assert_allclose(res.cands[0][0, k][ok], sc[ok], rtol=1e-5, atol=1e-6)
        allsc.append(sc)
    allsc = np.array(allsc)
    if not np.isfinite(allsc).any():
        assert res.feature[0] < 0
        return
    best = allsc.max()
    f, t = int(res.feature[0]), int(res.threshold[0])
    assert abs(allsc[f, t] - best) <= 1e-5 * max(1.0, abs(best))


@pytest.mark.parametrize("seed", range(5))
def test_histogram_invariants(oracle_mod, seed):
    rng = np.random.default_rng(100 + seed)
    N, F, E, nb, U = 400, 3, 4, 16, 2
    bins = rng.integers(0, nb, size=(N, F)).astype(np.uint8)
    grad = rng.standard_normal(N).astype(np.float32)
    node = rng.integers(0, U, size=N)
    era = rng.integers(0, E, size=N)
    ner = [[np.nonzero((node == u) & (era == e))[0] for e in range(E)] for u in range(U)]
    res = oracle_mod.split_batch(bins, grad, ner, np.arange(F, dtype=np.int32), nb,
                                 min_samples_leaf=1, want_planes=True)
    cnt, gp = res.planes  # prefix planes [E, U, K, nb]; index nb-1 = total
    for e in range(E):
        for u in range(U):
            rows = ner[u][e]
            for k in range(F):
                c, g = np.bincount(bins[rows, k], minlength=nb), np.zeros(nb)
                np.add.at(g, bins[rows, k], grad[rows].astype(np.float64))
                np.testing.assert_array_equal(cnt[e, u, k, :-1], np.cumsum(c)[:-1])
                assert cnt[e, u, k, -1] == rows.size
                mass = max(1.0, float(np.abs(grad[rows]).sum()))
                assert np.all(np.abs(gp[e, u, k, :-1] - np.cumsum(g)[:-1]) <= 1e-5 * mass)
                # right = total - left equals the reverse cumulative sum (reference
                # test_execution_modes.py:109-132)
                right = cnt[e, u, k, -1] - cnt[e, u, k, :-1]
                np.testing.assert_array_equal(right, np.cumsum(c[::-1])[::-1][1:])


@pytest.mark.parametrize("nb,k", [(32, 5), (48, 6), (64, 2), (10, 9), (200, 7), (6, 1)])
def test_even_cuts_closed_form(oracle_mod, nb, k):
    T = nb - 1
    got = oracle_mod.even_cuts(nb, k)
    if k == 1:
        want = [0]
    else:
        want = sorted({min(max(int(np.floor(i * (T - 1) / (k - 1) + 0.5)), 0), T - 1)
                       for i in range(k)})
        want += [want[-1]] * (k - len(want))
    np.testing.assert_array_equal(got, want)
    assert got[0] == 0 and (k == 1 or got[-1] == T - 1)


# checks that must fail on a build of the restatement with the given planted mistake
# (frontier_ref.c, ORACLE_MUTANT): parent term dropped, alpha ignored, Welford M2 with the
# old mean, direction sign flipped, threshold index off by one
MUTANT_CHECKS = {
    1: [("test_reference_des_fixture", 0.0)],
    2: [("test_era_alpha_weights_golden", None)],
    3: [("test_reference_des_fixture", 0.0)],
    4: [("test_reference_des_fixture", 0.0)],
    5: [("test_reference_des_fixture", 0.0), ("test_brute_force_best_split", 1)],
}


@pytest.mark.parametrize("mutant", sorted(MUTANT_CHECKS))
def test_planted_mistakes_are_caught(oracle_mod, tmp_path, mutant):
    """Each planted mistake makes at least one of the checks above fail, so a passing run
    of those checks rules it out for the real restatement."""
    path = oracle_mod.build_mutant(mutant, tmp_path)
    passed = []
    with oracle_mod.use_library(path):
        for name, arg in MUTANT_CHECKS[mutant]:
            fn = globals()[name]
            try:
                fn(oracle_mod) if arg is None else fn(oracle_mod, arg)
            except AssertionError:
                continue
            passed.append(name)
    assert not passed, f"mutant {mutant} passed {passed}"


@pytest.mark.parametrize("seed", range(4))
def test_score_planes_agrees_with_split_batch(oracle_mod, seed):
    """The plane-fed scorer (used to feed the GPU scorer the oracle's histograms) gives the
    split finder's candidates bit-for-bit on the split finder's own planes."""
    rng = np.random.default_rng(300 + seed)
    N, F, E, nb, U = 600, 4, 5, int(rng.integers(3, 20)), 3
    bins = rng.integers(0, nb, size=(N, F)).astype(np.uint8)
    grad = rng.standard_normal(N).astype(np.float32)
    node = rng.integers(0, U, size=N)
    era = rng.integers(0, E, size=N)
    ner = [[np.nonzero((node == u) & (era == e))[0] for e in range(E)] for u in range(U)]
    feats = rng.permutation(F).astype(np.int32)
    kw = dict(lambda_l2=0.2, lambda_dro=0.3, direction_weight=0.1 * (seed % 2),
              era_alpha=1.0 * (seed % 3 == 1), min_samples_leaf=5)
    ref = oracle_mod.split_batch(bins, grad, ner, feats, nb, want_planes=True, want_cands=True, **kw)
    sp = oracle_mod.score_planes(ref.planes[0], ref.planes[1], feats, None, **kw)
    v = ref.cands[3].astype(bool)
    np.testing.assert_array_equal(sp["valid"].astype(bool), v)
    np.testing.assert_array_equal(sp["score"][v].view(np.uint32), ref.cands[0][v].view(np.uint32))
    np.testing.assert_array_equal(sp["left_total"][v], ref.cands[1][v])
    for u in range(U):
        if ref.feature[u] >= 0:
            assert (sp["best_feature"][u], sp["best_threshold"][u]) == (ref.feature[u], ref.threshold[u])
