"""The reference's host-schema split finder, find_best_splits_batched_cpu
(frontier_cpu.cpp:111-515, called from booster.py:1080-1093), served on the HIP device by
packboost_amd.backends.find_best_splits_batched, against the oracle's restatement
(oracle.split_batch).

Per node: the same (feature, threshold) unless the two picks' scores tie within 1e-6 of each
other; for the same pick, left/right counts and the per-era left/right row lists (in list
order) bit-exact, left/right grad sums within 1e-5 of the node's |grad| mass (the device sums
are exact and rounded once, the reference's add float32 in row order), the score within 1e-5.
Nodes without rows or without a valid split give None; the stats carry the reference's keys
and counts. Bad inputs raise the reference's exception types.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import make_problem, node_era_rows

pytestmark = pytest.mark.gpu

STAT_KEYS = {"nodes_processed", "nodes_skipped", "rows_total", "feature_blocks", "bincount_calls", "hist_ms",
             "scan_ms", "score_ms", "partition_ms", "nodes_subtract_ok", "nodes_subtract_fallback",
             "nodes_rebuild", "block_size"}


@pytest.mark.parametrize("case", [
    # seed, N, F, E, nb, U, K, k_cuts, cut_selection, msl, alpha, dir, dro
    (1, 6000, 14, 6, 5, 6, 10, 0, "mass", 10, 0.0, 0.0, 0.4),
    (2, 8000, 20, 9, 32, 5, 12, 4, "mass", 5, 1.5, 0.1, 0.4),
    (3, 7000, 12, 5, 128, 4, 9, 6, "even", 20, 0.0, 0.0, 0.0),
    (4, 5000, 8, 4, 255, 3, 8, 0, "mass", 3, 0.7, 0.2, 0.5),
    (5, 3000, 6, 3, 16, 40, 6, 0, "mass", 40, 0.0, 0.0, 0.3),
    # bins >= max_bins (skipped in the histogram, sent right: frontier_cpu.cpp:278-281, 464-470)
    (6, 6000, 14, 6, 5, 6, 10, 0, "mass", 10, 0.0, 0.0, 0.4, True),
    (7, 8000, 20, 9, 32, 5, 12, 4, "mass", 5, 1.5, 0.1, 0.4, True),
    (8, 5000, 8, 4, 64, 3, 8, 0, "mass", 3, 0.7, 0.2, 0.5, True),
    (9, 7000, 12, 5, 128, 4, 9, 6, "even", 20, 0.0, 0.0, 0.0, True),
    (10, 150000, 5, 2, 16, 2, 5, 4, "mass", 20, 0.5, 0.0, 0.3, True),  # eras above 65535 rows
], ids=["nb5", "nb32_kcuts_alpha_dir", "nb128_even_cuts", "nb255_alpha_dir", "40_nodes_msl40",
        "skipped_nb5", "skipped_nb32_kcuts_alpha_dir", "skipped_nb64_alpha_dir", "skipped_nb128_even_cuts",
        "skipped_32bit_counts_kcuts_alpha"])
def test_host_schema_split_finder(hip, oracle_mod, case):
    from packboost_amd import backends
    from tests.helpers import with_skipped_bins

    seed, N, F, E, nb, U, K, kc, cut, msl, alpha, dirw, dro = case[:13]
    skipped = len(case) > 13 and case[13]
    print(f"[batched host] {case}", flush=True)
    assert backends.cpu_available()
    p = make_problem(seed, N, F, E, nb, U, empty_era=True)
    if skipped:
        p = with_skipped_bins(p, seed)
    ner = node_era_rows(p)
    ner.insert(1, [np.empty(0, np.int64) for _ in range(E)])  # a node without rows
    ner.append([])  # a node without eras
    M = len(ner)
    rng = np.random.default_rng(seed + 100)
    feats = rng.permutation(F)[:K].astype(np.int32)
    kw = dict(lambda_l2=1e-3, lambda_dro=dro, direction_weight=dirw, era_alpha=alpha, min_samples_leaf=msl)
    got, stats = backends.find_best_splits_batched(p["bins"].view(np.int8), p["grad"], ner, feats, nb, kc, cut,
                                                   kw["lambda_l2"], dro, dirw, alpha, msl)
    ref = oracle_mod.split_batch(p["bins"], p["grad"], ner[:-1], feats, nb, kc, cut, want_cands=True,
                                 want_planes=True, **kw)

    def thresholds_of(k: int) -> np.ndarray:
        """The candidate thresholds of feature slot k (frontier_cpu.cpp:322-338): every one, or
        the even / mass K-cuts (mass over this call's nodes, from the oracle's planes)."""
        if not (0 < kc < nb - 1):
            return np.arange(nb - 1)
        if cut == "even":
            return oracle_mod.even_cuts(nb, kc)
        pref = ref.planes[0][:, :, k, :].astype(np.int64)  # [E, M, nb] prefix counts
        mass = np.diff(pref, axis=2, prepend=0).sum(axis=(0, 1))
        return oracle_mod.mass_cuts(mass, nb, kc)

    assert isinstance(got, list) and len(got) == M and set(stats) == STAT_KEYS
    assert got[1] is None and got[-1] is None
    assert stats["nodes_processed"] == U and stats["nodes_skipped"] == 2
    assert stats["rows_total"] == sum(sum(a.size for a in eras) for eras in ner)
    assert stats["block_size"] == K and stats["feature_blocks"] == 1
    off = 0
    for m in range(M - 1):
        eras = ner[m]
        sizes = [a.size for a in eras]
        go_left = ref.go_left[off: off + sum(sizes)]
        off += sum(sizes)
        d = got[m]
        if ref.feature[m] < 0:
            assert d is None, m
            continue
        assert d is not None, m
        mass = float(np.abs(p["grad"][np.concatenate(eras)]).sum())
        if (d["feature"], d["threshold"]) != (int(ref.feature[m]), int(ref.threshold[m])):
            # a near-tie: the oracle's own score of the device's pick, not the device's score
            k = int(np.nonzero(feats == d["feature"])[0][0])
            t = int(np.nonzero(thresholds_of(k) == d["threshold"])[0][0])
            alt, best = float(ref.cands[0][m, k, t]), float(ref.score[m])
            assert ref.cands[3][m, k, t] and abs(alt - best) <= 1e-6 * max(1.0, abs(best)), m
            print(f"[batched host] near-tie at node {m}: {alt!r} vs {best!r}", flush=True)
            continue
        assert d["left_count"] == int(ref.left_count[m]) and d["right_count"] == int(ref.right_count[m]), m
        assert d["left_hess"] == float(ref.left_hess[m]) and d["right_hess"] == float(ref.right_hess[m]), m
        bar = 1e-5 * mass + 1e-6
        assert abs(d["left_grad"] - float(ref.left_grad[m])) <= bar, m
        assert abs(d["right_grad"] - float(ref.right_grad[m])) <= bar, m
        assert abs(d["score"] - float(ref.score[m])) <= 1e-5 * max(1.0, abs(float(ref.score[m]))), m
        assert len(d["left_rows"]) == E and len(d["right_rows"]) == E
        pos = 0
        for e, r in enumerate(eras):
            gl = go_left[pos: pos + r.size].astype(bool)
            pos += r.size
            np.testing.assert_array_equal(d["left_rows"][e], r[gl])
            np.testing.assert_array_equal(d["right_rows"][e], r[~gl])
            assert d["left_rows"][e].dtype == np.int64


def test_host_schema_bins_past_254_bins(hip):
    """With max_bins 255 a bin of 255 has no spare plane bin to go to: ValueError."""
    from packboost_amd import backends

    bins = np.zeros((10, 2), np.uint8)
    bins[3, 1] = 255
    ner = [[np.arange(10, dtype=np.int64)]]
    with pytest.raises(ValueError, match="max_bins <= 254"):
        backends.find_best_splits_batched(bins.view(np.int8), np.ones(10, np.float32), ner,
                                          np.arange(2, dtype=np.int32), 255, 0, "mass", 1e-6, 0.0, 0.0, 0.0, 1)


def test_host_schema_no_nodes_and_no_features(hip):
    from packboost_amd import backends

    bins = np.zeros((10, 3), np.int8)
    grad = np.zeros(10, np.float32)
    dec, stats = backends.find_best_splits_batched(bins, grad, [], np.arange(3, dtype=np.int32), 5, 0, "mass",
                                                   1e-6, 0.0, 0.0, 0.0, 1)
    assert dec == [] and stats["nodes_processed"] == 0
    ner = [[np.arange(5, dtype=np.int64), np.arange(5, 10, dtype=np.int64)]]
    dec, stats = backends.find_best_splits_batched(bins, grad, ner, np.zeros(0, np.int32), 5, 0, "mass",
                                                   1e-6, 0.0, 0.0, 0.0, 1)
    assert dec == [None] and stats["nodes_processed"] == 1 and stats["rows_total"] == 10


def test_host_schema_rejects_bad_inputs(hip):
    from packboost_amd import backends

    bins = np.zeros((10, 3), np.int8)
    grad = np.zeros(10, np.float32)
    ok = [[np.arange(10, dtype=np.int64)]]
    f = np.arange(3, dtype=np.int32)
    args = (5, 0, "mass", 1e-6, 0.0, 0.0, 0.0, 1)
    with pytest.raises(ValueError, match="2D"):
        backends.find_best_splits_batched(bins[:, 0], grad, ok, f, *args)
    with pytest.raises(ValueError, match="grad length"):
        backends.find_best_splits_batched(bins, grad[:5], ok, f, *args)
    with pytest.raises(IndexError, match="row index"):
        backends.find_best_splits_batched(bins, grad, [[np.array([3, 10])]], f, *args)
    with pytest.raises(IndexError, match="feature index"):
        backends.find_best_splits_batched(bins, grad, ok, np.array([0, 3], np.int32), *args)
    with pytest.raises(ValueError, match="list"):
        backends.find_best_splits_batched(bins, grad, [np.arange(10)], f, *args)


def _sequential_pick(score, lt, feat, thr, valid):
    """frontier_cpu.cpp:415-426 over one node's candidates in visiting order (float32 scores)."""
    best_s, best_l, best_f, best_t, best_i = np.float32(-np.inf), -1, -1, -1, -1
    for i in range(score.size):
        if not valid[i]:
            continue
        s = np.float32(score[i])
        better = bool(s > best_s)
        if not better and abs(np.float32(s - best_s)) <= np.float32(1e-12):
            better = lt[i] > best_l or (lt[i] == best_l and (feat[i] > best_f or (feat[i] == best_f and thr[i] > best_t)))
        if better:
            best_s, best_l, best_f, best_t, best_i = s, lt[i], feat[i], thr[i], i
    return best_i


@pytest.mark.parametrize("spread", [0.0, 3e-13, 2e-12, 1e-9])
def test_pick_sequential_tie_window(hip, spread):
    """pb_pick_sequential against the reference's scan on candidates whose scores lie within a
    few 1e-12 windows of each other (the non-transitive tie rule makes the order matter)."""
    import torch

    from packboost_amd.backends import _hip

    lib = _hip.load()
    rng = np.random.default_rng(int(spread * 1e13) + 7)
    M, K, T = 37, 9, 5
    n = K * T
    rec = np.zeros(M * n, dtype=_hip.CANDIDATE_DTYPE)
    base = rng.choice([1e-7, 3e-6, 0.25], size=M)
    rec["score"] = (np.repeat(base, n) + rng.integers(0, 6, M * n) * spread).astype(np.float32)
    rec["left_total"] = rng.integers(10, 14, M * n)
    feats = rng.permutation(50)[:K]
    rec["feature"] = np.tile(np.repeat(feats, T), M)
    rec["threshold"] = np.tile(np.tile(np.arange(T), K), M)
    rec["valid"] = rng.random(M * n) < 0.9
    rec["valid"][:n] = 0  # a node without a valid candidate
    rec["score"][n + 3] = np.nan  # NaN scores are skipped
    dev = torch.device("cuda")
    cand = torch.from_numpy(rec.view(np.uint8).copy()).to(dev)
    band = torch.empty(M * n, dtype=torch.int32, device=dev)
    out = torch.zeros(M * _hip.CANDIDATE_DTYPE.itemsize, dtype=torch.uint8, device=dev)
    _hip.check(lib.pb_pick_sequential(cand.data_ptr(), M, K, T, band.data_ptr(), out.data_ptr(),
                                      _hip.stream_ptr()), "pb_pick_sequential")
    got = np.frombuffer(out.cpu().numpy().tobytes(), dtype=_hip.CANDIDATE_DTYPE)
    for u in range(M):
        r = rec[u * n:(u + 1) * n]
        i = _sequential_pick(r["score"], r["left_total"], r["feature"], r["threshold"], r["valid"] != 0)
        if i < 0:
            assert got["valid"][u] == 0 and got["feature"][u] == -1 and got["threshold"][u] == -1, u
            continue
        assert got["valid"][u] == 1, u
        assert (got["feature"][u], got["threshold"][u], got["left_total"][u]) == \
            (r["feature"][i], r["threshold"][i], r["left_total"][i]), (u, spread)
        assert got["score"][u] == r["score"][i]
