"""Teacher-forced parity of one depth (kernels 1-3) against the CPU oracle.

Inputs: seeded random bins/grad/era layouts and a row -> node assignment. The oracle is the
restated reference split finder (frontier_cpu.cpp:111-515). Bars:
  * counts and node assignments bit-exact;
  * grad planes within 1e-5 of the per-cell absolute grad mass (sum |g| over the cell's rows);
  * scorer fed the oracle's planes: every candidate's score / left count / left grad /
    validity bit-identical, and the chosen (feature, threshold) identical;
  * scorer on the GPU's own planes: same choice unless the oracle's scores of the two
    choices are within 1e-6 (a tie).
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import GpuDepth, make_problem, node_era_rows, split_params

pytestmark = pytest.mark.gpu

CASES = [
    # seed, N, F, E, nb, U, K, msl, lambda_l2, lambda_dro, dir_w, era_alpha
    (1, 4000, 12, 6, 5, 1, 12, 20, 1e-6, 0.5, 0.0, 0.0),
    (2, 6000, 20, 9, 16, 4, 9, 10, 1.0, 0.5, 0.0, 0.0),
    (3, 9000, 30, 17, 128, 8, 16, 5, 1e-6, 0.1, 0.2, 1.5),
    (4, 3000, 8, 3, 2, 2, 8, 1, 0.5, 0.0, 0.0, 0.0),
    (5, 20000, 40, 40, 5, 32, 24, 20, 1e-6, 0.5, 0.0, 0.0),
    (6, 5000, 10, 5, 255, 3, 10, 3, 1.0, 1.0, 0.0, 2.5),
    # 100 nodes x 255 bins: one feature's histogram exceeds the LDS -> node tiles
    (7, 30000, 12, 6, 255, 100, 6, 5, 1e-6, 0.5, 0.0, 0.0),
    (8, 12000, 9, 4, 200, 70, 9, 3, 1.0, 0.2, 0.1, 1.0),
    # 210 nodes x 40 features x 254 thresholds: max_nodes x wavefront winners >= 32768, so the
    # per-node winners are reduced by one workgroup per node before the decision step
    (9, 40000, 48, 4, 255, 210, 40, 2, 1e-6, 0.5, 0.0, 0.0),
    # one node x 128 bins x 20 features (config 1's first depth): single-feature tiles of 16
    # uint8 columns, the widest single-feature launch shape
    (10, 10000, 20, 10, 128, 1, 20, 20, 1.0, 0.5, 0.0, 0.0),
    # 5 bins, 16 nodes: 16-feature pair tiles, the last one of 7 features (a pair whose second
    # feature lies past the tile's end)
    (11, 16000, 30, 9, 5, 16, 23, 5, 1e-6, 0.5, 0.0, 0.0),
    # 5 bins, 8 nodes: 12-feature triple tiles over 1000 joint cells per group (the 40 KB
    # budget), the last tile of one feature (a group with two partners past the tile's end)
    (12, 12000, 20, 7, 5, 8, 13, 5, 1e-6, 0.5, 0.0, 0.0),
]


def _abs_mass(p, U):
    """sum |g| per (era, node) — the scale of any grad cell of that (era, node)."""
    nid = p["nid"].astype(np.int64)
    m = np.zeros((p["E"], U))
    act = nid < U
    np.add.at(m, (p["era"][act], nid[act]), np.abs(p["grad"][act].astype(np.float64)))
    return m


# the nibble bin layout (max_bins <= 16) runs every case it applies to
LAYOUT_CASES = [(c, "u8") for c in CASES] + [(c, "nibble") for c in CASES if c[4] <= 16]


@pytest.mark.parametrize("case,layout", LAYOUT_CASES,
                         ids=[f"case{c[0]}-{lay}" for c, lay in LAYOUT_CASES])
def test_depth_parity(hip, oracle_mod, case, layout):
    seed, N, F, E, nb, U, K, msl, lam, dro, dw, alpha = case
    print(f"[depth parity] seed={seed} N={N} F={F} E={E} nb={nb} U={U} K={K} {layout}", flush=True)
    p = make_problem(seed, N, F, E, nb, U, empty_era=(seed % 2 == 0))
    rng = np.random.default_rng(seed + 100)
    feats = rng.permutation(F)[:K].astype(np.int32)
    kw = dict(lambda_l2=lam, lambda_dro=dro, direction_weight=dw, era_alpha=alpha,
              min_samples_leaf=msl)
    ref = oracle_mod.split_batch(p["bins"], p["grad"], node_era_rows(p), feats, nb,
                                 want_planes=True, want_cands=True, **kw)
    g = GpuDepth(hip, p, K, msl=msl, layout=layout)
    try:
        g.hist(feats)
        cnt, gp = g.planes()
        rc, rg = ref.planes
        # every (era, node) total is that node's rows in the era, counted from the row ids
        # (independent of the oracle: a build that miscounts fails here first)
        nid = p["nid"].astype(np.int64)
        act = nid < U
        rows_en = np.zeros((E, U), dtype=np.int64)
        np.add.at(rows_en, (p["era"][act], nid[act]), 1)
        np.testing.assert_array_equal(cnt[:, :, :, nb - 1], np.repeat(rows_en[:, :, None], K, axis=2))
        np.testing.assert_array_equal(cnt, rc)
        mass = _abs_mass(p, U)[:, :, None, None]
        err = np.abs(gp.astype(np.float64) - rg.astype(np.float64))
        assert np.all(err <= 1e-5 * np.maximum(mass, 1.0)), float((err / np.maximum(mass, 1.0)).max())

        params = split_params(hip, lambda_l2=lam, lambda_dro=dro, direction_weight=dw,
                              era_alpha=alpha, msl=msl)
        T = nb - 1
        # (a) scorer on the GPU's own histogram -> decisions
        own = g.score(feats, params, T)
        dec = g.decide(params)
        # (b) scorer fed the oracle planes: bit-exact candidates. The device planes hold one era
        # total per (era, node); the reference's float32 running sum can end a bit differently
        # per feature, so both scorers get feature 0's total for every feature.
        rg1 = rg.copy()
        rg1[..., nb - 1] = rg[:, :, :1, nb - 1]
        g.load_planes(rc, rg1)
        c = g.score(feats, params, T)
        sp = oracle_mod.score_planes(rc, rg1, feats, None, **kw)
        np.testing.assert_array_equal(c["valid"].astype(bool), sp["valid"].astype(bool))
        v = sp["valid"].astype(bool)
        np.testing.assert_array_equal(c["score"][v].view(np.uint32), sp["score"][v].view(np.uint32))
        np.testing.assert_array_equal(c["left_total"][v], sp["left_total"][v])
        np.testing.assert_array_equal(c["left_grad"][v].view(np.uint32),
                                      sp["left_grad"][v].view(np.uint32))
        rs, rl, rlg, rv = ref.cands

        for u in range(U):
            if ref.feature[u] < 0:
                assert dec["split"][u] == 0
                continue
            assert dec["split"][u] == 1
            if (dec["feature"][u], dec["threshold"][u]) != (ref.feature[u], ref.threshold[u]):
                k = int(np.nonzero(feats == dec["feature"][u])[0][0])
                s_gpu_choice = rs[u, k, dec["threshold"][u]]
                assert abs(float(s_gpu_choice) - float(ref.score[u])) <= 1e-6 * max(1.0, abs(float(ref.score[u]))), \
                    f"node {u}: not a tie"
                continue
            assert dec["left_count"][u] == ref.left_count[u]
            assert dec["right_count"][u] == ref.right_count[u]
            assert abs(float(dec["left_grad"][u]) - float(ref.left_grad[u])) <= 1e-5 * max(1.0, float(np.abs(p["grad"]).sum()))

        # partition with the GPU's decisions vs the restated rule bin <= thr -> left
        nid_after, tn_after = g.partition()
        u_next, tsize = g.frontier()
        nid0 = p["nid"].astype(np.int64)
        exp_tn = np.zeros(N, np.int64)
        exp_nid = np.full(N, 0xFFFF, np.int64)
        act = nid0 < U
        exp_tn[act] = g.node_ids[nid0[act]]
        slot = 0
        for u in range(U):
            rows = np.nonzero(nid0 == u)[0]
            if not dec["split"][u]:
                continue
            side = (p["bins"][rows, dec["feature"][u]] > dec["threshold"][u]).astype(np.int64)
            exp_tn[rows] = dec["left_id"][u] + side
            cnts = [int(np.sum(side == 0)), int(np.sum(side == 1))]
            assert cnts[0] == dec["left_count"][u] and cnts[1] == dec["right_count"][u]
            for s_ in (0, 1):
                if cnts[s_] >= 2 * msl:
                    exp_nid[rows[side == s_]] = slot
                    slot += 1
        np.testing.assert_array_equal(tn_after.astype(np.int64), exp_tn)
        np.testing.assert_array_equal(nid_after.astype(np.int64), exp_nid)
        assert u_next[g.depth + 1] == slot
    finally:
        g.close()


def test_hist_extreme_grad_scale(hip, oracle_mod):
    """Fixed-point grad sums hold up for tiny and huge gradient magnitudes."""
    for scale in (1e-20, 1e20):
        p = make_problem(11, 3000, 6, 4, 7, 2, grad_scale=scale)
        feats = np.arange(6, dtype=np.int32)
        ref = oracle_mod.split_batch(p["bins"], p["grad"], node_era_rows(p), feats, 7, want_planes=True)
        g = GpuDepth(hip, p, 6, msl=1)
        try:
            g.hist(feats)
            cnt, gp = g.planes()
            np.testing.assert_array_equal(cnt, ref.planes[0])
            mass = _abs_mass(p, 2)[:, :, None, None]
            err = np.abs(gp.astype(np.float64) - ref.planes[1].astype(np.float64))
            assert np.all(err <= 1e-5 * mass + 1e-30 * scale)
        finally:
            g.close()


@pytest.mark.parametrize("nb,hi", [(128, 126), (128, 64), (200, 190), (6, 4)])
def test_exact_ties_pick_largest_threshold(hip, oracle_mod, nb, hi):
    """Rows only in bins 0 and `hi`: thresholds 0..hi-1 give the same split, so their scores
    are bit-identical and the reference's tie-break (frontier_cpu.cpp:415-426) keeps the
    largest threshold, hi-1 — across wavefront boundaries of the candidate space too."""
    N, E = 4000, 3
    rng = np.random.default_rng(nb + hi)
    p = make_problem(7, N, 2, E, nb, 1, inactive_frac=0.0)
    p["bins"][:, 0] = np.where(rng.random(N) < 0.4, 0, hi).astype(np.uint8)
    feats = np.array([0, 1], dtype=np.int32)
    ref = oracle_mod.split_batch(p["bins"], p["grad"], node_era_rows(p), feats, nb, want_cands=True,
                                 min_samples_leaf=5)
    g = GpuDepth(hip, p, 2, msl=5)
    try:
        g.hist(feats)
        params = split_params(hip, msl=5)
        c = g.score(feats, params, nb - 1)
        dec = g.decide(params)
        s0 = c["score"][0, 0, :hi]
        assert np.all(s0.view(np.uint32) == s0[0].view(np.uint32))
        assert (dec["feature"][0], dec["threshold"][0]) == (ref.feature[0], ref.threshold[0]), \
            (dec["feature"][0], dec["threshold"][0], ref.feature[0], ref.threshold[0])
    finally:
        g.close()


@pytest.mark.parametrize("block", [128, 256])
@pytest.mark.parametrize("pairs", [1, 2, 3])
@pytest.mark.parametrize("copies", [1, 2, 4, 8, 16, 32])
def test_hist_copies(hip, oracle_mod, monkeypatch, pairs, copies, block):
    """Every histogram replication count (the copies are folded by DPP lane shifts), joint
    width and workgroup size gives the oracle's planes: counts bit-exact, grads within the
    per-cell mass bar."""
    monkeypatch.setenv("PB_HIST_COPIES", str(copies))
    monkeypatch.setenv("PB_HIST_PAIRS", str(pairs))
    monkeypatch.setenv("PB_HIST_BLOCK", str(block))
    print(f"[hist copies] C={copies} P={pairs} block={block}", flush=True)
    p = make_problem(40 + copies, 9000, 14, 5, 5, 2, empty_era=True)
    feats = np.random.default_rng(copies).permutation(14)[:13].astype(np.int32)
    ref = oracle_mod.split_batch(p["bins"], p["grad"], node_era_rows(p), feats, 5, want_planes=True)
    g = GpuDepth(hip, p, 13, msl=3, layout="nibble" if copies % 2 == 0 else "u8")
    try:
        g.hist(feats)
        cnt, gp = g.planes()
        np.testing.assert_array_equal(cnt, ref.planes[0])
        mass = _abs_mass(p, 2)[:, :, None, None]
        err = np.abs(gp.astype(np.float64) - ref.planes[1].astype(np.float64))
        assert np.all(err <= 1e-5 * np.maximum(mass, 1.0))
    finally:
        g.close()


@pytest.mark.parametrize("layout", ["u8", "nibble"])
@pytest.mark.parametrize("pairs,ftile", [(2, 32), (1, 16)])
def test_hist_widest_tiles(hip, oracle_mod, monkeypatch, pairs, ftile, layout):
    """The widest feature tiles (32 features in pairs, 16 single features: the instantiations
    with the most registers per thread), forced on a 5-bin panel with an odd feature count so
    the last pair's partner runs past the tile. Counts bit-exact, grads within the per-cell
    mass bar."""
    monkeypatch.setenv("PB_HIST_PAIRS", str(pairs))
    monkeypatch.setenv("PB_HIST_FTILE", str(ftile))
    print(f"[hist widest tiles] P={pairs} FT={ftile} {layout}", flush=True)
    K = 33
    p = make_problem(70 + ftile + pairs, 12000, 40, 6, 5, 2, empty_era=True)
    feats = np.random.default_rng(ftile + pairs).permutation(40)[:K].astype(np.int32)
    ref = oracle_mod.split_batch(p["bins"], p["grad"], node_era_rows(p), feats, 5, want_planes=True)
    g = GpuDepth(hip, p, K, msl=3, layout=layout)
    try:
        g.hist(feats)
        cnt, gp = g.planes()
        np.testing.assert_array_equal(cnt, ref.planes[0])
        mass = _abs_mass(p, 2)[:, :, None, None]
        err = np.abs(gp.astype(np.float64) - ref.planes[1].astype(np.float64))
        assert np.all(err <= 1e-5 * np.maximum(mass, 1.0))
    finally:
        g.close()


@pytest.mark.parametrize("layout", ["u8", "nibble"])
@pytest.mark.parametrize("pairs,nb", [(2, 2), (2, 3), (2, 4), (2, 5), (2, 6), (2, 7), (2, 8), (2, 9),
                                      (3, 2), (3, 3), (3, 4), (3, 6)])
def test_hist_joint_flush_bins(hip, oracle_mod, monkeypatch, pairs, nb, layout):
    """The joint-bin flush at every small bin count: pairs (one thread per (node, feature) over
    the pair's nb x nb cells for nb <= 8, the element-wise path above) and triples (marginal
    elements compacted, then prefixes per (node, feature)), with an odd feature count so the last
    group's partners run past the tile. Counts bit-exact, grads within the per-cell mass bar."""
    monkeypatch.setenv("PB_HIST_PAIRS", str(pairs))
    print(f"[hist joint flush] P={pairs} nb={nb} {layout}", flush=True)
    p = make_problem(60 + 10 * pairs + nb, 7000, 15, 6, nb, 3, empty_era=True)
    feats = np.random.default_rng(nb).permutation(15)[:11].astype(np.int32)
    ref = oracle_mod.split_batch(p["bins"], p["grad"], node_era_rows(p), feats, nb, want_planes=True)
    g = GpuDepth(hip, p, 11, msl=3, layout=layout)
    try:
        g.hist(feats)
        cnt, gp = g.planes()
        np.testing.assert_array_equal(cnt, ref.planes[0])
        mass = _abs_mass(p, 3)[:, :, None, None]
        err = np.abs(gp.astype(np.float64) - ref.planes[1].astype(np.float64))
        assert np.all(err <= 1e-5 * np.maximum(mass, 1.0))
    finally:
        g.close()


def test_wide_scorer_many_eras(hip, oracle_mod):
    """The many-threshold scorer over 3500 eras with unit era weights, fed the oracle's planes:
    every candidate bit-identical to the oracle scorer. Its Welford factor 1/n is computed
    (reciprocal plus one Newton step) for every active-era count n up to 3500, so this pins that
    computation against the IEEE division the reference uses."""
    E, nb, U, K = 3500, 70, 2, 2
    p = make_problem(77, E * 8, 3, E, nb, U, ragged=False, inactive_frac=0.0)
    feats = np.array([2, 0], np.int32)
    kw = dict(lambda_l2=1e-6, lambda_dro=0.5, direction_weight=0.0, era_alpha=0.0, min_samples_leaf=1)
    print(f"[wide many eras] E={E} nb={nb}", flush=True)
    ref = oracle_mod.split_batch(p["bins"], p["grad"], node_era_rows(p), feats, nb, want_planes=True, **kw)
    rc, rg = ref.planes
    rg1 = rg.copy()
    rg1[..., nb - 1] = rg[:, :, :1, nb - 1]
    g = GpuDepth(hip, p, K, msl=1)
    try:
        g.load_planes(rc, rg1)
        params = split_params(hip, lambda_l2=1e-6, lambda_dro=0.5, msl=1)
        c = g.score(feats, params, nb - 1)
        sp = oracle_mod.score_planes(rc, rg1, feats, None, **kw)
        np.testing.assert_array_equal(c["valid"].astype(bool), sp["valid"].astype(bool))
        v = sp["valid"].astype(bool)
        assert v.sum() > 0
        np.testing.assert_array_equal(c["score"][v].view(np.uint32), sp["score"][v].view(np.uint32))
    finally:
        g.close()


WIDE_CASES = [c for c in CASES if c[4] - 1 >= 64]


@pytest.mark.parametrize("k_cuts", [0, 70])
@pytest.mark.parametrize("case", WIDE_CASES, ids=[f"case{c[0]}" for c in WIDE_CASES])
def test_wide_scorer_matches_staged(hip, oracle_mod, monkeypatch, case, k_cuts):
    """Features with 64+ thresholds: the wide scorer (one thread per threshold, eras batched in
    registers) and the LDS-staged two-phase scorer give bit-identical candidates (score, left
    count, left grad, validity) and the same decisions, with the full sweep and with K-cuts."""
    seed, N, F, E, nb, U, K, msl, lam, dro, dw, alpha = case
    T = nb - 1 if (k_cuts == 0 or k_cuts >= nb - 1) else k_cuts
    print(f"[wide scorer] seed={seed} nb={nb} U={U} K={K} k_cuts={k_cuts}", flush=True)
    p = make_problem(seed, N, F, E, nb, U, empty_era=(seed % 2 == 0))
    feats = np.random.default_rng(seed + 100).permutation(F)[:K].astype(np.int32)
    params = split_params(hip, lambda_l2=lam, lambda_dro=dro, direction_weight=dw,
                          era_alpha=alpha, msl=msl, k_cuts=k_cuts, cut_selection="mass")
    out = {}
    for staged in (1, 0):
        monkeypatch.setenv("PB_SCORE_STAGED", str(staged))
        g = GpuDepth(hip, p, K, msl=msl, layout="u8")
        try:
            g.hist(feats)
            out[staged] = (g.score(feats, params, T), g.decide(params))
        finally:
            g.close()
    (c1, d1), (c0, d0) = out[1], out[0]
    for field in ("valid", "left_total", "feature", "threshold"):
        np.testing.assert_array_equal(c0[field], c1[field])
    for field in ("score", "left_grad"):
        np.testing.assert_array_equal(c0[field].view(np.uint32), c1[field].view(np.uint32))
    assert d0.tobytes() == d1.tobytes()


def _exact_prefix(p, feats, U):
    """float64 prefix grad sums and prefix |grad| masses [E][U][K][nb] (bin nb-1: the era total)."""
    nid = p["nid"].astype(np.int64)
    act = nid < U
    E, nb, K = p["E"], p["nb"], len(feats)
    g = p["grad"].astype(np.float64)[act]
    e, u = p["era"][act], nid[act]
    s = np.zeros((E, U, K, nb))
    m = np.zeros((E, U, K, nb))
    for k, f in enumerate(feats):
        b = p["bins"][act, f].astype(np.int64)
        np.add.at(s, (e, u, k, b), g)
        np.add.at(m, (e, u, k, b), np.abs(g))
    return np.cumsum(s, axis=3), np.cumsum(m, axis=3)


HEAVY = [
    # seed, N, F, E, nb, U, K: a few rows with |grad| 1e4..1e6 among N(0, 1) gradients
    (31, 20000, 16, 8, 5, 4, 16),
    (32, 30000, 12, 6, 128, 8, 12),
    (33, 24000, 10, 4, 16, 2, 10),
    (34, 70000, 8, 2, 16, 3, 8),  # eras of 35000 rows: summed over segments
]
HEAVY_LAYOUT = [(c, "u8") for c in HEAVY] + [(c, "nibble") for c in HEAVY if c[4] <= 16]


@pytest.mark.parametrize("case,layout", HEAVY_LAYOUT, ids=[f"seed{c[0]}-{lay}" for c, lay in HEAVY_LAYOUT])
def test_hist_heavy_tailed_grads(hip, oracle_mod, case, layout):
    """Grad planes when a few rows' |grad| exceed the rest by up to 10^6: every cell within
    1e-5 of its own |grad| mass (no floor), against exact float64 sums; counts bit-exact
    against the oracle. The fixed-point scale is set per era, so only the eras that hold an
    outlier get a coarser step."""
    seed, N, F, E, nb, U, K = case
    print(f"[heavy tails] seed={seed} N={N} E={E} nb={nb} U={U} {layout}", flush=True)
    p = make_problem(seed, N, F, E, nb, U)
    rng = np.random.default_rng(seed + 7)
    idx = rng.choice(N, 6, replace=False)
    p["grad"][idx] = (rng.choice([-1.0, 1.0], 6) * np.array([1e4, 3e4, 1e5, 3e5, 1e6, 1e6])).astype(np.float32)
    feats = rng.permutation(F)[:K].astype(np.int32)
    ref = oracle_mod.split_batch(p["bins"], p["grad"], node_era_rows(p), feats, nb, want_planes=True,
                                 min_samples_leaf=1)
    exact, mass = _exact_prefix(p, feats, U)
    g = GpuDepth(hip, p, K, msl=1, layout=layout)
    try:
        g.hist(feats)
        cnt, gp = g.planes()
        np.testing.assert_array_equal(cnt, ref.planes[0])
        err = np.abs(gp.astype(np.float64) - exact)
        worst = np.max(np.where(mass > 0, err / np.where(mass > 0, mass, 1.0), 0.0))
        assert np.all(err <= 1e-5 * mass), f"worst relative error {worst:.3g}"
        # the reference's float32 row-order sums meet the same bar on these inputs
        assert np.all(np.abs(ref.planes[1].astype(np.float64) - exact) <= 1e-5 * mass)
    finally:
        g.close()


def test_hist_max_nodes_above_frontier_bound(hip, oracle_mod):
    """pb_hist_build with max_nodes above pb_max_nodes (the header allows any bound at least
    that large) on eras split into segments gives the same planes as the pb_max_nodes call:
    the segment sums are strided by the context's own allocation, not by max_nodes."""
    import torch

    p = make_problem(51, 70000, 6, 2, 7, 3, inactive_frac=0.05)
    feats = np.arange(6, dtype=np.int32)
    g = GpuDepth(hip, p, 6, msl=1)
    try:
        g.hist(feats)
        cnt0, gp0 = g.planes()
        g.max_nodes += 8
        plane = int(g.lib.pb_hist_plane_elems(g.ctx, g.max_nodes))
        g.cnt = torch.zeros(plane, dtype=torch.int32, device="cuda")
        g.g = torch.zeros(plane, dtype=torch.float32, device="cuda")
        g.hist(feats)
        cnt1, gp1 = g.planes()
        np.testing.assert_array_equal(cnt1, cnt0)
        np.testing.assert_array_equal(gp1.view(np.uint32), gp0.view(np.uint32))
    finally:
        g.close()


UNIT_CASES = [
    # seed, N, F, E, nb, U, K: 1, 2, 5 and 8 pairs per producer thread at T = 4 (4, 12, 40
    # and 60 candidates per workgroup), partial last chunks of eras, an empty era
    (21, 20_000, 60, 37, 5, 1, 60),
    (22, 40_000, 240, 50, 5, 8, 240),
    (23, 60_000, 240, 75, 5, 32, 240),
    (24, 30_000, 120, 26, 16, 4, 120),
]


@pytest.mark.parametrize("mode", ["0", "1", "2"])
@pytest.mark.parametrize("case", UNIT_CASES, ids=[f"seed{c[0]}" for c in UNIT_CASES])
def test_unit_weight_scorers(hip, oracle_mod, monkeypatch, case, mode):
    """The two producer/consumer scorers for T <= 63 with unit era weights (PB_SCORE_PC: 0 the
    launch rule, 1 des_score_pc_kernel only, 2 des_score_pcu_kernel only, at every pairs-per-
    thread instantiation), fed the oracle's planes: every candidate bit-identical to the
    restated scorer (frontier_cpu.cpp:342-444)."""
    seed, N, F, E, nb, U, K = case
    monkeypatch.setenv("PB_SCORE_PC", mode)
    print(f"[unit scorers] mode={mode} {case}", flush=True)
    p = make_problem(seed, N, F, E, nb, U, empty_era=True)
    feats = np.random.default_rng(seed + 100).permutation(F)[:K].astype(np.int32)
    kw = dict(lambda_l2=1e-6, lambda_dro=0.5, direction_weight=0.0, era_alpha=0.0, min_samples_leaf=5)
    ref = oracle_mod.split_batch(p["bins"], p["grad"], node_era_rows(p), feats, nb, want_planes=True, **kw)
    rc, rg = ref.planes
    rg1 = rg.copy()
    rg1[..., nb - 1] = rg[:, :, :1, nb - 1]  # one era total per (era, node), as the device planes
    g = GpuDepth(hip, p, K, msl=5)
    try:
        g.load_planes(rc, rg1)
        params = split_params(hip, lambda_l2=1e-6, lambda_dro=0.5, msl=5)
        c = g.score(feats, params, nb - 1)
        sp = oracle_mod.score_planes(rc, rg1, feats, None, **kw)
        np.testing.assert_array_equal(c["valid"].astype(bool), sp["valid"].astype(bool))
        v = sp["valid"].astype(bool)
        assert v.sum() > 0
        np.testing.assert_array_equal(c["score"][v].view(np.uint32), sp["score"][v].view(np.uint32))
        np.testing.assert_array_equal(c["left_total"][v], sp["left_total"][v])
        np.testing.assert_array_equal(c["left_grad"][v].view(np.uint32), sp["left_grad"][v].view(np.uint32))
        dec = g.decide(params)
        for u in range(U):
            if sp["best_feature"][u] >= 0 and v[u].any():
                assert (dec["feature"][u], dec["threshold"][u]) == (sp["best_feature"][u], sp["best_threshold"][u])
    finally:
        g.close()


def test_decide_keeps_scored_feature_ids(hip, oracle_mod):
    """pb_decide uses the feature ids pb_des_score was given even when the caller rewrites its
    buffer between the two calls (pb_des_score keeps a copy on its stream)."""
    seed, N, F, E, nb, U, K = 31, 8000, 30, 7, 5, 3, 20
    p = make_problem(seed, N, F, E, nb, U)
    feats = np.random.default_rng(seed).permutation(F)[:K].astype(np.int32)
    params = split_params(hip, lambda_dro=0.5, msl=5)
    decs = []
    for clobber in (False, True):
        g = GpuDepth(hip, p, K, msl=5)
        try:
            g.hist(feats)
            g.score(feats, params, nb - 1)
            if clobber:
                g.feats.fill_(F + 7)  # the caller reuses its buffer before pb_decide
            decs.append(g.decide(params))
        finally:
            g.close()
    ref = oracle_mod.split_batch(p["bins"], p["grad"], node_era_rows(p), feats, nb, lambda_dro=0.5,
                                 min_samples_leaf=5)
    for key in ("split", "feature", "threshold", "left_count"):
        np.testing.assert_array_equal(decs[1][key], decs[0][key])
    assert set(decs[1]["feature"][decs[1]["split"] == 1]) <= set(feats.tolist())
    assert decs[1]["split"].sum() == int((ref.feature >= 0).sum())
