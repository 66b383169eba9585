"""One depth of the headline workload at its full size (2,400,000 rows x 2376 features, 574
contiguous eras, 5 bins, 238 sampled features, nibble bin layout as in a fit), checked through
properties that do not depend on the size, since the CPU oracle cannot histogram 5.7 GB in a
test:

- every era's total count is the number of its rows in the node (all of them at depth 0);
  prefix counts never decrease over thresholds and never exceed the total;
- sampled (era, feature) cells against a NumPy bincount of the same rows: counts bit-exact,
  grads within 1e-5 of the cell's |g| mass; era grad totals against float64 sums for every era;
- every candidate the HIP scorer makes from the device planes is bit-identical to the oracle
  scorer run on the same planes (frontier_cpu.cpp:342-444), and the decision matches the
  oracle's argmax with the reference tie-break;
- the partition sends row r left iff bin[r, f*] <= t* of its node, and its node counts equal
  the decision's left/right counts.
"""

from __future__ import annotations

import numpy as np
import pytest

from helpers import PB_INACTIVE, GpuDepth, decode_planes, split_params

pytestmark = pytest.mark.gpu

N, F, E, NB, K = 2_400_000, 2376, 574, 5, 238


@pytest.fixture(scope="module")
def panel():
    import torch

    print(f"[fullsize] generating {N} x {F} bins on the device", flush=True)
    ld = (N + 15) // 16 * 16
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    bins = torch.randint(0, NB, (F, ld), dtype=torch.uint8, device="cuda", generator=g)
    bins[:, N:] = 0
    sizes = np.array([len(a) for a in np.array_split(np.arange(N), E)], dtype=np.int64)
    offs = np.zeros(E + 1, np.int64)
    np.cumsum(sizes, out=offs[1:])
    yield bins, offs.astype(np.int32)
    del bins
    torch.cuda.empty_cache()


@pytest.mark.parametrize("U", [1, 32])
def test_fullsize_depth(hip, oracle_mod, panel, U):
    import torch

    bins, offs = panel
    rng = np.random.default_rng(100 + U)
    grad = rng.standard_normal(N).astype(np.float32)
    nid = np.zeros(N, np.uint16) if U == 1 else rng.integers(0, U, N).astype(np.uint16)
    if U > 1:
        nid[rng.random(N) < 0.05] = PB_INACTIVE
    era = np.repeat(np.arange(E), np.diff(offs))
    p = {"N": N, "F": F, "E": E, "nb": NB, "U": U, "era_off": offs, "grad": grad, "nid": nid,
         "era": era, "bins": None}
    feats = rng.permutation(F)[:K].astype(np.int32)
    kw = dict(lambda_l2=1e-6, lambda_dro=0.5, direction_weight=0.0, era_alpha=0.0,
              min_samples_leaf=20)
    print(f"[fullsize] U={U}: hist / score / decide / partition", flush=True)
    gd = GpuDepth(hip, p, K, msl=20, max_depth=6, layout="nibble", bins_dev=bins)
    try:
        gd.hist(feats)
        E_, M, K_, nb, _, _ = gd._plane_layout()
        cnt, gp = decode_planes(gd.cnt.cpu().numpy(), gd.g.cpu().numpy(), E_, M, K_, nb)
        cnt, gp = cnt[:, :U], gp[:, :U]

        # totals and monotone prefixes
        act = nid != PB_INACTIVE
        want_tot = np.zeros((E, U), np.int64)
        np.add.at(want_tot, (era[act], nid[act].astype(np.int64)), 1)
        np.testing.assert_array_equal(cnt[:, :, 0, NB - 1], want_tot)
        assert np.all(np.diff(cnt, axis=3) >= 0)
        gsum = np.zeros((E, U), np.float64)
        gabs = np.zeros((E, U), np.float64)
        np.add.at(gsum, (era[act], nid[act].astype(np.int64)), grad[act].astype(np.float64))
        np.add.at(gabs, (era[act], nid[act].astype(np.int64)), np.abs(grad[act]).astype(np.float64))
        assert np.all(np.abs(gp[:, :, 0, NB - 1] - gsum) <= 1e-5 * np.maximum(gabs, 1.0))

        # sampled cells against a bincount of the same rows
        for e in rng.choice(E, 6, replace=False):
            r0, r1 = int(offs[e]), int(offs[e + 1])
            cols = bins[torch.from_numpy(feats.astype(np.int64)).cuda(), r0:r1].cpu().numpy()  # [K, rows]
            u_e = nid[r0:r1].astype(np.int64)
            g_e = grad[r0:r1].astype(np.float64)
            for u in range(U):
                m = u_e == u
                for k in range(K):
                    b = cols[k, m]
                    c = np.cumsum(np.bincount(b, minlength=NB))
                    np.testing.assert_array_equal(cnt[e, u, k], c)
                    gs = np.cumsum(np.bincount(b, weights=g_e[m], minlength=NB))
                    assert np.all(np.abs(gp[e, u, k] - gs) <= 1e-5 * max(1.0, float(np.abs(g_e[m]).sum())))

        # every candidate from the device planes, bit for bit, and the decision
        params = split_params(hip, lambda_l2=1e-6, lambda_dro=0.5, msl=20)
        c = gd.score(feats, params, NB - 1)
        dec = gd.decide(params)
        sp = oracle_mod.score_planes(cnt, gp, feats, None, **kw)
        v = sp["valid"].astype(bool)
        np.testing.assert_array_equal(c["valid"].astype(bool), v)
        np.testing.assert_array_equal(c["score"][v].view(np.uint32), sp["score"][v].view(np.uint32))
        np.testing.assert_array_equal(c["left_total"][v], sp["left_total"][v])
        np.testing.assert_array_equal(c["left_grad"][v].view(np.uint32), sp["left_grad"][v].view(np.uint32))
        for u in range(U):
            if sp["best_feature"][u] < 0:
                assert dec["split"][u] == 0
                continue
            assert dec["split"][u] == 1
            assert (dec["feature"][u], dec["threshold"][u]) == (sp["best_feature"][u], sp["best_threshold"][u])
            assert dec["left_count"][u] == sp["best_left"][u]
            assert dec["left_count"][u] + dec["right_count"][u] == want_tot[:, u].sum()

        # partition: bin <= thr goes left, on the uint8 columns
        print(f"[fullsize] U={U}: partition check", flush=True)
        nid_after, tn_after = gd.partition()
        fu = np.where(dec["split"] == 1, dec["feature"], 0).astype(np.int64)
        used = np.unique(fu[dec["split"] == 1])
        colmap = {int(f): bins[int(f), :N].cpu().numpy() for f in used}
        exp_tn = np.zeros(N, np.int64)
        exp_tn[act] = gd.node_ids[nid[act].astype(np.int64)]
        for u in range(U):
            if not dec["split"][u]:
                continue
            rows = np.nonzero(nid == u)[0]
            side = (colmap[int(dec["feature"][u])][rows] > dec["threshold"][u]).astype(np.int64)
            exp_tn[rows] = dec["left_id"][u] + side
            assert int(np.sum(side == 0)) == dec["left_count"][u]
            assert int(np.sum(side == 1)) == dec["right_count"][u]
        np.testing.assert_array_equal(tn_after.astype(np.int64), exp_tn)
        moved = nid_after != PB_INACTIVE
        assert np.all(act[moved])  # only rows of split nodes stay active
    finally:
        gd.close()
