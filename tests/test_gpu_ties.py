"""The reference's sequential split pick and its 1e-12 tie window, on the device.

frontier_cpu.cpp:415-426 visits a node's candidates in order (subset feature, then threshold)
and replaces its best when a candidate scores higher, or scores within 1e-12 and has more left
rows, then a larger feature id, then a larger threshold. With scores near 1e-12 (tiny
gradients) distinct scores fall inside that window and the pick differs from a plain argmax.
Each case first checks on the CPU that it does differ (so the case exercises the window), then
feeds the oracle's planes to the device scorer and requires the device's decisions to equal the
oracle's sequential pick exactly.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import GpuDepth, make_problem, node_era_rows, split_params

pytestmark = pytest.mark.gpu


def strict_argmax(sp, feats):
    """Highest score; exact ties to the larger left count, feature, threshold."""
    s, lt, v = sp["score"], sp["left_total"], sp["valid"].astype(bool)
    out = []
    for u in range(s.shape[0]):
        best = None
        for k in range(s.shape[1]):
            for t in range(s.shape[2]):
                if v[u, k, t]:
                    key = (float(s[u, k, t]), int(lt[u, k, t]), int(feats[k]), t)
                    best = key if best is None or key > best else best
        out.append(None if best is None else (best[2], best[3]))
    return out


CASES = [
    # seed, grad scale, N, F, E, nb, U, K
    (11, 2e-6, 3000, 12, 4, 5, 2, 12),    # two unequal candidates within 1e-12 at the top
    (5, 2e-6, 3000, 12, 4, 5, 2, 12),
    (3, 1e-7, 6000, 40, 5, 5, 3, 40),     # every candidate within the window: band > 64
    (7, 1e-7, 4000, 8, 3, 64, 2, 8),      # 63 thresholds per feature
    (9, 1e-7, 5000, 6, 3, 200, 2, 6),     # the wide scorer (T >= 64)
]


@pytest.mark.parametrize("case", CASES, ids=[f"seed{c[0]}-nb{c[5]}" for c in CASES])
def test_sequential_pick_matches_reference(hip, oracle_mod, case):
    seed, scale, N, F, E, nb, U, K = case
    print(f"[ties] seed={seed} scale={scale} N={N} F={F} E={E} nb={nb} U={U} K={K}", flush=True)
    p = make_problem(seed, N, F, E, nb, U, grad_scale=scale)
    feats = np.random.default_rng(seed + 100).permutation(F)[:K].astype(np.int32)
    kw = dict(lambda_l2=1e-6, lambda_dro=0.5, direction_weight=0.0, era_alpha=0.0,
              min_samples_leaf=20)
    ref = oracle_mod.split_batch(p["bins"], p["grad"], node_era_rows(p), feats, nb,
                                 want_planes=True, **kw)
    rc, rg = ref.planes
    rg1 = rg.copy()
    rg1[..., nb - 1] = rg[:, :, :1, nb - 1]  # one era total per (era, node), as on the device
    sp = oracle_mod.score_planes(rc, rg1, feats, None, **kw)
    seq = [None if sp["best_feature"][u] < 0 else (int(sp["best_feature"][u]), int(sp["best_threshold"][u]))
           for u in range(U)]
    assert strict_argmax(sp, feats) != seq, "case does not exercise the tie window"

    g = GpuDepth(hip, p, K, msl=20)
    try:
        params = split_params(hip, **{k: v for k, v in kw.items() if k != "min_samples_leaf"}, msl=20)
        g.load_planes(rc, rg1)
        c = g.score(feats, params, nb - 1)
        v = sp["valid"].astype(bool)
        np.testing.assert_array_equal(c["score"][v].view(np.uint32), sp["score"][v].view(np.uint32))
        dec = g.decide(params)
        for u in range(U):
            if seq[u] is None:
                assert dec["split"][u] == 0
                continue
            assert dec["split"][u] == 1
            assert (int(dec["feature"][u]), int(dec["threshold"][u])) == seq[u], f"node {u}"
            assert dec["left_count"][u] == sp["best_left"][u]
            assert dec["score"][u].view(np.uint32) == sp["best_score"][u].view(np.uint32)
            assert dec["left_grad"][u].view(np.uint32) == sp["best_left_grad"][u].view(np.uint32)
    finally:
        g.close()
