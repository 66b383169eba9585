"""Host-side logic that needs no GPU: era encoding and the era-major permutation, the
rebuild of a round's tree from the device decision log (TreeBuilder numbering and
Python-double leaf values, booster.py:172-190, 527-563), the packed forest layout
(booster.py:730-783), the subset size rule (booster.py:787-792), and the bench contract's
refusal of more than one GPU."""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent


def test_encode_eras_and_era_major_order():
    from packboost_amd.data import encode_eras, era_major_order

    era = np.array([103, 100, 106, 100, 103, 103])
    codes, uniq = encode_eras(era, 6)
    np.testing.assert_array_equal(uniq, [100, 103, 106])
    np.testing.assert_array_equal(codes, [1, 0, 2, 0, 1, 1])
    perm, offs = era_major_order(codes, 3)
    np.testing.assert_array_equal(offs, [0, 2, 5, 6])
    # stable: rows of an era keep their order (the reference's ascending era row lists)
    np.testing.assert_array_equal(perm, [1, 3, 0, 4, 5, 2])
    codes0, uniq0 = encode_eras(None, 4)
    np.testing.assert_array_equal(codes0, 0)
    assert len(uniq0) == 1
    # already era-major input needs no permutation
    perm2, offs2 = era_major_order(np.array([0, 0, 1, 1, 1]), 2)
    assert perm2 is None or np.array_equal(perm2, np.arange(5))
    np.testing.assert_array_equal(offs2, [0, 2, 5])


def test_subset_size_rule():
    from packboost_amd import PackBoostConfig
    from packboost_amd.engine import subset_size

    assert subset_size(PackBoostConfig(layer_feature_fraction=0.1), 2376) == 238
    assert subset_size(PackBoostConfig(layer_feature_fraction=1.0), 20) == 20
    assert subset_size(PackBoostConfig(layer_feature_fraction=0.01), 20) == 1


def _decision(**kw):
    from packboost_amd.backends import _hip

    d = np.zeros(1, dtype=_hip.DECISION_DTYPE)
    for k, v in kw.items():
        d[k] = v
    return d[0]


def test_tree_arrays_from_log():
    from packboost_amd import PackBoostConfig
    from packboost_amd.backends import _hip
    from packboost_amd.engine import RoundLog, tree_arrays_from_log

    cfg = PackBoostConfig(max_depth=2, lambda_l2=0.5)
    dec = np.zeros(3, dtype=_hip.DECISION_DTYPE)
    # depth 0: root splits on feature 3 at bin 1 -> children 1, 2
    dec[0] = _decision(node_id=0, split=1, feature=3, threshold=1, left_grad=-2.0, left_hess=10,
                       right_grad=4.0, right_hess=30, left_count=10, right_count=30, left_id=1,
                       right_id=2, node_grad=2.0, node_count=40)
    # depth 1: node 1 becomes a leaf, node 2 splits on feature 0 at bin 0 -> 3, 4
    dec[1] = _decision(node_id=1, split=0, node_grad=-2.0, node_count=10, left_id=-1, right_id=-1)
    dec[2] = _decision(node_id=2, split=1, feature=0, threshold=0, left_grad=1.5, left_hess=12,
                       right_grad=2.5, right_hess=18, left_count=12, right_count=18, left_id=3,
                       right_id=4, node_grad=4.0, node_count=30)
    u = np.array([1, 2, 0], np.int32)
    log = RoundLog(u_active=u, tree_size=5, decisions=dec, root_grad=2.0, depths_drawn=2)
    a = tree_arrays_from_log(log, cfg, 40)
    np.testing.assert_array_equal(a["feature"], [3, -1, 0, -1, -1])
    np.testing.assert_array_equal(a["threshold"], [1, 0, 0, 0, 0])
    np.testing.assert_array_equal(a["left"], [1, -1, 3, -1, -1])
    np.testing.assert_array_equal(a["right"], [2, -1, 4, -1, -1])
    np.testing.assert_array_equal(a["is_leaf"], [False, True, False, True, True])
    lam = 0.5
    assert a["value"][0] == -2.0 / (40.0 + lam)
    assert a["value"][1] == -(-2.0) / (10.0 + lam)
    assert a["value"][2] == -4.0 / (30.0 + lam)
    assert a["value"][3] == -1.5 / (12.0 + lam)
    assert a["value"][4] == -2.5 / (18.0 + lam)


def test_pack_forest_layout():
    import torch

    from packboost_amd.booster import pack_forest

    tree = {"feature": np.array([2, -1, -1]), "threshold": np.array([1, 0, 0]),
            "left": np.array([1, -1, -1]), "right": np.array([2, -1, -1]),
            "value": np.array([0.0, 0.25, -0.5]), "is_leaf": np.array([False, True, True])}
    f = pack_forest([tree], 2, torch.device("cpu"))
    np.testing.assert_array_equal(f["offsets"].numpy(), [0, 3, 6])
    np.testing.assert_array_equal(f["left_abs"].numpy(), [1, -1, -1, 4, -1, -1])
    np.testing.assert_array_equal(f["right_abs"].numpy(), [2, -1, -1, 5, -1, -1])
    np.testing.assert_array_equal(f["feature"].numpy(), [2, -1, -1, 2, -1, -1])
    np.testing.assert_array_equal(f["is_leaf"].numpy(), [0, 1, 1, 0, 1, 1])
    assert f["value"].dtype == torch.float32


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in r.stderr


@pytest.mark.parametrize("max_bins", [2, 128, 255])
def test_prebinned_detection_and_range(max_bins):
    from packboost_amd.data import preprocess_features

    X = np.random.default_rng(1).integers(0, max_bins, size=(50, 4)).astype(np.int64)
    res = preprocess_features(X, max_bins)
    np.testing.assert_array_equal(res.bins, X.astype(np.uint8))
    assert res.bins.dtype == np.uint8


def test_draw_window_matches_sequential_draws():
    """Round r+1's subsets are window(p_r, 2D)[d_r : d_r + D] (what pb_select_subsets picks),
    equal to drawing sequentially with the generator left after round r's d_r draws; the final
    rewind leaves the generator exactly after the consumed draws."""
    import torch

    from packboost_amd.engine import _DrawStream

    F, K, D = 37, 5, 4
    depths = [4, 2, 4, 1, 3, 4, 1]  # subsets each round drew
    # sequential: each round looks at D draws, then keeps only the d it took
    seq = torch.Generator().manual_seed(11)
    expected_rounds = []
    for d in depths:
        state = seq.get_state()
        subs = [torch.randperm(F, generator=seq)[:K].numpy() for _ in range(D)]
        expected_rounds.append(np.stack(subs))
        seq.set_state(state)
        for _ in range(d):
            torch.randperm(F, generator=seq)
    rng = torch.Generator().manual_seed(11)
    ds = _DrawStream(rng, F, K)
    p, prev = 0, 0
    for r, d in enumerate(depths):
        start = p - prev  # window of round r begins at p_{r-1}; offset prev = d_{r-1}
        win = ds.window(start, 2 * D)
        np.testing.assert_array_equal(win[prev: prev + D], expected_rounds[r])
        p, prev = p + d, d
        ds.release(p - d)
    ds.rewind_to(p)
    assert torch.equal(rng.get_state(), seq.get_state())


def test_build_rejects_spilling_hot_kernels():
    """packboost_amd.build fails a build in which a histogram, scorer or K-cut kernel spills
    registers (hipcc's kernel-resource-usage remarks report its scratch), and lets other kernels
    keep scratch arrays."""
    from packboost_amd.build import spilling_kernels

    r = "\n".join([
        "a.hip:1:1: remark: Function Name: _ZN2pb12_GLOBAL__N_115hist_era_kernelILi16ELi1ELb0ELi256EEEvNS_8HistArgsE",
        "a.hip:1:1: remark:     ScratchSize [bytes/lane]: 20 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:2:1: remark: Function Name: _ZN2pb12_GLOBAL__N_117forest_tile_kernelEv",
        "a.hip:2:1: remark:     ScratchSize [bytes/lane]: 5136 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:5:1: remark: Function Name: _ZN2pb12_GLOBAL__N_112kcuts_kernelEPKt",
        "a.hip:5:1: remark:     ScratchSize [bytes/lane]: 16 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:3:1: remark: Function Name: _ZN2pb12_GLOBAL__N_116seg_score_kernelILi4ELb0ELb1EEEvNS_12SegScoreArgsE",
        "a.hip:3:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
        "a.hip:4:1: remark: Function Name: _ZN2pb12_GLOBAL__N_120des_score_pcu_kernelILb0ELi8ELi2EEEvNS_9ScoreArgsE",
        "a.hip:4:1: remark:     ScratchSize [bytes/lane]: 8 [-Rpass-analysis=kernel-resource-usage]",
    ])
    assert spilling_kernels(r) == [
        "_ZN2pb12_GLOBAL__N_115hist_era_kernelILi16ELi1ELb0ELi256EEEvNS_8HistArgsE",
        "_ZN2pb12_GLOBAL__N_112kcuts_kernelEPKt",
        "_ZN2pb12_GLOBAL__N_120des_score_pcu_kernelILb0ELi8ELi2EEEvNS_9ScoreArgsE",
    ]
