"""Nibble bin layout (pb_pack_bins4) and the histogram / partition reads of it in
pb_grow_round, for max_bins <= 16.

Bars: the packed bytes equal the layout's definition bit for bit; fits through the nibble
layout grow the same trees as through the uint8 layout (feature, threshold, children, leaf
flags bit-exact; values and predictions bit-exact, since both layouts feed the same exact
fixed-point sums) and match the oracle's restatement of the reference fit.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.test_gpu_fit import _compare_rounds, config1_data

pytestmark = pytest.mark.gpu


def _expected_pack4(bins_fm: np.ndarray, n: int) -> np.ndarray:
    F, ld = bins_fm.shape
    b = bins_fm.copy()
    b[:, n:] = 0
    g = b.reshape(F, ld // 8, 2, 4)  # [F, group, half, byte]
    return ((g[:, :, 0, :] & 0xF) | ((g[:, :, 1, :] & 0xF) << 4)).reshape(F, ld // 2).astype(np.uint8)


@pytest.mark.parametrize("F,ld,n", [(1, 16, 16), (7, 4096, 4001), (33, 16 * 1001, 16 * 1001 - 9),
                                    (3, 64, 0)])
def test_pack_bins4_layout(hip, F, ld, n):
    import torch
    from packboost_amd.backends import _hip

    print(f"[pack4] F={F} ld={ld} n={n}", flush=True)
    rng = np.random.default_rng(F * 31 + ld)
    bins = rng.integers(0, 16, size=(F, ld), dtype=np.uint8)
    bins[:, n:] = 0xFF  # padding the caller never initialised
    dev = torch.device("cuda")
    src = torch.from_numpy(bins).to(dev)
    out = torch.full((F, ld // 2), 0xAB, dtype=torch.uint8, device=dev)
    lib = _hip.load()
    _hip.check(lib.pb_pack_bins4(src.data_ptr(), n, ld, F, out.data_ptr(), _hip.stream_ptr()),
               "pb_pack_bins4")
    got = out.cpu().numpy()
    np.testing.assert_array_equal(got, _expected_pack4(bins, n))
    # row r of a column sits in byte (r // 8) * 4 + r % 4, high nibble iff r % 8 >= 4
    r = np.arange(ld)
    nib = (got[:, (r // 8) * 4 + r % 4] >> np.where(r % 8 >= 4, 4, 0)) & 0xF
    np.testing.assert_array_equal(nib[:, :n], bins[:, :n])
    assert not nib[:, n:].any()
    assert lib.pb_pack_bins4(src.data_ptr(), n, ld + 8, F, out.data_ptr(), None) < 0  # ld % 16
    assert lib.pb_pack_bins4(src.data_ptr(), ld + 1, ld, F, out.data_ptr(), None) < 0  # n > ld


def _device_fit_trees(bins, y, off, cfg, layout, rounds):
    import torch
    from packboost_amd.engine import DeviceFit, tree_arrays_from_log

    N, F = bins.shape
    ld = (N + 15) // 16 * 16
    fm = np.full((F, ld), 0xFF, np.uint8)  # padding rows hold garbage
    fm[:, :N] = bins.T
    dev = torch.device("cuda")
    fit = DeviceFit(torch.from_numpy(fm).to(dev), N, torch.from_numpy(y).to(dev), off, cfg,
                    bin_layout=layout)
    assert (fit.bins4 is not None) == (layout == "nibble")
    trees = [tree_arrays_from_log(log, cfg, N)
             for log, _, _ in fit.rounds(torch.Generator().manual_seed(cfg.random_state), rounds)]
    preds = fit.preds[:N].cpu().numpy().copy()
    fit.close()
    return trees, preds


@pytest.mark.parametrize("nb,eras", [(5, 7), (16, 5), (3, 1), (12, 13)])
def test_nibble_fit_matches_u8_and_oracle(hip, oracle_mod, nb, eras):
    """Ragged eras (sizes not multiples of 8) exercise the 8-row alignment of era starts."""
    from packboost_amd import PackBoostConfig
    from packboost_amd.data import preprocess_features

    print(f"[nibble fit] nb={nb} eras={eras}", flush=True)
    X, y, _ = config1_data(seed=nb * 7 + eras, n=4003, f=14, eras=1)
    rng = np.random.default_rng(nb)
    cuts = np.sort(rng.choice(np.arange(1, 4003), eras - 1, replace=False))
    era = np.zeros(4003, np.int64)
    for c in cuts:
        era[c:] += 1
    cfg_kw = dict(pack_size=3, max_depth=5, learning_rate=0.1, lambda_l2=0.5, lambda_dro=0.3,
                  min_samples_leaf=6, max_bins=nb, layer_feature_fraction=0.8, random_state=5)
    cfg = PackBoostConfig(**cfg_kw, prebinned=True)
    bins = preprocess_features(X, nb).bins
    off = np.concatenate([[0], np.cumsum(np.bincount(era, minlength=eras))]).astype(np.int32)
    rounds = 4
    t8, p8 = _device_fit_trees(bins, y, off, cfg, "u8", rounds)
    t4, p4 = _device_fit_trees(bins, y, off, cfg, "nibble", rounds)
    for a, b in zip(t8, t4):
        for key in ("feature", "threshold", "left", "right", "is_leaf", "value"):
            np.testing.assert_array_equal(np.asarray(a[key]), np.asarray(b[key]), err_msg=key)
    np.testing.assert_array_equal(p8, p4)
    ref = oracle_mod.fit(bins, y, era, num_rounds=rounds, **cfg_kw)
    _compare_rounds(t4, ref.rounds)
    np.testing.assert_allclose(p4, ref.preds, atol=1e-5, rtol=0)


def test_nibble_rejected_above_16_bins(hip):
    import torch
    from packboost_amd import PackBoostConfig
    from packboost_amd.engine import DeviceFit

    cfg = PackBoostConfig(max_bins=17, max_depth=2, pack_size=1, prebinned=True)
    fm = torch.zeros((2, 64), dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError, match="max_bins <= 16"):
        DeviceFit(fm, 64, torch.zeros(64, device="cuda"), np.array([0, 64], np.int32), cfg,
                  bin_layout="nibble")
