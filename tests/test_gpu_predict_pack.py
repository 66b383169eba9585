"""pb_predict_pack through the reference's shim name predict_pack_cuda
(frontier_cuda.cu:989-1068): out[r] = tree_weight * sum over the pack's B trees of the leaf
value reached by row r (left iff bin <= threshold), on feature-major int8/uint8 bins [F, N].

Bars: leaf indices (absolute, per tree) bit-exact against the oracle's walk of each tree
(booster.py:131-169); outputs within 1e-5 of tree_weight times the float64 sum of the
oracle's leaf values."""

from __future__ import annotations

import numpy as np
import pytest

from tests.test_gpu_forest import _forest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,B,D,ragged,int8", [
    (20011, 8, 6, False, False),    # config-5 style pack: full depth-6 trees
    (7777, 8, 5, True, True),       # ragged trees, int8 bins as the reference passes them
    (64, 64, 4, False, False),      # a wide pack (B = 64, config 4's pack size)
    (1, 3, 2, True, False),
], ids=["full-d6", "ragged-int8", "wide-pack", "one-row"])
def test_predict_pack_matches_oracle(hip, oracle_mod, N, B, D, ragged, int8):
    import torch

    from packboost_amd.backends import predict_pack_cuda
    from packboost_amd.booster import pack_forest

    print(f"[predict_pack] N={N} B={B} D={D} ragged={ragged} int8={int8}", flush=True)
    F = 300
    rounds = _forest(N + B, B, 1, D, F, ragged)  # B distinct trees, packed as one pack
    rng = np.random.default_rng(N)
    bins = rng.integers(0, 5, size=(N, F), dtype=np.uint8)
    dev = torch.device("cuda")
    f = pack_forest(rounds, 1, dev)
    fm = torch.from_numpy(np.ascontiguousarray(bins.T)).to(dev)
    if int8:
        fm = fm.view(torch.int8)
    tw = 0.37
    out = predict_pack_cuda(fm, f["feature"], f["threshold"], f["left_abs"], f["right_abs"],
                            f["value"], f["is_leaf"], f["offsets"], tw).cpu().numpy()
    want = np.zeros(N, np.float64)
    for arrs in rounds:
        want += arrs["value"][oracle_mod.leaf_index(arrs, bins)]
    np.testing.assert_allclose(out.astype(np.float64), tw * want, rtol=0, atol=1e-5)

    # leaf dump of the same call through the C ABI
    lib = hip.load()
    ld = (N + 15) // 16 * 16
    bfm = torch.zeros((F, ld), dtype=torch.uint8, device=dev)
    bfm[:, :N] = torch.from_numpy(np.ascontiguousarray(bins.T)).to(dev)
    leaves = torch.full((B, N), -7, dtype=torch.int32, device=dev)
    out2 = torch.empty(N, dtype=torch.float32, device=dev)
    hip.check(lib.pb_predict_pack(bfm.data_ptr(), N, ld, F, f["feature"].data_ptr(), f["threshold"].data_ptr(),
                                  f["left_abs"].data_ptr(), f["right_abs"].data_ptr(), f["value"].data_ptr(),
                                  f["is_leaf"].data_ptr(), f["offsets"].data_ptr(), B, int(f["value"].numel()),
                                  tw, out2.data_ptr(), leaves.data_ptr(), hip.stream_ptr()), "pb_predict_pack")
    np.testing.assert_array_equal(out2.cpu().numpy(), out)
    offs = f["offsets"].cpu().numpy()
    lv = leaves.cpu().numpy()
    for t, arrs in enumerate(rounds):
        np.testing.assert_array_equal(lv[t] - offs[t], oracle_mod.leaf_index(arrs, bins))


def test_predict_pack_empty_and_errors(hip):
    import torch

    from packboost_amd.backends import predict_pack_cuda
    from packboost_amd.booster import pack_forest

    dev = torch.device("cuda")
    f = pack_forest(_forest(1, 2, 1, 3, 10), 1, dev)
    empty = predict_pack_cuda(torch.zeros((10, 0), dtype=torch.uint8, device=dev), f["feature"],
                              f["threshold"], f["left_abs"], f["right_abs"], f["value"], f["is_leaf"],
                              f["offsets"], 1.0)
    assert empty.numel() == 0
    # malformed trees end their walk with 0 (the reference's child guard): a split feature
    # outside [0, F), or a child outside the tree's span, at the first tree's root
    bins = torch.from_numpy(np.random.default_rng(2).integers(0, 5, (10, 37), dtype=np.uint8)).to(dev)
    args = ("feature", "threshold", "left_abs", "right_abs", "value", "is_leaf")
    second_only = predict_pack_cuda(bins, *(f[k] for k in args), f["offsets"][1:].contiguous(), 1.0)
    off1 = int(f["offsets"][1])
    for field, val in (("feature", 10), ("left_abs", off1 + 1)):
        bad = {k: v.clone() for k, v in f.items()}
        bad[field][0] = val
        if field == "left_abs":
            bad["right_abs"][0] = val
        got = predict_pack_cuda(bins, *(bad[k] for k in args), bad["offsets"], 1.0)
        np.testing.assert_array_equal(got.cpu().numpy(), second_only.cpu().numpy())
