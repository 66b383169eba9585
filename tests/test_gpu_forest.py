"""Compiled-forest prediction (pb_forest_create / pb_forest_predict) on a config-5 style
forest (full depth-6 trees, random features and thresholds, leaves N(0, 0.01)) against the
per-row walk of pb_predict_forest and the CPU oracle (booster.py:131-169, 709-712):
predictions within 1e-5 of the oracle's float32 tree-order sum (the per-row walk bit-identical
to pb_predict_forest, the tiled walk within 1e-5 of it); leaf indices bit-exact. Malformed
forests are rejected."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _forest(seed, packs, B, D, F, ragged=False, max_thr=3):
    rng = np.random.default_rng(seed)
    n_nodes = (1 << (D + 1)) - 1
    inner = (1 << D) - 1
    rounds = []
    for p in range(packs):
        idx = np.arange(n_nodes)
        leaf = idx >= inner
        if ragged and p % 2 and D >= 2:  # a shallower tree: depth-2 subtree under the root's right child
            leaf = leaf | ((idx >= 3) & (idx % 2 == 0))
        r = {"feature": np.where(leaf, -1, rng.integers(0, F, n_nodes)),
             "threshold": np.where(leaf, 0, rng.integers(0, max_thr + 1, n_nodes)),
             "left": np.where(leaf, -1, 2 * idx + 1), "right": np.where(leaf, -1, 2 * idx + 2),
             "value": np.where(leaf, rng.normal(0.0, 0.01, n_nodes), 0.0), "is_leaf": leaf}
        rounds.append(r)
    return rounds


@pytest.mark.parametrize("B", [8, 1], ids=["packs", "distinct"])
@pytest.mark.parametrize("tile", [1, 0], ids=["tiled", "per-row"])
@pytest.mark.parametrize("ragged", [False, True])
def test_compiled_forest(hip, oracle_mod, monkeypatch, ragged, tile, B):
    """tile 1: the tiled walk (double sums rounded once; the tree-order float32 sum of
    pb_predict_forest carries up to T float32 roundings, so the two agree to 1e-5); tile 0: the
    per-row walk, bit-identical to pb_predict_forest. B 8: each pack repeats one tree 8 times,
    which the tiled walk holds once with its count; B 1: every tree distinct (no counts)."""
    import torch

    monkeypatch.setenv("PB_FOREST_TILE", str(tile))
    from packboost_amd.booster import pack_forest
    from packboost_amd.predictor import CompiledForest

    N, F, D = 20011, 300, 6
    print(f"[forest] ragged={ragged} tile={tile} B={B}", flush=True)
    rounds = _forest(3, 25, B, D, F, ragged)
    rng = np.random.default_rng(4)
    bins = rng.integers(0, 5, size=(N, F), dtype=np.uint8)
    dev = torch.device("cuda")
    ld = (N + 15) // 16 * 16
    bfm = torch.zeros((F, ld), dtype=torch.uint8, device=dev)
    bfm[:, :N] = torch.from_numpy(np.ascontiguousarray(bins.T)).to(dev)
    f = pack_forest(rounds, B, dev)
    T = int(f["offsets"].numel() - 1)
    cf = CompiledForest(f)
    leaves = torch.empty((T, N), dtype=torch.int32, device=dev)
    got = cf.predict(bfm, N, 0.5, leaves=leaves).cpu().numpy()
    lib = hip.load()
    ref = torch.empty(N, dtype=torch.float32, device=dev)
    hip.check(lib.pb_predict_forest(bfm.data_ptr(), N, ld, F, f["feature"].data_ptr(),
                                    f["threshold"].data_ptr(), f["left_abs"].data_ptr(),
                                    f["right_abs"].data_ptr(), f["value"].data_ptr(),
                                    f["is_leaf"].data_ptr(), f["offsets"].data_ptr(), T,
                                    int(f["value"].numel()), 0.5, ref.data_ptr(), hip.stream_ptr()),
              "pb_predict_forest")
    if tile:
        np.testing.assert_allclose(got, ref.cpu().numpy(), rtol=0, atol=1e-5)
    else:
        np.testing.assert_array_equal(got, ref.cpu().numpy())
    np.testing.assert_allclose(got, oracle_mod.predict(rounds, B, 0.5, bins), rtol=0, atol=1e-5)
    lv = leaves.cpu().numpy() - f["offsets"][:-1].cpu().numpy()[:, None]
    for r, arrs in enumerate(rounds):
        want = oracle_mod.leaf_index(arrs, bins)
        for t in range(B):
            np.testing.assert_array_equal(lv[r * B + t], want)
    cf.close()


@pytest.mark.parametrize("D,F,max_thr,odd_ld", [
    (0, 7, 3, False), (1, 40, 3, False), (2, 300, 6, True), (3, 300, 14, False),
    (4, 1000, 14, False), (5, 700, 200, False), (7, 2376, 255, False), (8, 90, 3, False)])
def test_forest_shapes(hip, oracle_mod, D, F, max_thr, odd_ld):
    """The tiled walk at every depth it serves (0-8), all three tile packings (3 bits for
    thresholds < 7, 4 bits < 15, else 8), 64- and 32-row tiles (2376 features at 8 bits do not
    fit two 64-row tiles per CU), a tree count that leaves the last tree block part-filled, and
    an odd row stride (the per-row walk then serves the call): predictions within 1e-5 of the
    oracle, leaf indices bit-exact."""
    import torch

    from packboost_amd.booster import pack_forest
    from packboost_amd.predictor import CompiledForest

    N, B = 3001, 4
    packs = 13 if D <= 6 else 3
    print(f"[forest-shape] D={D} F={F} max_thr={max_thr} odd_ld={odd_ld}", flush=True)
    rounds = _forest(11 + D, packs, B, D, F, ragged=True, max_thr=max_thr)
    rng = np.random.default_rng(12 + D)
    bins = rng.integers(0, min(max_thr + 2, 256), size=(N, F)).astype(np.uint8)
    dev = torch.device("cuda")
    ld = N if odd_ld else (N + 15) // 16 * 16
    bfm = torch.zeros((F, ld), dtype=torch.uint8, device=dev)
    bfm[:, :N] = torch.from_numpy(np.ascontiguousarray(bins.T)).to(dev)
    f = pack_forest(rounds, B, dev)
    T = int(f["offsets"].numel() - 1)
    cf = CompiledForest(f)
    leaves = torch.empty((T, N), dtype=torch.int32, device=dev)
    got = cf.predict(bfm, N, 0.25, leaves=leaves).cpu().numpy()
    np.testing.assert_allclose(got, oracle_mod.predict(rounds, B, 0.25, bins), rtol=0, atol=1e-5)
    plain = cf.predict(bfm, N, 0.25).cpu().numpy()  # the walk without leaf output
    np.testing.assert_array_equal(plain, got)
    lv = leaves.cpu().numpy() - f["offsets"][:-1].cpu().numpy()[:, None]
    for r, arrs in enumerate(rounds):
        want = oracle_mod.leaf_index(arrs, bins)
        for t in range(B):
            np.testing.assert_array_equal(lv[r * B + t], want)
    cf.close()


def test_forest_rejects_malformed(hip):
    import torch

    from packboost_amd.booster import pack_forest

    rounds = _forest(5, 1, 1, 2, 10)
    rounds[0]["left"] = rounds[0]["left"].copy()
    rounds[0]["left"][1] = 0  # child points back to the root: a cycle
    f = pack_forest(rounds, 1, torch.device("cuda"))
    lib = hip.load()
    h = ctypes.c_void_p()
    rc = lib.pb_forest_create(f["feature"].data_ptr(), f["threshold"].data_ptr(),
                              f["left_abs"].data_ptr(), f["right_abs"].data_ptr(),
                              f["value"].data_ptr(), f["is_leaf"].data_ptr(), f["offsets"].data_ptr(),
                              1, int(f["value"].numel()), ctypes.byref(h))
    assert rc == -1 and not h.value
    assert b"malformed" in lib.pb_last_error()
