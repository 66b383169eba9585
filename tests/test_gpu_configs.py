"""GPU parity at BASELINE configs 3, 4 and 5 at their real workloads (configs 2 and 3 against
the oracle's whole rounds: tests/test_gpu_fixture_rounds.py).

- Config 4 (1,000,000 x 500, 255 bins, 200 eras): one depth-7 step at full size (128 nodes,
  node-tiled histogram), checked through size-independent properties: era totals against
  row counts and float64 sums, monotone prefixes, sampled cells against NumPy bincounts, the
  oracle scorer on the whole device planes of sampled nodes (every candidate bit-identical,
  the decision equal), every node's decision a top-scoring device candidate, and the
  partition rule with exact left/right counts.
- Config 4 whole rounds: 3 rounds of the full workload (B 64, D 8) in segment mode (fused
  kernel from depth 3, the default there) and on the plane path: every decision record and the
  training predictions bit-identical.
- Config 3 whole rounds: 3 rounds of the full 2.4M x 2376 panel (574 eras, 5 bins, B 8, D 6,
  238 features per depth, DRO 0.5) on the plane path over the nibble bins and in segment mode
  (the fused kernel over the uint8 bins from depth 2): two independent device paths, every
  decision record and the training predictions bit-identical.
- Config 5 (5,000,000 x 2376 uint8 bins, 250 packs x 8 distinct depth-6 trees): the full
  prediction, compared on a 50,000-row sample with the oracle's tree-order float32 sum
  (booster.py:709-712) within 1e-5, and leaf indices of every tree bit-exact on that sample
  (booster.py:131-169).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from tests.helpers import PB_INACTIVE, GpuDepth, compare_fit_rounds, split_params

pytestmark = pytest.mark.gpu


# ----------------------------------------------------------------------------- config 4
N4, F4, E4, NB4, U4, D4 = 1_000_000, 500, 200, 255, 128, 7


def test_config4_depth7_fullsize(hip, oracle_mod):
    import torch

    rng = np.random.default_rng(44)
    ld = (N4 + 15) // 16 * 16
    print(f"[config4] {N4} x {F4} bins, {NB4} levels, depth {D4} with {U4} nodes", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(44)
    bins = torch.randint(0, NB4, (F4, ld), dtype=torch.uint8, device="cuda", generator=g)
    bins[:, N4:] = 0
    sizes = np.array([len(a) for a in np.array_split(np.arange(N4), E4)], dtype=np.int64)
    offs = np.zeros(E4 + 1, np.int64)
    np.cumsum(sizes, out=offs[1:])
    era = np.repeat(np.arange(E4), sizes)
    grad = rng.standard_normal(N4).astype(np.float32)
    nid = rng.integers(0, U4, N4).astype(np.uint16)
    nid[rng.random(N4) < 0.05] = PB_INACTIVE
    p = {"N": N4, "F": F4, "E": E4, "nb": NB4, "U": U4, "era_off": offs.astype(np.int32), "grad": grad,
         "nid": nid, "era": era, "bins": None}
    feats = rng.permutation(F4).astype(np.int32)  # frac 1.0: all 500 features
    K = F4
    kw = dict(lambda_l2=1e-6, lambda_dro=0.0, direction_weight=0.0, era_alpha=0.0, min_samples_leaf=20)
    gd = GpuDepth(hip, p, K, msl=20, depth=D4, max_depth=D4 + 1, layout="u8", bins_dev=bins)
    try:
        assert gd.max_nodes == U4
        gd.hist(feats)
        torch.cuda.synchronize()
        T = NB4 - 1
        M = gd.max_nodes
        cells = E4 * M * K * T
        tot = (cells + 63) // 64 * 64
        cnt16 = gd.cnt.view(torch.int16)
        gflat = gd.g

        def plane_slice(e_idx, u, ks):
            """Prefix planes [len(e_idx)][len(ks)][nb] (total at nb-1) of node u, from the device."""
            e_t = torch.as_tensor(np.asarray(e_idx), device="cuda").long()
            k_t = torch.as_tensor(np.asarray(ks), device="cuda").long()
            base = ((e_t[:, None] * M + u) * K + k_t[None, :]) * T  # [e, k]
            idx = base[:, :, None] + torch.arange(T, device="cuda")[None, None, :]
            c = (cnt16[idx].int() & 0xFFFF).cpu().numpy().astype(np.int64)
            gg = gflat[idx].cpu().numpy()
            ct = gd.cnt[tot + e_t * M + u].cpu().numpy().astype(np.int64)
            gt = gflat[tot + e_t * M + u].cpu().numpy()
            c = np.concatenate([c, np.repeat(ct[:, None, None], len(ks), axis=1)], axis=2)
            gg = np.concatenate([gg, np.repeat(gt[:, None, None], len(ks), axis=1)], axis=2)
            return c, gg

        # era totals against row counts and float64 sums
        act = nid != PB_INACTIVE
        want_tot = np.zeros((E4, U4), np.int64)
        np.add.at(want_tot, (era[act], nid[act].astype(np.int64)), 1)
        got_tot = gd.cnt[tot: tot + E4 * M].cpu().numpy().reshape(E4, M)[:, :U4]
        np.testing.assert_array_equal(got_tot, want_tot)
        gsum = np.zeros((E4, U4))
        gabs = np.zeros((E4, U4))
        np.add.at(gsum, (era[act], nid[act].astype(np.int64)), grad[act].astype(np.float64))
        np.add.at(gabs, (era[act], nid[act].astype(np.int64)), np.abs(grad[act]).astype(np.float64))
        gtot = gflat[tot: tot + E4 * M].cpu().numpy().reshape(E4, M)[:, :U4]
        assert np.all(np.abs(gtot - gsum) <= 1e-5 * gabs)

        # sampled cells: monotone prefixes and NumPy bincounts of the same rows
        print("[config4] sampled cells", flush=True)
        for e in rng.choice(E4, 3, replace=False):
            r0, r1 = int(offs[e]), int(offs[e + 1])
            cols = bins[:, r0:r1].cpu().numpy()  # [F, rows]
            u_e = nid[r0:r1].astype(np.int64)
            g_e = grad[r0:r1].astype(np.float64)
            for u in rng.choice(U4, 3, replace=False):
                c, gg = plane_slice([e], int(u), np.arange(K))
                assert np.all(np.diff(c[0], axis=1) >= 0)
                m = u_e == u
                for k in range(K):
                    b = cols[feats[k], m]
                    np.testing.assert_array_equal(c[0, k], np.cumsum(np.bincount(b, minlength=NB4)))
                    gs = np.cumsum(np.bincount(b, weights=g_e[m], minlength=NB4))
                    ms = np.cumsum(np.bincount(b, weights=np.abs(g_e[m]), minlength=NB4))
                    assert np.all(np.abs(gg[0, k] - gs) <= 1e-5 * ms)

        # scorer: every candidate of sampled nodes bit-identical to the oracle scorer on the
        # device planes, and the decisions
        print("[config4] scorer and decisions", flush=True)
        params = split_params(hip, **{k: v for k, v in kw.items() if k != "min_samples_leaf"}, msl=20)
        gd.feats = torch.from_numpy(feats).cuda()
        cand_all = torch.zeros(M * K * T * 32, dtype=torch.uint8, device="cuda")
        hip.check(gd.lib.pb_des_score(gd.ctx, gd.cnt.data_ptr(), gd.g.data_ptr(), gd.feats.data_ptr(), K,
                                      gd.depth, M, ctypes.byref(params), cand_all.data_ptr(),
                                      hip.stream_ptr()), "pb_des_score")
        dec = gd.decide(params)
        cv = cand_all.view(torch.int32).view(M, K, T, 8)
        score_all = cv[:U4, :, :, 0].view(torch.float32)
        lt_all = cv[:U4, :, :, 1]
        valid_all = cv[:U4, :, :, 5] != 0
        for u in rng.choice(U4, 3, replace=False):
            u = int(u)
            c, gg = plane_slice(np.arange(E4), u, np.arange(K))
            sp = oracle_mod.score_planes(c[:, None], gg[:, None], feats, None, **kw)
            v = sp["valid"][0].astype(bool)
            np.testing.assert_array_equal(valid_all[u].cpu().numpy(), v)
            np.testing.assert_array_equal(score_all[u].cpu().numpy()[v].view(np.uint32),
                                          sp["score"][0][v].view(np.uint32))
            np.testing.assert_array_equal(lt_all[u].cpu().numpy()[v], sp["left_total"][0][v])
            assert dec["split"][u] == (1 if sp["best_feature"][0] >= 0 else 0)
            if dec["split"][u]:
                assert (dec["feature"][u], dec["threshold"][u]) == (sp["best_feature"][0], sp["best_threshold"][0])
        best = torch.where(valid_all, score_all, torch.tensor(float("-inf"), device="cuda")).amax(dim=(1, 2)).cpu().numpy()
        pos = {int(f): k for k, f in enumerate(feats)}
        for u in range(U4):
            if not dec["split"][u]:
                assert not np.isfinite(best[u])
                continue
            k = pos[int(dec["feature"][u])]
            t = int(dec["threshold"][u])
            assert bool(valid_all[u, k, t])
            assert abs(float(score_all[u, k, t]) - float(best[u])) <= 1e-12 * 64
            assert int(lt_all[u, k, t]) == dec["left_count"][u]
            assert dec["left_count"][u] + dec["right_count"][u] == want_tot[:, u].sum()

        # partition rule on every row of the split nodes
        print("[config4] partition", flush=True)
        nid_after, tn_after = gd.partition()
        used = np.unique(dec["feature"][dec["split"] == 1])
        colmap = {int(f): bins[int(f), :N4].cpu().numpy() for f in used}
        exp_tn = np.zeros(N4, np.int64)
        exp_tn[act] = gd.node_ids[nid[act].astype(np.int64)]
        for u in range(U4):
            if not dec["split"][u]:
                continue
            rows = np.nonzero(nid == u)[0]
            side = (colmap[int(dec["feature"][u])][rows] > dec["threshold"][u]).astype(np.int64)
            exp_tn[rows] = dec["left_id"][u] + side
            assert int(np.sum(side == 0)) == dec["left_count"][u]
        np.testing.assert_array_equal(tn_after.astype(np.int64), exp_tn)
    finally:
        gd.close()
        del bins
        torch.cuda.empty_cache()


# ----------------------------------------------------------------------------- config 5
def test_config4_rounds_segments_match_planes(hip):
    """Config 4's whole rounds (B 64, D 8, 1M x 500, 255 bins, 200 eras) in segment mode and on
    the plane path of the same data: the decision logs and predictions are equal bit for bit."""
    import torch

    from packboost_amd import PackBoostConfig
    from packboost_amd.engine import DeviceFit

    ld = (N4 + 15) // 16 * 16
    g = torch.Generator(device="cuda")
    g.manual_seed(45)
    bins = torch.randint(0, NB4, (F4, ld), dtype=torch.uint8, device="cuda", generator=g)
    bins[:, N4:] = 0
    noise = torch.randn(N4, device="cuda", generator=g)
    b0, b1, b2 = (bins[k, :N4].float() for k in (0, 1, 2))
    y = ((b0 - 127.0) / 128.0 + 0.5 * (b1 > 100).float() - 0.3 * (b2 < 40).float() + 0.5 * noise).contiguous()
    sizes = np.array([len(a) for a in np.array_split(np.arange(N4), E4)], dtype=np.int64)
    offs = np.zeros(E4 + 1, np.int64)
    np.cumsum(sizes, out=offs[1:])
    cfg = PackBoostConfig(pack_size=64, max_depth=8, learning_rate=0.1, lambda_l2=1e-6, lambda_dro=0.0,
                          min_samples_leaf=20, max_bins=NB4, layer_feature_fraction=1.0, random_state=42,
                          prebinned=True)
    out = {}
    for mode in ("segments", "planes"):
        print(f"[config4 rounds] {mode}", flush=True)
        fit = DeviceFit(bins, N4, y, offs.astype(np.int32), cfg, fit_mode=mode)
        try:
            assert fit.segments == (mode == "segments")
            if mode == "segments":
                assert fit.seg_from == 3
            logs = [log.decisions.copy() for log, _, _ in fit.rounds(torch.Generator().manual_seed(7), 3)]
            torch.cuda.synchronize()
            out[mode] = (logs, fit.preds[:N4].cpu().numpy().copy())
        finally:
            fit.close()
    seg_logs, seg_preds = out["segments"]
    pl_logs, pl_preds = out["planes"]
    for r, (a, b) in enumerate(zip(seg_logs, pl_logs)):
        assert a.tobytes() == b.tobytes(), f"round {r}: decision records differ"
    assert int(np.count_nonzero(pl_logs[0]["split"])) > 64  # the trees grow past depth 6
    np.testing.assert_array_equal(seg_preds, pl_preds)


def test_config3_rounds_segments_match_planes(hip, monkeypatch):
    """The headline workload's whole rounds through the plane path (nibble bins, joint-bin
    histograms, the producer/consumer scorer) and through segment mode (the fused kernel from
    depth 2): the decision logs and the training predictions are equal bit for bit."""
    import torch

    from packboost_amd import PackBoostConfig
    from packboost_amd.engine import DeviceFit

    N, F, E, nb = 2_400_000, 2376, 574, 5
    ld = (N + 15) // 16 * 16
    g = torch.Generator(device="cuda")
    g.manual_seed(33)
    bins = torch.randint(0, nb, (F, ld), dtype=torch.uint8, device="cuda", generator=g)
    bins[:, N:] = 0
    sizes = np.array([len(a) for a in np.array_split(np.arange(N), E)], dtype=np.int64)
    offs = np.zeros(E + 1, np.int64)
    np.cumsum(sizes, out=offs[1:])
    era_id = torch.from_numpy(np.repeat(np.arange(E), sizes)).cuda()
    rng = np.random.default_rng(33)
    sel = rng.permutation(F)[:50]
    w = rng.standard_normal(50)
    flip = torch.from_numpy(np.where(rng.random((E, 10)) < 0.5, -1.0, 1.0).astype(np.float32)).cuda()
    lin = torch.zeros(N, device="cuda")
    for j in range(50):
        col = bins[int(sel[j]), :N].float() - 2.0
        lin += float(w[j]) * col * (flip[era_id, j] if j < 10 else 1.0)
    lin += 0.5 * float(lin.std()) * torch.randn(N, device="cuda", generator=g)
    q = torch.quantile(lin[::12], torch.tensor([0.2, 0.4, 0.6, 0.8], device="cuda"))
    y = (torch.bucketize(lin, q).float() / 4.0).contiguous()
    cfg = PackBoostConfig(pack_size=8, max_depth=6, learning_rate=0.01, lambda_l2=1e-6, lambda_dro=0.5,
                          min_samples_leaf=20, max_bins=nb, layer_feature_fraction=0.1, random_state=42,
                          prebinned=True)
    out = {}
    for mode in ("planes", "segments"):
        print(f"[config3 rounds] {mode}", flush=True)
        monkeypatch.setenv("PB_SEG_FROM_DEPTH", "2")
        fit = DeviceFit(bins, N, y, offs.astype(np.int32), cfg, fit_mode=mode)
        try:
            assert fit.segments == (mode == "segments") and fit.bins4 is not None
            logs = [log.decisions.copy() for log, _, _ in fit.rounds(torch.Generator().manual_seed(5), 3)]
            torch.cuda.synchronize()
            out[mode] = (logs, fit.preds[:N].cpu().numpy().copy())
        finally:
            fit.close()
    for r, (a, b) in enumerate(zip(out["segments"][0], out["planes"][0])):
        assert a.tobytes() == b.tobytes(), f"round {r}: decision records differ"
    assert int(np.count_nonzero(out["planes"][0][0]["split"])) >= 32  # deep trees
    np.testing.assert_array_equal(out["segments"][1], out["planes"][1])


def test_config5_predict(hip, oracle_mod):
    import torch

    from packboost_amd.booster import pack_forest
    from packboost_amd.predictor import CompiledForest
    from tests.test_gpu_forest import _forest

    N, F, D, T = 5_000_000, 2376, 6, 2000
    tw = 0.01
    print(f"[config5] {N} x {F} bins, {T} depth-{D} trees", flush=True)
    ld = (N + 15) // 16 * 16
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    bins = torch.randint(0, 5, (F, ld), dtype=torch.uint8, device="cuda", generator=g)
    rounds = _forest(55, T, 1, D, F)  # 250 packs x 8 distinct trees
    forest = CompiledForest(pack_forest(rounds, 1, torch.device("cuda")))
    try:
        out = forest.predict(bins, N, tw).cpu().numpy()
        rng = np.random.default_rng(5)
        idx = np.sort(rng.choice(N, 50_000, replace=False))
        sub = bins[:, torch.from_numpy(idx).cuda()].contiguous()  # [F, 50000]
        sample = sub.t().contiguous().cpu().numpy()  # row-major for the oracle
        print("[config5] oracle on the sample", flush=True)
        want = oracle_mod.predict(rounds, 1, tw, sample)
        np.testing.assert_allclose(out[idx], want, rtol=0, atol=1e-5)
        n = idx.size
        ld_s = (n + 15) // 16 * 16
        bs = torch.zeros((F, ld_s), dtype=torch.uint8, device="cuda")
        bs[:, :n] = sub
        leaves = torch.empty((T, n), dtype=torch.int32, device="cuda")
        out_s = forest.predict(bs, n, tw, leaves=leaves).cpu().numpy()
        np.testing.assert_array_equal(out_s, out[idx])
        offs = np.asarray([0] + [len(r["feature"]) for r in rounds]).cumsum()
        lv = leaves.cpu().numpy()
        for t, arrs in enumerate(rounds):
            np.testing.assert_array_equal(lv[t] - offs[t], oracle_mod.leaf_index(arrs, sample))
    finally:
        forest.close()
        del bins
        torch.cuda.empty_cache()
