"""The reference's row-list CUDA entry points (frontier_cuda.cu:576-716, 719-851), served by the
HIP kernels through packboost_amd.backends, against the oracle.

Split finder: per (node, feature) the chosen threshold equals the oracle's best threshold for
that feature (same tie-break) unless the oracle's scores of the two thresholds tie within 1e-6;
left counts bit-exact for the same threshold; scores within 1e-5. Partition: left/right row
lists and absolute per-era splits bit-exact against the rule bin <= threshold.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import make_problem, node_era_rows

pytestmark = pytest.mark.gpu


def _rowlist_inputs(p, ner):
    import torch

    rows, nrs, nes = [], [0], []
    for eras in ner:
        rel = [0]
        for r in eras:
            rows.append(r)
            rel.append(rel[-1] + r.size)
        nes.append(rel)
        nrs.append(nrs[-1] + rel[-1])
    dev = torch.device("cuda")
    rows = np.concatenate(rows).astype(np.int32)
    return (torch.from_numpy(rows).to(dev), torch.tensor(nrs, dtype=torch.int32, device=dev),
            torch.tensor(nes, dtype=torch.int32, device=dev))


def _oracle_per_feature(cands):
    """Best threshold per (node, feature) with the CUDA path's tie-break."""
    s, lt, _, v = cands
    U, K, T = s.shape
    best = np.full((U, K), -1)
    for u in range(U):
        for k in range(K):
            b, bs, bl = -1, -np.inf, -1
            for t in range(T):
                if not v[u, k, t]:
                    continue
                sc = float(s[u, k, t])
                better = sc > bs
                if not better and abs(sc - bs) <= 1e-12:
                    better = lt[u, k, t] > bl or (lt[u, k, t] == bl and t > b)
                if better:
                    b, bs, bl = t, sc, lt[u, k, t]
            best[u, k] = b
    return best


@pytest.mark.parametrize("case", [
    # seed, N, F, E, nb, U, K, msl, alpha, dir
    (1, 5000, 12, 6, 5, 3, 8, 10, 0.0, 0.0),
    (2, 8000, 20, 9, 32, 5, 12, 5, 1.5, 0.1),
    (3, 6000, 10, 4, 128, 2, 10, 20, 0.0, 0.0),
    (4, 60000, 6, 3, 5, 4200, 3, 2, 0.0, 0.0),
    # bins >= max_bins: left out of the histogram (frontier_cuda.cu:451, frontier_cpu.cpp:278-281)
    (5, 5000, 12, 6, 5, 3, 8, 10, 0.0, 0.0, True),
    (6, 8000, 20, 9, 32, 5, 12, 5, 1.5, 0.1, True),
    (7, 6000, 10, 4, 128, 2, 10, 20, 0.0, 0.0, True),
], ids=["nb5", "nb32_alpha_dir", "nb128", "4200_nodes_two_chunks", "skipped_nb5",
        "skipped_nb32_alpha_dir", "skipped_nb128"])
def test_split_finder_rowlist(hip, oracle_mod, case):
    import torch

    from packboost_amd import backends
    from tests.helpers import with_skipped_bins

    seed, N, F, E, nb, U, K, msl, alpha, dirw = case[:10]
    print(f"[rowlist split] {case}", flush=True)
    p = make_problem(seed, N, F, E, nb, U)
    if len(case) > 10 and case[10]:
        p = with_skipped_bins(p, seed)
    ner = node_era_rows(p)
    feats = np.random.default_rng(seed).permutation(F)[:K].astype(np.int32)
    ref = oracle_mod.split_batch(p["bins"], p["grad"], ner, feats, nb, lambda_l2=1e-3, lambda_dro=0.4,
                                 direction_weight=dirw, era_alpha=alpha, min_samples_leaf=msl,
                                 want_cands=True)
    dev = torch.device("cuda")
    rows, nrs, nes = _rowlist_inputs(p, ner)
    bins_fm = torch.from_numpy(np.ascontiguousarray(p["bins"].T)).to(dev)
    grad_c = torch.from_numpy(p["grad"]).to(dev)[rows.long()]
    counts = (nes[:, 1:] - nes[:, :-1]).float()
    w = torch.where(counts > 0, counts + alpha if alpha > 0 else torch.ones_like(counts),
                    torch.zeros_like(counts))
    out = backends.find_best_splits_batched_cuda(
        bins_fm, grad_c, torch.ones_like(grad_c), rows, nrs, nes, w,
        torch.zeros(U, device=dev), torch.zeros(U, device=dev), torch.zeros(U, dtype=torch.int64, device=dev),
        torch.from_numpy(feats).to(dev), nb, 0, "mass", 1e-3, 0.4, dirw, msl, int(rows.numel()))
    thr = out["thresholds"].cpu().numpy()
    lc = out["left_count"].cpu().numpy()
    sc = out["scores"].cpu().numpy()
    lg = out["left_grad"].cpu().numpy()
    lh = out["left_hess"].cpu().numpy()
    want = _oracle_per_feature(ref.cands)
    s_ref, lt_ref, lg_ref = ref.cands[0], ref.cands[1], ref.cands[2]
    for u in range(U):
        for k in range(K):
            if want[u, k] < 0:
                assert thr[u, k] == -1 and np.isneginf(sc[u, k])
                continue
            if thr[u, k] != want[u, k]:
                a, b = float(s_ref[u, k, thr[u, k]]), float(s_ref[u, k, want[u, k]])
                assert abs(a - b) <= 1e-6 * max(1.0, abs(b)), (u, k, thr[u, k], want[u, k])
                continue
            assert lc[u, k] == lt_ref[u, k, want[u, k]] and lh[u, k] == lc[u, k]
            g_ref = float(lg_ref[u, k, want[u, k]])
            assert abs(lg[u, k] - g_ref) <= 1e-5 * max(1.0, abs(g_ref)), (u, k)
            assert abs(sc[u, k] - s_ref[u, k, want[u, k]]) <= 1e-5 * max(1.0, abs(s_ref[u, k, want[u, k]]))


def test_partition_rowlist(hip):
    import torch

    from packboost_amd import backends

    p = make_problem(21, 7000, 9, 5, 16, 4)
    ner = node_era_rows(p)
    rows, nrs, nes = _rowlist_inputs(p, ner)
    dev = torch.device("cuda")
    bins_fm = torch.from_numpy(np.ascontiguousarray(p["bins"].T)).to(dev)
    feat = np.array([3, 0, 8, 5], np.int32)
    thr = np.array([7, 0, 15, 4], np.int32)
    out = backends.partition_frontier_cuda(bins_fm, rows, nrs, nes, torch.from_numpy(feat).to(dev),
                                           torch.from_numpy(thr).to(dev))
    li, ri = out["left_index"].cpu().numpy(), out["right_index"].cpu().numpy()
    ls, rs = out["left_splits"].cpu().numpy(), out["right_splits"].cpu().numpy()
    lpos = rpos = 0
    for u, eras in enumerate(ner):
        for e, r in enumerate(eras):
            go = p["bins"][r, feat[u]] <= thr[u]
            L, R = r[go], r[~go]
            assert ls[u, e] == lpos and rs[u, e] == rpos
            np.testing.assert_array_equal(li[lpos: lpos + L.size], L)
            np.testing.assert_array_equal(ri[rpos: rpos + R.size], R)
            lpos += L.size
            rpos += R.size
        assert ls[u, -1] == lpos and rs[u, -1] == rpos
    assert lpos == li.size and rpos == ri.size


def _partition_expect(bins_nf, rows, nrs, nes, feat, thr):
    """Stable per-segment split (frontier_cpu.cpp:446-497) in numpy, vectorised: rows sorted by
    (segment, side) with a stable sort keep list order inside each side."""
    S, E1 = nes.shape
    E = E1 - 1
    sizes = (nes[:, 1:] - nes[:, :-1]).reshape(-1)
    seg = np.repeat(np.arange(S * E), sizes)
    node = seg // E
    pos = np.concatenate([nrs[s] + np.arange(nes[s, 0], nes[s, E]) for s in range(S)]) if S else seg
    r = rows[pos]
    go = bins_nf[r, feat[node]].astype(np.int64) <= thr[node]
    left = r[go]
    right = r[~go]
    lc = np.bincount(seg[go], minlength=S * E).reshape(S, E)
    rc = sizes.reshape(S, E) - lc

    def absolute(c):
        flat = np.concatenate([[0], np.cumsum(c.reshape(-1))])
        return np.stack([flat[s * E: s * E + E + 1] for s in range(S)]).astype(np.int32)

    return left, right, absolute(lc), absolute(rc)


@pytest.mark.parametrize("case", [
    # seed, N, F, E, nb, S, int8 bins, shuffled lists
    (31, 3000, 4, 1, 8, 1, True, False),
    (32, 20000, 6, 7, 16, 300, False, True),
    (33, 1_500_000, 8, 500, 64, 64, False, True),
], ids=["one_node_one_era_int8", "300_nodes_shuffled", "1.5M_rows_500_eras"])
def test_partition_rowlist_shapes(hip, case):
    """Empty nodes, empty eras, thresholds that send every row one way (-1, nb-1, 255) and list
    orders that are not ascending, against the stable split in numpy."""
    import torch

    from packboost_amd import backends

    seed, N, F, E, nb, S, int8, shuffled = case
    print(f"[rowlist partition] {case}", flush=True)
    rng = np.random.default_rng(seed)
    bins_nf = rng.integers(0, nb, size=(N, F), dtype=np.uint8)
    node = rng.integers(-1, S, size=N)              # -1: the row is in no listed node
    if S > 2:
        node[node == 1] = -1                        # node 1 lists no rows
    era = np.sort(rng.integers(0, E, size=N))
    if E > 3:
        era[era == 2] = 3                           # era 2 is empty for every node
    rows, nrs, nes = [], [0], np.zeros((S, E + 1), np.int32)
    for s in range(S):
        mine = np.nonzero(node == s)[0]
        if shuffled:
            mine = rng.permutation(mine)
        mine = mine[np.argsort(era[mine], kind="stable")]
        rows.append(mine)
        nes[s, 1:] = np.cumsum(np.bincount(era[mine], minlength=E))
        nrs.append(nrs[-1] + mine.size)
    rows = np.concatenate(rows).astype(np.int32)
    nrs = np.array(nrs, np.int32)
    feat = rng.integers(0, F, size=S).astype(np.int32)
    thr = rng.integers(0, nb, size=S).astype(np.int32)
    thr[::5] = -1
    thr[1::5] = nb - 1
    thr[2::7] = 255
    dev = torch.device("cuda")
    b = torch.from_numpy(np.ascontiguousarray(bins_nf.T)).to(dev)
    if int8:
        b = b.view(torch.int8)
    out = backends.partition_frontier_cuda(b, torch.from_numpy(rows).to(dev), torch.from_numpy(nrs).to(dev),
                                           torch.from_numpy(nes).to(dev), torch.from_numpy(feat).to(dev),
                                           torch.from_numpy(thr).to(dev))
    left, right, ls, rs = _partition_expect(bins_nf, rows, nrs, nes, feat, thr)
    np.testing.assert_array_equal(out["left_splits"].cpu().numpy(), ls)
    np.testing.assert_array_equal(out["right_splits"].cpu().numpy(), rs)
    np.testing.assert_array_equal(out["left_index"].cpu().numpy(), left)
    np.testing.assert_array_equal(out["right_index"].cpu().numpy(), right)


@pytest.mark.parametrize("bad", ["row", "feature", "segment"])
def test_rowlist_rejects_bad_indices(hip, bad):
    """Out-of-range row ids, features and segments are caught by the kernels' own bounds checks
    (nothing is read or written out of range) and raised on the host."""
    import torch

    from packboost_amd import backends

    print(f"[rowlist bad input] {bad}", flush=True)
    dev = torch.device("cuda")
    rng = np.random.default_rng(5)
    N, F, E = 1000, 3, 2
    b = torch.from_numpy(rng.integers(0, 4, size=(F, N), dtype=np.uint8)).to(dev)
    rows = torch.arange(0, 600, dtype=torch.int32, device=dev)
    nrs = torch.tensor([0, 300, 600], dtype=torch.int32, device=dev)
    nes = torch.tensor([[0, 100, 300], [0, 150, 300]], dtype=torch.int32, device=dev)
    feat = torch.tensor([0, 2], dtype=torch.int32, device=dev)
    thr = torch.tensor([1, 2], dtype=torch.int32, device=dev)
    if bad == "row":
        rows[17] = N + 5
        msg = "row id"
    elif bad == "feature":
        feat[1] = F
        msg = "feature id"
    else:
        nes[1, 2] = 900
        msg = "segment"
    with pytest.raises(RuntimeError, match=msg):
        backends.partition_frontier_cuda(b, rows, nrs, nes, feat, thr)
    w = torch.ones((2, E), device=dev)
    g = torch.randn(600, device=dev)
    fid = torch.tensor([0, 1, 2], dtype=torch.int32, device=dev)
    if bad == "feature":
        fid[2] = F + 1
    z = torch.zeros(2, device=dev)
    with pytest.raises(RuntimeError, match=msg):
        backends.find_best_splits_batched_cuda(b, g, torch.ones_like(g), rows, nrs, nes, w, z, z,
                                               torch.zeros(2, dtype=torch.int64, device=dev), fid, 4, 0,
                                               "mass", 1e-3, 0.0, 0.0, 1, 600)


def test_best_thresholds_tie_break(hip):
    """pb_best_thresholds against frontier_cuda.cu:537-560's sequential pick, on records built
    to hit every branch: exact score ties broken by left count and then threshold, invalid
    records, -inf / +inf / NaN scores."""
    import ctypes

    import torch

    from packboost_amd.backends import _hip

    lib = hip.load()
    rng = np.random.default_rng(9)
    M, K, T = 40, 7, 9
    score = rng.choice(np.array([0.5, 0.25, 1.0, -2.0], np.float32), size=(M, K, T))
    left = rng.integers(1, 5, size=(M, K, T)).astype(np.int32)
    thr = np.tile(np.arange(T, dtype=np.int32), (M, K, 1))
    valid = (rng.random((M, K, T)) < 0.8).astype(np.int32)
    valid[0, 0] = 0                                       # nothing valid
    score[1, 0, :] = np.inf                               # +inf best
    score[1, 1, 3] = np.nan                               # NaN never wins
    score[1, 2, :] = -np.inf                              # -inf only
    rec = np.zeros((M, K, T), dtype=_hip.CANDIDATE_DTYPE)
    rec["score"], rec["left_total"], rec["threshold"], rec["valid"] = score, left, thr, valid
    rec["left_grad"] = rng.standard_normal((M, K, T)).astype(np.float32)
    dev = torch.device("cuda")
    cand = torch.from_numpy(rec.view(np.uint8).reshape(-1).copy()).to(dev)
    out_s = torch.empty((M, K), dtype=torch.float32, device=dev)
    out_t = torch.empty((M, K), dtype=torch.int32, device=dev)
    out_g = torch.empty((M, K), dtype=torch.float32, device=dev)
    out_h = torch.empty((M, K), dtype=torch.float32, device=dev)
    out_c = torch.empty((M, K), dtype=torch.int64, device=dev)
    _hip.check(lib.pb_best_thresholds(cand.data_ptr(), M, K, T, out_s.data_ptr(), out_t.data_ptr(),
                                      out_g.data_ptr(), out_h.data_ptr(), out_c.data_ptr(),
                                      ctypes.c_void_p(_hip.stream_ptr())), "pb_best_thresholds")
    torch.cuda.synchronize()
    got_t, got_c = out_t.cpu().numpy(), out_c.cpu().numpy()
    got_s, got_g = out_s.cpu().numpy(), out_g.cpu().numpy()
    for m in range(M):
        for k in range(K):
            bs, bt, bl, bg = np.float32(-np.inf), -1, 0, np.float32(0)
            for t in range(T):
                if not valid[m, k, t]:
                    continue
                sc = score[m, k, t]
                better = sc > bs
                with np.errstate(invalid="ignore"):
                    near = abs(np.float32(sc - bs)) <= np.float32(1e-12)
                if not better and near:
                    better = left[m, k, t] > bl or (left[m, k, t] == bl and thr[m, k, t] > bt)
                if better:
                    bs, bt, bl, bg = sc, thr[m, k, t], left[m, k, t], rec["left_grad"][m, k, t]
            if not np.isfinite(bs):
                bt, bl, bg = -1, 0, np.float32(0)
            assert got_t[m, k] == bt and got_c[m, k] == bl, (m, k)
            assert got_g[m, k] == bg and (got_s[m, k] == bs or (np.isnan(bs) and np.isnan(got_s[m, k])))
    assert got_t[0, 0] == -1 and np.isneginf(got_s[0, 0])
    assert got_t[1, 0] == -1 and np.isposinf(got_s[1, 0]) and got_c[1, 0] == 0
    assert got_t[1, 2] == -1
