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
], ids=["nb5", "nb32_alpha_dir", "nb128"])
def test_split_finder_rowlist(hip, oracle_mod, case):
    import torch

    from packboost_amd import backends

    seed, N, F, E, nb, U, K, msl, alpha, dirw = case
    print(f"[rowlist split] {case}", flush=True)
    p = make_problem(seed, N, F, E, nb, U)
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
    want = _oracle_per_feature(ref.cands)
    s_ref, lt_ref = ref.cands[0], ref.cands[1]
    for u in range(U):
        for k in range(K):
            if want[u, k] < 0:
                assert thr[u, k] == -1 and np.isneginf(sc[u, k])
                continue
            if thr[u, k] != want[u, k]:
                a, b = float(s_ref[u, k, thr[u, k]]), float(s_ref[u, k, want[u, k]])
                assert abs(a - b) <= 1e-6 * max(1.0, abs(b)), (u, k, thr[u, k], want[u, k])
                continue
            assert lc[u, k] == lt_ref[u, k, want[u, k]]
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
