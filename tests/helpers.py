"""Shared builders for the parity tests: seeded problems, the oracle's view of one depth and
the GPU's view of the same depth through the C ABI."""

from __future__ import annotations

import ctypes

import numpy as np

PB_INACTIVE = 0xFFFF


def make_problem(seed: int, N: int, F: int, E: int, nb: int, U: int, *, inactive_frac: float = 0.1,
                 ragged: bool = True, empty_era: bool = False, grad_scale: float = 1.0) -> dict:
    """Random bins/grad, an era-major layout and a row -> active-slot assignment."""
    rng = np.random.default_rng(seed)
    if ragged:
        w = rng.uniform(0.3, 1.7, size=E)
        if empty_era and E > 2:
            w[E // 2] = 0.0
        sizes = np.floor(w / w.sum() * N).astype(np.int64)
        sizes[-1] += N - sizes.sum()
    else:
        sizes = np.full(E, N // E, dtype=np.int64)
        sizes[-1] += N - sizes.sum()
    offs = np.zeros(E + 1, dtype=np.int64)
    np.cumsum(sizes, out=offs[1:])
    era = np.repeat(np.arange(E), sizes)
    bins = rng.integers(0, nb, size=(N, F), dtype=np.uint8)
    grad = (rng.standard_normal(N) * grad_scale).astype(np.float32)
    nid = rng.integers(0, U, size=N).astype(np.int64)
    if inactive_frac > 0:
        nid[rng.random(N) < inactive_frac] = PB_INACTIVE
    return {"bins": bins, "grad": grad, "nid": nid.astype(np.uint16), "era": era,
            "era_off": offs.astype(np.int32), "N": N, "F": F, "E": E, "nb": nb, "U": U}


def with_skipped_bins(p: dict, seed: int, frac: float = 0.08) -> dict:
    """Sets a seeded `frac` of the bins to values >= nb (nb, nb + 3 and 255, the last being -1 as
    the reference's int8), and every bin of feature 0 in era 1 to nb, so that the era has rows
    but none in that feature's histogram."""
    rng = np.random.default_rng(seed + 1000)
    bins = p["bins"].copy()
    nb = p["nb"]
    hit = rng.random(bins.shape) < frac
    bins[hit] = rng.choice(np.array([nb, min(255, nb + 3), 255], dtype=np.uint8), size=int(hit.sum()))
    bins[p["era_off"][1]:p["era_off"][2], 0] = nb
    return {**p, "bins": bins}


def node_era_rows(p: dict) -> list[list[np.ndarray]]:
    nid, era = p["nid"].astype(np.int64), p["era"]
    out = []
    for u in range(p["U"]):
        m = nid == u
        out.append([np.nonzero(m & (era == e))[0].astype(np.int64) for e in range(p["E"])])
    return out


def decode_planes(cnt_raw: np.ndarray, g_raw: np.ndarray, E: int, M: int, K: int, nb: int,
                  cnt32: bool = False):
    """Compact histogram planes (uint16 prefix counts, uint32 when an era holds more than 65535
    rows, and float32 prefix grads [E][M][K][nb-1]; era totals [E][M] at element
    round_up(E*M*K*(nb-1), 64) of each buffer) expanded to the reference's [E][M][K][nb]
    prefix form (bin nb-1 = era total, repeated per feature)."""
    cells = E * M * K * (nb - 1)
    tot = (cells + 63) // 64 * 64
    cnt_raw = np.ascontiguousarray(cnt_raw, dtype=np.int32)
    c16 = (cnt_raw.view(np.uint32) if cnt32 else cnt_raw.view(np.uint16))[:cells].reshape(E, M, K, nb - 1)
    ct = cnt_raw[tot: tot + E * M].reshape(E, M)
    g = np.asarray(g_raw, dtype=np.float32)[:cells].reshape(E, M, K, nb - 1)
    gt = np.asarray(g_raw, dtype=np.float32)[tot: tot + E * M].reshape(E, M)
    c = np.concatenate([c16.astype(np.int64), np.repeat(ct[:, :, None, None].astype(np.int64), K, axis=2)], axis=3)
    gg = np.concatenate([g, np.repeat(gt[:, :, None, None], K, axis=2)], axis=3)
    return c, gg


def depth_for(U: int) -> int:
    d = 0
    while (1 << d) < U:
        d += 1
    return d


class GpuDepth:
    """Runs hist -> score -> decide -> partition for one teacher-forced depth."""

    def __init__(self, hip, p: dict, K: int, *, msl: int, depth: int | None = None,
                 max_depth: int | None = None, layout: str = "u8", bins_dev=None):
        import torch

        self.torch = torch
        self.hip = hip
        self.lib = hip.load()
        self.p = p
        N, F, E, nb = p["N"], p["F"], p["E"], p["nb"]
        self.depth = depth_for(p["U"]) if depth is None else depth
        D = max(self.depth + 1, max_depth or 0)
        self.ld = (N + 15) // 16 * 16
        dims = hip.PbDims(num_rows=N, ld=self.ld, num_features=F, num_eras=E, max_bins=nb,
                          max_depth=D, max_feats=K, min_samples_leaf=msl)
        self.offs = np.ascontiguousarray(p["era_off"], dtype=np.int32)
        ctx = ctypes.c_void_p()
        hip.check(self.lib.pb_ctx_create(ctypes.byref(dims), self.offs.ctypes.data, ctypes.byref(ctx)),
                  "pb_ctx_create")
        self.ctx = ctx
        dev = torch.device("cuda")
        if bins_dev is not None:  # column-major [F, ld] uint8 already on the device
            assert tuple(bins_dev.shape) == (F, self.ld)
            self.bins = bins_dev
        else:
            bfm = np.zeros((F, self.ld), dtype=np.uint8)
            bfm[:, :N] = p["bins"].T
            self.bins = torch.from_numpy(bfm).to(dev)
        if layout == "nibble":  # the histogram and partition read the packed copy
            packed = torch.empty((F, self.ld // 2), dtype=torch.uint8, device=dev)
            hip.check(self.lib.pb_pack_bins4(self.bins.data_ptr(), N, self.ld, F, packed.data_ptr(),
                                             hip.stream_ptr()), "pb_pack_bins4")
            hip.check(self.lib.pb_set_bin_layout(ctx, 1), "pb_set_bin_layout")
            self.bins = packed
        rp = self.ld
        self.grad = torch.zeros(rp, dtype=torch.float32, device=dev)
        preds = torch.zeros(rp, dtype=torch.float32, device=dev)
        preds[:N] = torch.from_numpy(p["grad"]).to(dev)
        y = torch.zeros(rp, dtype=torch.float32, device=dev)
        self.nid = torch.zeros(rp, dtype=torch.int16, device=dev)
        self.tnode = torch.zeros(rp, dtype=torch.int16, device=dev)
        s = hip.stream_ptr()
        hip.check(self.lib.pb_round_begin(ctx, preds.data_ptr(), y.data_ptr(), self.grad.data_ptr(),
                                          self.nid.data_ptr(), self.tnode.data_ptr(), s), "round_begin")
        nid = np.full(rp, PB_INACTIVE, dtype=np.uint16)
        nid[:N] = p["nid"]
        self.nid.copy_(torch.from_numpy(nid.view(np.int16)).to(dev))
        d = self.depth
        base = (1 << d) - 1
        ids = (base + np.arange(p["U"])).astype(np.int32)
        self.node_ids = ids
        tn = np.zeros(rp, dtype=np.uint16)
        act = nid[:N] != PB_INACTIVE
        tn[:N][act] = ids[nid[:N][act]]
        self.tnode.copy_(torch.from_numpy(tn.view(np.int16)).to(dev))
        hip.check(self.lib.pb_frontier_set(ctx, d, p["U"], ids.ctypes.data, (1 << (d + 1)) - 1, s),
                  "pb_frontier_set")
        self.max_nodes = int(self.lib.pb_max_nodes(ctx, d))
        assert self.max_nodes >= p["U"]
        plane = int(self.lib.pb_hist_plane_elems(ctx, self.max_nodes))
        self.cnt = torch.zeros(plane, dtype=torch.int32, device=dev)
        self.g = torch.zeros(plane, dtype=torch.float32, device=dev)
        self.K = K
        self.values = torch.zeros(1 << (D + 1), dtype=torch.float32, device=dev)
        self.dec = torch.zeros(((1 << D) - 1) * 64, dtype=torch.uint8, device=dev)

    def _plane_layout(self):
        p = self.p
        E, M, K, nb = p["E"], self.max_nodes, self.K, p["nb"]
        cells = E * M * K * (nb - 1)
        return E, M, K, nb, cells, (cells + 63) // 64 * 64

    def planes(self):
        """The device planes in the reference's [E][U][K][nb] prefix form."""
        E, M, K, nb, _, _ = self._plane_layout()
        cnt32 = int(np.diff(self.offs).max(initial=0)) > 0xFFFF
        c, g = decode_planes(self.cnt.cpu().numpy(), self.g.cpu().numpy(), E, M, K, nb, cnt32)
        U = self.p["U"]
        return c[:, :U], g[:, :U]

    def load_planes(self, cnt: np.ndarray, g: np.ndarray) -> None:
        """Writes [E][U][K][nb] prefix planes into the compact device layout. The era totals are
        stored once per (era, node): they are taken from feature 0."""
        torch = self.torch
        E, M, K, nb, cells, tot = self._plane_layout()
        U = cnt.shape[1]
        assert int(np.diff(self.offs).max(initial=0)) <= 0xFFFF, "writes the 16-bit count layout"
        assert cnt[..., : nb - 1].max(initial=0) <= 0xFFFF
        c16 = np.zeros((E, M, K, nb - 1), np.uint16)
        c16[:, :U] = cnt[..., : nb - 1]
        ct = np.zeros((E, M), np.int32)
        ct[:, :U] = cnt[:, :, 0, nb - 1]
        gp = np.zeros((E, M, K, nb - 1), np.float32)
        gp[:, :U] = g[..., : nb - 1]
        gt = np.zeros((E, M), np.float32)
        gt[:, :U] = g[:, :, 0, nb - 1]
        craw = np.zeros(self.cnt.numel(), np.int32)
        craw.view(np.uint16)[:cells] = c16.reshape(-1)
        craw[tot: tot + E * M] = ct.reshape(-1)
        graw = np.zeros(self.g.numel(), np.float32)
        graw[:cells] = gp.reshape(-1)
        graw[tot: tot + E * M] = gt.reshape(-1)
        self.cnt.copy_(torch.from_numpy(craw))
        self.g.copy_(torch.from_numpy(graw))

    def hist(self, feats: np.ndarray) -> None:
        self.feats = self.torch.from_numpy(np.ascontiguousarray(feats, np.int32)).to("cuda")
        self.hip.check(self.lib.pb_hist_build(
            self.ctx, self.bins.data_ptr(), self.grad.data_ptr(), self.nid.data_ptr(),
            self.feats.data_ptr(), self.K, self.depth, self.max_nodes, self.cnt.data_ptr(),
            self.g.data_ptr(), self.hip.stream_ptr()), "pb_hist_build")

    def score(self, feats: np.ndarray, params, T: int):
        torch = self.torch
        self.feats = torch.from_numpy(np.ascontiguousarray(feats, np.int32)).to("cuda")
        n = self.max_nodes * self.K * T
        self.cand_all = torch.zeros(n * 32, dtype=torch.uint8, device="cuda")
        self.hip.check(self.lib.pb_des_score(
            self.ctx, self.cnt.data_ptr(), self.g.data_ptr(), self.feats.data_ptr(), self.K,
            self.depth, self.max_nodes, ctypes.byref(params), self.cand_all.data_ptr(),
            self.hip.stream_ptr()), "pb_des_score")
        raw = self.cand_all.cpu().numpy().tobytes()
        c = np.frombuffer(raw, dtype=self.hip.CANDIDATE_DTYPE).reshape(self.max_nodes, self.K, T)
        return c[: self.p["U"]]

    def decide(self, params):
        self.hip.check(self.lib.pb_decide(self.ctx, self.depth, self.max_nodes, ctypes.byref(params),
                                          self.dec.data_ptr(), self.values.data_ptr(),
                                          self.hip.stream_ptr()), "pb_decide")
        raw = self.dec.cpu().numpy().tobytes()
        d = np.frombuffer(raw, dtype=self.hip.DECISION_DTYPE)
        base = (1 << self.depth) - 1
        return d[base: base + self.p["U"]].copy()

    def partition(self):
        self.hip.check(self.lib.pb_partition(self.ctx, self.bins.data_ptr(), self.depth,
                                             self.nid.data_ptr(), self.tnode.data_ptr(),
                                             self.hip.stream_ptr()), "pb_partition")
        N = self.p["N"]
        nid = self.nid.cpu().numpy().view(np.uint16)[:N].copy()
        tn = self.tnode.cpu().numpy().view(np.uint16)[:N].copy()
        return nid, tn

    def frontier(self):
        u = np.zeros(17, np.int32)
        ts = ctypes.c_int32(0)
        self.hip.check(self.lib.pb_frontier_counts(self.ctx, u.ctypes.data, ctypes.byref(ts),
                                                   self.hip.stream_ptr()), "pb_frontier_counts")
        return u, int(ts.value)

    def close(self):
        self.torch.cuda.synchronize()
        self.lib.pb_ctx_destroy(self.ctx)


def split_params(hip, *, lambda_l2=1e-6, lambda_dro=0.0, direction_weight=0.0, era_alpha=0.0,
                 msl=20, k_cuts=0, cut_selection="mass"):
    p = hip.PbSplitParams()
    p.lambda_l2, p.lambda_dro, p.direction_weight, p.era_alpha = (
        float(lambda_l2), float(lambda_dro), float(direction_weight), float(era_alpha))
    p.min_samples_leaf, p.k_cuts = int(msl), int(k_cuts)
    p.cut_selection = 1 if cut_selection == "mass" else 0
    return p


def node_sum_bounds(arrs: dict, bins: np.ndarray, grad: np.ndarray, lambda_l2: float,
                    leaf_index, return_leaf: bool = False):
    """Per node of one tree: the |grad| mass of the rows its value is formed from (its parent's
    rows: a child's value is -G/(n + lambda) with G a left sum or a parent total minus a left
    sum, booster.py:545-546; the root's own rows) over (rows + lambda_l2). Grad sums within 1e-5
    of their mass move the value by at most 1e-5 times this."""
    n = len(arrs["feature"])
    leaf = leaf_index(arrs, bins)
    m = np.bincount(leaf, weights=np.abs(grad.astype(np.float64)), minlength=n)
    c = np.bincount(leaf, minlength=n).astype(np.float64)
    parent = np.full(n, -1, np.int64)
    for node in range(n - 1, -1, -1):
        if not arrs["is_leaf"][node]:
            for ch in (arrs["left"][node], arrs["right"][node]):
                m[node] += m[ch]
                c[node] += c[ch]
                parent[ch] = node
    pm = np.where(parent >= 0, m[np.maximum(parent, 0)], m)
    bound = pm / (c + lambda_l2)
    return (bound, leaf) if return_leaf else bound


def compare_fit_rounds(oracle_mod, got_rounds, ref, trace, bins, kw) -> int:
    """Whole-fit parity of the device trees against the oracle's, round by round:
      * structure (feature, threshold, children, leaf flags) identical; at the first node that
        differs the device's split must be a near-tie (the oracle's score of it on the same
        rows within 1e-6, relative, of the oracle's best) and the comparison stops there, as the
        trajectories part;
      * node values within 1e-5 (relative) of the oracle's, plus twice 1e-5 of the |grad| mass
        the value is formed from over its rows (node_sum_bounds): the values are
        -G/(n + lambda) of grad sums that agree within 1e-5 of their mass, and a right child's
        G is a float32 difference of two such sums (booster.py:545-546).
    Returns the number of rounds compared whole and, per row, the bound those rounds' value
    bars put on the predictions: lr * B * the bar of the row's leaf, summed over the rounds
    (pack aggregation, booster.py:581-599); callers add the float32 rounding of the adds."""
    lam = float(kw.get("lambda_l2", 1e-6))
    lr = float(kw.get("learning_rate", 0.1))
    B = int(kw.get("pack_size", 8))
    pred_bar = np.zeros(bins.shape[0])
    matched = 0
    for r, (a, b) in enumerate(zip(got_rounds, ref.rounds)):
        same = all(np.array_equal(np.asarray(a[k]), np.asarray(b[k]))
                   for k in ("feature", "threshold", "left", "right", "is_leaf"))
        depth_traces = [t for t in trace if t["round"] == r]
        if not same:
            assert_near_tie(oracle_mod, bins, a, b, depth_traces, kw)
            break
        va, vb = np.asarray(a["value"], np.float64), np.asarray(b["value"], np.float64)
        if depth_traces:
            bound, leaf = node_sum_bounds(b, bins, depth_traces[0]["grad"], lam, oracle_mod.leaf_index,
                                          return_leaf=True)
            err = np.abs(va - vb)
            bar = 1e-5 * (np.abs(vb) + 2.0 * bound) + 1e-7
            pred_bar += lr * B * bar[leaf]
            worst = int(np.argmax(err / bar))
            print(f"[fit parity] round {r}: worst value error {err[worst]:.3g} at node {worst} "
                  f"(bar {bar[worst]:.3g}, |value| {abs(vb[worst]):.3g}, mass bound {bound[worst]:.3g})",
                  flush=True)
            assert np.all(err <= bar), (f"round {r}: node {worst} value {va[worst]!r} vs {vb[worst]!r} "
                                        f"(bar {bar[worst]:.3g})")
        else:
            np.testing.assert_allclose(va, vb, rtol=1e-5, atol=1e-5, err_msg=f"round {r} value")
            pred_bar += lr * B * 1e-5 * np.maximum(1.0, np.abs(vb[oracle_mod.leaf_index(b, bins)]))
        matched += 1
    return matched, pred_bar


def assert_near_tie(oracle_mod, bins, got, want, depth_traces, kw):
    """The first node (depth by depth, in frontier order) where the device tree differs from
    the oracle's: the device's split must score, by the oracle on that node's rows, within 1e-6
    (relative) of the oracle's best."""
    for t in depth_traces:
        res = t["result"]
        for m, nid in enumerate(t["node_ids"]):
            fw, tw = int(want["feature"][nid]), int(want["threshold"][nid])
            fg, tg = int(got["feature"][nid]), int(got["threshold"][nid])
            if (fw, tw) == (fg, tg):
                continue
            assert fg >= 0 and fw >= 0, f"node {nid}: split vs no split"
            opts = {k: kw[k] for k in ("k_cuts", "cut_selection", "lambda_l2", "lambda_dro",
                                       "direction_weight", "era_alpha") if k in kw}
            cands = oracle_mod.split_batch(bins, t["grad"], [t["nodes_era_rows"][m]], t["feats"],
                                           kw["max_bins"], want_cands=True,
                                           min_samples_leaf=kw.get("min_samples_leaf", 20), **opts).cands
            k = int(np.nonzero(t["feats"] == fg)[0][0])
            s_dev = float(cands[0][0, k, tg])
            best = float(res.score[m])
            assert abs(s_dev - best) <= 1e-6 * max(1.0, abs(best)), \
                f"node {nid}: device split ({fg}, {tg}) scores {s_dev} vs best {best}"
            print(f"[fit parity] near-tie at node {nid}: {s_dev} vs {best}", flush=True)
            return
    raise AssertionError("trees differ outside the traced depths")


# ------------------------------------------------------------------ whole-round fixtures
class _EraRows:
    """nodes_era_rows of one traced depth, built on demand (only a near-tie check reads it):
    per frontier node, its rows per era in ascending order."""

    def __init__(self, node_at_depth: np.ndarray, node_ids, era: np.ndarray, E: int):
        self.node_at_depth, self.node_ids, self.era, self.E = node_at_depth, node_ids, era, E

    def __getitem__(self, m: int):
        rows = np.nonzero(self.node_at_depth == int(self.node_ids[m]))[0].astype(np.int64)
        cuts = np.searchsorted(self.era[rows], np.arange(self.E + 1))
        return [rows[cuts[e]:cuts[e + 1]] for e in range(self.E)]


class _Scores:
    def __init__(self, score: np.ndarray):
        self.score = score


def node_at_depth(tree: dict, bins: np.ndarray, d: int) -> np.ndarray:
    """The tree node each row sits in after d levels of the bin <= threshold walk."""
    node = np.zeros(bins.shape[0], dtype=np.int64)
    for _ in range(d):
        inner = np.nonzero(~np.asarray(tree["is_leaf"], bool)[node])[0]
        if inner.size == 0:
            break
        nd = node[inner]
        go_left = bins[inner, tree["feature"][nd]] <= tree["threshold"][nd]
        node[inner] = np.where(go_left, tree["left"][nd], tree["right"][nd])
    return node


def fixture_fit_parity(oracle_mod, name: str, fit_rounds) -> int:
    """A HIP fit against tests/golden/<name>_rounds.npz (tests/golden/make_rounds_golden.py).

    fit_rounds(n) fits the workload's first n rounds on the device and returns the PackBoost
    model. The oracle's trace is rebuilt from the fixture: the predictions entering each round
    from its trees (oracle.replay_preds arithmetic, checked against the fixture's prediction
    sums and samples bit for bit), frontier node ids, subsets and best scores per depth, and
    each node's era row lists on demand. Then:
      * compare_fit_rounds: trees identical, or at the first differing node a near-tie (the
        oracle's score of the device's split on that node's rows within 1e-6 of its best),
        where the trajectories part; node values within 1e-5;
      * the depth logs of the matched rounds: frontier size and row count per depth, exact;
      * training predictions after the matched rounds within 1e-5 (plus the value bars carried
        through the pack sums) of the oracle's (a second, shorter device fit when the
        trajectories part early).
    Returns the number of rounds compared whole (at least 1)."""
    from tests.golden.make_rounds_golden import case_data, load_fixture, sample_rows

    fx = load_fixture(name)
    R = fx["rounds"]
    want = fx["trees"]
    print(f"[{name} fixture] generating the workload ({R} fixture rounds)", flush=True)
    X, bins, y, era, cfg = case_data(name)
    E = int(era.max()) + 1
    samp = sample_rows(name, bins.shape[0])
    B, lr = int(cfg["pack_size"]), float(cfg["learning_rate"])
    trace, after = [], []
    preds = np.zeros(bins.shape[0], dtype=np.float32)
    by_round: dict = {}
    for e in fx["depths"]:
        by_round.setdefault(e["round"], []).append(e)
    for r in range(R):
        grad = (preds - y).astype(np.float32)
        for e in by_round.get(r, []):
            d, nodes = e["depth"], e["nodes"]
            trace.append({"round": r, "depth": d, "node_ids": nodes, "feats": e["feats"], "grad": grad,
                          "result": _Scores(e["score"]), "rows": e["rows"],
                          "nodes_era_rows": _EraRows(node_at_depth(want[r], bins, d), nodes, era, E)})
        leaf_val = want[r]["value"].astype(np.float32)[oracle_mod.leaf_index(want[r], bins)]
        preds = oracle_mod.pack_update(preds, leaf_val, B, np.float32(lr))
        assert float(preds.astype(np.float64).sum()) == float(fx["preds_sum"][r]), f"replay {r}"
        if r in fx["preds_sample"]:
            np.testing.assert_array_equal(preds[samp], fx["preds_sample"][r], err_msg=f"replay {r}")
        after.append(preds)
    print(f"[{name} fixture] HIP fit", flush=True)
    model = fit_rounds(R)
    got = model._rounds
    assert len(got) == R

    class Ref:
        rounds = want

    matched, pred_bar = compare_fit_rounds(oracle_mod, got, Ref, trace, bins, dict(cfg))
    print(f"[{name} fixture] {matched} of {R} rounds identical", flush=True)
    assert matched >= 1, "the device and the oracle part (at a near-tie) in the first round"
    logs = iter(model._depth_logs)
    for t in trace:
        if t["round"] >= matched:
            break
        dl = next(logs)
        assert (dl["depth"], dl["nodes_processed"]) == (t["depth"], len(t["node_ids"]))
        assert dl["rows_total"] == int(t["rows"].sum())
    dev_model = model if matched == R else fit_rounds(matched)
    ref = after[matched - 1].astype(np.float64)
    bar = np.maximum(1e-5, pred_bar + matched * (B + 1) * 6e-8 * np.abs(ref))
    dev = train_preds_rows(dev_model).astype(np.float64)
    diff = np.abs(dev - ref)
    print(f"[{name} fixture] training predictions after {matched} rounds: max diff {diff.max():.3g}, "
          f"{int(np.sum(diff > 1e-5))} rows beyond 1e-5", flush=True)
    assert np.all(diff <= bar)
    return matched


def train_preds_rows(model) -> np.ndarray:
    """A fitted model's training predictions in the caller's row order (the fit keeps them in
    its era-major order, model._perm)."""
    dev = model._train_preds.cpu().numpy()
    perm = getattr(model, "_perm", None)
    if perm is None:
        return dev
    out = np.empty_like(dev)
    out[np.asarray(perm)] = dev
    return out


def live_fit_parity(oracle_mod, fit_rounds, bins, y, era_codes, kw, rounds, *, min_matched=None):
    """A HIP fit against the oracle's fit (run here) on the same data, over `rounds` rounds.

    fit_rounds(n) fits the first n rounds on the device and returns the PackBoost model. Trees
    must be identical, or part at an asserted near-tie (compare_fit_rounds); node values within
    1e-5; training predictions and predict() after the matched rounds within 1e-5 of the oracle's
    (a second, shorter device fit when the trajectories part early); leaf indices of every
    matched round's tree bit-exact. Requires at least `min_matched` whole rounds (default: all
    of them, unless they part at an asserted near-tie; then at least one). Returns matched."""
    model = fit_rounds(rounds)
    trace: list = []
    ref = oracle_mod.fit(bins, y, era_codes, num_rounds=rounds, trace=trace, **kw)
    matched, pred_bar = compare_fit_rounds(oracle_mod, model._rounds, ref, trace, bins, kw)
    print(f"[fit parity] {matched} of {rounds} rounds identical", flush=True)
    assert matched >= (1 if min_matched is None else min_matched)
    B, lr = int(kw.get("pack_size", 8)), float(kw.get("learning_rate", 0.1))
    dev_model = model if matched == rounds else fit_rounds(matched)
    ref_train = oracle_mod.replay_preds(ref.rounds[:matched], bins, B, lr).astype(np.float64)
    if matched == rounds:
        np.testing.assert_array_equal(ref_train, ref.preds)
    bar = np.maximum(1e-5, pred_bar + matched * (B + 1) * 6e-8 * np.abs(ref_train))
    d = np.abs(train_preds_rows(dev_model).astype(np.float64) - ref_train)
    assert np.all(d <= bar), f"training predictions: max diff {d.max():.3g}"
    return model, ref, matched, bar
