"""Device-resident training rounds on the HIP backend.

`DeviceFit` owns the per-fit device state (column-major uint8 bins, targets, predictions,
per-row frontier ids, histogram planes, decision log) and runs one boosting round as a
sequence of asynchronous kernel launches on the caller's stream:

    round_begin                         grad = preds - y, every row in the root
    for depth in 0..D-1:
        hist_build -> des_score -> decide -> partition
    round_end                           preds += lr * pack_sum

A whole round is one C-ABI call (pb_grow_round). The only host round trip per round is the
copy of the decision log (a few KB) from which the host rebuilds the round's trees. Feature
subsets are drawn on the host from the fit's CPU generator before the round; the generator
is rewound afterwards to the state the reference would have after its actual number of draws
(it draws only while a depth still has active nodes, booster.py:516-519).

`DeviceFit.rounds` pipelines the host and the GPU: round r+1 is enqueued before round r's log
is read, on the assumption that round r drew all D subsets. Its predictions are snapshotted
first; in the rare case that round r stopped early, the snapshot is restored and round r+1
is enqueued again with the generator rewound, so results never depend on the speculation.
"""

from __future__ import annotations

import ctypes
import os
import math
from dataclasses import dataclass

import numpy as np
import torch

from .backends import _hip
from .config import PackBoostConfig


def padded_rows(n: int) -> int:
    return (n + 15) // 16 * 16


def split_params(cfg: PackBoostConfig) -> _hip.PbSplitParams:
    p = _hip.PbSplitParams()
    p.lambda_l2 = float(cfg.lambda_l2)
    p.lambda_dro = float(cfg.lambda_dro)
    p.direction_weight = float(cfg.direction_weight)
    p.era_alpha = max(0.0, float(cfg.era_alpha))
    p.min_samples_leaf = int(cfg.min_samples_leaf)
    p.k_cuts = int(cfg.k_cuts)
    p.cut_selection = 1 if str(cfg.cut_selection) == "mass" else 0
    p.skip_last_bin = 0
    return p


def subset_size(cfg: PackBoostConfig, num_features: int) -> int:
    """k = max(1, round(frac * F)), capped at F (booster.py:787-792)."""
    k = max(1, int(round(float(cfg.layer_feature_fraction) * num_features)))
    return min(k, num_features)


# A round whose gradients (preds - y) are not all finite: the predictions overflowed (a learning
# rate x pack_size that overshoots) or the targets hold NaN/inf. The histograms are exact
# fixed-point sums and hold no NaN or infinity, so such a round cannot follow the reference's
# float arithmetic (whose NaN scores end the splits); the fit stops with this error instead.
NONFINITE_MSG = ("gradients are not finite (the predictions overflowed or y holds NaN/inf); "
                 "lower learning_rate x pack_size or clean the targets")


@dataclass
class RoundLog:
    """Decisions of one round, as the host reads them back."""

    u_active: np.ndarray      # int32 [D+1] active unique nodes per depth
    tree_size: int            # nodes of each tree of the round
    decisions: np.ndarray     # DECISION_DTYPE [2^D - 1], depth d at offset 2^d - 1
    root_grad: float          # float32 sum of grad over all rows (root value numerator)
    depths_drawn: int         # feature subsets the reference would have drawn
    phase_ms: np.ndarray | None = None  # float64 [4][D] GPU ms of hist / score / decide /
                                        # partition per depth (timed rounds only: rounds()
                                        # with phase_times or phase_every)


class _DrawStream:
    """The feature-subset draws of a fit as one indexed stream: draw i is
    torch.randperm(F, generator=rng)[:K] taken after draws 0..i-1, materialised on demand,
    with the generator state before each draw kept so the generator can be left exactly
    where the consumed draws end."""

    def __init__(self, rng: torch.Generator, F: int, K: int) -> None:
        self.rng, self.F, self.K = rng, F, K
        self.base = 0                        # absolute index of draws[0]
        self.draws: list[np.ndarray] = []
        self.states = [rng.get_state()]      # states[i]: before draw base + i

    def window(self, lo: int, n: int) -> np.ndarray:
        while self.base + len(self.draws) < lo + n:
            self.draws.append(torch.randperm(self.F, generator=self.rng)[: self.K].numpy()
                              .astype(np.int32))
            self.states.append(self.rng.get_state())
        i = lo - self.base
        return np.stack(self.draws[i: i + n])

    def release(self, lo: int) -> None:
        """Forgets draws before absolute index lo."""
        k = lo - self.base
        if k > 0:
            del self.draws[:k]
            del self.states[:k]
            self.base = lo

    def rewind_to(self, pos: int) -> None:
        """Leaves the generator as if exactly draws 0..pos-1 had been taken."""
        self.rng.set_state(self.states[pos - self.base])


class DeviceFit:
    """One fit's device state and round driver (all B trees of a pack share one frontier)."""

    def __init__(self, bins_fm: torch.Tensor, num_rows: int, y: torch.Tensor,
                 era_offsets: np.ndarray, cfg: PackBoostConfig, *,
                 stream: torch.cuda.Stream | None = None, bin_layout: str = "auto",
                 fit_mode: str | None = None) -> None:
        """bin_layout: "u8" (the histogram reads bins_fm), "nibble" (a two-rows-per-byte copy,
        pb_pack_bins4, max_bins <= 16) or "auto" (nibble whenever max_bins <= 16).

        fit_mode: "planes" (histogram planes in HBM, then the scorer), "segments" (from a
        depth on, rows kept sorted by frontier node and one fused histogram + scorer kernel
        per depth: pb_set_segment_mode; PB_SEG_FROM_DEPTH sets that depth, else the first
        whose planes would pass 1 GiB) or "auto" (default; the environment variable
        PB_FIT_MODE overrides it): segments when the deepest depth's planes would pass 1 GiB,
        there are 64 or more thresholds per feature and the fit allows them (full threshold
        sweep, eras of at most 65535 rows)."""
        lib = _hip.load()
        if bins_fm.dtype != torch.uint8 or bins_fm.dim() != 2 or not bins_fm.is_cuda:
            raise ValueError("bins_fm must be a CUDA uint8 tensor [F, ld]")
        if not bins_fm.is_contiguous():
            raise ValueError("bins_fm must be contiguous")
        F, ld = bins_fm.shape
        N = int(num_rows)
        if ld < N or ld % 16 != 0 or bins_fm.data_ptr() % 16 != 0:
            raise ValueError("bins_fm row stride must be >= N and a multiple of 16")
        self.lib = lib
        self.cfg = cfg
        self.device = bins_fm.device
        self.stream = stream if stream is not None else torch.cuda.current_stream(self.device)
        self.N, self.F, self.ld = N, int(F), int(ld)
        self.E = int(len(era_offsets) - 1)
        self.D = int(cfg.max_depth)
        self.K = subset_size(cfg, self.F)
        self.nb = int(cfg.max_bins)
        self.B = int(cfg.pack_size)
        self.lr = float(cfg.learning_rate)
        self.params = split_params(cfg)
        self.bins = bins_fm
        self.rows_padded = padded_rows(N)
        dev = self.device
        if bin_layout not in ("auto", "u8", "nibble"):
            raise ValueError(f"bin_layout must be 'auto', 'u8' or 'nibble', got {bin_layout!r}")
        if bin_layout == "nibble" and self.nb > 16:
            raise ValueError("the nibble bin layout needs max_bins <= 16")
        self.bins4 = None
        if bin_layout == "nibble" or (bin_layout == "auto" and self.nb <= 16):
            self.bins4 = torch.empty((self.F, self.ld // 2), dtype=torch.uint8, device=dev)
            _hip.check(lib.pb_pack_bins4(bins_fm.data_ptr(), N, self.ld, self.F, self.bins4.data_ptr(),
                                         _hip.stream_ptr(self.stream)), "pb_pack_bins4")

        dims = _hip.PbDims(num_rows=N, ld=self.ld, num_features=self.F, num_eras=self.E,
                           max_bins=self.nb, max_depth=self.D, max_feats=self.K,
                           min_samples_leaf=int(cfg.min_samples_leaf))
        offs = np.ascontiguousarray(era_offsets, dtype=np.int32)
        self._offs = offs
        ctx = ctypes.c_void_p()
        _hip.check(lib.pb_ctx_create(ctypes.byref(dims), offs.ctypes.data, ctypes.byref(ctx)),
                   "pb_ctx_create")
        self.ctx = ctx

        def rows(dtype):
            return torch.zeros(self.rows_padded, dtype=dtype, device=dev)

        self.y = rows(torch.float32)
        self.y[:N].copy_(y.to(device=dev, dtype=torch.float32).reshape(-1))
        self.preds = rows(torch.float32)
        self.grad = rows(torch.float32)
        self.nid = rows(torch.int16)    # uint16 ids carried in int16 storage
        self.tnode = rows(torch.int16)
        self.max_nodes = [int(lib.pb_max_nodes(ctx, d)) for d in range(self.D)]
        mode = fit_mode or os.environ.get("PB_FIT_MODE", "auto")
        if mode not in ("auto", "planes", "segments"):
            raise ValueError(f"fit_mode must be 'auto', 'planes' or 'segments', got {mode!r}")
        full_sweep = not (0 < int(cfg.k_cuts) < self.nb - 1)
        era_rows = int(np.max(np.diff(np.asarray(era_offsets, dtype=np.int64)))) if self.E else 0
        segments_ok = full_sweep and era_rows <= 65535
        if mode == "segments" and not segments_ok:
            raise ValueError("fit_mode 'segments' needs k_cuts 0 and eras of at most 65535 rows")
        plane_bytes = [self.E * m * self.K * max(1, self.nb - 1) * 6 for m in self.max_nodes]
        # auto: only where the fused kernel's threads have thresholds to score (one per threshold,
        # 4 features per workgroup: with few bins most of a workgroup would idle)
        self.segments = mode == "segments" or (mode == "auto" and segments_ok and self.nb - 1 >= 64
                                               and plane_bytes[-1] >= (1 << 30))
        # histogram planes for the depths the plane path scores (all of them, or those before
        # the first fused depth of a segment-mode fit: the deepest planes can take tens of GB)
        plane_depths = self.D
        if self.segments:
            env = os.environ.get("PB_SEG_FROM_DEPTH")
            if env is not None:
                plane_depths = min(self.D, max(0, int(env)))
            else:
                plane_depths = next((d for d, b in enumerate(plane_bytes) if b >= (1 << 30)), self.D)
            _hip.check(lib.pb_set_segment_mode(ctx, 1, plane_depths), "pb_set_segment_mode")
        self.seg_from = plane_depths if self.segments else None
        plane = max(int(lib.pb_hist_plane_elems(ctx, m)) for m in self.max_nodes[:max(1, plane_depths)])
        self.hist_cnt = torch.empty(plane, dtype=torch.int32, device=dev)
        self.hist_g = torch.empty(plane, dtype=torch.float32, device=dev)

        self.values = torch.zeros(1 << (self.D + 1), dtype=torch.float32, device=dev)
        n_dec = (1 << self.D) - 1
        self.dec_dev = torch.zeros(n_dec * _hip.DECISION_DTYPE.itemsize, dtype=torch.uint8, device=dev)
        self.dec_host = torch.empty_like(self.dec_dev, device="cpu").pin_memory()
        self.feats_dev = torch.zeros((self.D, self.K), dtype=torch.int32, device=dev)
        self.feats_host = torch.zeros((self.D, self.K), dtype=torch.int32).pin_memory()
        self.root_grad_dev = torch.zeros(1, dtype=torch.float32, device=dev)

        # pb_grow_round state: two slots (round parity) of feature subsets and of the round's
        # log = [decisions (2^D - 1) x 64 B | header 96 B], device and pinned host copies
        self._n_dec = n_dec
        log_bytes = n_dec * _hip.DECISION_DTYPE.itemsize + _hip.HEADER_DTYPE.itemsize
        self._log_dev = [torch.zeros(log_bytes, dtype=torch.uint8, device=dev) for _ in range(2)]
        self._log_host = [torch.zeros(log_bytes, dtype=torch.uint8).pin_memory() for _ in range(2)]
        self._feats_slot_dev = [torch.zeros((self.D, self.K), dtype=torch.int32, device=dev)
                                for _ in range(2)]
        self._feats_slot_host = [torch.zeros((self.D, self.K), dtype=torch.int32).pin_memory()
                                 for _ in range(2)]
        # pipelined rounds: each round's window of 2D subset draws (pb_select_subsets)
        self._win_dev = [torch.zeros((2 * self.D, self.K), dtype=torch.int32, device=dev)
                         for _ in range(2)]
        self._win_host = [torch.zeros((2 * self.D, self.K), dtype=torch.int32).pin_memory()
                          for _ in range(2)]
        self._log_ready = [None, None]
        self.preds_snap = torch.zeros_like(self.preds)
        b = _hip.PbFitBuffers()
        b.bins_dev = self.bins.data_ptr()
        b.bins4_dev = None if self.bins4 is None else self.bins4.data_ptr()
        b.y_dev = self.y.data_ptr()
        b.preds_dev = self.preds.data_ptr()
        b.grad_dev = self.grad.data_ptr()
        b.nid_dev = self.nid.data_ptr()
        b.tnode_dev = self.tnode.data_ptr()
        b.hist_cnt_dev = self.hist_cnt.data_ptr()
        b.hist_grad_dev = self.hist_g.data_ptr()
        b.values_dev = self.values.data_ptr()
        b.pack_size = self.B
        b.learning_rate = self.lr
        b.params = self.params
        self._bufs = b
        # a root below 2*min_samples_leaf never splits: the per-phase path sets its value
        self._root_splittable = self.N >= 2 * int(cfg.min_samples_leaf)

    # ------------------------------------------------------------------ lifecycle
    def close(self) -> None:
        if getattr(self, "ctx", None) is not None and self.ctx.value:
            torch.cuda.synchronize(self.device)
            self.lib.pb_ctx_destroy(self.ctx)
            self.ctx = None

    def __del__(self) -> None:  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass

    # ------------------------------------------------------------------ rounds
    def draw_subsets(self, rng: torch.Generator) -> tuple[np.ndarray, list]:
        """Draws the subsets of every depth, keeping the generator state before each draw."""
        states = []
        subs = np.empty((self.D, self.K), dtype=np.int32)
        for d in range(self.D):
            states.append(rng.get_state())
            subs[d] = torch.randperm(self.F, generator=rng)[: self.K].numpy().astype(np.int32)
        states.append(rng.get_state())
        return subs, states

    def enqueue_round(self, subsets: np.ndarray, events: list | None = None) -> None:
        """Enqueues one full round on the stream (no host synchronisation).

        events: optional list that receives (phase, depth, start, end) timing events
        recorded on the fit's stream around every kernel phase.
        """
        if self.segments and self._root_splittable:
            raise RuntimeError("a segment-mode fit runs whole rounds (pb_grow_round) only")
        lib, ctx, s = self.lib, self.ctx, _hip.stream_ptr(self.stream)
        chk = _hip.check
        self.feats_host.numpy()[...] = subsets
        with torch.cuda.stream(self.stream):
            self.feats_dev.copy_(self.feats_host, non_blocking=True)
        chk(lib.pb_round_begin(ctx, self.preds.data_ptr(), self.y.data_ptr(), self.grad.data_ptr(),
                               self.nid.data_ptr(), self.tnode.data_ptr(), s), "pb_round_begin")
        p = ctypes.byref(self.params)
        def mark():
            if events is None:
                return None
            ev = torch.cuda.Event(enable_timing=True)
            ev.record(self.stream)
            return ev

        for d in range(self.D):
            fptr = self.feats_dev[d].data_ptr()
            m = self.max_nodes[d]
            t0 = mark()
            chk(lib.pb_hist_build(ctx, self.bins.data_ptr(), self.grad.data_ptr(),
                                  self.nid.data_ptr(), fptr, self.K, d, m,
                                  self.hist_cnt.data_ptr(), self.hist_g.data_ptr(), s),
                "pb_hist_build")
            t1 = mark()
            chk(lib.pb_des_score(ctx, self.hist_cnt.data_ptr(), self.hist_g.data_ptr(), fptr,
                                 self.K, d, m, p, None, s), "pb_des_score")
            t2 = mark()
            chk(lib.pb_decide(ctx, d, m, p, self.dec_dev.data_ptr(), self.values.data_ptr(), s),
                "pb_decide")
            t3 = mark()
            chk(lib.pb_partition(ctx, self.bins.data_ptr(), d, self.nid.data_ptr(),
                                 self.tnode.data_ptr(), s), "pb_partition")
            t4 = mark()
            if events is not None:
                events += [("hist", d, t0, t1), ("score", d, t1, t2), ("decide", d, t2, t3),
                           ("partition", d, t3, t4)]
        self._root_value_if_inactive()
        chk(lib.pb_round_end(ctx, self.tnode.data_ptr(), self.values.data_ptr(), self.B,
                             ctypes.c_float(self.lr), self.preds.data_ptr(), s), "pb_round_end")

    def enqueue_grow(self, subsets: np.ndarray, slot: int) -> None:
        """Enqueues one full round as a single pb_grow_round call plus the copy of its log
        into host slot `slot` (no host synchronisation)."""
        fh = self._feats_slot_host[slot]
        fh.numpy()[...] = subsets
        log_dev = self._log_dev[slot]
        dec_ptr = log_dev.data_ptr()
        hdr_ptr = dec_ptr + self._n_dec * _hip.DECISION_DTYPE.itemsize
        with torch.cuda.stream(self.stream):
            self._feats_slot_dev[slot].copy_(fh, non_blocking=True)
            _hip.check(self.lib.pb_grow_round(self.ctx, ctypes.byref(self._bufs),
                                              self._feats_slot_dev[slot].data_ptr(), self.K,
                                              dec_ptr, hdr_ptr, _hip.stream_ptr(self.stream)),
                       "pb_grow_round")
            self._log_host[slot].copy_(log_dev, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(self.stream)
        self._log_ready[slot] = ev

    def _hdr_ptr(self, slot: int) -> int:
        return self._log_dev[slot].data_ptr() + self._n_dec * _hip.DECISION_DTYPE.itemsize

    def enqueue_grow_window(self, window: np.ndarray, slot: int, prev_slot: int | None) -> None:
        """Like enqueue_grow, with the round's subsets picked on the device from `window`
        ([2D][K] draws) by the previous round's header in log slot `prev_slot`
        (pb_select_subsets), so the host need not know how many subsets that round drew."""
        wh = self._win_host[slot]
        wh.numpy()[: len(window)] = window
        log_dev = self._log_dev[slot]
        dec_ptr = log_dev.data_ptr()
        sp = _hip.stream_ptr(self.stream)
        with torch.cuda.stream(self.stream):
            self._win_dev[slot].copy_(wh, non_blocking=True)
            _hip.check(self.lib.pb_select_subsets(
                None if prev_slot is None else self._hdr_ptr(prev_slot), self._win_dev[slot].data_ptr(),
                self.D, self.K, self._feats_slot_dev[slot].data_ptr(), sp), "pb_select_subsets")
            _hip.check(self.lib.pb_grow_round(self.ctx, ctypes.byref(self._bufs),
                                              self._feats_slot_dev[slot].data_ptr(), self.K,
                                              dec_ptr, self._hdr_ptr(slot), sp), "pb_grow_round")
            self._log_host[slot].copy_(log_dev, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(self.stream)
        self._log_ready[slot] = ev

    def read_slot(self, slot: int) -> RoundLog:
        """Waits for the log copy of `slot` (not for later work on the stream) and parses it."""
        self._log_ready[slot].synchronize()
        raw = self._log_host[slot].numpy()
        nd = self._n_dec * _hip.DECISION_DTYPE.itemsize
        dec = np.frombuffer(raw[:nd].tobytes(), dtype=_hip.DECISION_DTYPE)
        hdr = np.frombuffer(raw[nd:].tobytes(), dtype=_hip.HEADER_DTYPE)[0]
        if int(hdr["reserved"][0]):
            raise FloatingPointError(NONFINITE_MSG)
        u = np.asarray(hdr["u_active"], dtype=np.int32)
        drawn = int(np.count_nonzero(u[: self.D] > 0))
        return RoundLog(u_active=u[: self.D + 1].copy(), tree_size=int(hdr["tree_size"]),
                        decisions=dec, root_grad=float(dec[0]["node_grad"]), depths_drawn=drawn)

    def read_phase_ms(self) -> tuple[np.ndarray, np.ndarray]:
        """GPU ms and launch counts [4][D] (hist, score, decide, partition per depth) of the
        rounds timed since the last read (pb_profile_read; waits for them)."""
        ms = np.zeros(4 * _hip.PB_MAX_DEPTH, dtype=np.float64)
        n = np.zeros(4 * _hip.PB_MAX_DEPTH, dtype=np.int64)
        _hip.check(self.lib.pb_profile_read(self.ctx, ms.ctypes.data, n.ctypes.data), "pb_profile_read")
        return ms.reshape(4, -1)[:, : self.D], n.reshape(4, -1)[:, : self.D]

    def rounds(self, rng: torch.Generator, num_rounds: int, *, profile_every: int = 0,
               profile_mode: int = 2, phase_times: bool = False, phase_every: int = 0):
        """Runs `num_rounds` rounds with the host one round ahead of the GPU.

        profile_every > 0 turns the library's phase timing (pb_profile_enable, mode
        `profile_mode`) on for every profile_every-th round only, so that the events' queue
        barriers touch few rounds.

        phase_times: every round timed phase by phase, each read back with its log
        (RoundLog.phase_ms); rounds then run one at a time (no round is enqueued ahead), so
        the times are the round's own.

        phase_every > 1: rounds 0, phase_every, 2 * phase_every, ... are timed phase by phase
        and their RoundLog.phase_ms filled, while the loop stays one round ahead (the next round
        is never timed, so reading a timed round's events waits for that round only);
        phase_every == 1 is phase_times.

        Yields (RoundLog, preds_after, ready) per round in order. `preds_after` holds the
        predictions after that round until the consumer resumes the generator (the GPU may
        already be running the next round on `preds`); `ready` is an event on the fit's
        stream after which `preds_after` is valid, so a side stream can read it without
        waiting for the next round.
        """
        def now() -> torch.cuda.Event:
            ev = torch.cuda.Event()
            ev.record(self.stream)
            return ev

        if not self._root_splittable:
            for _ in range(num_rounds):
                log = self.run_round(rng)
                yield log, self.preds, now()
            return
        if num_rounds <= 0:
            return
        def set_profile(r: int) -> None:
            if profile_every > 0:
                on = profile_mode if r % profile_every == 0 else 0
                _hip.check(self.lib.pb_profile_enable(self.ctx, on), "pb_profile_enable")

        # Round r draws subsets [p_r, p_r + d_r) of the generator's stream (d_r: its depths with
        # active nodes). Round r + 1 is enqueued before round r's log is read, with the window
        # [p_r, p_r + 2D): the device picks its D subsets at offset d_r from round r's header.
        draws = _DrawStream(rng, self.F, self.K)
        D = self.D
        p = 0
        if phase_every == 1:
            phase_times = True
        if phase_times:
            profile_every, profile_mode = 1, 1
        elif phase_every > 1:
            profile_every, profile_mode = phase_every, 1
        set_profile(0)
        self.enqueue_grow_window(draws.window(0, 2 * D), 0, None)
        for r in range(num_rounds):
            slot = r & 1
            if phase_times and r > 0:  # this round's subsets start where the last round's ended
                self.enqueue_grow_window(draws.window(p, 2 * D), slot, None)
            ahead = r + 1 < num_rounds and not phase_times
            if ahead:
                with torch.cuda.stream(self.stream):
                    self.preds_snap.copy_(self.preds)
                ready = now()
                set_profile(r + 1)
                self.enqueue_grow_window(draws.window(p, 2 * D), slot ^ 1, slot)
            log = self.read_slot(slot)
            if phase_times or (phase_every > 1 and r % phase_every == 0):
                log.phase_ms = self.read_phase_ms()[0]
            p += log.depths_drawn
            draws.release(p)
            if ahead:
                yield log, self.preds_snap, ready
            else:
                draws.rewind_to(p)
                if profile_every > 0 and r + 1 == num_rounds:
                    _hip.check(self.lib.pb_profile_enable(self.ctx, 0), "pb_profile_enable")
                yield log, self.preds, now()

    def _root_value_if_inactive(self) -> None:
        # Root below capacity (N < 2*msl): the tree is a single leaf -G/(N+lambda)
        # (booster.py:503-513). The decision kernels never run for it.
        if self.N >= 2 * int(self.cfg.min_samples_leaf):
            return
        with torch.cuda.stream(self.stream):
            g = self.grad[: self.N].sum()
            self.root_grad_dev.copy_(g.reshape(1))
            h = float(self.N)
            self.values[0:1].copy_((-g.double() / (h + float(self.cfg.lambda_l2))).float().reshape(1))

    def read_round(self, depths_states: list | None = None) -> RoundLog:
        """Synchronises the stream and returns the round's decision log."""
        with torch.cuda.stream(self.stream):
            self.dec_host.copy_(self.dec_dev, non_blocking=True)
        u = np.zeros(_hip.PB_MAX_DEPTH + 1, dtype=np.int32)
        ts = ctypes.c_int32(0)
        _hip.check(self.lib.pb_frontier_counts(self.ctx, u.ctypes.data, ctypes.byref(ts),
                                               _hip.stream_ptr(self.stream)), "pb_frontier_counts")
        dec = np.frombuffer(self.dec_host.numpy().tobytes(), dtype=_hip.DECISION_DTYPE).copy()
        if not bool(torch.isfinite(self.grad[: self.N]).all()):
            raise FloatingPointError(NONFINITE_MSG)
        drawn = int(np.count_nonzero(u[: self.D] > 0))
        if u[0] > 0:
            root_grad = float(dec[0]["node_grad"])
        else:
            root_grad = float(self.root_grad_dev.cpu()[0])
        return RoundLog(u_active=u[: self.D + 1].copy(), tree_size=int(ts.value), decisions=dec,
                        root_grad=root_grad, depths_drawn=drawn)

    def run_round(self, rng: torch.Generator, events: list | None = None) -> RoundLog:
        """One round, synchronously. With `events` (or a root that cannot split) the round
        runs as per-phase C-ABI calls; otherwise as one pb_grow_round call."""
        subs, states = self.draw_subsets(rng)
        if events is None and self._root_splittable:
            self.enqueue_grow(subs, 0)
            log = self.read_slot(0)
        else:
            self.enqueue_round(subs, events)
            log = self.read_round()
        if log.depths_drawn < self.D:
            rng.set_state(states[log.depths_drawn])
        return log


def tree_arrays_from_log(log: RoundLog, cfg: PackBoostConfig, num_rows: int) -> dict[str, np.ndarray]:
    """Rebuilds one tree of the round (TreeBuilder semantics, booster.py:172-190, 499-563).

    Values are Python-double results of -G/(H + lambda) on the float32 sums, as the reference
    stores them in TreeNode.value.
    """
    lam = float(cfg.lambda_l2)
    n = max(1, int(log.tree_size))
    feature = np.full(n, -1, dtype=np.int64)
    threshold = np.zeros(n, dtype=np.int64)
    left = np.full(n, -1, dtype=np.int64)
    right = np.full(n, -1, dtype=np.int64)
    value = np.zeros(n, dtype=np.float64)
    is_leaf = np.ones(n, dtype=bool)
    # root leaf value at round start: -sum(g) / (sum(h) + lambda), h == 1 per row
    if num_rows > 0:
        value[0] = -float(np.float32(log.root_grad)) / (float(np.float32(num_rows)) + lam)
    D = int(cfg.max_depth)
    # one depth at a time (a depth's leaf values overwrite the child values its parents set),
    # each as whole-array float64 operations: the same IEEE results as Python floats
    for d in range(D):
        ua = int(log.u_active[d])
        if ua <= 0:
            break
        recs = log.decisions[(1 << d) - 1: (1 << d) - 1 + ua]
        nid = recs["node_id"].astype(np.int64)
        sp = recs["split"] != 0
        sn = nid[sp]
        if sn.size:
            r = recs[sp]
            li = r["left_id"].astype(np.int64)
            ri = r["right_id"].astype(np.int64)
            feature[sn] = r["feature"]
            threshold[sn] = r["threshold"]
            is_leaf[sn] = False
            left[sn], right[sn] = li, ri
            value[li] = -r["left_grad"].astype(np.float64) / (r["left_hess"].astype(np.float64) + lam)
            value[ri] = -r["right_grad"].astype(np.float64) / (r["right_hess"].astype(np.float64) + lam)
        ln = nid[~sp]
        if ln.size:
            r = recs[~sp]
            cnt = r["node_count"].astype(np.int64)
            den = cnt.astype(np.float32).astype(np.float64) + lam
            with np.errstate(divide="ignore", invalid="ignore"):
                v = -r["node_grad"].astype(np.float64) / den
            value[ln] = np.where(cnt == 0, 0.0, v)
            feature[ln], threshold[ln], left[ln], right[ln] = -1, 0, -1, -1
            is_leaf[ln] = True
    return {"feature": feature, "threshold": threshold, "left": left, "right": right,
            "value": value, "is_leaf": is_leaf}


def depth_log_from_round(log: RoundLog, d: int, cfg: PackBoostConfig, k: int,
                         histogram_mode: str, phase: tuple[np.ndarray, int] | None = None) -> dict:
    """Per-depth instrumentation in the reference's key set (booster.py:220-270, 565-579).

    The *_ms fields are GPU times from the library's phase events (HIP events on the fit's
    stream around each launch): hist_ms the histogram kernel, which also forms the prefix scan
    (scan_ms is therefore 0.0 and `scan_fused` says so), score_ms the DES scorer plus the
    decision step, partition_ms the partition. `phase` = (phase_ms [4][D], round) gives the
    times and the 1-based round they were measured on: the round itself when it was timed
    (log.phase_ms), else the last timed round that reached this depth (`phase_ms_round` names
    it); None when no timed round has reached the depth, and then the *_ms fields are None.
    One frontier serves the pack's B identical trees: the reference's shard dedup collapses
    B - 1 of every B shards (nodes_collapsed) and processes the rest."""
    ua = int(log.u_active[d])
    recs = log.decisions[(1 << d) - 1: (1 << d) - 1 + ua]
    rows = int(recs["node_count"].astype(np.int64).sum()) if ua else 0
    B = int(cfg.pack_size)
    rebuild = histogram_mode == "rebuild"
    ph_hist = ph_score = ph_part = ph_scan = None
    src = None
    if phase is not None and ua:
        ms, src = phase
        ph_hist = float(ms[0, d])
        ph_score = float(ms[1, d] + ms[2, d])
        ph_part = float(ms[3, d])
        ph_scan = 0.0
    out = {
        "nodes_processed": ua, "nodes_skipped": 0, "rows_total": rows,
        "feature_blocks": 1 if ua else 0, "bincount_calls": 2 if ua else 0,
        "hist_ms": ph_hist, "scan_ms": ph_scan, "score_ms": ph_score, "partition_ms": ph_part,
        "nodes_subtract_ok": 0 if rebuild else ua, "nodes_rebuild": ua if rebuild else 0,
        "nodes_subtract_fallback": 0, "nodes_collapsed": (B - 1) * ua,
        "feature_block_size": k, "depth": d, "feature_subset_size": k, "pack_size": B,
        "layer_feature_fraction": float(cfg.layer_feature_fraction),
        "histogram_mode": histogram_mode, "seed": cfg.random_state,
        "torch_threads": torch.get_num_threads(),
        "phase_ms_round": src, "scan_fused": True,
    }
    return out


def column_major_bins(bins_rowmajor: np.ndarray | torch.Tensor, perm: np.ndarray | None,
                      device: torch.device, chunk_rows: int = 1 << 18) -> torch.Tensor:
    """Row-major bins [N, F] -> device uint8 [F, ld] with rows permuted era-major.

    Transposes on the device in row chunks so host memory holds only the input.
    """
    if isinstance(bins_rowmajor, torch.Tensor):
        src = bins_rowmajor
        N, F = src.shape
    else:
        src = np.asarray(bins_rowmajor)
        N, F = src.shape
    ld = padded_rows(N)
    out = torch.zeros((F, ld), dtype=torch.uint8, device=device)
    perm_t = None
    if perm is not None:
        perm_t = torch.as_tensor(perm, dtype=torch.int64)
    for r0 in range(0, N, chunk_rows):
        r1 = min(N, r0 + chunk_rows)
        if perm_t is None:
            part = src[r0:r1]
        else:
            idx = perm_t[r0:r1]
            part = src[idx.numpy()] if isinstance(src, np.ndarray) else src[idx.to(src.device)]
        t = torch.as_tensor(part).to(device=device).view(torch.uint8)
        out[:, r0:r1] = t.t()
    return out


def bins_max(bins_fm: torch.Tensor, N: int) -> int:
    return int(bins_fm[:, :N].max().item()) if N > 0 else 0


def clamp_log2(x: float) -> int:
    return int(math.ceil(math.log2(max(1.0, x))))
