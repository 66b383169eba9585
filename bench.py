"""Headline benchmark: boosting rounds/sec of pack-parallel tree growth on one MI355X.

Workload (the north-star era panel): 2,400,000 rows x 2,376
uint8 features quantised to 5 levels, 574 contiguous eras, pack_size 8, max_depth 6,
per-depth feature fraction 0.1 (238 features), lr 0.01, lambda_dro 0.5, min_samples_leaf 20.
Inputs are synthetic and generated directly in HBM (column-major bins); one step is one full
boosting round (gradient, 6 depths of histogram -> DES score -> decide -> partition, pack
aggregation, decision read-back and host tree build), the same span as the reference's
round_seconds (booster.py:495, 654).

Also reported: the histogram kernel's achieved GB/s against the 8 TB/s HBM peak, from the
bytes this build's layouts move per launch (bin codes at half a byte per row in the nibble
layout, grad f32 and a 2-byte node id per row, the compact planes written) over the average
launch time from HIP events on the fit's stream; beside it the same time priced in the
reference's formats (one byte per bin code, 8 bytes of row state, 8 bytes per histogram cell),
and the HBM traffic rocprofv3 measured. The CPU baseline is the oracle's C restatement of the
reference's CPU split finder (frontier_cpu.cpp) under its restated fit loop, on the host cores,
at two bounded row samples extrapolated to the full rows (--cpu-full: rounds 1-3 at full size),
with the build container's reference/restatement timing ratio (oracle/calibration.json).
"""

from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
PROFILE_EVERY = 4  # timed rounds whose histogram launches carry HIP timing events
METRIC = "boosting rounds/sec (B=8,D=6, 2.4M×2376) on 1 GPU; hist-build HBM GB/s"

CONFIGS = {
    3: dict(rows=2_400_000, features=2376, eras=574, bins=5, pack_size=8, max_depth=6,
            frac=0.1, lr=0.01, lambda_dro=0.5, lambda_l2=1e-6, msl=20),
    # float features, binned on the device before the timed region
    2: dict(rows=200_000, features=100, eras=50, bins=128, pack_size=8, max_depth=5,
            frac=1.0, lr=0.1, lambda_dro=0.0, lambda_l2=1e-6, msl=20, float_features=True),
    4: dict(rows=1_000_000, features=500, eras=200, bins=255, pack_size=64, max_depth=8,
            frac=1.0, lr=0.1, lambda_dro=0.0, lambda_l2=1e-6, msl=20, float_features=True),
    # prediction only: 5M rows through 250 packs x 8 full depth-6 trees
    5: dict(rows=5_000_000, features=2376, bins=5, packs=250, pack_size=8, max_depth=6),
}


def era_offsets(n: int, e: int) -> np.ndarray:
    sizes = np.array([len(a) for a in np.array_split(np.arange(n), e)], dtype=np.int64)
    off = np.zeros(e + 1, dtype=np.int64)
    np.cumsum(sizes, out=off[1:])
    return off.astype(np.int32)


def make_device_data(c: dict, seed: int = 42):
    """Config-3 style panel in HBM: uniform 5-level bins, quantised sparse-linear target with
    era-specific sign flips on 10 of its 50 features."""
    import torch

    N, F, E, nb = c["rows"], c["features"], c["eras"], c["bins"]
    ld = (N + 15) // 16 * 16
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    bins = torch.randint(0, nb, (F, ld), dtype=torch.uint8, device="cuda", generator=g)
    cpu = torch.Generator().manual_seed(seed)
    sel = torch.randperm(F, generator=cpu)[:50]
    w = torch.randn(50, generator=cpu)
    off = era_offsets(N, E)
    era_id = torch.from_numpy(np.repeat(np.arange(E), np.diff(off))).cuda()
    flips = torch.where(torch.rand(E, 10, generator=cpu) < 0.5, -1.0, 1.0).cuda()
    lin = torch.zeros(N, device="cuda")
    center = (nb - 1) / 2.0
    for j in range(50):
        col = bins[int(sel[j]), :N].float() - center
        s = flips[era_id, j] if j < 10 else 1.0
        lin += float(w[j]) * col * s
    lin += torch.randn(N, device="cuda", generator=g) * lin.std() * 0.5
    q = torch.quantile(lin[:: max(1, N // 200_000)], torch.tensor([0.2, 0.4, 0.6, 0.8], device="cuda"))
    y = torch.bucketize(lin, q).float() / 4.0
    return bins, y, off


def host_cpu() -> dict:
    """Host CPU facts for the baseline: model, sockets, physical cores, threads per core
    (lscpu) and the CPUs this process may run on."""
    import subprocess

    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            info[key.strip()] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    def num(key):
        try:
            return int(info.get(key, ""))
        except ValueError:
            return None
    sockets, per_socket, tpc = num("Socket(s)"), num("Core(s) per socket"), num("Thread(s) per core")
    return {
        "model": info.get("Model name"),
        "sockets": sockets,
        "physical_cores": sockets * per_socket if sockets and per_socket else None,
        "threads_per_core": tpc,
        "cpus_allowed": len(os.sched_getaffinity(0)),
    }


def _calibration() -> list | None:
    """oracle/calibration.json: the build container's timing of the reference's own splitter
    against the restatement under the same fit loop (oracle/calibrate.py --write)."""
    path = ROOT / "oracle" / "calibration.json"
    try:
        return json.loads(path.read_text())
    except (OSError, ValueError):
        return None


def cpu_baseline(c: dict, budget_s: float = 12.0, full: bool = False) -> dict:
    """The reference's CPU path as it runs on the GPU box: the oracle's C restatement of its split
    finder (frontier_cpu.cpp:111-515: row-major int8 bins, serial over the sampled features,
    OpenMP over nodes) under the restated fit loop (booster.py:375-599), steady-state seconds
    per round (rounds 2.., the span of round_seconds, booster.py:495, 654). The reference itself
    is not run here; the container-measured ratio of the two (oracle/calibration.json) rides in
    the line.

    Default: rounds at two row samples n1 = N/40 and n2 = N/20 (E * 25 / E * 50 rows at least),
    extrapolated linearly in rows to N. A round's histogram and partition work grow with the
    rows; its scan and scoring (nodes x eras x features x thresholds) do not, so scaling one
    sample by N / n would overstate a full round. full=True times rounds 1-3 at N rows."""
    from oracle import oracle as ref

    N, F, E, nb = c["rows"], c["features"], c["eras"], c["bins"]
    threads = int(ref.lib().oracle_num_threads())

    def steady_at(n: int, max_rounds: int, budget: float) -> tuple[float, int]:
        rng = np.random.default_rng(0)
        bins = rng.integers(0, nb, size=(n, F), dtype=np.uint8)
        y = (rng.integers(0, 5, size=n) / 4.0).astype(np.float32)
        codes = np.repeat(np.arange(E), np.diff(era_offsets(n, E)))
        gen = __import__("torch").Generator().manual_seed(42)
        times = []
        t_start = time.perf_counter()
        while len(times) < max_rounds and (len(times) < 3 or time.perf_counter() - t_start < budget):
            r = ref.fit(bins, y, codes, num_rounds=1, pack_size=c["pack_size"], max_depth=c["max_depth"],
                        learning_rate=c["lr"], lambda_l2=c["lambda_l2"], lambda_dro=c["lambda_dro"],
                        min_samples_leaf=c["msl"], max_bins=nb, layer_feature_fraction=c["frac"], rng=gen,
                        splitter="restated")
            times.append(r.round_seconds[0])
            print(f"[bench] cpu round {len(times)} at {n} rows: {times[-1]:.2f} s", file=sys.stderr, flush=True)
        return float(np.mean(times[1:])), len(times) - 1

    if full:
        sec, k = steady_at(N, 3, 0.0)
        sample = (f"full size: {N} rows x {F} features (row-major int8), {E} eras, rounds 1-3, "
                  f"steady rounds 2-3 mean {sec:.2f} s")
    else:
        n1, n2 = max(E * 25, N // 40), max(E * 50, N // 20)
        s1, k1 = steady_at(n1, 5, budget_s / 3)
        s2, k2 = steady_at(n2, 5, 2 * budget_s / 3)
        slope = (s2 - s1) / (n2 - n1)
        sec = s2 + slope * (N - n2) if slope > 0 else s2 * N / n2
        sample = (f"{n1} and {n2} rows x {F} features (row-major int8), {E} eras, full "
                  f"{c['max_depth']}-depth rounds: steady {s1:.3f} s ({k1} rounds) and {s2:.3f} s "
                  f"({k2} rounds), extrapolated linearly in rows to {N}: {sec:.2f} s per round")
    out = {
        "value": 1.0 / sec,
        "unit": "rounds/s",
        "cores": threads,
        "kind": "port",
        "sample": sample + "; C restatement of frontier_cpu.cpp under the restated fit loop",
        "host": host_cpu(),
    }
    cal = _calibration()
    if cal:
        ratios = {r["workload"]: r["reference_over_restated"] for r in cal}
        out["calibration"] = {
            "reference_over_restated_s_per_round": ratios,
            "identical_trees": all(r.get("identical_trees") for r in cal),
            "measured": f"oracle/calibrate.py in the build container ({cal[0].get('cpu')}, "
                        f"{cal[0].get('omp_threads')} threads)",
        }
        if "config3_slice" in ratios:
            out["calibration"]["reference_estimate_value"] = out["value"] / ratios["config3_slice"]
    return out


def profiled_traffic(config: int, rows: int, summary: str = "hist_score") -> float | None:
    """HBM bytes per launch of the line's roofline kernel from the committed rocprofv3
    FETCH_SIZE/WRITE_SIZE summary of this workload (profiles/<summary>_config<N>.md, its
    `traffic_bytes_per_launch` line), or None when the workload differs from the profiled one."""
    path = ROOT / "profiles" / f"{summary}_config{config}.md"
    if rows != CONFIGS[config]["rows"] or not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def copy_probe(mib: int) -> int:
    """Reads and writes exactly `mib` MiB per launch: the reference point that scales the
    FETCH_SIZE / WRITE_SIZE counters to HBM bytes."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_mib": mib, "launches": 5}), flush=True)
    return 0


def copy_peak_gbs(mib: int = 1024, reps: int = 10) -> float:
    """HBM bytes per second (read + write) of a plain device copy of `mib` MiB, the measured
    ceiling on this box that the histogram rate is also compared with."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    gbs = 2 * n * 4 * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
    del src, dst
    torch.cuda.empty_cache()
    return gbs


def make_float_data(c: dict, seed: int = 42):
    """Configs 2 and 4: float features generated in HBM (config 2: N(0,1) with 10 columns
    correlated at 0.6, sparse-linear + tanh target with per-era shifts; config 4: half N(0,1),
    half lognormal, piecewise-constant target over 30 features), quantile-binned on the device
    (data.quantile_bin_device) into the column-major layout."""
    import torch

    from packboost_amd.data import quantile_bin_device

    N, F, E, nb = c["rows"], c["features"], c["eras"], c["bins"]
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    X = torch.randn((N, F), device="cuda", generator=g)
    off = era_offsets(N, E)
    era_id = torch.from_numpy(np.repeat(np.arange(E), np.diff(off))).cuda()
    cpu = torch.Generator().manual_seed(seed)
    if c["bins"] == 255:  # config 4
        X[:, F // 2:] = torch.exp(X[:, F // 2:])
        sel = torch.randperm(F, generator=cpu)[:30]
        cut = torch.randn(30, generator=cpu)
        w = torch.randn(30, generator=cpu)
        y = torch.zeros(N, device="cuda")
        for j in range(30):
            col = X[:, int(sel[j])]
            y += float(w[j]) * (col > float(cut[j]) + (1.0 if int(sel[j]) >= F // 2 else 0.0)).float()
    else:  # config 2
        z = torch.randn(N, device="cuda", generator=g)
        X[:, :10] = 0.6 ** 0.5 * z[:, None] + 0.4 ** 0.5 * X[:, :10]
        sel = torch.randperm(F, generator=cpu)[:20]
        w = torch.randn(20, generator=cpu)
        y = X[:, sel.cuda()] @ w.cuda() + torch.tanh(X[:, 0] * X[:, 1]) + torch.tanh(X[:, 2] - X[:, 3])
        y += (torch.randn(E, generator=cpu) * 0.2).cuda()[era_id]
    y += 0.1 * torch.randn(N, device="cuda", generator=g)
    bins, _ = quantile_bin_device(X, nb, torch.device("cuda"))
    del X
    return bins, y.float(), off


def bench_predict(args, c: dict) -> int:
    """Config 5: batched inference of 5M rows x 2376 uint8 bins (uniform over 5 levels) through a
    random-init forest of 250 packs x 8 full depth-6 trees, every tree drawn on its own (heap
    numbering = TreeBuilder's BFS ids for full trees; features U[0, F), thresholds U{0..3},
    leaves N(0, 0.01)), on the compiled forest (pb_forest_predict). Inputs are resident in HBM."""
    import torch

    from packboost_amd.booster import pack_forest

    N, F, D = c["rows"], c["features"], c["max_depth"]
    T = c["packs"] * c["pack_size"]
    ld = (N + 15) // 16 * 16
    g = torch.Generator(device="cuda")
    g.manual_seed(42)
    bins = torch.randint(0, c["bins"], (F, ld), dtype=torch.uint8, device="cuda", generator=g)
    rng = np.random.default_rng(42)
    n_nodes = (1 << (D + 1)) - 1
    inner = (1 << D) - 1
    rounds = []
    for _ in range(T):
        idx = np.arange(n_nodes)
        leaf = idx >= inner
        rounds.append({"feature": np.where(leaf, -1, rng.integers(0, F, n_nodes)),
                       "threshold": np.where(leaf, 0, rng.integers(0, 4, n_nodes)),
                       "left": np.where(leaf, -1, 2 * idx + 1), "right": np.where(leaf, -1, 2 * idx + 2),
                       "value": np.where(leaf, rng.normal(0.0, 0.01, n_nodes), 0.0), "is_leaf": leaf})
    from packboost_amd.predictor import CompiledForest

    forest = CompiledForest(pack_forest(rounds, 1, torch.device("cuda")))

    def run():
        forest.predict(bins, N, 1.0)

    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        run()
    e1.record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    # the same shape as a fitted model holds it: each pack repeats one tree pack_size times
    # (booster.py:503-519), so the compiled forest walks 250 trees, each counted 8 times
    packed = CompiledForest(pack_forest(rounds[: c["packs"]], c["pack_size"], torch.device("cuda")))
    packed.predict(bins, N, 1.0)
    e0.record()
    for _ in range(args.steps):
        packed.predict(bins, N, 1.0)
    e1.record()
    torch.cuda.synchronize()
    ms_packed = e0.elapsed_time(e1) / args.steps
    packed.close()
    bytes_compulsory = float(N) * F + N * 4
    achieved = bytes_compulsory / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "rows/sec predicted (5M x 2376 bins, 250 packs x 8 depth-6 trees) on 1 GPU",
        "value": round(N / (elapsed / args.steps), 1), "unit": "rows/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(elapsed * 1e3 / args.steps, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (bins and forest generated in HBM / seeded)",
        "config": {"workload": f"config5: {N} rows x {F} features, {T} trees of depth {D}"},
        "kernel_ms": round(ms, 3),
        "fitted_packs": {"kernel_ms": round(ms_packed, 3), "rows_per_s": round(N / (ms_packed * 1e-3), 1),
                         "forest": f"{c['packs']} packs x {c['pack_size']} identical depth-{D} trees, "
                                   "as a fitted model holds them (each pack walked once)"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(5, N, "predict"),
                     "kernel": "forest_tile_kernel",
                     "algorithmic_bytes": "N*F bin bytes read once + N*4 output (compulsory)"},
    }), flush=True)
    return 0


def other_configs(configs=(2, 4, 5), timeout_s: float = 300.0) -> dict:
    """BASELINE.json's other single-GPU configs, measured by the same run: `bench.py --config N
    --no-cpu-baseline` in a child process each (its own GPU context, after config 3's buffers are
    freed), their progress on this process's stderr. Each entry keeps the child's rate and the
    figures that locate it; a child that fails or passes `timeout_s` leaves its error instead."""
    res = {}
    for n in configs:
        print(f"[bench] config {n} in a child process", file=sys.stderr, flush=True)
        t0 = time.perf_counter()
        try:
            p = subprocess.run([sys.executable, "-u", str(Path(__file__).resolve()), "--config", str(n),
                                "--no-cpu-baseline"], stdout=subprocess.PIPE, text=True, timeout=timeout_s)
        except subprocess.TimeoutExpired:
            res[f"config{n}"] = {"error": f"no result within {timeout_s:.0f} s"}
            continue
        lines = [ln for ln in p.stdout.splitlines() if ln.startswith("{")]
        if p.returncode != 0 or not lines:
            res[f"config{n}"] = {"error": f"exit status {p.returncode}"}
            continue
        j = json.loads(lines[-1])
        keep = {k: j[k] for k in ("metric", "value", "unit", "steps", "warmup", "ms_per_step") if k in j}
        keep["workload"] = j.get("config", {}).get("workload")
        for k in ("kernel_ms", "fitted_packs", "phase_ms_per_round", "hist_ms_per_depth", "full_depth_rounds"):
            if k in j:
                keep[k] = j[k]
        if "fit_mode" in j.get("config", {}):
            keep["fit_mode"] = j["config"]["fit_mode"]
        r = j.get("roofline") or {}
        keep["roofline"] = {k: r.get(k) for k in ("kernel", "bound", "achieved", "unit", "frac")}
        keep["child_wall_s"] = round(time.perf_counter() - t0, 1)
        res[f"config{n}"] = keep
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None,
                    help="timed rounds (default 100, the rounds configs 2 and 3 run; config 4: 10, the "
                         "rounds before its default learning rate x B = 6.4 diverges and the trees stop "
                         "at the root; config 5: 20 predict calls)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed rounds first (default 3; config 4: 1)")
    ap.add_argument("--config", type=int, default=3, choices=sorted(CONFIGS))
    ap.add_argument("--rows", type=int, default=0, help="override row count (quick runs)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--cpu-full", action="store_true",
                    help="CPU baseline from rounds 1-3 at the full size (minutes) instead of two samples")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 5 plain device copies of MIB MiB (counter calibration)")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="config 3 only (by default its line also carries configs 2, 4 and 5)")
    args = ap.parse_args()
    if args.copy_probe:
        return copy_probe(args.copy_probe)
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the path would shard by feature, one slice of the bin columns per GPU).",
              file=sys.stderr)
        return 2

    import torch

    from packboost_amd import PackBoostConfig
    from packboost_amd.backends import _hip
    from packboost_amd.engine import DeviceFit, tree_arrays_from_log

    c = dict(CONFIGS[args.config])
    if args.rows:
        c["rows"] = args.rows
    if args.steps is None:
        args.steps = {4: 10, 5: 20}.get(args.config, 100)  # config 5: predict calls
    if args.warmup is None:
        args.warmup = 1 if args.config == 4 else 3
    torch.cuda.set_device(0)
    copy_gbs = copy_peak_gbs()
    if args.config == 5:
        return bench_predict(args, c)
    bins, y, off = make_float_data(c) if c.get("float_features") else make_device_data(c)
    N = c["rows"]
    cfg = PackBoostConfig(pack_size=c["pack_size"], max_depth=c["max_depth"], learning_rate=c["lr"],
                          lambda_l2=c["lambda_l2"], lambda_dro=c["lambda_dro"],
                          min_samples_leaf=c["msl"], max_bins=c["bins"],
                          layer_feature_fraction=c["frac"], random_state=42, prebinned=True)
    fit = DeviceFit(bins, N, y, off, cfg)
    rng = torch.Generator().manual_seed(42)
    print(f"[bench] config {args.config}: N={N} F={c['features']} E={c['eras']} K={fit.K} "
          f"warmup={args.warmup} steps={args.steps}", file=sys.stderr, flush=True)
    for log, _, _ in fit.rounds(rng, args.warmup):
        tree_arrays_from_log(log, cfg, N)
    torch.cuda.synchronize()
    D = fit.D

    def read_profile():
        ms = np.zeros(4 * _hip.PB_MAX_DEPTH, dtype=np.float64)
        n = np.zeros(4 * _hip.PB_MAX_DEPTH, dtype=np.int64)
        _hip.check(fit.lib.pb_profile_read(fit.ctx, ms.ctypes.data, n.ctypes.data), "pb_profile_read")
        return ms.reshape(4, -1)[:, :D], n.reshape(4, -1)[:, :D]

    # Timed region: the histogram launches of every PROFILE_EVERY-th round are bracketed by HIP
    # events on the fit's stream (each event is a queue barrier, so only those rounds pay it).
    logs = []
    t0 = time.perf_counter()
    for log, _, _ in fit.rounds(rng, args.steps, profile_every=PROFILE_EVERY, profile_mode=2):
        tree_arrays_from_log(log, cfg, N)
        logs.append(log)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps
    prof_ms, prof_n = read_profile()
    # Untimed: the per-phase breakdown, every phase bracketed by events, on a fresh fit that
    # replays the first rounds of the same seed (later rounds can grow smaller trees).
    fit.close()
    n_phase = min(args.warmup + args.steps, 20)
    fit = DeviceFit(bins, N, y, off, cfg)
    for log, _, _ in fit.rounds(torch.Generator().manual_seed(42), n_phase, profile_every=1,
                                profile_mode=1):
        tree_arrays_from_log(log, cfg, N)
    torch.cuda.synchronize()
    phase_raw, _ = read_profile()
    fit.close()

    # Untimed for `value`: the same rounds with the per-round train era correlation that
    # PackBoost.fit logs (pb_era_corr on a side stream, read back each round), the reference's
    # log_metrics outside its round_seconds span (booster.py:654-655).
    from packboost_amd.booster import _era_corr_device

    fit = DeviceFit(bins, N, y, off, cfg)
    side = torch.cuda.Stream()
    era_off_dev = torch.from_numpy(np.asarray(off, dtype=np.int32)).cuda()
    corr_scratch = torch.empty(len(off), dtype=torch.float64, device="cuda")
    rng_m = torch.Generator().manual_seed(42)
    corr = float("nan")

    def rounds_with_metrics(n: int) -> None:
        nonlocal corr
        for log, preds_after, ready in fit.rounds(rng_m, n):
            tree_arrays_from_log(log, cfg, N)
            with torch.cuda.stream(side):
                side.wait_event(ready)
                corr = _era_corr_device(y, preds_after, era_off_dev, corr_scratch)

    rounds_with_metrics(args.warmup)
    torch.cuda.synchronize()
    t_m = time.perf_counter()  # the same rounds as the timed region, bracketed the same way
    rounds_with_metrics(args.steps)
    torch.cuda.synchronize()
    with_metrics_s = time.perf_counter() - t_m

    # histogram roofline, summed over the profiled rounds. Algorithmic bytes per launch, with the
    # reference formats' per-unit figures: rows of active nodes x K (one byte per bin code)
    # + rows x 8 (grad f32, node id 4 B) + cells U x E x K x nb x 8 (count i32 + grad f32);
    # hess is not moved by this build, so it is not counted. Moved bytes: what this build's
    # layouts carry (K/2 or K bin bytes per row, grad 4 B + node id 2 B, compact planes).
    K, E, nb = fit.K, fit.E, fit.nb
    bin_bytes = 0.5 if fit.bins4 is not None else 1.0
    moved_bytes = 0.0
    phase_ms = {name: float(phase_raw[i].sum()) for i, name in
                enumerate(("hist", "score", "decide", "partition"))}
    hist_bytes = 0.0
    # a segment-mode fit builds no planes from its first fused depth on: those depths' fused
    # histogram + scorer launches are not part of this histogram roofline
    hist_depths = fit.seg_from if fit.segments else D
    for r, log in enumerate(logs):
        if r % PROFILE_EVERY:
            continue
        for d in range(hist_depths):
            u = int(log.u_active[d])
            if u == 0:
                continue
            base = (1 << d) - 1
            rows = int(log.decisions[base: base + u]["node_count"].astype(np.int64).sum())
            hist_bytes += rows * K + rows * 8 + u * E * K * nb * 8
            moved_bytes += rows * K * bin_bytes + rows * 6 + u * E * (K * (nb - 1) * 6 + 8)
    # launches per depth that had active nodes (a round that stops early still launches its
    # deeper depths, which exit at once; they are not counted as launches of the kernel)
    n_act = np.zeros(D, dtype=np.int64)
    for r, log in enumerate(logs):
        if r % PROFILE_EVERY == 0:
            n_act += (np.asarray(log.u_active[:D]) > 0)
    hist_ms = float(prof_ms[0][:hist_depths].sum())
    n_hist = int(n_act[:hist_depths].sum())
    achieved = moved_bytes / (hist_ms * 1e-3) / 1e9 if hist_ms > 0 else 0.0
    ref_format_gbs = hist_bytes / (hist_ms * 1e-3) / 1e9 if hist_ms > 0 else 0.0
    rounds_per_s = args.steps / elapsed
    metric = METRIC if args.config == 3 else (
        f"boosting rounds/sec (B={c['pack_size']},D={c['max_depth']}, {N}x{c['features']}) on 1 GPU; "
        "hist-build HBM GB/s")
    out = {
        "metric": metric,
        "value": round(rounds_per_s, 4),
        "unit": "rounds/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": ("synthetic (float features generated in HBM, quantile-binned on the device)"
                 if c.get("float_features") else
                 "synthetic (generated in HBM: uniform 5-level bins, quantised sparse-linear target)"),
        "config": {
            "workload": (f"config{args.config}: {N} rows x {c['features']} features, {c['eras']} eras, "
                         f"{c['bins']} bins, B={c['pack_size']}, D={c['max_depth']}, K={K}/depth"),
            "rows": N, "features": c["features"], "eras": c["eras"], "max_bins": c["bins"],
            "pack_size": c["pack_size"], "max_depth": c["max_depth"], "features_per_depth": K,
            "fit_mode": (f"segments (fused from depth {fit.seg_from})" if fit.segments else "planes"),
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": profiled_traffic(args.config, N),
            "kernel": "hist_era_kernel",
            "bin_layout": "nibble" if fit.bins4 is not None else "u8",
            "avg_launch_ms": round(hist_ms / max(n_hist, 1), 4),
            "algorithmic_bytes_per_launch": round(moved_bytes / max(n_hist, 1)),
            "algorithmic_bytes": ("per depth: rows*K*b (bin codes, b = 1/2 nibble or 1 uint8) + rows*6 "
                                  "(grad f32, node id u16) + U*E*(K*(nb-1)*6 + 8) (compact planes "
                                  "written); rows = rows of the depth's active nodes"),
            "copy_peak_gbs": round(copy_gbs, 1),
            "frac_of_copy_peak": round(achieved / copy_gbs, 4) if copy_gbs > 0 else None,
            "reference_format_bytes_per_launch": round(hist_bytes / max(n_hist, 1)),
            "reference_format_gbs": round(ref_format_gbs, 1),
            "reference_format_frac": round(ref_format_gbs / HBM_PEAK_GBS, 4),
            "reference_format_bytes": "rows*K*1 + rows*8 + U*E*K*nb*8 per depth (reference layouts, no hess)",
        },
        "with_round_metrics": {
            "rounds_per_s": round(args.steps / with_metrics_s, 4),
            "ms_per_round": round(with_metrics_s * 1e3 / args.steps, 4),
            "metric": "train era correlation per round on the device (pb_era_corr), as PackBoost.fit logs it",
            "last_train_corr": round(corr, 6),
        },
        "profiled_rounds": {"hist_events": f"every {PROFILE_EVERY}th timed round",
                            "phase_breakdown": f"first {n_phase} rounds replayed untimed"},
        "phase_ms_per_round": {k: round(v / n_phase, 4) for k, v in phase_ms.items()},
        "hist_ms_per_depth": [round(float(prof_ms[0, d]) / max(1, int(n_act[d])), 4)
                              for d in range(D)],
        # score + decide per depth, over the replayed rounds (a depth's launches in rounds that
        # stopped above it take no time)
        "score_ms_per_depth": [round(float(phase_raw[1, d]) / n_phase, 4) for d in range(D)],
        "full_depth_rounds": int(sum(1 for log in logs if int(log.u_active[D - 1]) > 0)),
        "cpu_baseline": None,
    }
    fit.close()
    del bins
    torch.cuda.empty_cache()
    if args.config == 3 and not args.rows and not args.no_other_configs:
        out["other_configs"] = other_configs()
    if not args.no_cpu_baseline and args.config == 3:
        print("[bench] timing the CPU restatement of the reference frontier", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(c, args.cpu_budget, full=args.cpu_full)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
