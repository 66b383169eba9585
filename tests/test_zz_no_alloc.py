"""pb_rowlist_partition_noalloc: the row-list partition without a caller workspace (a fixed
device array per device instead), for callers that cannot allocate. Called through the C ABI
twice in a row, the second call smaller than the first (the array keeps the first call's
contents), each against pb_rowlist_partition with its own workspace: left/right row lists and
per-era splits bit-identical, status words all zero; plus the size limit, rejected on the host.
"""

from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import make_problem, node_era_rows


def _inputs(seed, N, F, E, nb, U):
    import torch

    p = make_problem(seed, N, F, E, nb, U)
    ner = node_era_rows(p)
    rows, nrs, nes = [], [0], []
    for eras in ner:
        rel = [0]
        for r in eras:
            rows.append(r)
            rel.append(rel[-1] + r.size)
        nes.append(rel)
        nrs.append(nrs[-1] + rel[-1])
    dev = torch.device("cuda")
    rng = np.random.default_rng(seed + 1)
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a, dtype=dt)).to(dev)  # noqa: E731
    ld = (N + 15) // 16 * 16
    bfm = np.zeros((F, ld), np.uint8)
    bfm[:, :N] = p["bins"].T
    return dict(bins=t(bfm, np.uint8), N=N, ld=ld, F=F, rows=t(np.concatenate(rows), np.int32),
                nrs=t(nrs, np.int32), nes=t(nes, np.int32), S=U, E=E,
                feat=t(rng.integers(0, F, U), np.int32), thr=t(rng.integers(0, nb - 1, U), np.int32))


def _partition(hip, d, noalloc):
    import torch

    lib = hip.load()
    dev = torch.device("cuda")
    R = int(d["rows"].numel())
    left = torch.full((R,), -1, dtype=torch.int32, device=dev)
    right = torch.full((R,), -1, dtype=torch.int32, device=dev)
    ls = torch.full((d["S"], d["E"] + 1), -1, dtype=torch.int32, device=dev)
    rs = torch.full((d["S"], d["E"] + 1), -1, dtype=torch.int32, device=dev)
    common = (d["bins"].data_ptr(), d["N"], d["ld"], d["F"], d["rows"].data_ptr(), R, d["nrs"].data_ptr(),
              d["nes"].data_ptr(), d["S"], d["E"], d["feat"].data_ptr(), d["thr"].data_ptr(),
              left.data_ptr(), right.data_ptr(), R, ls.data_ptr(), rs.data_ptr())
    if noalloc:
        status = torch.full((4,), 7, dtype=torch.int32, device=dev)
        hip.check(lib.pb_rowlist_partition_noalloc(*common, status.data_ptr(), hip.stream_ptr()),
                  "pb_rowlist_partition_noalloc")
    else:
        work = torch.empty(int(lib.pb_rowlist_work_elems(d["S"], d["E"])), dtype=torch.int32, device=dev)
        hip.check(lib.pb_rowlist_partition(*common, work.data_ptr(), hip.stream_ptr()), "pb_rowlist_partition")
        status = work[:4]
    torch.cuda.synchronize()
    return [x.cpu().numpy() for x in (left, right, ls, rs, status)]


@pytest.mark.gpu
def test_noalloc_partition_matches_workspace_call(hip):
    big = (11, 200_000, 9, 30, 16, 40)
    small = (12, 20_000, 6, 12, 7, 7)
    for case in (big, small):
        print(f"[noalloc] seed={case[0]} N={case[1]} E={case[3]} S={case[5]}", flush=True)
        d = _inputs(*case)
        want = _partition(hip, d, noalloc=False)
        got = _partition(hip, d, noalloc=True)
        for a, b in zip(got, want):
            np.testing.assert_array_equal(a, b)
        assert not got[4].any()


def test_noalloc_partition_rejects_oversize():
    """Checked on the host before any device work (runs without a GPU)."""
    from packboost_amd.backends import _hip

    lib = _hip.load()
    cap = int(lib.pb_rowlist_noalloc_max_segments())
    assert cap >= 1_000_000
    E = 1000
    S = cap // E + 1
    rc = lib.pb_rowlist_partition_noalloc(None, 10, 16, 1, None, 0, None, None, S, E, None, None, None, None,
                                          0, None, None, None, None)
    assert rc == _hip.PB_ERR_UNSUPPORTED
    assert b"static workspace" in lib.pb_last_error()
