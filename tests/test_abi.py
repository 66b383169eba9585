"""The C ABI without a GPU: the library loads, exports every entry point include/*.h
declares, the Python bindings' struct layouts match the header's (checked by compiling the
header with the host C compiler), and argument errors come back as status codes with a
message (no device work is started)."""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_functions() -> set[str]:
    names = set()
    for h in HEADERS:
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)  # drop comments
        text = re.sub(r"//[^\n]*", " ", text)
        for m in re.finditer(r"^[\w \t\*]*?\b(pb_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_header_declares_entry_points():
    names = declared_functions()
    assert {"pb_ctx_create", "pb_hist_build", "pb_des_score", "pb_partition", "pb_predict_pack",
            "pb_grow_round", "pb_last_error", "pb_version"} <= names


def test_library_exports_every_declared_symbol():
    from packboost_amd.backends import _hip

    lib = _hip.load()
    names = declared_functions()
    assert names == set(_hip.EXPORTED_SYMBOLS), names ^ set(_hip.EXPORTED_SYMBOLS)
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing


def test_status_codes_without_device():
    from packboost_amd.backends import _hip

    lib = _hip.load()
    assert lib.pb_version() == 100
    out = ctypes.c_void_p()
    # null dims: rejected on the host before any HIP call
    assert lib.pb_ctx_create(None, None, ctypes.byref(out)) == -1
    assert lib.pb_last_error().decode()
    dims = _hip.PbDims(num_rows=100, ld=100, num_features=3, num_eras=1, max_bins=300,
                       max_depth=3, max_feats=3, min_samples_leaf=1)  # ld % 16 != 0, nb > 255
    offs = np.array([0, 100], np.int32)
    assert lib.pb_ctx_create(ctypes.byref(dims), offs.ctypes.data, ctypes.byref(out)) < 0
    assert lib.pb_last_error().decode()
    assert lib.pb_grow_round(None, None, None, 0, None, None, None) == -1
    assert lib.pb_profile_enable(None, 1) == -1


def _c_layout() -> dict[str, int]:
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no host C compiler")
    probe = r"""
#include <stdio.h>
#include <stddef.h>
#include "packboost_hip.h"
#define S(t) printf(#t " %zu\n", sizeof(t));
#define O(t, f) printf(#t "." #f " %zu\n", offsetof(t, f));
int main(void) {
  S(pb_dims) O(pb_dims, ld) O(pb_dims, num_features) O(pb_dims, min_samples_leaf)
  S(pb_split_params) O(pb_split_params, era_alpha) O(pb_split_params, min_samples_leaf)
  O(pb_split_params, cut_selection) O(pb_split_params, skip_last_bin)
  S(pb_decision) O(pb_decision, score) O(pb_decision, left_count) O(pb_decision, node_grad)
  O(pb_decision, node_count)
  S(pb_candidate) O(pb_candidate, left_total) O(pb_candidate, valid)
  S(pb_round_header) O(pb_round_header, tree_size)
  S(pb_fit_buffers) O(pb_fit_buffers, values_dev) O(pb_fit_buffers, pack_size)
  O(pb_fit_buffers, learning_rate) O(pb_fit_buffers, params)
  return 0;
}
"""
    import tempfile

    with tempfile.TemporaryDirectory() as td:
        src = Path(td) / "probe.c"
        exe = Path(td) / "probe"
        src.write_text(probe)
        subprocess.run([cc, "-std=c11", "-I", str(ROOT / "include"), str(src), "-o", str(exe)],
                       check=True)
        out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    return {k: int(v) for k, v in (line.split() for line in out.splitlines())}


def test_struct_layouts_match_header():
    from packboost_amd.backends import _hip

    c = _c_layout()
    assert c["pb_dims"] == ctypes.sizeof(_hip.PbDims)
    for f in ("ld", "num_features", "min_samples_leaf"):
        assert c[f"pb_dims.{f}"] == getattr(_hip.PbDims, f).offset
    assert c["pb_split_params"] == ctypes.sizeof(_hip.PbSplitParams)
    for f in ("era_alpha", "min_samples_leaf", "cut_selection", "skip_last_bin"):
        assert c[f"pb_split_params.{f}"] == getattr(_hip.PbSplitParams, f).offset
    assert c["pb_fit_buffers"] == ctypes.sizeof(_hip.PbFitBuffers)
    for f in ("values_dev", "pack_size", "learning_rate", "params"):
        assert c[f"pb_fit_buffers.{f}"] == getattr(_hip.PbFitBuffers, f).offset
    assert c["pb_decision"] == _hip.DECISION_DTYPE.itemsize
    for f in ("score", "left_count", "node_grad", "node_count"):
        assert c[f"pb_decision.{f}"] == _hip.DECISION_DTYPE.fields[f][1]
    assert c["pb_candidate"] == _hip.CANDIDATE_DTYPE.itemsize
    for f in ("left_total", "valid"):
        assert c[f"pb_candidate.{f}"] == _hip.CANDIDATE_DTYPE.fields[f][1]
    assert c["pb_round_header"] == _hip.HEADER_DTYPE.itemsize
    assert c["pb_round_header.tree_size"] == _hip.HEADER_DTYPE.fields["tree_size"][1]


def test_product_path_has_no_cpu_fallback():
    """Without the HIP device the public API raises instead of computing on the CPU."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    from packboost_amd import PackBoost, PackBoostConfig

    X = np.random.default_rng(0).integers(0, 4, size=(64, 3)).astype(np.uint8)
    with pytest.raises(RuntimeError):
        PackBoost(PackBoostConfig(max_bins=4)).fit(X, np.zeros(64, np.float32), None, num_rounds=1)


def test_error_codes_match_header():
    import re

    from packboost_amd.backends import _hip

    text = (Path(__file__).resolve().parents[1] / "include" / "packboost_hip.h").read_text()
    codes = {m.group(1): int(m.group(2)) for m in
             re.finditer(r"#define (PB_(?:OK|ERR_\w+))\s+\(?(-?\d+)\)?", text)}
    assert codes["PB_OK"] == 0 and len(codes) >= 6
    for name, value in codes.items():
        assert getattr(_hip, name) == value, name
