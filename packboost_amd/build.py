"""Builds libpackboost_hip.so (gfx950) in-tree with hipcc.

Every HIP source is compiled with:
  -ffp-contract=off      no FMA contraction: the DES scorer and the pack aggregation issue
                         the reference's float32 operations one rounding at a time;
  -packed-fp32-ops off   no packed-FP32 VALU instructions (gfx950 code is plain FP32 VALU).
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libpackboost_hip.so"
LIB_PATH = PKG_DIR / LIB_NAME
SOURCES = ["hist.hip", "score.hip", "partition.hip", "predict.hip", "metrics.hip", "binning.hip", "rowlist.hip", "segment.hip",
           "capi.cpp"]
ARCH = "gfx950"


def hipcc() -> str:
    cand = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(cand).exists():
        raise RuntimeError("hipcc not found (ROCm toolchain required to build the HIP backend)")
    return cand


def compile_flags() -> list[str]:
    return [
        "-x", "hip",
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wall",
        "-Wno-unused-function",
        "-I", str(PKG_DIR.parent / "include"),
    ]


# Kernels that must not use scratch (register spills): the histogram, the scorers and the K-cut
# selection. One build of the single-feature histogram tile that spilled returned wrong plane
# counts for a code generation it took only with the spills, so a spill here fails the build.
NO_SCRATCH = re.compile(r"hist_era_kernel|seg_score_kernel|des_score|kcuts_kernel")


def spilling_kernels(remarks: str) -> list[str]:
    """Names of NO_SCRATCH kernels whose kernel-resource-usage remarks report ScratchSize > 0."""
    out, name = [], None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and name and int(m.group(1)) > 0 and NO_SCRATCH.search(name):
            out.append(name)
    return out


def build(verbose: bool = False) -> Path:
    """Compiles every source for gfx950 and links the shared library. Always rebuilds."""
    cc = hipcc()
    out_dir = PKG_DIR / "_build"
    out_dir.mkdir(exist_ok=True)

    def one(src: str) -> Path:
        obj = out_dir / (Path(src).stem + ".o")
        cmd = [cc, *compile_flags(), "-Rpass-analysis=kernel-resource-usage", "-c", str(CSRC / src),
               "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
        spilled = spilling_kernels(res.stderr)
        if spilled:
            raise RuntimeError(f"{src}: register spills (scratch) in {', '.join(spilled)}; the histogram "
                               "and scorer kernels must fit their registers")
        if verbose:
            warn = "\n".join(l for l in res.stderr.splitlines() if "remark:" not in l)
            if warn.strip():
                print(warn, file=sys.stderr)
        return obj

    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(one, SOURCES))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
