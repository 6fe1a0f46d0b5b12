"""Build the gfx950 HIP library `tallax_amd/_build/libtallax_hip.so`.

One hipcc invocation per source (parallel), then one link.  Every HIP source is
compiled with:
  * --offload-arch=gfx950 (MI355X only);
  * -ffp-contract=off, so every float operation on the sampler path is a single
    IEEE binary32 operation that the numpy oracle reproduces bit for bit;
  * -Xclang -target-feature -Xclang -packed-fp32-ops, which keeps the compiler
    from emitting packed-FP32 VALU instructions.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_build"
LIB_NAME = "libtallax_hip.so"
LIB_PATH = OUT_DIR / LIB_NAME

SOURCES = [
    "capi.hip",
    "row_select.hip",
    "scan_gather.hip",
    "sort_rows.hip",
    "sort_wide.hip",
    "binned.hip",
    "softmax_topk.hip",
    "sample_wide.hip",
    "testing.hip",
]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    f"-I{CSRC}",
    f"-I{PKG.parent / 'include'}",
]


def _compile(src: str, obj_dir: pathlib.Path) -> pathlib.Path:
    obj = obj_dir / (pathlib.Path(src).stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = True) -> pathlib.Path:
    """Compile every HIP source for gfx950 and link the shared library."""
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    OUT_DIR.mkdir(exist_ok=True)
    obj_dir = OUT_DIR / "obj"
    obj_dir.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(lambda s: _compile(s, obj_dir), SOURCES))
    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
