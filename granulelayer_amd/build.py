"""Build the HIP library in-tree: granulelayer_amd/lib/libgranulelayer_amd.so (gfx950 only).

Usage: ``python -m granulelayer_amd.build`` (or ``__graft_entry__.build()``).  Every source is
compiled with hipcc for gfx950 in parallel, then linked into one shared library that exports the
C ABI declared in include/granulelayer_amd.h.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "lib"
LIB = OUT_DIR / "libgranulelayer_amd.so"
# the LDS gather-rate probe behind `bench.py --lds-probe`: a measurement tool in a library of its
# own, never loaded by the layer
PROBE_SRC = CSRC / "probe" / "gl_lds_probe.hip"
PROBE_LIB = OUT_DIR / "libgl_lds_probe.so"
ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
SOURCES = ["gl_abi.hip", "gl_forward.hip", "gl_backward.hip", "gl_max_bwd.hip", "gl_edges.hip", "gl_adam.hip",
           "gl_sched.hip", "gl_cover.hip"]
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # keep the compiler from emitting packed fp32 (v_pk_*_f32) instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    f"-I{ROOT / 'include'}",
]


def _compile(src: str, obj_dir: Path) -> Path:
    obj = obj_dir / (Path(src).stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def _build_probe() -> Path:
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, *FLAGS, "-shared", "-o", str(tmp), str(PROBE_SRC)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {PROBE_SRC.name}:\n{r.stderr}")
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


def build(verbose: bool = False) -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    obj_dir = PKG / "_build"
    obj_dir.mkdir(exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES) + 1)) as ex:
        probe = ex.submit(_build_probe)
        objs = list(ex.map(lambda s: _compile(s, obj_dir), SOURCES))
        probe.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} and {PROBE_LIB.name}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
