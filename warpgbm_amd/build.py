"""Build the HIP library ``warpgbm_amd/libwarpgbm_amd.so`` for gfx950 and the
host extension ``warpgbm_amd._trees``.

Every ``csrc/*.hip`` file is compiled by hipcc to an object in ``_build/`` and
the objects are linked into one shared library that exports the C ABI of
``include/warpgbm_amd.h``.  ``csrc/trees.c`` (tree records -> the reference's
tree dicts, a CPython extension) is compiled by the host C compiler.  Run
``python -m warpgbm_amd.build`` (or call :func:`build`); both are written
in-tree so that they travel with the source tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = ROOT / "_build" / "hip"
LIB = PKG / "libwarpgbm_amd.so"
ARCH = os.environ.get("WGBM_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    # IEEE float32 semantics are part of the contract: no implicit FMA contraction
    "-ffp-contract=off",
    # keep the compiler from emitting packed-FP32 VALU instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    f"-I{ROOT / 'include'}",
]


def _hipcc() -> str:
    h = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(h).exists():
        raise RuntimeError("hipcc not found; ROCm is required to build warpgbm_amd")
    return h


def _compile(src: Path) -> Path:
    out = OBJ / (src.stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr}")
    return out


def build_trees(verbose: bool = False) -> Path:
    """Compile the ``_trees`` CPython extension (plain C, no GPU code)."""
    out = PKG / ("_trees" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out.with_name(out.name + ".tmp")
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        raise RuntimeError("no host C compiler (gcc) found to build warpgbm_amd._trees")
    cmd = [cc, "-O2", "-shared", "-fPIC", "-Wall", f"-I{sysconfig.get_paths()['include']}",
           str(CSRC / "trees.c"), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"gcc failed for trees.c:\n{r.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}")
    return out


def build(verbose: bool = False) -> Path:
    """Compile all HIP sources and link the shared library (returns its
    path), then the ``_trees`` host extension."""
    build_trees(verbose)
    OBJ.mkdir(parents=True, exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
