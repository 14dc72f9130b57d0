"""The HIP library loads and exports every symbol include/warpgbm_amd.h declares
(CPU: no compute call is made)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "warpgbm_amd.h"
LIB = ROOT / "warpgbm_amd" / "libwarpgbm_amd.so"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wgbm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_reference_ops():
    syms = declared_symbols()
    for name in ("wgbm_compute_histogram3", "wgbm_compute_split", "wgbm_custom_cuda_binner",
                 "wgbm_predict_forest"):
        assert name in syms


def test_library_exports_every_declared_symbol():
    if not LIB.exists():
        from warpgbm_amd import build

        build.build()
    lib = ctypes.CDLL(str(LIB))
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, f"not exported: {missing}"


def test_python_binding_covers_the_header():
    from warpgbm_amd import _lib

    assert set(declared_symbols()) == set(_lib.SIGNATURES)


def test_error_reporting_without_gpu_work():
    """Argument validation happens before any HIP call and reports through
    wgbm_last_error."""
    from warpgbm_amd import _lib

    lib = _lib.load()
    assert lib.wgbm_version().decode().startswith("warpgbm_amd")
    rc = lib.wgbm_compute_split(None, None, 0, 1, 1, 0.0, 1.0, 0.0, None, None, 0, None)
    assert rc == 1000
    assert "bad split shape" in lib.wgbm_last_error().decode()
    rc = lib.wgbm_compute_histogram3(None, 10, 5, None, None, 4, None, 5, None, 1, None, None,
                                     200, 64, 4, None)
    assert rc == 1000 and "num_bins" in lib.wgbm_last_error().decode()


def test_noalloc_size_check_without_gpu_work():
    """The no-allocation entry point refuses a call whose working memory
    exceeds its fixed array before any HIP call, naming both sizes."""
    from warpgbm_amd import _lib

    lib = _lib.load()
    one = ctypes.c_void_p(1)  # never dereferenced: the size check comes first
    rc = lib.wgbm_histogram_segments_noalloc(one, 1 << 24, 1024, 1000, one, one, one, 1, 1 << 24,
                                             32, 0, one, one, None)
    assert rc == 1000
    msg = lib.wgbm_last_error().decode()
    assert "needs" in msg and str(64 * 1024 * 1024) in msg
