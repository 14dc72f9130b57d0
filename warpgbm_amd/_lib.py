"""ctypes binding of the C ABI in ``include/warpgbm_amd.h``.

``torch`` is imported before the library is loaded: both link the HIP
runtime ``libamdhip64.so.7``, and loading torch first makes the dynamic loader
resolve our dependency to torch's copy, so device pointers and streams are
shared between torch and the kernels.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libwarpgbm_amd.so"

# flags of wgbm_histogram_segments (include/warpgbm_amd.h)
CODES_NATIVE = 1

_p = C.c_void_p
_i32 = C.c_int32
_i64 = C.c_int64
_f32 = C.c_float

# name -> (restype, argtypes)
SIGNATURES = {
    "wgbm_version": (C.c_char_p, []),
    "wgbm_last_error": (C.c_char_p, []),
    "wgbm_compute_histogram3": (C.c_int, [_p, _i64, _i64, _p, _p, _i64, _p, _i64, _p, _i32,
                                          _p, _p, _i32, _i32, _i32, _p]),
    "wgbm_compute_split": (C.c_int, [_p, _p, _i32, _i32, _i32, _f32, _f32, _f32, _p, _p, _i32, _p]),
    "wgbm_custom_cuda_binner": (C.c_int, [_p, _i64, _p, _i32, _p, _p]),
    "wgbm_predict_forest": (C.c_int, [_p, _i64, _i64, _p, _i64, _i64, _f32, _p, _p]),
    "wgbm_histogram_segments": (C.c_int, [_p, _i64, _i64, _i32, _p, _p, _p, _i32, _i64, _i32,
                                          _i32, _p, _p, _p]),
    "wgbm_histogram_segments_noalloc": (C.c_int, [_p, _i64, _i64, _i32, _p, _p, _p, _i32, _i64,
                                                  _i32, _i32, _p, _p, _p]),
    "wgbm_quantile_edges": (C.c_int, [_p, _i64, _i32, _p, _i32, _p, _p]),
    "wgbm_quantile_edges_matrix": (C.c_int, [_p, _i64, _i32, _i64, _p, _i32, _p, _p]),
    "wgbm_quantile_stage_rows": (C.c_int, [_p, _i64, _i32, _i64, _i64, _p, _i64, _p, _p, _p]),
    "wgbm_quantile_edges_staged": (C.c_int, [_p, _i64, _i32, _i64, _p, _p, _p, _i32, _p, _p]),
    "wgbm_bin_matrix": (C.c_int, [_p, _i64, _i32, _i64, _p, _i32, _p, _i64, _p, _p]),
    "wgbm_copy_prebinned": (C.c_int, [_p, _i64, _i32, _i64, _p, _i64, _p, _i32, _p, _p]),
    "wgbm_predict_heap": (C.c_int, [_p, _i64, _i64, _i32, _p, _p, _p, _i32, _i32, _i32, _i32,
                                    _f32, _p, _p]),
    "wgbm_importance_add": (C.c_int, [_p, _i32, _i32, _p, _p, _p, _p]),
    "wgbm_softmax_rows": (C.c_int, [_p, _i64, _i32, _p]),
    "wgbm_engine_create": (C.c_int, [C.POINTER(_p), _p]),
    "wgbm_engine_round": (C.c_int, [_p, _p, _p, _p, _i32, _p, _p]),
    "wgbm_engine_set_tuning": (C.c_int, [_p, _i32, _i64]),
    "wgbm_engine_destroy": (None, [_p]),
    "wgbm_timer_enable": (None, [_i32]),
    "wgbm_timer_read": (C.c_int, [C.c_char_p, C.POINTER(C.c_double), C.POINTER(_i64)]),
    "wgbm_timer_reset": (None, []),
    "wgbm_probe_lds_atomics": (C.c_int, [_i32, _i32, C.POINTER(C.c_double), _p]),
    "wgbm_probe_hbm_read": (C.c_int, [_p, _i64, _i32, C.POINTER(C.c_double), _p]),
    "wgbm_release_scratch": (None, []),
}


class EngineConfig(C.Structure):
    _fields_ = [
        ("n_rows", _i64),
        ("n_feats", _i32),
        ("codes_stride", _i64),
        ("num_bins", _i32),
        ("num_eras", _i32),
        ("max_depth", _i32),
        ("n_trees", _i32),
        ("objective", _i32),
        ("min_child_weight", _f32),
        ("min_split_gain", _f32),
        ("l2_reg", _f32),
        ("learning_rate", _f32),
        ("codes_rm", _p),
        ("codes_cm", _p),
        ("root_order", _p),
        ("era_start", _p),
        ("level_bytes", _i64),
    ]


class TreeRecord(C.Structure):
    _fields_ = [
        ("feat", _p),
        ("bin", _p),
        ("leaf", _p),
        ("count", _p),
        ("gain", _p),
        ("H", _i32),
    ]


class WgbmError(RuntimeError):
    """A warpgbm_amd C-ABI call failed."""


_LIB = None


def load(path: str | os.PathLike | None = None) -> C.CDLL:
    """Load (once) and return the library.  Raises if it has not been built."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    import torch  # noqa: F401  (see module docstring)

    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise WgbmError(
            f"{p} not found: build the HIP library first (python -m warpgbm_amd.build)")
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().wgbm_last_error().decode(errors="replace")
        raise WgbmError(f"{what} failed (code {rc}): {msg}")


_raw_stream = None


def current_stream_ptr(device=None) -> int:
    """torch's current HIP stream on ``device`` (a torch.device, an index or
    None for the current device) as an integer handle.  Uses torch's raw
    accessor when this build has it (a fraction of a microsecond: the
    drop-in ops are called once per node or column), else the public API."""
    global _raw_stream
    import torch

    if _raw_stream is None:
        _raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", False)
    if _raw_stream:
        if device is None:
            idx = torch.cuda.current_device()
        elif isinstance(device, int):
            idx = device
        else:
            if not isinstance(device, torch.device):
                device = torch.device(device)
            idx = device.index if device.index is not None else torch.cuda.current_device()
        return int(_raw_stream(idx))
    return int(torch.cuda.current_stream(device).cuda_stream)
