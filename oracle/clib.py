"""ctypes loader of the oracle's C helpers (test infrastructure only)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from .build import OUT, build

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not OUT.exists():
            build()
        L = C.CDLL(str(OUT))
        p, i32, i64 = C.c_void_p, C.c_int32, C.c_int64
        L.oracle_hist_exact.argtypes = [p, i64, p, p, i64, p, i32, p, i32, i32, p, p]
        L.oracle_hist_exact.restype = None
        L.oracle_expf.argtypes = [C.c_float]
        L.oracle_expf.restype = C.c_float
        L.oracle_expf_array.argtypes = [p, i64, p]
        L.oracle_softmax_residual.argtypes = [p, p, i64, i32, p]
        L.oracle_softmax_rows.argtypes = [p, i64, i32]
        L.oracle_quantile_sorted.argtypes = [p, i64, p, i32, p]
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def hist_exact_q(codes, q, rows, feats, era, E, B):
    """Same contract as ops.histogram_exact_q, computed by a C loop."""
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    q32 = np.ascontiguousarray(q, dtype=np.int32)
    rows = None if rows is None else np.ascontiguousarray(rows, dtype=np.int32)
    feats = np.ascontiguousarray(feats, dtype=np.int32)
    era32 = None if E == 1 else np.ascontiguousarray(era, dtype=np.int32)
    F = len(feats)
    Q = np.empty((E, F, B), np.int64)
    Cn = np.empty((E, F, B), np.int64)
    n = codes.shape[0] if rows is None else len(rows)
    lib().oracle_hist_exact(_ptr(codes), codes.shape[1], _ptr(q32), _ptr(rows), n, _ptr(feats),
                            F, _ptr(era32), E, B, _ptr(Q), _ptr(Cn))
    return Q, Cn


def quantile_sorted(s, q):
    s = np.ascontiguousarray(s, dtype=np.float32)
    q = np.ascontiguousarray(q, dtype=np.float32)
    out = np.empty(len(q), np.float32)
    lib().oracle_quantile_sorted(_ptr(s), len(s), _ptr(q), len(q), _ptr(out))
    return out


def expf(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().oracle_expf_array(_ptr(x), x.size, _ptr(out))
    return out


def softmax_residual(logits, labels):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    labels = np.ascontiguousarray(labels, dtype=np.int32)
    n, K = logits.shape
    r = np.empty((K, n), np.float32)
    lib().oracle_softmax_residual(_ptr(logits), _ptr(labels), n, K, _ptr(r))
    return r


def softmax_rows(x):
    x = np.array(x, dtype=np.float32, copy=True, order="C")
    n, K = x.shape
    lib().oracle_softmax_rows(_ptr(x), n, K)
    return x
