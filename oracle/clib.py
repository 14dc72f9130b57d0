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
        L.oracle_quantile_edges_matrix.argtypes = [p, i64, i64, i64, p, i32, p]
        L.oracle_bin_matrix.argtypes = [p, i64, i64, i64, p, i32, p, i64]
        L.oracle_predict_tables.argtypes = [p, i64, i64, p, i32, i32, p, i32, C.c_float, p]
        L.oracle_num_threads.restype = C.c_int
        L.oracle_split_scan_q.argtypes = [p, p, i64, i32, i32, p, C.c_float, C.c_float, p, p]
        L.oracle_era_absmax.argtypes = [p, p, i64, p, i32, p]
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


def quantile_edges_matrix(X, num_bins):
    """[F, B-1] torch.quantile edges of every column of the row-major float32
    matrix X (the C loop of ops.quantile_edges, for full-size inputs)."""
    from . import ops

    X = np.ascontiguousarray(X, dtype=np.float32)
    n, F = X.shape
    q = np.ascontiguousarray(ops.quantile_levels(num_bins), dtype=np.float32)
    out = np.empty((F, num_bins - 1), np.float32)
    lib().oracle_quantile_edges_matrix(_ptr(X), n, F, F, _ptr(q), len(q), _ptr(out))
    return out


def bin_matrix(X, edges):
    """int8 codes [n, F] of X against edges [F, B-1] (ops.bin_matrix in C)."""
    X = np.ascontiguousarray(X, dtype=np.float32)
    edges = np.ascontiguousarray(edges, dtype=np.float32)
    n, F = X.shape
    assert edges.shape[0] == F
    out = np.empty((n, F), np.int8)
    lib().oracle_bin_matrix(_ptr(X), n, F, F, _ptr(edges), edges.shape[1], _ptr(out), F)
    return out


def predict_tables(codes, tables, lr, out, cls=None):
    """ops.predict_table in C over many trees: out [n, K] (or [n]) is updated
    in tree order with float32(lr * leaf); tree t adds to column cls[t]."""
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    tables = np.ascontiguousarray(tables, dtype=np.float32)
    T, M, _ = tables.shape
    o = np.array(out, dtype=np.float32, copy=True, order="C")
    K = 1 if o.ndim == 1 else o.shape[1]
    c = None if cls is None else np.ascontiguousarray(cls, dtype=np.int32)
    assert c is None or len(c) == T
    lib().oracle_predict_tables(_ptr(codes), codes.shape[0], codes.shape[1], _ptr(tables), T, M,
                                _ptr(c), K, np.float32(lr), _ptr(o))
    return o


def split_scan_q(Q, Cn, s, min_child_samples, eps):
    """ops.split_scan(ops.dequantise(Q, s), float32(Cn), ...) in one C loop:
    gain, dir [E, F, B-1] from exact histograms Q, Cn [E, F, B]; s is one
    shift for every era or an array of E per-era shifts."""
    Q = np.ascontiguousarray(Q, dtype=np.int64)
    Cn = np.ascontiguousarray(Cn, dtype=np.int64)
    E, F, B = Q.shape
    s_era = np.ascontiguousarray(np.broadcast_to(np.asarray(s, dtype=np.int32).reshape(-1), (E,)),
                                 dtype=np.int32)
    gain = np.empty((E, F, B - 1), np.float32)
    dirn = np.empty((E, F, B - 1), np.float32)
    lib().oracle_split_scan_q(_ptr(Q), _ptr(Cn), E * F, B, F, _ptr(s_era),
                              np.float32(min_child_samples), np.float32(eps), _ptr(gain), _ptr(dirn))
    return gain, dirn


def era_absmax(r, rows, era, E):
    """[E] largest |r| over the rows of each era among ``rows`` (float32),
    computed by a C loop (ops.era_absmax is the same in numpy)."""
    r = np.ascontiguousarray(r, dtype=np.float32)
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    era = np.ascontiguousarray(era, dtype=np.int32)
    out = np.empty(E, np.uint32)
    lib().oracle_era_absmax(_ptr(r), _ptr(rows), len(rows), _ptr(era), E, _ptr(out))
    return out.view(np.float32)


def num_threads():
    """Threads of the OpenMP loops (OMP_NUM_THREADS, else every core)."""
    return int(lib().oracle_num_threads())
