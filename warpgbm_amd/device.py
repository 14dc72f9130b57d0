"""Device-side building blocks of the estimator: ingestion and binning, era
bookkeeping, the level-wise engine and ensemble inference.

Everything here runs the HIP library through its C ABI; torch only provides
device memory, copies and the stream.  Calling any of it without the built
library (or without a GPU) raises -- there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import concurrent.futures as cf
import os
import threading
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib


def _stream(dev) -> int:
    return _lib.current_stream_ptr(dev)


def codes_stride(n_feats: int) -> int:
    """Row stride (bytes) of the int8 code matrix: a multiple of 16, and of 128
    once a row spans several cache lines, so that the 256-byte feature chunks
    read by one histogram workgroup never straddle a row boundary."""
    if n_feats <= 128:
        return (n_feats + 15) // 16 * 16
    return (n_feats + 127) // 128 * 128


def quantile_levels(num_bins: int) -> torch.Tensor:
    """``torch.linspace(0, 1, num_bins + 1)[1:-1]`` in float32 (warpgbm/core.py:529-531)."""
    return torch.linspace(0, 1, num_bins + 1, dtype=torch.float32)[1:-1].contiguous()


@dataclass
class Codes:
    """Binned matrix on the device.  ``rm`` is the library's native row-major
    layout for ``num_bins`` (every byte in [0, num_bins + 1]: codes in
    [0, num_bins) as is, negative codes as num_bins, codes >= num_bins and
    padding as num_bins + 1); ``cm`` the raw column-major copy."""
    rm: torch.Tensor        # int8 [n, stride]
    cm: torch.Tensor | None  # int8 [F, n]
    n: int
    n_feats: int
    stride: int
    num_bins: int


def _alloc_codes(n: int, F: int, dev, with_cm: bool, num_bins: int) -> Codes:
    S = codes_stride(F)
    rm = torch.empty((n, S), dtype=torch.int8, device=dev)
    cm = torch.empty((F, n), dtype=torch.int8, device=dev) if with_cm else None
    return Codes(rm, cm, n, F, S, num_bins)


def upload_prebinned(X: np.ndarray, dev, with_cm: bool, num_bins: int) -> Codes:
    """Integer input whose columns are all < num_bins is used as codes directly
    (warpgbm/core.py:499-517); values are cast to int8 like the reference's
    ``bin_indices[:, f] = torch.as_tensor(X[:, f])``."""
    X = np.asarray(X)
    x8 = upload_int8(X if X.dtype == np.int8 else X.astype(np.int8), dev)
    return codes_from_int8(x8, with_cm, num_bins)[0]


def upload_int8(X: np.ndarray, dev) -> torch.Tensor:
    """int8 [n, F] contiguous copy of an int8 host matrix on the device."""
    return _upload_staged(X, dev, np.int8, torch.int8)


def codes_from_int8(x8: torch.Tensor, with_cm: bool, num_bins: int, check: bool = False):
    """Native codes for num_bins from an int8 [n, F] device matrix
    (``wgbm_copy_prebinned``).  With check, also whether some value is
    >= num_bins (found in the same pass over the matrix); else None."""
    n, F = x8.shape
    dev = x8.device
    c = _alloc_codes(n, F, dev, with_cm, num_bins)
    flag = torch.empty(1, dtype=torch.int32, device=dev) if check else None
    lib = _lib.load()
    rc = lib.wgbm_copy_prebinned(x8.data_ptr(), n, F, F, c.rm.data_ptr(), c.stride,
                                 c.cm.data_ptr() if c.cm is not None else None, int(num_bins),
                                 flag.data_ptr() if flag is not None else None, _stream(dev))
    _lib.check(rc, "copy_prebinned")
    return c, (bool(flag.item()) if flag is not None else None)


_STAGE_BYTES = 64 << 20   # one pinned staging buffer
_STAGE_COUNT = 4          # buffers in rotation
_NARROW_CHUNK_ROWS = 131072  # rows per chunk of a column-subset upload
_stage_lock = threading.Lock()
_stage_bufs: list = []
_pool = None


def _staging():
    """Reusable pinned host buffers (allocated pinned, never registered)."""
    global _pool
    with _stage_lock:
        if not _stage_bufs:
            for _ in range(_STAGE_COUNT):
                _stage_bufs.append(torch.empty(_STAGE_BYTES, dtype=torch.uint8, pin_memory=True))
        if _pool is None:
            _pool = cf.ThreadPoolExecutor(max(1, min(8, os.cpu_count() or 1)))
    return _stage_bufs, _pool


def upload_float(X: np.ndarray, dev) -> torch.Tensor:
    """float32 [n, F] contiguous copy of X on the device (float64 input is
    rounded to float32 first, as ``torch.as_tensor(..., dtype=float32)``)."""
    return _upload_staged(X, dev, np.float32, torch.float32)


def _streams(X: np.ndarray, esize: int) -> bool:
    """Whether _upload_staged streams X through the staging buffers."""
    n, F = X.shape
    return n * esize * max(F, 1) >= 4 * _STAGE_BYTES and X.flags.c_contiguous


def _upload_staged(X: np.ndarray, dev, np_dtype, torch_dtype, on_chunk=None,
                   row_align: int = 1) -> torch.Tensor:
    """[n, F] contiguous copy of X on the device in np_dtype.

    Large inputs are streamed through pinned staging buffers: host threads
    fill one buffer (converting the dtype on the way) while the DMA engine
    copies the previous ones on a side stream.  ``on_chunk(out, r0, r1,
    stream)`` (streamed inputs only) enqueues work on rows [r0, r1) of the
    device copy on that side stream right after their copy; chunks then
    start on multiples of ``row_align`` rows."""
    X = np.asarray(X)
    n, F = X.shape
    esize = np.dtype(np_dtype).itemsize
    row_bytes = esize * max(F, 1)
    if not _streams(X, esize):
        return torch.from_numpy(np.ascontiguousarray(X, dtype=np_dtype)).to(dev)
    out = torch.empty((n, F), dtype=torch_dtype, device=dev)
    bufs, pool = _staging()
    rows_per = max(1, _STAGE_BYTES // row_bytes)
    rows_per = max(row_align, rows_per // row_align * row_align)
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    events = [None] * len(bufs)
    nthreads = pool._max_workers

    def fill(dst, lo, hi):
        np.copyto(dst[lo:hi], X[r0 + lo:r0 + hi], casting="same_kind")

    for i, r0 in enumerate(range(0, n, rows_per)):
        r1 = min(n, r0 + rows_per)
        k = i % len(bufs)
        if events[k] is not None:
            events[k].synchronize()  # the DMA that used this buffer has finished
        host = bufs[k][: (r1 - r0) * row_bytes].view(torch_dtype).view(r1 - r0, F)
        dst = host.numpy()
        step = max(1, (r1 - r0 + nthreads - 1) // nthreads)
        list(pool.map(lambda a: fill(dst, a, min(a + step, r1 - r0)), range(0, r1 - r0, step)))
        with torch.cuda.stream(side):
            out[r0:r1].copy_(host, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(side)
            if on_chunk is not None:
                on_chunk(out, r0, r1, side.cuda_stream)
        events[k] = ev
    torch.cuda.current_stream(dev).wait_stream(side)
    out.record_stream(side)
    for ev in events:
        if ev is not None:
            ev.synchronize()  # buffers are reused by the next upload
    return out


def upload_and_bin(X: np.ndarray, edges: torch.Tensor, dev, cols=None, on_chunk=None) -> Codes:
    """Row-major native codes of a host float matrix for known edges
    [F, num_bins - 1] (predict-time binning, warpgbm/core.py:902-915): the rows
    stream through the pinned staging buffers and a few device chunk buffers;
    the copies run back to back on a copy stream and each chunk is binned on
    a compute stream as soon as its copy lands, so the float matrix is never
    whole on the device and the binning overlaps the transfer.

    With ``cols`` (feature indices) only those columns are gathered (host
    threads, straight into the staging buffers), uploaded and binned: code
    column j holds feature cols[j].  ``on_chunk(codes_rows, r0, r1)`` is
    called after each chunk's binning is enqueued, with the compute stream
    current, so work on those rows (the predictors) overlaps the next copies;
    when the input is not streamed it is called once for all rows."""
    X = np.asarray(X)
    n, F = X.shape
    edges = edges.to(device=dev, dtype=torch.float32).contiguous()
    if edges.shape[0] != F:
        raise ValueError(f"edges for {edges.shape[0]} features, X has {F}")
    if cols is not None:
        cols = np.ascontiguousarray(cols, dtype=np.intp)
        if cols.ndim != 1 or len(cols) == 0 or cols.min() < 0 or cols.max() >= F:
            raise ValueError("cols must be a non-empty list of feature indices")
        edges = edges[torch.from_numpy(cols).to(dev)].contiguous()
    Fw = F if cols is None else len(cols)
    row_bytes = 4 * max(Fw, 1)
    if (n * 4 * max(F, 1) < 4 * _STAGE_BYTES and cols is None) or not X.flags.c_contiguous:
        Xs = X if cols is None else np.take(X, cols, axis=1)
        c = bin_matrix(upload_float(Xs, dev), edges, with_cm=False)
        if on_chunk is not None:
            on_chunk(c, 0, n)
        return c
    c = _alloc_codes(n, Fw, dev, False, edges.shape[1] + 1)
    bufs, pool = _staging()
    rows_per = max(1, _STAGE_BYTES // row_bytes)
    if cols is not None:
        rows_per = min(rows_per, _NARROW_CHUNK_ROWS)  # several chunks in flight
    dbufs = [torch.empty((rows_per, Fw), dtype=torch.float32, device=dev)
             for _ in range(len(bufs))]
    lib = _lib.load()
    # copies on one stream, binning (and on_chunk's work) on another: chunk
    # i's copy waits for the binning that last read its device buffer, chunk
    # i's binning for its copy
    cur = torch.cuda.current_stream(dev)
    copy_st = torch.cuda.Stream(device=dev)
    comp_st = torch.cuda.Stream(device=dev)
    copy_st.wait_stream(cur)
    comp_st.wait_stream(cur)
    comp_ptr = comp_st.cuda_stream
    events = [None] * len(bufs)   # copy done: the staging buffer can be refilled
    freed = [None] * len(bufs)    # binning done: the device buffer can be overwritten
    nthreads = pool._max_workers

    def fill(dst, lo, hi):
        src = X[r0 + lo:r0 + hi]
        if cols is None:
            np.copyto(dst[lo:hi], src, casting="same_kind")
        elif X.dtype == np.float32:
            np.take(src, cols, axis=1, out=dst[lo:hi], mode="clip")  # cols are in range
        else:
            np.copyto(dst[lo:hi], np.take(src, cols, axis=1), casting="same_kind")

    for i, r0 in enumerate(range(0, n, rows_per)):
        r1 = min(n, r0 + rows_per)
        k = i % len(bufs)
        if events[k] is not None:
            events[k].synchronize()  # the copy that used this staging buffer is done
        host = bufs[k][: (r1 - r0) * row_bytes].view(torch.float32).view(r1 - r0, Fw)
        dst = host.numpy()
        step = max(1, (r1 - r0 + nthreads - 1) // nthreads)
        list(pool.map(lambda a: fill(dst, a, min(a + step, r1 - r0)), range(0, r1 - r0, step)))
        with torch.cuda.stream(copy_st):
            if freed[k] is not None:
                copy_st.wait_event(freed[k])  # the binning of chunk i - len(bufs) read it
            dbufs[k][: r1 - r0].copy_(host, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(copy_st)
        events[k] = ev
        comp_st.wait_event(ev)
        rc = lib.wgbm_bin_matrix(dbufs[k].data_ptr(), r1 - r0, Fw, Fw, edges.data_ptr(),
                                 edges.shape[1], c.rm.data_ptr() + r0 * c.stride, c.stride, None,
                                 comp_ptr)
        _lib.check(rc, "bin_matrix")
        fe = torch.cuda.Event()
        fe.record(comp_st)
        freed[k] = fe
        if on_chunk is not None:
            with torch.cuda.stream(comp_st):
                on_chunk(Codes(c.rm[r0:r1], None, r1 - r0, Fw, c.stride, c.num_bins), r0, r1)
    cur.wait_stream(comp_st)
    cur.wait_stream(copy_st)
    c.rm.record_stream(comp_st)
    for b in dbufs:
        b.record_stream(copy_st)
        b.record_stream(comp_st)
    for ev in events:
        if ev is not None:
            ev.synchronize()  # staging buffers are reused by the next upload
    return c


def upload_float_with_edges(X: np.ndarray, dev, num_bins: int):
    """float32 device copy of X and its quantile edges [F, num_bins - 1]
    (warpgbm/core.py:519-534).  A streamed upload stages each row block's
    values for the selection as soon as the block lands
    (``wgbm_quantile_stage_rows`` on the copy stream, hidden behind the
    transfer of the next blocks); the edges are then taken from the staged
    columns (``wgbm_quantile_edges_staged``), bit-identical to
    ``quantile_edges`` of the whole copy."""
    X = np.asarray(X)
    n, F = X.shape
    if not _streams(X, 4) or F == 0 or num_bins < 2:
        Xd = upload_float(X, dev)
        return Xd, quantile_edges(Xd, num_bins)
    st = QuantileStage(n, F, dev)
    Xd = _upload_staged(X, dev, np.float32, torch.float32,
                        on_chunk=lambda out, r0, r1, sp: st.stage(out, r0, r1, sp), row_align=32)
    return Xd, st.edges(num_bins)


class QuantileStage:
    """Column-major staging of an [n, F] float32 matrix for the quantile
    selection (``wgbm_quantile_stage_rows`` per row block, in any order),
    then the edges of all n rows (``wgbm_quantile_edges_staged``)."""

    def __init__(self, n: int, F: int, dev):
        if n > (1 << 24):
            raise ValueError("quantile() input tensor is too large (more than 2^24 rows per "
                             "feature)")
        self.n, self.F, self.dev = n, F, dev
        self.ks = (n + 31) // 32 * 32
        self.cols = torch.empty((F, self.ks), dtype=torch.int32, device=dev)
        self.kmin = torch.full((F,), -1, dtype=torch.int32, device=dev)  # 0xffffffff
        self.kmax = torch.zeros((F,), dtype=torch.int32, device=dev)
        self.lib = _lib.load()

    def stage(self, Xd: torch.Tensor, r0: int, r1: int, stream_ptr=None) -> None:
        """Rows [r0, r1) of the device matrix Xd (r0 a multiple of 4)."""
        sp = _stream(self.dev) if stream_ptr is None else stream_ptr
        rc = self.lib.wgbm_quantile_stage_rows(Xd[r0].data_ptr(), r1 - r0, self.F,
                                               Xd.stride(0), r0, self.cols.data_ptr(), self.ks,
                                               self.kmin.data_ptr(), self.kmax.data_ptr(), sp)
        _lib.check(rc, "quantile_stage_rows")

    def edges(self, num_bins: int) -> torch.Tensor:
        q = quantile_levels(num_bins).to(self.dev)
        nq = num_bins - 1
        edges = torch.empty((self.F, nq), dtype=torch.float32, device=self.dev)
        rc = self.lib.wgbm_quantile_edges_staged(self.cols.data_ptr(), self.n, self.F, self.ks,
                                                 self.kmin.data_ptr(), self.kmax.data_ptr(),
                                                 q.data_ptr(), nq, edges.data_ptr(),
                                                 _stream(self.dev))
        _lib.check(rc, "quantile_edges_staged")
        return edges


def quantile_edges(Xd: torch.Tensor, num_bins: int) -> torch.Tensor:
    """Per-feature quantile edges [F, num_bins - 1] (the torch.quantile call of
    warpgbm/core.py:529-534), by radix selection on the device
    (``wgbm_quantile_edges_matrix``)."""
    n, F = Xd.shape
    if n > (1 << 24):
        raise ValueError("quantile() input tensor is too large (more than 2^24 rows per feature)")
    dev = Xd.device
    q = quantile_levels(num_bins).to(dev)
    nq = num_bins - 1
    edges = torch.empty((F, nq), dtype=torch.float32, device=dev)
    lib = _lib.load()
    rc = lib.wgbm_quantile_edges_matrix(Xd.data_ptr(), n, F, F, q.data_ptr(), nq,
                                        edges.data_ptr(), _stream(dev))
    _lib.check(rc, "quantile_edges_matrix")
    return edges


def quantile_edges_sorted(sorted_cols: torch.Tensor, num_bins: int) -> torch.Tensor:
    """Edges from columns already sorted ascending, [F, n] (``wgbm_quantile_edges``)."""
    F, n = sorted_cols.shape
    dev = sorted_cols.device
    q = quantile_levels(num_bins).to(dev)
    edges = torch.empty((F, num_bins - 1), dtype=torch.float32, device=dev)
    rc = _lib.load().wgbm_quantile_edges(sorted_cols.data_ptr(), n, F, q.data_ptr(),
                                         num_bins - 1, edges.data_ptr(), _stream(dev))
    _lib.check(rc, "quantile_edges")
    return edges


def bin_matrix(Xd: torch.Tensor, edges: torch.Tensor, with_cm: bool) -> Codes:
    """All columns binned in one launch (the per-feature binner loop of
    warpgbm/core.py:527-538 and :908-913)."""
    n, F = Xd.shape
    edges = edges.to(device=Xd.device, dtype=torch.float32).contiguous()
    if edges.shape[0] != F:
        raise ValueError(f"edges for {edges.shape[0]} features, X has {F}")
    c = _alloc_codes(n, F, Xd.device, with_cm, edges.shape[1] + 1)
    lib = _lib.load()
    rc = lib.wgbm_bin_matrix(Xd.data_ptr(), n, F, F, edges.data_ptr(), edges.shape[1],
                             c.rm.data_ptr(), c.stride,
                             c.cm.data_ptr() if c.cm is not None else None, _stream(Xd.device))
    _lib.check(rc, "bin_matrix")
    return c


def era_id_int32(era_id: np.ndarray) -> np.ndarray:
    """The era ids as the reference sees them: torch.from_numpy(era_id)
    .type(torch.int32) (warpgbm/core.py:493), i.e. floats truncated toward
    zero (1.2 and 1.7 are one era), wider integers wrapped to 32 bits, bools
    0/1; dtypes torch cannot take (strings, objects) raise TypeError as there."""
    era = np.asarray(era_id).reshape(-1)
    if era.dtype == np.int32:
        return era
    return torch.from_numpy(np.ascontiguousarray(era)).type(torch.int32).numpy()


def era_layout(era_id: np.ndarray):
    """Sorted unique eras, era index per row, rows sorted by era (stable) and
    era offsets (warpgbm/core.py:540: torch.unique(..., return_inverse=True)
    over the int32 era ids of :493).  Era ids that are already non-decreasing
    (one era, or contiguous eras) take a linear path with the same result as
    the sort."""
    era = era_id_int32(era_id)
    n = era.shape[0]
    if n > 0 and (n == 1 or bool(np.all(era[1:] >= era[:-1]))):
        first = np.ones(n, dtype=bool)
        first[1:] = era[1:] != era[:-1]
        idx = np.flatnonzero(first)
        uniq = era[idx]
        inv = (np.cumsum(first) - 1).astype(np.int32)
        order = np.arange(n, dtype=np.int32)
        start = np.empty(len(idx) + 1, dtype=np.int64)
        start[:-1] = idx
        start[-1] = n
        return uniq, inv, order, start
    uniq, inv = np.unique(era, return_inverse=True)
    inv = inv.astype(np.int32).reshape(-1)
    order = np.argsort(inv, kind="stable").astype(np.int32)
    counts = np.bincount(inv, minlength=len(uniq)).astype(np.int64)
    start = np.zeros(len(uniq) + 1, dtype=np.int64)
    np.cumsum(counts, out=start[1:])
    return uniq, inv, order, start


class Engine:
    """Owner of a native level-wise engine (``wgbm_engine_*``)."""

    def __init__(self, codes: Codes, root_order: torch.Tensor, era_start: torch.Tensor,
                 num_bins: int, num_eras: int, max_depth: int, n_trees: int, objective: int,
                 min_child_weight: float, min_split_gain: float, l2_reg: float,
                 learning_rate: float, level_bytes: int = 0):
        self.lib = _lib.load()
        self._keep = (codes, root_order, era_start)
        cfg = _lib.EngineConfig(
            n_rows=codes.n, n_feats=codes.n_feats, codes_stride=codes.stride, num_bins=num_bins,
            num_eras=num_eras, max_depth=max_depth, n_trees=n_trees, objective=objective,
            min_child_weight=float(min_child_weight), min_split_gain=float(min_split_gain),
            l2_reg=float(l2_reg), learning_rate=float(learning_rate),
            codes_rm=codes.rm.data_ptr(), codes_cm=codes.cm.data_ptr(),
            root_order=root_order.data_ptr(), era_start=era_start.data_ptr(),
            level_bytes=int(level_bytes))
        h = C.c_void_p()
        _lib.check(self.lib.wgbm_engine_create(C.byref(h), C.byref(cfg)), "engine_create")
        self.h = h
        self.H = (1 << (max_depth + 1)) - 1
        self.n_trees = n_trees
        self.num_eras = num_eras

    def set_tuning(self, key: int, value: int) -> None:
        _lib.check(self.lib.wgbm_engine_set_tuning(self.h, key, value), "engine_set_tuning")

    def round(self, target: torch.Tensor, pred: torch.Tensor, feat_sel: torch.Tensor,
              rec: dict) -> None:
        r = _lib.TreeRecord(feat=rec["feat"].data_ptr(), bin=rec["bin"].data_ptr(),
                            leaf=rec["leaf"].data_ptr(), count=rec["count"].data_ptr(),
                            gain=rec["gain"].data_ptr(), H=self.H)
        rc = self.lib.wgbm_engine_round(self.h, target.data_ptr(), pred.data_ptr(),
                                        feat_sel.data_ptr(), feat_sel.numel(), C.byref(r),
                                        _stream(pred.device))
        _lib.check(rc, "engine_round")

    def close(self) -> None:
        if getattr(self, "h", None):
            self.lib.wgbm_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def predict_heap(codes: Codes, feat: torch.Tensor, bin_: torch.Tensor, leaf: torch.Tensor,
                 n_rounds: int, K: int, max_depth: int, learning_rate: float,
                 out: torch.Tensor) -> None:
    """Add the contributions of ``n_rounds`` rounds of K heap-ordered trees to
    ``out`` [n, K] (one launch; cf. warpgbm/core.py:917-932, 991-1030)."""
    H = (1 << (max_depth + 1)) - 1
    lib = _lib.load()
    rc = lib.wgbm_predict_heap(codes.rm.data_ptr(), codes.n, codes.stride, codes.num_bins,
                               feat.data_ptr(), bin_.data_ptr(), leaf.data_ptr(), n_rounds, K, H,
                               max_depth, float(learning_rate), out.data_ptr(),
                               _stream(out.device))
    _lib.check(rc, "predict_heap")


def importance_add(acc: torch.Tensor, gain: torch.Tensor, node: torch.Tensor,
                   feat_start: torch.Tensor) -> None:
    """acc [E, F] float32 += the gain rows ``gain`` [*, E] of ``node`` (int64,
    grouped by feature: group f = node[feat_start[f]:feat_start[f+1]]), in
    order, one float32 add at a time (cf. warpgbm/core.py:624-627)."""
    E, F = acc.shape
    assert acc.is_contiguous() and gain.is_contiguous() and acc.dtype == torch.float32
    assert node.dtype == torch.int64 and feat_start.dtype == torch.int64
    assert feat_start.numel() == F + 1
    lib = _lib.load()
    rc = lib.wgbm_importance_add(acc.data_ptr(), F, E, gain.data_ptr(), node.data_ptr(),
                                 feat_start.data_ptr(), _stream(acc.device))
    _lib.check(rc, "importance_add")


def rows_of(values: np.ndarray, n: int, dev) -> torch.Tensor:
    """float32 [n, K] on the device, every row equal to ``values`` [K] (a
    broadcast on the device: no host-side tile and no n * K upload)."""
    v = torch.from_numpy(np.ascontiguousarray(values, dtype=np.float32)).to(dev)
    return v.reshape(1, -1).expand(n, v.numel()).contiguous()


def cols_of(values: np.ndarray, n: int, dev) -> torch.Tensor:
    """float32 [K, n] on the device, row k filled with ``values[k]`` (the
    class-major layout of rows_of)."""
    v = torch.from_numpy(np.ascontiguousarray(values, dtype=np.float32)).to(dev)
    return v.reshape(-1, 1).expand(v.numel(), n).contiguous()


def to_host(t: torch.Tensor) -> np.ndarray:
    """A device tensor as a numpy array, copied through page-locked memory
    (a DMA at full link speed; a plain ``.cpu()`` stages pageable memory at a
    fraction of it).  The array keeps its page-locked block until it is freed."""
    if not t.is_cuda:
        return t.numpy()
    h = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
    h.copy_(t)
    return h.numpy()


def softmax_rows(x: torch.Tensor) -> None:
    lib = _lib.load()
    n, K = x.shape
    _lib.check(lib.wgbm_softmax_rows(x.data_ptr(), n, K, _stream(x.device)), "softmax_rows")
