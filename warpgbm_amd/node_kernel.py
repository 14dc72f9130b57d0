"""Drop-in mirror of the reference's native op module ``warpgbm.cuda.node_kernel``.

The reference binds four CUDA launchers with pybind11
(warpgbm/cuda/node_kernel.cpp:41-47).  This module exposes the same four
names with the same argument order and meaning, taking torch tensors that
live on the GPU, and forwards to the HIP implementation through the C ABI of
``include/warpgbm_amd.h``.  Launches go on torch's current stream.

Differences from the reference, all stricter:
* dtype / device / contiguity / shape mismatches raise ``RuntimeError``
  (the reference's ``data_ptr<T>()`` raises only on dtype; launch errors are
  printed and swallowed there, raised here);
* results are deterministic: histogram sums are exact sums of the residuals
  quantised with a power-of-two scale (28 significant bits), rounded once to
  float32; predictions add trees in tree order.
"""
from __future__ import annotations

import torch

from . import _lib


def _need(t: torch.Tensor, name: str, dtype: torch.dtype, ndim: int | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"{name} must be a torch.Tensor")
    if t.dtype != dtype:
        raise RuntimeError(f"{name} must have dtype {dtype}, got {t.dtype}")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor, got device {t.device}")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if ndim is not None and t.dim() != ndim:
        raise RuntimeError(f"{name} must be {ndim}-D, got shape {tuple(t.shape)}")


def compute_histogram3(bin_indices, residuals, sample_indices, feature_indices, era_indices,
                       grad_hist, hess_hist, num_bins, threads_per_block=256,
                       rows_per_thread=1) -> None:
    """Accumulate per-(era, feature, bin) residual sums and row counts.

    Mirrors warpgbm/cuda/histogram_kernel.cu:63-104: ``grad_hist[e, f, b] +=
    residuals[s]`` and ``hess_hist[e, f, b] += 1`` for every s in
    ``sample_indices`` with ``e = era_indices[s]`` and
    ``b = bin_indices[s, feature_indices[f]]`` in ``[0, num_bins)``.  The number
    of eras is ``grad_hist.size(0)``.
    """
    _need(bin_indices, "bin_indices", torch.int8, 2)
    _need(residuals, "residuals", torch.float32, 1)
    _need(sample_indices, "sample_indices", torch.int32, 1)
    _need(feature_indices, "feature_indices", torch.int32, 1)
    _need(era_indices, "era_indices", torch.int32, 1)
    _need(grad_hist, "grad_hist", torch.float32, 3)
    _need(hess_hist, "hess_hist", torch.float32, 3)
    E, F, B = grad_hist.shape
    if tuple(hess_hist.shape) != (E, F, B):
        raise RuntimeError("hess_hist must have the shape of grad_hist")
    if F != feature_indices.numel():
        raise RuntimeError("grad_hist.size(1) must equal len(feature_indices)")
    if B < num_bins:
        raise RuntimeError(f"grad_hist.size(2)={B} is smaller than num_bins={num_bins}")
    if B != num_bins:
        raise RuntimeError("grad_hist.size(2) must equal num_bins")
    N, Fm = bin_indices.shape
    if residuals.numel() != N or era_indices.numel() != N:
        raise RuntimeError("residuals and era_indices must have one entry per row of bin_indices")
    lib = _lib.load()
    rc = lib.wgbm_compute_histogram3(
        bin_indices.data_ptr(), N, Fm, residuals.data_ptr(), sample_indices.data_ptr(),
        sample_indices.numel(), feature_indices.data_ptr(), F, era_indices.data_ptr(), E,
        grad_hist.data_ptr(), hess_hist.data_ptr(), int(num_bins), int(threads_per_block),
        int(rows_per_thread), _lib.current_stream_ptr(bin_indices.device))
    _lib.check(rc, "compute_histogram3")


def compute_split(G, H, min_split_gain, min_child_samples, eps, per_era_gain, per_era_direction,
                  threads=128) -> None:
    """Per-era split gain and direction (warpgbm/cuda/best_split_kernel.cu:61-88)."""
    _need(G, "G", torch.float32, 3)
    _need(H, "H", torch.float32, 3)
    _need(per_era_gain, "per_era_gain", torch.float32, 3)
    _need(per_era_direction, "per_era_direction", torch.float32, 3)
    E, F, B = G.shape
    if tuple(H.shape) != (E, F, B):
        raise RuntimeError("H must have the shape of G")
    if B < 2:
        raise RuntimeError("num_bins must be >= 2")
    if tuple(per_era_gain.shape) != (E, F, B - 1) or tuple(per_era_direction.shape) != (E, F, B - 1):
        raise RuntimeError(f"per-era outputs must have shape {(E, F, B - 1)}")
    lib = _lib.load()
    rc = lib.wgbm_compute_split(G.data_ptr(), H.data_ptr(), E, F, B, float(min_split_gain),
                                float(min_child_samples), float(eps), per_era_gain.data_ptr(),
                                per_era_direction.data_ptr(), int(threads),
                                _lib.current_stream_ptr(G.device))
    _lib.check(rc, "compute_split")


def custom_cuda_binner(X, bin_edges, bin_indices) -> None:
    """Bin one float32 column by its sorted edges (warpgbm/cuda/binner.cu:27-52)."""
    _need(X, "X", torch.float32, 1)
    _need(bin_edges, "bin_edges", torch.float32, 1)
    _need(bin_indices, "bin_indices", torch.int8, 1)
    if bin_indices.numel() != X.numel():
        raise RuntimeError("bin_indices must have one entry per value of X")
    if bin_edges.numel() > 126:
        raise RuntimeError("at most 126 edges (num_bins <= 127)")
    lib = _lib.load()
    rc = lib.wgbm_custom_cuda_binner(X.data_ptr(), X.numel(), bin_edges.data_ptr(),
                                     bin_edges.numel(), bin_indices.data_ptr(),
                                     _lib.current_stream_ptr(X.device))
    _lib.check(rc, "custom_cuda_binner")


def predict_forest(bin_indices, tree_tensor, learning_rate, out) -> None:
    """Add ``learning_rate * leaf`` of every tree to ``out`` (warpgbm/cuda/predict.cu:48-76)."""
    _need(bin_indices, "bin_indices", torch.int8, 2)
    _need(tree_tensor, "tree_tensor", torch.float32, 3)
    _need(out, "out", torch.float32, 1)
    N, F = bin_indices.shape
    T, M, six = tree_tensor.shape
    if six != 6:
        raise RuntimeError("tree_tensor must be [T, max_nodes, 6]")
    if out.numel() != N:
        raise RuntimeError("out must have one entry per row")
    lib = _lib.load()
    rc = lib.wgbm_predict_forest(bin_indices.data_ptr(), N, F, tree_tensor.data_ptr(), T, M,
                                 float(learning_rate), out.data_ptr(),
                                 _lib.current_stream_ptr(out.device))
    _lib.check(rc, "predict_forest")


def install_as_reference_module() -> None:
    """Serve this module as ``warpgbm.cuda.node_kernel``, the name the
    reference estimator imports it by (``from warpgbm.cuda import
    node_kernel``, warpgbm/core.py:7), so that the reference's own Python
    runs on these kernels without an edit.  Call it before the reference's
    ``warpgbm.core`` is imported; the reference's ``warpgbm`` package itself
    must still be importable (only its compiled op module is replaced)."""
    import sys

    me = sys.modules[__name__]
    sys.modules["warpgbm.cuda.node_kernel"] = me
    parent = sys.modules.get("warpgbm.cuda")
    if parent is not None:
        setattr(parent, "node_kernel", me)
