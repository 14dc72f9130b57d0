"""WarpGBM estimator on the MI355X hot path.

Same public API as the reference estimator (warpgbm/core.py:14-1252):
``WarpGBM(objective, num_bins, max_depth, learning_rate, n_estimators,
min_child_weight, min_split_gain, threads_per_block, rows_per_thread, L2_reg,
device, colsample_bytree, random_state, warm_start)`` with ``fit``,
``predict``, ``predict_proba``, importance getters, ``save_model`` /
``load_model`` and ``flatten_tree``; the fitted forest uses the reference's
nested-dict tree format.

What differs is how the trees are grown: the native level-wise engine builds
every node of a depth (and all K class trees of a softmax round) per launch
sequence, with no host synchronisation inside a round, instead of the
reference's recursive per-node Python loop.  The trees are the same: the
residual is fixed per tree (core.py:719), each node's decision depends only
on its own rows, and histogram sums are exact (see include/warpgbm_amd.h).
"""
from __future__ import annotations

import pickle

import numpy as np
import torch
from sklearn.base import BaseEstimator, RegressorMixin
from sklearn.preprocessing import LabelEncoder

import os
import time

from . import device as D
from . import node_kernel
from .metrics import accuracy_torch, log_loss_torch, rmsle_torch, softmax

_TIMING = os.environ.get("WGBM_TIMING", "") not in ("", "0")
# predict inputs from this many rows on read only the forest's split columns
_NARROW_MIN_ROWS = 1 << 16


class _Phases:
    """Wall-clock phase timer for fit (printed when WGBM_TIMING=1)."""

    def __init__(self):
        self.t = time.perf_counter()
        self.items = []

    def mark(self, name):
        if _TIMING:
            torch.cuda.synchronize()
            now = time.perf_counter()
            self.items.append((name, now - self.t))
            self.t = now

    def report(self, what="fit"):
        if _TIMING:
            print(f"{what} phases: " + ", ".join(f"{n} {dt * 1e3:.1f} ms" for n, dt in self.items))


def _record_round_bytes(n_trees, H):
    """Bytes of one round's tree records (count, feature, bin, leaf of each
    tree's H heap nodes), rounded up to 16 bytes."""
    return (20 * n_trees * H + 15) // 16 * 16


def _record_views(raw, n_trees, H):
    """The record fields as [rounds, trees, H] views of one round-major byte
    buffer raw [rounds, _record_round_bytes]: a round's records are one
    contiguous range (one copy for a block of rounds), and within a round
    each field is contiguous (the engine's per-round pointers)."""
    th = n_trees * H
    R = raw.shape[0]

    def field(lo, hi, dtype):
        return raw[:, lo:hi].view(dtype).view(R, n_trees, H)

    return {"count": field(0, 8 * th, torch.int64), "feat": field(8 * th, 12 * th, torch.int32),
            "bin": field(12 * th, 16 * th, torch.int32),
            "leaf": field(16 * th, 20 * th, torch.float32), "raw": raw}


_SIDE_STREAMS = {}


def _side_stream(dev):
    """One side stream per device for the record copies, created once (a
    stream's creation can take milliseconds)."""
    dev = torch.device(dev)
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    if key not in _SIDE_STREAMS:
        _SIDE_STREAMS[key] = torch.cuda.Stream(device=key)
    return _SIDE_STREAMS[key]


class _RecordStream:
    """The engine's per-round tree records (device heaps [rounds, trees, H])
    copied to pinned host memory in blocks of rounds while later rounds run,
    and each landed block turned into reference tree dicts (by the C
    extension ``_trees``) on the launching thread, a few thousand heap nodes
    at a time, only while the GPU still has the previous round queued: the
    conversion uses the host's slack between launches and never holds the
    interpreter lock against them (a converter thread did, and left the GPU
    idle at round starts).  What remains when the last round is enqueued is
    converted by ``finish``."""

    BLOCK = 8          # rounds per copy
    CHUNK_NODES = 2048  # heap nodes per conversion step (~0.3-0.4 ms of host time)

    def __init__(self, rec):
        self.rec = rec
        n_trees, H = rec["feat"].shape[1], rec["feat"].shape[2]
        self.host_raw = torch.empty(rec["raw"].shape, dtype=torch.uint8, pin_memory=True)
        self.host = {k: v for k, v in _record_views(self.host_raw, n_trees, H).items()
                     if k != "raw"}
        self.pending = []   # (first round, end round, event) of issued copies
        self.copied = 0     # rounds whose copy has been issued
        self.landed = []    # [r0, r1, trees converted so far, fields] of landed blocks, in order
        self.flat = []      # tree dicts of the converted trees, rounds then trees
        self.trees = []     # per finished round: its list of tree dicts
        # per converted block: the records' rows of its internal nodes (rounds,
        # then trees in order, nodes in pre-order) and their split features
        self.nodes = []
        self.prev_ev = None  # completion of the round before the last enqueued one
        self.last_ev = None
        self.side = None     # the copies' stream
        self.closed = False

    def round_done(self, j, n_rounds):
        """Round j of n_rounds has been enqueued: issue a block copy every
        BLOCK rounds (every round in the last block, so that little is left
        to convert when the GPU finishes), then convert landed trees while
        the GPU is still busy with round j - 1 (so round j stays queued
        behind it)."""
        if (j + 1) % self.BLOCK == 0 or j + self.BLOCK >= n_rounds:
            self.issue(j + 1)
        ev = torch.cuda.Event()
        ev.record()
        self.prev_ev, self.last_ev = self.last_ev, ev
        while self.prev_ev is not None and not self.prev_ev.query():
            if not self._step():
                break

    def issue(self, end):
        """Copy rounds [copied, end) to the host on a side stream (after the
        compute stream's work so far), so that the copies' host-visible
        writes never stall the compute stream."""
        if end <= self.copied:
            return
        r0 = self.copied
        if self.side is None:
            self.side = _side_stream(self.rec["feat"].device)
        ready = torch.cuda.Event()
        ready.record()
        with torch.cuda.stream(self.side):
            self.side.wait_event(ready)
            # the rounds' records are one contiguous range: one copy
            self.host_raw[r0:end].copy_(self.rec["raw"][r0:end], non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(self.side)
        self.pending.append((r0, end, ev))
        self.copied = end

    def _step(self, wait=False):
        """Convert a few trees (CHUNK_NODES heap nodes) of the oldest landed
        block; False when no landed block has trees left."""
        # landed copies; with wait, block for the oldest one only when none
        # has landed (the rest keep landing while this one is converted)
        n_trees, H = self.host["feat"].shape[1], self.host["feat"].shape[2]
        while self.pending and (self.pending[0][2].query() or (wait and not self.landed)):
            r0, r1, ev = self.pending.pop(0)
            ev.synchronize()
            # the block's fields as contiguous [trees of the block, H] arrays
            f = {k: np.ascontiguousarray(v[r0:r1].numpy()).reshape(-1, H)
                 for k, v in self.host.items()}
            self.landed.append([r0, r1, 0, f])
        if not self.landed:
            return False
        blk = self.landed[0]
        r0, r1, done, f = blk
        total = (r1 - r0) * n_trees
        hi = min(total, done + max(1, self.CHUNK_NODES // H))
        self.flat.extend(_heaps_to_dicts(f["feat"][done:hi], f["bin"][done:hi],
                                         f["leaf"][done:hi], f["count"][done:hi]))
        blk[2] = hi
        if hi == total:
            self.landed.pop(0)
            self.nodes.append(self._block_nodes(r0, r1))
        return True

    def _block_nodes(self, r0, r1):
        """The block's internal nodes in the importance order."""
        feat = self.host["feat"][r0:r1].numpy()
        n_trees, H = feat.shape[1], feat.shape[2]
        po = _preorder_heap(H).astype(np.int64)
        fp = feat[:, :, po]
        internal = fp >= 0
        base = (np.arange(r0, r1, dtype=np.int64)[:, None, None] * n_trees
                + np.arange(n_trees, dtype=np.int64)[None, :, None]) * H
        return (base + po[None, None, :])[internal], fp[internal]

    def finish(self, done):
        try:
            self.issue(done)
            while self._step(wait=True):
                pass
            n_trees = self.host["feat"].shape[1]
            self.trees = [self.flat[j * n_trees:(j + 1) * n_trees] for j in range(done)]
        finally:
            self.close()

    def close(self):
        """Wait for the copies in flight (also after an error: the pinned
        buffer must outlive them)."""
        if not self.closed:
            self.closed = True
            for _, _, ev in self.pending:
                ev.synchronize()


class WarpGBM(BaseEstimator, RegressorMixin):
    def __init__(
        self,
        objective="regression",
        num_bins=10,
        max_depth=3,
        learning_rate=0.1,
        n_estimators=100,
        min_child_weight=20,
        min_split_gain=0.0,
        threads_per_block=64,
        rows_per_thread=4,
        L2_reg=1e-6,
        device="cuda",
        colsample_bytree=1.0,
        random_state=None,
        warm_start=False,
    ):
        self._validate_hyperparams(
            objective=objective,
            num_bins=num_bins,
            max_depth=max_depth,
            learning_rate=learning_rate,
            n_estimators=n_estimators,
            min_child_weight=min_child_weight,
            min_split_gain=min_split_gain,
            threads_per_block=threads_per_block,
            rows_per_thread=rows_per_thread,
            L2_reg=L2_reg,
            colsample_bytree=colsample_bytree,
        )
        self.objective = objective
        self.num_bins = num_bins
        self.max_depth = max_depth
        self.learning_rate = learning_rate
        self.n_estimators = n_estimators
        self.min_child_weight = min_child_weight
        self.min_split_gain = min_split_gain
        # CUDA launch-shape knobs of the reference; accepted and validated,
        # no effect on the HIP kernels
        self.threads_per_block = threads_per_block
        self.rows_per_thread = rows_per_thread
        self.L2_reg = L2_reg
        self.device = device
        self.colsample_bytree = colsample_bytree
        self.random_state = random_state
        self.warm_start = warm_start
        self.forest = [{} for _ in range(self.n_estimators)]
        self.bin_edges = None
        self.base_prediction = None
        self.unique_eras = None
        self.num_classes = None
        self.classes_ = None
        self.num_features = None
        self.num_samples = None
        self.label_encoder = None
        self.feature_importance_ = None
        self.per_era_feature_importance_ = None
        self._is_fitted = False
        self._trees_trained = 0
        self._heap = None  # device heap tables of the fitted forest (cache)
        self._heap_used = None  # (heap, split features, tables over them) (cache)

    # ------------------------------------------------------------------ validation
    def _validate_hyperparams(self, **kwargs):
        """Same checks and messages as warpgbm/core.py:83-143."""
        if kwargs["objective"] not in ["regression", "multiclass", "binary"]:
            raise ValueError(
                f"objective must be 'regression', 'binary', or 'multiclass', got {kwargs['objective']}."
            )
        int_params = ["num_bins", "max_depth", "n_estimators", "min_child_weight",
                      "threads_per_block", "rows_per_thread"]
        float_params = ["learning_rate", "min_split_gain", "L2_reg", "colsample_bytree"]
        for param in int_params:
            if not isinstance(kwargs[param], int):
                raise TypeError(f"{param} must be an integer, got {type(kwargs[param])}.")
        for param in float_params:
            if not isinstance(kwargs[param], (float, int)):
                raise TypeError(f"{param} must be a float, got {type(kwargs[param])}.")
        if not (2 <= kwargs["num_bins"] <= 127):
            raise ValueError("num_bins must be between 2 and 127 inclusive.")
        if kwargs["max_depth"] < 1:
            raise ValueError("max_depth must be at least 1.")
        if not (0.0 < kwargs["learning_rate"] <= 1.0):
            raise ValueError("learning_rate must be in (0.0, 1.0].")
        if kwargs["n_estimators"] <= 0:
            raise ValueError("n_estimators must be positive.")
        if kwargs["min_child_weight"] < 1:
            raise ValueError("min_child_weight must be a positive integer.")
        if kwargs["min_split_gain"] < 0:
            raise ValueError("min_split_gain must be non-negative.")
        if kwargs["threads_per_block"] <= 0 or kwargs["threads_per_block"] % 32 != 0:
            raise ValueError("threads_per_block should be a positive multiple of 32 (warp size).")
        if not (1 <= kwargs["rows_per_thread"] <= 16):
            raise ValueError("rows_per_thread must be positive between 1 and 16 inclusive.")
        if kwargs["L2_reg"] < 0:
            raise ValueError("L2_reg must be non-negative.")
        if kwargs["colsample_bytree"] <= 0 or kwargs["colsample_bytree"] > 1:
            raise ValueError(
                f"Invalid colsample_bytree: {kwargs['colsample_bytree']}. Must be a float value > 0 and <= 1."
            )

    def validate_fit_params(self, X, y, era_id, X_eval, y_eval, eval_every_n_trees,
                            early_stopping_rounds, eval_metric):
        """Same checks and messages as warpgbm/core.py:216-291."""
        if not isinstance(X, np.ndarray) or not isinstance(y, np.ndarray):
            raise TypeError("X and y must be numpy arrays.")
        if X.ndim != 2:
            raise ValueError(f"X must be 2-dimensional, got shape {X.shape}")
        if y.ndim != 1:
            raise ValueError(f"y must be 1-dimensional, got shape {y.shape}")
        if X.shape[0] != y.shape[0]:
            raise ValueError(
                f"X and y must have the same number of rows. Got {X.shape[0]} and {y.shape[0]}.")
        if era_id is not None:
            if not isinstance(era_id, np.ndarray):
                raise TypeError("era_id must be a numpy array.")
            if era_id.ndim != 1:
                raise ValueError(f"era_id must be 1-dimensional, got shape {era_id.shape}")
            if len(era_id) != len(y):
                raise ValueError(
                    f"era_id must have same length as y. Got {len(era_id)} and {len(y)}.")
        eval_args = [X_eval, y_eval, eval_every_n_trees]
        if any(arg is not None for arg in eval_args):
            if X_eval is None or y_eval is None or eval_every_n_trees is None:
                raise ValueError(
                    "If using eval set, X_eval, y_eval, and eval_every_n_trees must all be defined.")
            if not isinstance(X_eval, np.ndarray) or not isinstance(y_eval, np.ndarray):
                raise TypeError("X_eval and y_eval must be numpy arrays.")
            if X_eval.ndim != 2:
                raise ValueError(f"X_eval must be 2-dimensional, got shape {X_eval.shape}")
            if y_eval.ndim != 1:
                raise ValueError(f"y_eval must be 1-dimensional, got shape {y_eval.shape}")
            if X_eval.shape[0] != y_eval.shape[0]:
                raise ValueError(
                    f"X_eval and y_eval must have same number of rows. Got {X_eval.shape[0]} and {y_eval.shape[0]}.")
            if not isinstance(eval_every_n_trees, int) or eval_every_n_trees <= 0:
                raise ValueError(
                    f"eval_every_n_trees must be a positive integer, got {eval_every_n_trees}.")
            if early_stopping_rounds is not None:
                if not isinstance(early_stopping_rounds, int) or early_stopping_rounds <= 0:
                    raise ValueError(
                        f"early_stopping_rounds must be a positive integer, got {early_stopping_rounds}.")
            else:
                early_stopping_rounds = self.n_estimators + 1
            valid_metrics = ["mse", "corr", "rmsle", "logloss", "accuracy"]
            if eval_metric not in valid_metrics:
                raise ValueError(f"Invalid eval_metric: {eval_metric}. Choose from {valid_metrics}.")
        return early_stopping_rounds

    # ------------------------------------------------------------------ fit
    def fit(self, X, y, era_id=None, X_eval=None, y_eval=None, eval_every_n_trees=None,
            early_stopping_rounds=None, eval_metric="mse"):
        early_stopping_rounds = self.validate_fit_params(
            X, y, era_id, X_eval, y_eval, eval_every_n_trees, early_stopping_rounds, eval_metric)
        # random_state seeds the global RNGs as the reference does
        # (warpgbm/core.py:308-314); colsample_bytree subsets are then drawn
        # with torch.randperm on the device (core.py:722, 778)
        if self.random_state is not None:
            torch.manual_seed(self.random_state)
            np.random.seed(self.random_state)
            if torch.cuda.is_available():
                torch.cuda.manual_seed(self.random_state)
                torch.cuda.manual_seed_all(self.random_state)

        fresh = not (self.warm_start and self._is_fitted)
        if fresh:
            self._reset_training_state()
        elif X.shape[1] != self.num_features:
            raise ValueError(
                f"X has {X.shape[1]} features, but model was trained with {self.num_features} features.")
        elif self._trees_trained >= self.n_estimators:
            print(f"Model already has {self._trees_trained} trees (n_estimators={self.n_estimators}). No additional training needed.")
            return self

        if era_id is None:
            era_id = np.ones(X.shape[0], dtype="int32")
        self._subsets_dev = []
        self._phases = _Phases()
        try:
            if self.objective in ("multiclass", "binary"):
                y_encoded = self._encode_labels(y, refit=fresh)
                self._check_class_count()
                return self._fit_classification(X, y_encoded, era_id, X_eval, y_eval,
                                                eval_every_n_trees, early_stopping_rounds,
                                                eval_metric)
            return self._fit_regression(X, y, era_id, X_eval, y_eval, eval_every_n_trees,
                                        early_stopping_rounds, eval_metric)
        finally:
            # the subsets drawn on the device, on the host once the fit is done
            self.feature_subsets_ = [t if isinstance(t, np.ndarray) else
                                     t.cpu().numpy().astype(np.int32) for t in self._subsets_dev]
            self._subsets_dev = []

    def _reset_training_state(self):
        """A fresh fit: no trees, no loss history (warpgbm/core.py:317-324)."""
        self._is_fitted = False
        self._trees_trained = 0
        self.forest = [{} for _ in range(self.n_estimators)] if self.objective == "regression" else []
        self.training_loss = []
        self.eval_loss = []

    def _encode_labels(self, y, refit):
        """Class labels as 0..K-1 by sklearn's LabelEncoder (warpgbm/core.py:341-352):
        fitted on a fresh start, the fitted one reused on a warm start."""
        if refit:
            self.label_encoder = LabelEncoder().fit(y)
            self.classes_ = self.label_encoder.classes_
            self.num_classes = len(self.classes_)
        return self.label_encoder.transform(y)

    def _check_class_count(self):
        K = self.num_classes
        if self.objective == "binary" and K != 2:
            raise ValueError(f"binary objective requires exactly 2 classes, got {K}")
        if self.objective == "multiclass" and K < 2:
            raise ValueError(f"multiclass objective requires at least 2 classes, got {K}")

    def preprocess_gpu_data(self, X_np, Y_np, era_id_np):
        """Codes, era layout and targets on the device (warpgbm/core.py:487-541)."""
        self.num_samples, self.num_features = X_np.shape
        dev = torch.device(self.device)
        ph = self._phases
        codes, Xd = self._prebinned_codes(X_np, dev, with_cm=True)
        if codes is not None:
            print("Detected pre-binned integer input — skipping quantile binning.")
            bin_edges = torch.arange(1, self.num_bins, dtype=torch.float32).repeat(
                self.num_features, 1).to(dev)
        else:
            print("quantile binning.")
            if Xd is None:
                # the selection's staging rides on the upload (edges are
                # ready shortly after the last row block lands)
                Xd, bin_edges = D.upload_float_with_edges(X_np, dev, self.num_bins)
                ph.mark("upload")
            else:
                ph.mark("upload")
                bin_edges = D.quantile_edges(Xd, self.num_bins)
            ph.mark("edges")
            codes = D.bin_matrix(Xd, bin_edges, with_cm=True)
            ph.mark("bin")
            del Xd
        ph.mark("codes")
        uniq, inv, order, start = D.era_layout(era_id_np)
        self.unique_eras = uniq
        self.num_eras = len(uniq)
        self._era_inv = inv
        root_order = torch.from_numpy(order).to(dev)
        era_start = torch.from_numpy(start).to(dev)
        Y_gpu = torch.from_numpy(np.asarray(Y_np)).type(torch.float32).to(dev)
        ph.mark("eras+targets")
        return codes, root_order, era_start, bin_edges, Y_gpu

    def _prebinned_codes(self, X_np, dev, with_cm):
        """The reference's pre-binned test (warpgbm/core.py:499-505, 938-945):
        integer input whose every column max is < num_bins is used as codes.
        int8 input is uploaded once and tested on the device in the pass that
        lays out the codes; other integer types are tested on the host.
        Returns (codes or None, float32 device copy of X or None)."""
        if not np.issubdtype(X_np.dtype, np.integer):
            return None, None
        if X_np.dtype == np.int8 and X_np.shape[0] > 0:
            x8 = D.upload_int8(X_np, dev)
            codes, over = D.codes_from_int8(x8, with_cm, self.num_bins, check=True)
            if not over:
                return codes, None
            del codes
            return None, x8.to(torch.float32)
        if X_np.shape[0] == 0 or bool(np.all(X_np.max(axis=0) < self.num_bins)):
            return D.upload_prebinned(X_np, dev, with_cm, self.num_bins), None
        return None, None

    def _new_engine(self, codes, root_order, era_start, n_trees, objective):
        # _engine_level_bytes (0: the library's default) bounds the per-level
        # split buffers; a smaller bound only changes how levels are chunked
        eng = D.Engine(codes, root_order, era_start, self.num_bins, self.num_eras,
                       self.max_depth, n_trees, objective, self.min_child_weight,
                       self.min_split_gain, self.L2_reg, self.learning_rate,
                       getattr(self, "_engine_level_bytes", 0))
        # engine knobs (wgbm_engine_set_tuning keys); none changes the model
        for key, value in getattr(self, "_engine_tuning", {}).items():
            eng.set_tuning(int(key), int(value))
        return eng

    def _feature_subset(self, dev):
        """Features of one round: torch.randperm(F)[:k] on the device,
        k = max(1, int(colsample * F)) (warpgbm/core.py:702-703, 721-722,
        777-778); the subsets of the last fit are kept in ``feature_subsets_``
        (copied to the host when the fit ends, so no round waits for them)."""
        F = self.num_features
        if self.colsample_bytree < 1.0:
            k = max(1, int(self.colsample_bytree * F))
            sel = torch.randperm(F, device=dev, dtype=torch.int32)[:k]
            self._subsets_dev.append(sel)
            return sel
        # every round uses all features: one device copy for the whole fit
        # (keyed by the device as given: torch.device("cuda") != "cuda:0")
        cached = getattr(self, "_all_features_dev", None)
        if cached is None or cached.numel() != F or getattr(self, "_all_features_on", None) != dev:
            cached = torch.arange(F, dtype=torch.int32, device=dev)
            self._all_features_dev = cached
            self._all_features_on = dev
            self._all_features_host = np.arange(F, dtype=np.int32)
        self._subsets_dev.append(self._all_features_host)
        return cached

    def _alloc_records(self, n_rounds, n_trees, dev):
        H = (1 << (self.max_depth + 1)) - 1
        need = n_rounds * n_trees * H * (20 + 4 * self.num_eras)
        free, _ = torch.cuda.mem_get_info(dev)
        if need > free:
            raise MemoryError(
                f"max_depth={self.max_depth} with {n_rounds} rounds x {n_trees} trees needs "
                f"{need / 2**30:.1f} GiB of device memory for the tree records "
                f"({free / 2**30:.1f} GiB free); reduce max_depth or n_estimators")
        rec = _record_views(torch.empty((n_rounds, _record_round_bytes(n_trees, H)),
                                        dtype=torch.uint8, device=dev), n_trees, H)
        rec["gain"] = torch.empty((n_rounds, n_trees, H, self.num_eras), dtype=torch.float32,
                                  device=dev)
        return rec

    @staticmethod
    def _records_heap(rec, done):
        """Predict tables of a fresh fit taken straight from the engine's
        device records: the same feature / bin / leaf values the tree dicts
        hold (absent nodes carry feature -2, which traversal never reaches),
        so the first predict need not rebuild them from the dicts."""
        if done == 0:
            return None
        return (rec["feat"][:done].contiguous(), rec["bin"][:done].contiguous(),
                rec["leaf"][:done].contiguous(), done)

    def _fit_regression(self, X, y, era_id, X_eval, y_eval, eval_every_n_trees,
                        early_stopping_rounds, eval_metric):
        dev = torch.device(self.device)
        codes, root_order, era_start, self.bin_edges, Y_gpu = self.preprocess_gpu_data(X, y, era_id)
        start_iter = self._trees_trained if (self.warm_start and self._is_fitted) else 0
        if start_iter > 0:
            # rebuild the training predictions from the existing trees; trees
            # are added in order, exactly as during training
            preds = torch.full((self.num_samples,), np.float32(self.base_prediction),
                               dtype=torch.float32, device=dev)
            self._predict_codes_into(codes, preds.view(-1, 1), self.forest[:start_iter])
        else:
            # mean of the float32 targets, float64 accumulation, one rounding
            # (the reference's Y_gpu.mean().item(), core.py:387)
            self.base_prediction = float(np.float32(
                np.mean(np.asarray(y, dtype=np.float32), dtype=np.float64)))
            preds = torch.full((self.num_samples,), np.float32(self.base_prediction),
                               dtype=torch.float32, device=dev)
        self._setup_eval(X_eval, y_eval, eval_every_n_trees, early_stopping_rounds, eval_metric,
                         classification=False)
        if not hasattr(self, "training_loss") or not self.warm_start or not self._is_fitted:
            self.training_loss = []
            self.eval_loss = []
            self.per_era_feature_importance_ = np.zeros((self.num_eras, self.num_features),
                                                        dtype=np.float32)
        if len(self.forest) < self.n_estimators:
            self.forest.extend([{} for _ in range(self.n_estimators - len(self.forest))])
        eng = self._new_engine(codes, root_order, era_start, 1, 0)
        n_new = self.n_estimators - start_iter
        rec = self._alloc_records(n_new, 1, dev)
        self._phases.mark("engine")
        self.stop = False
        eval_pred = None
        if self._eval is not None:
            eval_pred = torch.full((self._eval["codes"].n, 1), np.float32(self.base_prediction),
                                   dtype=torch.float32, device=dev)
            if start_iter > 0:
                self._predict_codes_into(self._eval["codes"], eval_pred, self.forest[:start_iter])
        done = 0
        stream = _RecordStream(rec)
        try:
            with torch.no_grad():
                for j in range(n_new):
                    i = start_iter + j
                    feat_sel = self._feature_subset(dev)
                    eng.round(Y_gpu, preds, feat_sel, {k: v[j] for k, v in rec.items()})
                    done = j + 1
                    stream.round_done(j, n_new)
                    if self._eval is not None:
                        D.predict_heap(self._eval["codes"], rec["feat"][j], rec["bin"][j],
                                       rec["leaf"][j], 1, 1, self.max_depth, self.learning_rate,
                                       eval_pred)
                        self._compute_eval_regression(i, Y_gpu, preds, eval_pred[:, 0])
                        if self.stop:
                            break
            stream.finish(done)
        finally:
            stream.close()
        self._phases.mark("rounds")
        eng.close()
        self._absorb_records(rec, stream, done, start_iter, classification=False)
        self._phases.mark("records")
        self._phases.report()
        self.feature_importance_ = self.per_era_feature_importance_.sum(axis=0)
        self._is_fitted = True
        self._heap = self._records_heap(rec, done) if start_iter == 0 else None
        print(f"Finished training forest. Total trees: {self._trees_trained}")
        del codes
        return self

    def _fit_classification(self, X, y_encoded, era_id, X_eval, y_eval, eval_every_n_trees,
                            early_stopping_rounds, eval_metric):
        dev = torch.device(self.device)
        codes, root_order, era_start, self.bin_edges, _ = self.preprocess_gpu_data(X, y_encoded, era_id)
        K = self.num_classes
        labels = torch.from_numpy(np.asarray(y_encoded).astype(np.int32)).to(dev)
        start_iter = self._trees_trained if (self.warm_start and self._is_fitted) else 0
        init = self._class_prior_logits(np.asarray(y_encoded))
        # the engine keeps the training scores class-major, [K, n]
        if start_iter > 0:
            scores_rm = D.rows_of(init, self.num_samples, dev)
            self._predict_codes_into(codes, scores_rm, self.forest[:start_iter])
            scores = scores_rm.t().contiguous()
            del scores_rm
        else:
            scores = D.cols_of(init, self.num_samples, dev)
        self._setup_eval(X_eval, y_eval, eval_every_n_trees, early_stopping_rounds, eval_metric,
                         classification=True)
        if not hasattr(self, "training_loss") or not self.warm_start or not self._is_fitted:
            self.training_loss = []
            self.eval_loss = []
            self.per_era_feature_importance_ = np.zeros((self.num_eras, self.num_features),
                                                        dtype=np.float32)
            self.forest = []
        eng = self._new_engine(codes, root_order, era_start, K, 1)
        n_new = self.n_estimators - start_iter
        rec = self._alloc_records(n_new, K, dev)
        self._phases.mark("engine")
        self.stop = False
        eval_scores = None
        if self._eval is not None:
            eval_scores = D.rows_of(self._uniform_prior_logits(), self._eval["codes"].n, dev)
            if start_iter > 0:
                self._predict_codes_into(self._eval["codes"], eval_scores, self.forest[:start_iter])
        done = 0
        stream = _RecordStream(rec)
        try:
            with torch.no_grad():
                for j in range(n_new):
                    i = start_iter + j
                    feat_sel = self._feature_subset(dev)
                    eng.round(labels, scores, feat_sel, {k: v[j] for k, v in rec.items()})
                    done = j + 1
                    stream.round_done(j, n_new)
                    if self._eval is not None:
                        D.predict_heap(self._eval["codes"], rec["feat"][j], rec["bin"][j],
                                       rec["leaf"][j], 1, K, self.max_depth, self.learning_rate,
                                       eval_scores)
                        self._compute_eval_multiclass(i, labels, scores.t().contiguous(),
                                                      eval_scores)
                        if self.stop:
                            break
            stream.finish(done)
        finally:
            stream.close()
        self._phases.mark("rounds")
        eng.close()
        self._absorb_records(rec, stream, done, start_iter, classification=True)
        self._phases.mark("records")
        self._phases.report()
        self.feature_importance_ = self.per_era_feature_importance_.sum(axis=0)
        self._is_fitted = True
        self._heap = self._records_heap(rec, done) if start_iter == 0 else None
        print(f"Finished training multiclass forest. Total rounds: {self._trees_trained} "
              f"({self._trees_trained * self.num_classes} trees)")
        del codes
        return self

    # ------------------------------------------------------------------ priors
    def _class_prior_logits(self, y_encoded):
        """log(prior_k + 1e-10) with prior_k the class frequency in float32
        (warpgbm/core.py:452-456)."""
        K = self.num_classes
        n = np.float32(len(y_encoded))
        out = np.zeros(K, dtype=np.float32)
        for k in range(K):
            p = np.float32(np.count_nonzero(y_encoded == k)) / n
            if p > 0:
                out[k] = np.float32(np.log(np.float64(np.float32(p + np.float32(1e-10)))))
        return out

    def _uniform_prior_logits(self):
        """The start logits of predict_proba (warpgbm/core.py:1003-1007):
        1/K + 1e-10 is a float64 there (numpy division, wrapped by
        torch.tensor), so its log is taken in float64 and rounded to float32
        once, when it lands in the float32 score matrix."""
        K = self.num_classes
        v = np.float32(np.log(np.float64(1.0) / np.float64(K) + 1e-10))
        return np.full(K, v, dtype=np.float32)

    # ------------------------------------------------------------------ eval
    def _setup_eval(self, X_eval, y_eval, eval_every_n_trees, early_stopping_rounds, eval_metric,
                    classification):
        if X_eval is None or y_eval is None:
            self._eval = None
            self.eval_every_n_trees = None
            self.early_stopping_rounds = None
            return
        dev = torch.device(self.device)
        codes = self.bin_inference_data(X_eval)
        if classification:
            y_enc = self.label_encoder.transform(y_eval)
            ye = torch.from_numpy(np.asarray(y_enc).astype(np.int32)).to(dev)
            self.eval_metric = eval_metric if eval_metric != "mse" else "logloss"
        else:
            ye = torch.from_numpy(np.asarray(y_eval)).to(torch.float32).to(dev)
            self.eval_metric = eval_metric
        self._eval = {"codes": codes, "y": ye}
        self.eval_every_n_trees = eval_every_n_trees
        self.early_stopping_rounds = early_stopping_rounds

    _REGRESSION_METRICS = {
        # mean squared error
        "mse": lambda t, p: ((t - p) ** 2).mean(),
        # one minus Pearson's r of targets and predictions
        "corr": lambda t, p: 1 - torch.corrcoef(torch.vstack([t, p]))[0, 1],
        "rmsle": lambda t, p: rmsle_torch(t, p),
    }

    def get_eval_metric(self, y_true, y_pred):
        """Regression eval loss of warpgbm/core.py:660-668 (lower is better)."""
        fn = self._REGRESSION_METRICS.get(self.eval_metric)
        if fn is None:
            raise ValueError(f"Invalid eval_metric: {self.eval_metric}.")
        return fn(y_true, y_pred).item()

    def _compute_eval_regression(self, i, Y_gpu, preds, eval_preds):
        """warpgbm/core.py:670-690."""
        train_loss = ((Y_gpu - preds) ** 2).mean().item()
        self.training_loss.append(train_loss)
        if i % self.eval_every_n_trees == 0:
            eval_loss = self.get_eval_metric(self._eval["y"], eval_preds)
            self.eval_loss.append(eval_loss)
            if len(self.eval_loss) > self.early_stopping_rounds:
                if self.eval_loss[-(self.early_stopping_rounds + 1)] < self.eval_loss[-1]:
                    self.stop = True
            print(f"🌲 Tree {i+1}/{self.n_estimators} | Train MSE: {train_loss:.6f} | "
                  f"Eval {self.eval_metric}: {eval_loss:.6f}")

    def _compute_eval_multiclass(self, i, labels, scores, eval_scores):
        """warpgbm/core.py:820-853."""
        train_loss = log_loss_torch(labels, softmax(scores, dim=1)).item()
        self.training_loss.append(train_loss)
        if i % self.eval_every_n_trees == 0:
            probs = eval_scores.clone()
            D.softmax_rows(probs)
            if self.eval_metric == "accuracy":
                eval_loss = 1.0 - accuracy_torch(self._eval["y"], torch.argmax(probs, dim=1)).item()
            else:
                eval_loss = log_loss_torch(self._eval["y"], probs).item()
            self.eval_loss.append(eval_loss)
            if len(self.eval_loss) > self.early_stopping_rounds:
                if self.eval_loss[-(self.early_stopping_rounds + 1)] < self.eval_loss[-1]:
                    self.stop = True
            print(f"🌲 Round {i+1}/{self.n_estimators} ({self.num_classes} trees) | "
                  f"Train LogLoss: {train_loss:.6f} | Eval {self.eval_metric}: {eval_loss:.6f}")

    # ------------------------------------------------------------------ records -> forest
    def _absorb_records(self, rec, stream, done, start_iter, classification):
        """Reference tree dicts of the ``done`` rounds (built by the record
        stream during training) into the forest, and importance in the
        reference's order: per tree, internal nodes in depth-first pre-order,
        float32 adds (warpgbm/core.py:624-627)."""
        dev = rec["gain"].device
        # importance: every internal node of every tree, trees in order and
        # nodes in pre-order, one float32 add per node and era in exactly that
        # sequence, on the device from the per-era gain records; the nodes
        # (listed by the record stream block by block while later rounds
        # ran) are grouped by feature here (a stable sort keeps their
        # order), so each (feature, era) word is one device thread's sum
        rows = (np.concatenate([r for r, _ in stream.nodes]) if stream.nodes
                else np.zeros(0, np.int64))
        fsel = (np.concatenate([f for _, f in stream.nodes]) if stream.nodes
                else np.zeros(0, np.int32))
        if rows.size:
            F, E = self.num_features, self.num_eras
            # (16-bit keys sort by radix: several times faster than 32-bit)
            by_f = np.argsort(fsel.astype(np.int16) if F < (1 << 15) else fsel, kind="stable")
            fstart = np.searchsorted(fsel[by_f], np.arange(F + 1)).astype(np.int64)
            acc = torch.from_numpy(np.ascontiguousarray(self.per_era_feature_importance_,
                                                        dtype=np.float32)).to(dev)
            D.importance_add(acc, rec["gain"][:done].reshape(-1, E),
                             torch.from_numpy(np.ascontiguousarray(rows[by_f])).to(dev),
                             torch.from_numpy(fstart).to(dev))
            self.per_era_feature_importance_ = acc.cpu().numpy()
        self._phases.mark("importance")
        for j in range(done):
            if classification:
                self.forest.append(stream.trees[j])
            else:
                self.forest[start_iter + j] = stream.trees[j][0]
        self._trees_trained = start_iter + done

    # ------------------------------------------------------------------ binning at predict time
    def bin_data_with_existing_edges(self, X_np):
        dev = torch.device(self.device)
        ph = _Phases()
        codes = D.upload_and_bin(X_np, torch.as_tensor(self.bin_edges), dev)
        ph.mark("upload+bin")
        ph.report("binning")
        return codes

    def bin_inference_data(self, X_np):
        """Codes for new data (warpgbm/core.py:934-955)."""
        dev = torch.device(self.device)
        codes, Xd = None, None
        if X_np.shape[1] == self.num_features:
            codes, Xd = self._prebinned_codes(X_np, dev, with_cm=False)
        if codes is not None:
            print("Detected pre-binned input at predict-time — skipping binning.")
            return codes
        if Xd is not None:
            codes = D.bin_matrix(Xd, torch.as_tensor(self.bin_edges), with_cm=False)
            del Xd
            return codes
        return self.bin_data_with_existing_edges(X_np)

    # ------------------------------------------------------------------ inference
    def _heap_tables(self, rounds):
        """Device heap tables [n_trees, H] of a list of rounds (tree dicts, or
        lists of K tree dicts); empty trees are skipped like the reference's
        ``if tree`` filters."""
        H = (1 << (self.max_depth + 1)) - 1
        K = 1 if self.objective == "regression" else self.num_classes
        rows = []
        for r in rounds:
            trees = [r] if self.objective == "regression" else list(r)
            if not trees or not all(trees):
                continue
            rows.append([_dict_to_heap(t, H) for t in trees])
        n = len(rows)
        feat = np.full((max(n, 1), K, H), -1, np.int32)
        bin_ = np.zeros((max(n, 1), K, H), np.int32)
        leaf = np.zeros((max(n, 1), K, H), np.float32)
        for j, trees in enumerate(rows):
            for k, (f, b, v) in enumerate(trees):
                feat[j, k], bin_[j, k], leaf[j, k] = f, b, v
        dev = torch.device(self.device)
        return (torch.from_numpy(feat).to(dev), torch.from_numpy(bin_).to(dev),
                torch.from_numpy(leaf).to(dev), n)

    def _predict_codes_into(self, codes, out, rounds):
        feat, bin_, leaf, n = self._heap_tables(rounds)
        if n:
            D.predict_heap(codes, feat, bin_, leaf, n, out.shape[1], self.max_depth,
                           self.learning_rate, out)

    def _cached_heap(self):
        if self._heap is None:
            self._heap = self._heap_tables(self.forest)
        return self._heap

    def _used_features(self):
        """The features the fitted forest splits on (sorted) and its heap
        tables with every split feature replaced by its index in that list.
        Cached with the tables they were derived from."""
        heap = self._cached_heap()
        if self._heap_used is None or self._heap_used[0] is not heap:
            feat = heap[0]
            fh = feat.cpu().numpy()  # (small: trees x heap nodes)
            used = np.unique(fh[fh >= 0])  # sorted
            if used.size == 0:
                used = np.zeros(1, dtype=fh.dtype)
            lut = np.full(self.num_features, -1, dtype=fh.dtype)
            lut[used] = np.arange(used.size, dtype=fh.dtype)
            local = np.where(fh >= 0, lut[np.maximum(fh, 0)], fh)
            local_d = torch.from_numpy(np.ascontiguousarray(local)).to(feat.device)
            self._heap_used = (heap, used.astype(np.intp), (local_d, heap[1], heap[2], heap[3]))
        return self._heap_used[1], self._heap_used[2]

    def _infer(self, X_np, K):
        """Raw scores [n, K] of new data: the start values plus every tree,
        added in tree order.  Float input (binned with the training edges,
        warpgbm/core.py:902-915) is streamed: each chunk of rows is walked
        as soon as it is binned, on the device, while the next chunk is
        copied.  A prediction reads only the codes of the features the forest
        splits on: where those are at most half of the columns of an input of
        _NARROW_MIN_ROWS rows or more, only their columns are gathered on the
        host, uploaded and binned, and the tables index that narrow code
        matrix.  The codes of the features read are the same as in the full
        matrix, so the predictions are identical either way."""
        X_np = np.asarray(X_np)
        dev = torch.device(self.device)
        heap = self._cached_heap()
        n = X_np.shape[0]
        if K == 1:
            out = torch.full((n, 1), np.float32(self.base_prediction), dtype=torch.float32,
                             device=dev)
        else:
            out = D.rows_of(self._uniform_prior_logits(), n, dev)
        if (X_np.ndim == 2 and np.issubdtype(X_np.dtype, np.floating)
                and X_np.shape[1] == self.num_features):
            cols, tables = None, heap
            if heap[3] and n >= _NARROW_MIN_ROWS:
                used, narrow = self._used_features()
                if 2 * len(used) <= X_np.shape[1]:
                    cols, tables = used, narrow
            feat, bin_, leaf, n_rounds = tables

            def walk(codes, r0, r1):
                if n_rounds:
                    D.predict_heap(codes, feat, bin_, leaf, n_rounds, K, self.max_depth,
                                   self.learning_rate, out[r0:r1])

            D.upload_and_bin(X_np, torch.as_tensor(self.bin_edges), dev, cols=cols,
                             on_chunk=walk)
            return out
        codes = self.bin_inference_data(X_np)
        feat, bin_, leaf, n_rounds = heap
        if n_rounds:
            D.predict_heap(codes, feat, bin_, leaf, n_rounds, K, self.max_depth,
                           self.learning_rate, out)
        del codes
        return out

    def _predict_values(self, codes, tables):
        out = torch.full((codes.n, 1), np.float32(self.base_prediction), dtype=torch.float32,
                         device=torch.device(self.device))
        feat, bin_, leaf, n = tables
        if n:
            D.predict_heap(codes, feat, bin_, leaf, n, 1, self.max_depth, self.learning_rate, out)
        return out[:, 0]

    def _predict_scores(self, codes, tables):
        dev = torch.device(self.device)
        scores = D.rows_of(self._uniform_prior_logits(), codes.n, dev)
        feat, bin_, leaf, n = tables
        if n:
            D.predict_heap(codes, feat, bin_, leaf, n, self.num_classes, self.max_depth,
                           self.learning_rate, scores)
        D.softmax_rows(scores)
        return scores

    def predict_binned(self, codes):
        return self._predict_values(codes, self._cached_heap())

    def predict_proba_binned(self, codes):
        return self._predict_scores(codes, self._cached_heap())

    def predict(self, X_np):
        """Regression values, or class labels for classification (warpgbm/core.py:957-974)."""
        if self.objective in ("multiclass", "binary"):
            probs = self.predict_proba(X_np)
            return self.label_encoder.inverse_transform(np.argmax(probs, axis=1))
        ph = _Phases()
        out = self._infer(X_np, 1)
        ph.mark("codes + trees")
        preds = D.to_host(out[:, 0])
        ph.mark("copy out")
        ph.report("predict")
        return preds

    def predict_proba(self, X_np):
        """Class probabilities (warpgbm/core.py:976-989)."""
        if self.objective not in ["multiclass", "binary"]:
            raise ValueError("predict_proba only available for classification objectives")
        scores = self._infer(X_np, self.num_classes)
        D.softmax_rows(scores)
        return D.to_host(scores)

    # ------------------------------------------------------------------ importance
    @staticmethod
    def _share_of_total(a):
        """Each row of ``a`` (float32) divided by its own sum; all-zero rows
        stay zero."""
        tot = a.sum(axis=-1, keepdims=True)
        return np.where(tot > 0, a / np.where(tot > 0, tot, 1), a).astype(a.dtype)

    def get_feature_importance(self, importance_type="gain", normalize=True):
        """Summed split gain per feature over all eras (warpgbm/core.py:1032-1065),
        as fractions of the total with ``normalize``."""
        if self.feature_importance_ is None:
            raise ValueError("Model has not been fitted yet.")
        if importance_type != "gain":
            raise ValueError(f"importance_type '{importance_type}' not supported. Use 'gain'.")
        imp = np.array(self.feature_importance_, copy=True)
        return self._share_of_total(imp) if normalize else imp

    def get_per_era_feature_importance(self, normalize=True):
        """Split gain per (era, feature) (warpgbm/core.py:1067-1101); with
        ``normalize`` every era's row sums to 1 (eras without gain stay 0)."""
        if self.per_era_feature_importance_ is None:
            raise ValueError("Model has not been fitted yet.")
        imp = np.array(self.per_era_feature_importance_, copy=True)
        return self._share_of_total(imp) if normalize else imp

    # ------------------------------------------------------------------ persistence
    def save_model(self, path):
        """Pickle the model state with the reference's keys (warpgbm/core.py:1103-1155)."""
        if not self._is_fitted:
            raise ValueError("Cannot save unfitted model. Call fit() first.")
        state = {
            "objective": self.objective,
            "num_bins": self.num_bins,
            "max_depth": self.max_depth,
            "learning_rate": self.learning_rate,
            "n_estimators": self.n_estimators,
            "min_child_weight": self.min_child_weight,
            "min_split_gain": self.min_split_gain,
            "L2_reg": self.L2_reg,
            "colsample_bytree": self.colsample_bytree,
            "random_state": self.random_state,
            "warm_start": self.warm_start,
            "forest": self.forest,
            "bin_edges": torch.as_tensor(self.bin_edges).detach().cpu(),
            "base_prediction": self.base_prediction,
            "num_features": self.num_features,
            "num_classes": self.num_classes,
            "classes_": self.classes_,
            "label_encoder": self.label_encoder,
            "feature_importance_": self.feature_importance_,
            "per_era_feature_importance_": self.per_era_feature_importance_,
            "_is_fitted": self._is_fitted,
            "_trees_trained": self._trees_trained,
            "training_loss": getattr(self, "training_loss", []),
            "eval_loss": getattr(self, "eval_loss", []),
        }
        with open(path, "wb") as f:
            pickle.dump(state, f)
        print(f"Model saved to {path}")

    def load_model(self, path):
        """Restore a model written by :meth:`save_model` (warpgbm/core.py:1157-1213).
        Only load files you trust: the format is a pickle, as in the reference."""
        with open(path, "rb") as f:
            state = pickle.load(f)
        for k in ["objective", "num_bins", "max_depth", "learning_rate", "n_estimators",
                  "min_child_weight", "min_split_gain", "L2_reg", "colsample_bytree",
                  "random_state", "warm_start", "forest", "bin_edges", "base_prediction",
                  "num_features", "num_classes", "classes_", "label_encoder",
                  "feature_importance_", "per_era_feature_importance_", "_is_fitted",
                  "_trees_trained"]:
            setattr(self, k, state[k])
        self.training_loss = state.get("training_loss", [])
        self.eval_loss = state.get("eval_loss", [])
        if self.per_era_feature_importance_ is not None:
            self.num_eras = self.per_era_feature_importance_.shape[0]
        self._heap = None
        print(f"Model loaded from {path} ({self._trees_trained} trees)")
        return self

    def flatten_tree(self, tree, max_nodes):
        """Pre-order table [max_nodes, 6] of (feature, bin, left, right, is_leaf,
        leaf_value), NaN-filled (the reference's predict table format,
        warpgbm/core.py:1215-1252)."""
        flat = torch.full((max_nodes, 6), float("nan"), dtype=torch.float32)
        counter = [0]

        def walk(node):
            i = counter[0]
            counter[0] += 1
            if "leaf_value" in node:
                flat[i, 4] = 1.0
                flat[i, 5] = float(node["leaf_value"])
                return
            flat[i, 0] = float(node["feature"])
            flat[i, 1] = float(node["bin"])
            flat[i, 4] = 0.0
            flat[i, 2] = counter[0]
            walk(node["left"])
            flat[i, 3] = counter[0]
            walk(node["right"])

        walk(tree)
        return flat


# ---------------------------------------------------------------------- tree helpers
def _heaps_to_dicts(feat, bin_, leaf, count):
    """Reference tree dicts of many heap records ([..., H] arrays, trees in
    row-major order; feat -1 leaf, -2 absent, >= 0 split; children of h at
    2h+1 / 2h+2), each built bottom-up by the C extension ``_trees``.  A tree
    with no root is None, as is an absent child of a split."""
    try:
        from . import _trees
    except ImportError as e:  # built with the HIP library by warpgbm_amd.build
        raise ImportError("warpgbm_amd._trees is not built; run `python -m warpgbm_amd.build`") \
            from e
    H = feat.shape[-1]
    return _trees.heaps_to_dicts(np.ascontiguousarray(feat, dtype=np.int32),
                                 np.ascontiguousarray(bin_, dtype=np.int32),
                                 np.ascontiguousarray(leaf, dtype=np.float32),
                                 np.ascontiguousarray(count, dtype=np.int64), H)


def _preorder_heap(H):
    """All heap indices < H in depth-first pre-order (left first).  For a
    complete heap (H = 2^(D+1) - 1) the pre-order position of a node follows
    from its parent's: left child = parent + 1, right child = parent + 1 + the
    size of the left child's subtree; computed level by level."""
    D = int(H + 1).bit_length() - 2
    if H < 1 or (1 << (D + 1)) - 1 != H:
        out, stack = [], [0]
        while stack:
            h = stack.pop()
            if h < H:
                out.append(h)
                stack.append(2 * h + 2)
                stack.append(2 * h + 1)
        return np.asarray(out, dtype=np.int64)
    pos = np.zeros(H, dtype=np.int64)
    for d in range(D):
        par = np.arange((1 << d) - 1, (1 << (d + 1)) - 1, dtype=np.int64)
        sub = (1 << (D - d)) - 1  # nodes under a child of a depth-d node
        pos[2 * par + 1] = pos[par] + 1
        pos[2 * par + 2] = pos[par] + 1 + sub
    out = np.empty(H, dtype=np.int64)
    out[pos] = np.arange(H, dtype=np.int64)
    return out


def _dict_to_heap(tree, H):
    feat = np.full(H, -1, np.int32)
    bin_ = np.zeros(H, np.int32)
    leaf = np.zeros(H, np.float32)

    def walk(node, h):
        if h >= H:
            raise ValueError("tree deeper than max_depth")
        if "leaf_value" in node:
            leaf[h] = np.float32(node["leaf_value"])
            return
        feat[h] = int(node["feature"])
        bin_[h] = int(node["bin"])
        walk(node["left"], 2 * h + 1)
        walk(node["right"], 2 * h + 2)

    walk(tree, 0)
    return feat, bin_, leaf
