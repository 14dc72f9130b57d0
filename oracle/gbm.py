"""The reference estimator's tree growth on the CPU (oracle; test-only).

Restates warpgbm/core.py: grow_forest (692-744), grow_forest_multiclass
(746-818), grow_tree (597-658), find_best_split (565-594) and the
predict drivers (917-932, 991-1030) -- recursively, depth first, left child
first, smaller child's histogram computed and the sibling obtained by
subtraction, exactly the reference's control flow.  Histogram arithmetic is
the exact quantised form of ``ops`` (per tree: one shift from max|residual|
over all rows, exact integer sums and exact subtraction, one rounding to
float32 before the split scan).
"""
from __future__ import annotations

import numpy as np

from . import ops

F32 = np.float32


class TreeGrower:
    """Grows one tree given the residual of the tree (fixed, core.py:719)."""

    def __init__(self, codes, era_idx, E, B, max_depth, min_child_weight, min_split_gain,
                 L2_reg, feat_sel, qbits, hist=None, scan=None):
        self.codes = codes
        self.era = era_idx
        self.E = E
        self.B = B
        self.max_depth = max_depth
        self.mcw = min_child_weight
        self.msg = min_split_gain
        self.eps = L2_reg
        self.feat_sel = np.asarray(feat_sel, dtype=np.int64)
        self.qbits = qbits
        self.hist = hist or ops.histogram_exact_q
        # (Q, C, shift) -> per-era gain, dir; clib.split_scan_q is the same in C
        self.scan = scan or (lambda Q, C, s, mcw, eps: ops.split_scan(
            ops.dequantise(Q, s), C.astype(F32), mcw, eps))
        self.splits = []  # (global feature, per-era gains) in DFS pre-order

    def grow(self, resid, rows):
        r = np.asarray(resid, dtype=F32)
        self.s = ops.shift_from_absmax(np.max(np.abs(r)) if len(r) else F32(0), self.qbits)
        self.q = ops.quantise(r, self.s)
        self.leaf_rows = []  # (rows, leaf value)
        Q, C = self._hist(rows)
        return self._node(Q, C, np.asarray(rows, dtype=np.int64), 0)

    def _hist(self, rows):
        return self.hist(self.codes, self.q, rows, self.feat_sel, self.era, self.E, self.B)

    def _leaf(self, rows):
        v = ops.leaf_value(int(self.q[rows].sum()), len(rows), self.s)
        self.leaf_rows.append((rows, v))
        return {"leaf_value": float(v), "samples": int(len(rows))}

    def _node(self, Q, C, rows, depth):
        if depth == self.max_depth:
            return self._leaf(rows)
        gain, dirn = self.scan(Q, C, self.s, self.mcw, self.eps)
        lf, b = ops.des_select(gain, dirn, self.msg)
        if lf == -1:
            return self._leaf(rows)
        gf = int(self.feat_sel[lf])
        self.splits.append((gf, gain[:, lf, b].copy()))
        go_left = self.codes[rows, gf].astype(np.int64) <= b
        left, right = rows[go_left], rows[~go_left]
        if depth + 1 < self.max_depth:
            if len(left) <= len(right):
                QL, CL = self._hist(left)
                QR, CR = Q - QL, C - CL
            else:
                QR, CR = self._hist(right)
                QL, CL = Q - QR, C - CR
        else:  # children at max_depth are leaves: their histograms are never read
            QL = CL = QR = CR = None
        return {
            "feature": gf,
            "bin": int(b),
            "left": self._node(QL, CL, left, depth + 1),
            "right": self._node(QR, CR, right, depth + 1),
        }


def softmax_residuals(logits, labels):
    """residual_k = -(softmax(F)_k - onehot_k) for every class, [K, n]
    (core.py:186-214 and :782), with the oracle's deterministic exp."""
    from . import clib

    return clib.softmax_residual(logits, labels)


class Forest:
    """Reference fit loop.  feat_sets: list of per-round feature subsets (or
    None for all features)."""

    def __init__(self, objective="regression", num_bins=10, max_depth=3, learning_rate=0.1,
                 n_estimators=100, min_child_weight=20, min_split_gain=0.0, L2_reg=1e-6):
        self.objective = objective
        self.B = num_bins
        self.max_depth = max_depth
        self.lr = learning_rate
        self.n_estimators = n_estimators
        self.mcw = min_child_weight
        self.msg = min_split_gain
        self.eps = L2_reg

    def fit_codes(self, codes, y, era_id=None, feat_sets=None, hist=None, scan=None):
        codes = np.asarray(codes)
        N, F = codes.shape
        if era_id is None:
            era_id = np.ones(N, dtype=np.int32)
        uniq, inv = np.unique(era_ids_int32(era_id), return_inverse=True)
        self.E = len(uniq)
        era = inv.astype(np.int64).reshape(-1)
        self.num_features = F
        self.imp = np.zeros((self.E, F), dtype=F32)
        qbits = ops.qbits_for_rows(N)
        rows = np.arange(N)
        self.forest = []
        if self.objective == "regression":
            Y = np.asarray(y, dtype=F32)
            self.base = base_score(Y)
            preds = np.full(N, self.base, F32)
            for i in range(self.n_estimators):
                fs = np.arange(F) if feat_sets is None else feat_sets[i]
                resid = Y - preds
                g = TreeGrower(codes, era, self.E, self.B, self.max_depth, self.mcw, self.msg,
                               self.eps, fs, qbits, hist, scan)
                tree = g.grow(resid, rows)
                for rws, v in g.leaf_rows:
                    preds[rws] = preds[rws] + F32(self.lr) * v
                self._importance(g)
                self.forest.append(tree)
            self.train_preds = preds
        else:
            labels = np.asarray(y).astype(np.int32)
            K = int(labels.max()) + 1
            self.K = K
            scores = np.tile(class_prior_logits(labels, K), (N, 1)).astype(F32)
            for i in range(self.n_estimators):
                fs = np.arange(F) if feat_sets is None else feat_sets[i]
                res = softmax_residuals(scores, labels)
                trees = []
                for k in range(K):
                    g = TreeGrower(codes, era, self.E, self.B, self.max_depth, self.mcw,
                                   self.msg, self.eps, fs, qbits, hist, scan)
                    tree = g.grow(res[k], rows)
                    for rws, v in g.leaf_rows:
                        scores[rws, k] = scores[rws, k] + F32(self.lr) * v
                    self._importance(g)
                    trees.append(tree)
                self.forest.append(trees)
            self.train_scores = scores
        self.feature_importance = self.imp.sum(axis=0)
        return self

    def _importance(self, g):
        """per_era_imp[e, f] += per_era_gain[e, local_f, bin], float32, DFS order
        (core.py:624-627)."""
        for gf, gains in g.splits:
            self.imp[:, gf] += gains

    def predict_codes(self, codes):
        codes = np.asarray(codes)
        if self.objective == "regression":
            out = np.full(codes.shape[0], self.base, F32)
            for tree in self.forest:
                out = out + F32(self.lr) * ops.predict_tree_dict(codes, tree)
            return out
        out = np.tile(uniform_prior_logits(self.K), (codes.shape[0], 1)).astype(F32)
        for trees in self.forest:
            for k, tree in enumerate(trees):
                out[:, k] = out[:, k] + F32(self.lr) * ops.predict_tree_dict(codes, tree)
        from . import clib

        return clib.softmax_rows(out)


def era_ids_int32(era_id):
    """The era ids after the reference's ``.type(torch.int32)`` (core.py:493):
    a C cast -- floats truncated toward zero, wider integers wrapped to 32
    bits, bools 0/1."""
    return np.asarray(era_id).reshape(-1).astype(np.int32, casting="unsafe")


def base_score(Y):
    """The regression start value Y.mean() (core.py:387) as the float32
    nearest the exact mean of the float32 targets (float64 pairwise sum, one
    division, one rounding).  The reference's torch float32 reduction is
    within a few ulps of it in an order no other device reproduces."""
    return F32(np.mean(np.asarray(Y, dtype=F32), dtype=np.float64))


def class_prior_logits(labels, K):
    """log(prior_k + 1e-10) for every class present, 0 for an absent class
    (core.py:450-456): prior_k = float32(count_k) / float32(n), + 1e-10 in
    float32, and the float32 nearest the natural log of that (torch.log is
    within 1 ulp of it)."""
    n = F32(len(labels))
    out = np.zeros(K, F32)
    for k in range(K):
        p = F32(np.count_nonzero(labels == k)) / n
        if p > 0:
            out[k] = F32(np.log(np.float64(F32(p + F32(1e-10)))))
    return out


def uniform_prior_logits(K):
    """The start logits of predict_proba (core.py:1003-1007): 1/K + 1e-10 and
    its log in float64 (a numpy float64 wrapped by torch.tensor), rounded to
    float32 once when stored into the float32 score matrix."""
    return np.full(K, F32(np.log(np.float64(1.0) / np.float64(K) + 1e-10)), F32)
