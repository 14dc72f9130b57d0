"""The reference estimator's tree growth on the CPU (oracle; test-only).

Restates warpgbm/core.py: grow_forest (692-744), grow_forest_multiclass
(746-818), grow_tree (597-658), find_best_split (565-594) and the
predict drivers (917-932, 991-1030) -- recursively, depth first, left child
first, smaller child's histogram computed and the sibling obtained by
subtraction, exactly the reference's control flow.  Histogram arithmetic is
the exact quantised form of ``ops``: per tree a shift s from max|residual|
over all rows.  One era: per node a histogram shift (ops.node_shift: the
parent's, unless the node's own residuals are all below 2^-8 of the
parent's scale); exact integer sums, and the sibling by exact subtraction
when both children keep the parent's shift (else both children histogrammed
directly).  Several eras: every (node, era) segment at the shift of its own
largest |residual| (ops.key_shift), the sibling's segment of an era by
subtraction where the parent's and both children's shifts of that era are
equal (else histogrammed directly).  One rounding to float32 per era before
the split scan.  Leaf means come from the wide quantisation of
ops.leaf_value63.
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
        # (Q, C, shift or per-era shifts) -> per-era gain, dir; clib.split_scan_q
        # is the same in C
        self.scan = scan or (lambda Q, C, s, mcw, eps: ops.split_scan(
            ops.dequantise(Q, s), C.astype(F32), mcw, eps))
        self.splits = []  # (global feature, per-era gains) in DFS pre-order

    def grow(self, resid, rows):
        r = np.asarray(resid, dtype=F32)
        rows = np.asarray(rows, dtype=np.int64)
        self.r = r
        self.s = ops.shift_from_absmax(np.max(np.abs(r[rows])) if len(rows) else F32(0),
                                       self.qbits)
        self.s63 = ops.shift63(self.s, self.qbits)
        self.q63 = ops.quantise(r, self.s63)
        self._qcache = {}
        self.leaf_rows = []  # (rows, leaf value)
        if self.E > 1:
            S = self._key_shifts(rows)
            Q, C = self._hist_era(rows, S)
            return self._node_era(Q, C, rows, 0, S)
        Q, C = self._hist(rows, self.s)
        return self._node(Q, C, rows, 0, self.s)

    # ---- several eras: per-(node, era) shifts
    def _key_shifts(self, rows):
        from . import clib

        m = clib.era_absmax(self.r, rows, self.era, self.E)
        return np.array([ops.key_shift(v, self.qbits) for v in m], np.int64)

    def _hist_era(self, rows, S):
        q = ops.quantise_by_era(self.r, rows, self.era, S)
        return self.hist(self.codes, q, rows, self.feat_sel, self.era, self.E, self.B)

    def _node_era(self, Q, C, rows, depth, S):
        if depth == self.max_depth:
            return self._leaf(rows)
        gain, dirn = self.scan(Q, C, S, self.mcw, self.eps)
        lf, b = ops.des_select(gain, dirn, self.msg)
        if lf == -1:
            return self._leaf(rows)
        gf = int(self.feat_sel[lf])
        self.splits.append((gf, gain[:, lf, b].copy()))
        go_left = self.codes[rows, gf].astype(np.int64) <= b
        left, right = rows[go_left], rows[~go_left]
        QL = CL = QR = CR = SL = SR = None
        if depth + 1 < self.max_depth:  # (children at max_depth are leaves)
            SL, SR = self._key_shifts(left), self._key_shifts(right)
            same = (SL == S) & (SR == S)  # eras where the sibling is parent - child
            small_left = len(left) <= len(right)
            small, other = (left, right) if small_left else (right, left)
            Qs, Cs = self._hist_era(small, SL if small_left else SR)
            Qo, Co = Q - Qs, C - Cs
            if not same.all():
                # the other child's segments of those eras, directly
                sel = other[~same[self.era[other]]]
                Qd, Cd = self._hist_era(sel, SR if small_left else SL)
                Qo[~same] = Qd[~same]
                Co[~same] = Cd[~same]
            QL, CL, QR, CR = (Qs, Cs, Qo, Co) if small_left else (Qo, Co, Qs, Cs)
        return {
            "feature": gf,
            "bin": int(b),
            "left": self._node_era(QL, CL, left, depth + 1, SL),
            "right": self._node_era(QR, CR, right, depth + 1, SR),
        }

    def _q(self, hs):
        if hs not in self._qcache:
            self._qcache[hs] = ops.quantise(self.r, hs)
        return self._qcache[hs]

    def _hist(self, rows, hs):
        return self.hist(self.codes, self._q(hs), rows, self.feat_sel, self.era, self.E, self.B)

    def _child_shift(self, rows, hs):
        m = np.max(np.abs(self.r[rows])) if len(rows) else F32(0)
        return ops.node_shift(m, hs, self.qbits)

    def _leaf(self, rows):
        v = ops.leaf_value63(self.q63[rows], len(rows), self.s63)
        self.leaf_rows.append((rows, v))
        return {"leaf_value": float(v), "samples": int(len(rows))}

    def _node(self, Q, C, rows, depth, hs):
        if depth == self.max_depth:
            return self._leaf(rows)
        gain, dirn = self.scan(Q, C, hs, self.mcw, self.eps)
        lf, b = ops.des_select(gain, dirn, self.msg)
        if lf == -1:
            return self._leaf(rows)
        gf = int(self.feat_sel[lf])
        self.splits.append((gf, gain[:, lf, b].copy()))
        go_left = self.codes[rows, gf].astype(np.int64) <= b
        left, right = rows[go_left], rows[~go_left]
        hl = hr = hs
        if depth + 1 < self.max_depth:
            hl, hr = self._child_shift(left, hs), self._child_shift(right, hs)
            if hl == hs and hr == hs:
                if len(left) <= len(right):
                    QL, CL = self._hist(left, hs)
                    QR, CR = Q - QL, C - CL
                else:
                    QR, CR = self._hist(right, hs)
                    QL, CL = Q - QR, C - CR
            else:  # a child with a finer shift: both histogrammed directly
                QL, CL = self._hist(left, hl)
                QR, CR = self._hist(right, hr)
        else:  # children at max_depth are leaves: their histograms are never read
            QL = CL = QR = CR = None
        return {
            "feature": gf,
            "bin": int(b),
            "left": self._node(QL, CL, left, depth + 1, hl),
            "right": self._node(QR, CR, right, depth + 1, hr),
        }


class LiteralF32Grower(TreeGrower):
    """The reference's literal float32 arithmetic: histograms accumulated in
    float32 in ascending position order (ops.histogram_f32_seq, one order its
    atomics can take, histogram_kernel.cu:43-44, 57-58), the sibling as the
    float32 difference parent - child (core.py:638-643), the split scan on
    those arrays, and the leaf as numpy's float32 mean of the leaf's residuals
    (core.py:599, 614; the reference's torch reduction order differs).

    Its trees are compared with the exact mode's (compare_growth), not held to
    bit equality.  ``trace`` records, per split node in DFS order, the
    criterion array and the pick, for the near-tie check."""

    def grow(self, resid, rows):
        self.r = np.asarray(resid, dtype=F32)
        rows = np.asarray(rows, dtype=np.int64)
        self.leaf_rows = []
        self.trace = []
        G, H = ops.histogram_f32_seq(self.codes, self.r, rows, self.feat_sel, self.era, self.E,
                                     self.B)
        return self._node_f32(G, H, rows, 0)

    def _leaf(self, rows):
        v = F32(np.mean(self.r[rows], dtype=F32))
        self.leaf_rows.append((rows, v))
        return {"leaf_value": float(v), "samples": int(len(rows))}

    def _node_f32(self, G, H, rows, depth):
        if depth == self.max_depth:
            return self._leaf(rows)
        gain, dirn = ops.split_scan(G, H, self.mcw, self.eps)
        lf, b = ops.des_select(gain, dirn, self.msg)
        if lf == -1:
            return self._leaf(rows)
        gf = int(self.feat_sel[lf])
        self.splits.append((gf, gain[:, lf, b].copy()))
        go_left = self.codes[rows, gf].astype(np.int64) <= b
        left, right = rows[go_left], rows[~go_left]
        if depth + 1 < self.max_depth:
            hist = lambda rr: ops.histogram_f32_seq(self.codes, self.r, rr, self.feat_sel,
                                                    self.era, self.E, self.B)
            if len(left) <= len(right):
                GL, HL = hist(left)
                GR, HR = G - GL, H - HL
            else:
                GR, HR = hist(right)
                GL, HL = G - GR, H - HR
        else:
            GL = HL = GR = HR = None
        return {"feature": gf, "bin": int(b),
                "left": self._node_f32(GL, HL, left, depth + 1),
                "right": self._node_f32(GR, HR, right, depth + 1)}


def split_criteria(codes, resid, rows, feat_sel, era, E, B, mcw, eps):
    """Float64 DES criterion of every candidate of one node from float64
    histogram sums of the float32 residuals (np.bincount: each sum within
    2^-52 relative of the true one), for judging near-ties: returns
    (crit [F, B-1] float64, mask of the candidates the DES rule admits)."""
    rows = np.asarray(rows, dtype=np.int64)
    F = len(feat_sel)
    r = np.asarray(resid, dtype=np.float64)[rows]
    es = np.zeros(len(rows), np.int64) if E == 1 else np.asarray(era, np.int64)[rows]
    G = np.zeros((E, F, B))
    H = np.zeros((E, F, B))
    for fi, f in enumerate(feat_sel):
        b = codes[rows, f].astype(np.int64)
        ok = (b >= 0) & (b < B)
        G[:, fi, :] = np.bincount(es[ok] * B + b[ok], weights=r[ok], minlength=E * B).reshape(E, B)
        H[:, fi, :] = np.bincount(es[ok] * B + b[ok], minlength=E * B).reshape(E, B)
    Gt, Ht = G.sum(axis=2, keepdims=True), H.sum(axis=2, keepdims=True)
    GL, HL = np.cumsum(G, axis=2)[:, :, :-1], np.cumsum(H, axis=2)[:, :, :-1]
    GR, HR = Gt - GL, Ht - HL
    ok = (HL >= mcw) & (HR >= mcw)
    with np.errstate(divide="ignore", invalid="ignore"):
        g = GL**2 / (HL + eps) + GR**2 / (HR + eps) - Gt**2 / (Ht + eps)
        d = np.where(GL / (HL + eps) > GR / (HR + eps), 1.0, -1.0)
    gain = np.where(ok, g, 0.0)
    dirn = np.where(ok, d, 0.0)
    crit = gain.mean(axis=0)
    agree = np.abs(dirn.sum(axis=0))
    mask = agree == agree.max() if E > 1 else np.ones_like(crit, bool)
    return crit, mask


def compare_growth(exact, literal, codes, tie_rtol=1e-4, leaf_rtol=1e-5, exact_may_win=False):
    """Walk two fitted forests (same data; exact mode and literal float32
    mode) tree by tree, node by node.  Where both split the same way, recurse;
    where both are leaves, the leaf values must agree within leaf_rtol of the
    leaf's mean |residual|.  At the first node whose decision differs, the two
    picks are judged on float64 criteria (split_criteria) of that node's rows:
    a near-tie when |crit_a - crit_b| <= tie_rtol * max(|crit_a|, |crit_b|)
    (a leaf counts as crit = min_split_gain).  With exact_may_win, a
    difference where the exact mode's pick is the better one in float64 is
    accepted too (data whose float32 sums lose the small residuals, where the
    literal arithmetic is the one that errs).  Every later tree sees other
    residuals, so the walk stops there.  Returns (trees compared identical,
    description of the first difference or None); raises AssertionError for a
    difference that is not a near-tie or a leaf value out of tolerance."""
    assert len(exact.forest) == len(literal.forest)
    B = exact.B
    ga_list = exact.growers
    n_ident = 0
    for i, (ga, r) in enumerate(ga_list):
        gb = literal.growers[i][0]
        ta = ga_tree = _tree_of(exact, i)
        tb = _tree_of(literal, i)
        diff = _walk(ga_tree, tb, np.arange(codes.shape[0]), codes, r, exact, ga, B,
                     tie_rtol, leaf_rtol, f"tree {i}", exact_may_win)
        if diff is not None:
            return n_ident, diff
        n_ident += 1
        del ta
    return n_ident, None


def _tree_of(forest, i):
    if forest.objective == "regression":
        return forest.forest[i]
    K = forest.K
    return forest.forest[i // K][i % K]


def _walk(a, b, rows, codes, r, forest, g, B, tie_rtol, leaf_rtol, where, may_win):
    la, lb = "leaf_value" in a, "leaf_value" in b
    if la and lb:
        assert a["samples"] == b["samples"] == len(rows), where
        scale = float(np.mean(np.abs(r[rows].astype(np.float64)))) if len(rows) else 0.0
        assert abs(a["leaf_value"] - b["leaf_value"]) <= leaf_rtol * max(scale, 1e-30), \
            f"{where}: leaf {a['leaf_value']} vs {b['leaf_value']}"
        return None
    if not la and not lb and a["feature"] == b["feature"] and a["bin"] == b["bin"]:
        go = codes[rows, int(a["feature"])].astype(np.int64) <= int(a["bin"])
        d = _walk(a["left"], b["left"], rows[go], codes, r, forest, g, B, tie_rtol, leaf_rtol,
                  where + " L", may_win)
        if d is not None:
            return d
        return _walk(a["right"], b["right"], rows[~go], codes, r, forest, g, B, tie_rtol,
                     leaf_rtol, where + " R", may_win)
    crit, mask = split_criteria(codes, r, rows, g.feat_sel, g.era, g.E, B, g.mcw, g.eps)
    pos = {int(f): k for k, f in enumerate(g.feat_sel)}

    def value(node):
        if "leaf_value" in node:
            return float(g.msg)
        k = pos[int(node["feature"])]
        return float(crit[k, int(node["bin"])]) if mask[k, int(node["bin"])] else -np.inf

    va, vb = value(a), value(b)
    gap = abs(va - vb)
    if np.isfinite(gap) and gap <= tie_rtol * max(abs(va), abs(vb)):
        return f"{where}: near-tie, crit {va:.9g} vs {vb:.9g}"
    assert may_win and va > vb, f"{where}: decisions differ beyond a near-tie: crit {va} vs {vb}"
    return f"{where}: exact mode's pick better in float64, crit {va:.9g} vs {vb:.9g}"


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

    def fit_codes(self, codes, y, era_id=None, feat_sets=None, hist=None, scan=None,
                  literal_f32=False, progress=None):
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
        Grower = LiteralF32Grower if literal_f32 else TreeGrower
        self.growers = []  # per tree: (grower, residual) for compare_growth
        self.forest = []
        if self.objective == "regression":
            Y = np.asarray(y, dtype=F32)
            self.base = base_score(Y)
            preds = np.full(N, self.base, F32)
            for i in range(self.n_estimators):
                fs = np.arange(F) if feat_sets is None else feat_sets[i]
                resid = Y - preds
                g = Grower(codes, era, self.E, self.B, self.max_depth, self.mcw, self.msg,
                           self.eps, fs, qbits, hist, scan)
                tree = g.grow(resid, rows)
                self.growers.append((g, resid))
                for rws, v in g.leaf_rows:
                    preds[rws] = preds[rws] + F32(self.lr) * v
                self._importance(g)
                self.forest.append(tree)
                if progress:
                    progress(i)
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
                    g = Grower(codes, era, self.E, self.B, self.max_depth, self.mcw,
                               self.msg, self.eps, fs, qbits, hist, scan)
                    tree = g.grow(res[k], rows)
                    self.growers.append((g, res[k]))
                    for rws, v in g.leaf_rows:
                        scores[rws, k] = scores[rws, k] + F32(self.lr) * v
                    self._importance(g)
                    trees.append(tree)
                self.forest.append(trees)
                if progress:
                    progress(i)
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
