"""numpy restatements of WarpGBM's native operators (CPU oracle; test-only).

Conventions
* float32 arithmetic is done with numpy float32 arrays/scalars; every
  operation rounds to float32 (x86-64 SSE, no extended precision, no FMA).
* "exact" histograms use the arithmetic of the HIP library: each residual is
  quantised to q = rint(r * 2^s) (exact scaling by a power of two), sums of q
  are exact integers, and a float32 value is produced once by rounding
  ldexp(sum, -s).  The shift s comes from max|r| (see shift_from_absmax); in
  tree growth each node has its own (node_shift), and leaf means use a wider
  quantisation (leaf_value63).
"""
from __future__ import annotations

import numpy as np

F32 = np.float32


# --------------------------------------------------------------------------- quantisation
def qbits_for_rows(n: int) -> int:
    """Significant bits per quantised residual for up to n rows: keeps
    |sum q| < 2^53 (so sums convert to float64 exactly); at most 28."""
    bl = int(n).bit_length()
    return int(min(28, max(8, 52 - bl)))


def shift_from_absmax(m, qbits: int) -> int:
    """s such that max|r| * 2^s < 2^qbits: with m = f * 2^e, f in [0.5, 1)."""
    m = F32(m)
    if not (m > 0):
        return 0
    _, e = np.frexp(m)
    return int(qbits - int(e))


def quantise(r: np.ndarray, s: int) -> np.ndarray:
    """q = rint(r * 2^s) as int64 (ties to even); r * 2^s is exact in float32."""
    return np.rint(np.ldexp(np.asarray(r, dtype=F32), s)).astype(np.int64)


def dequantise(Q, s) -> np.ndarray:
    """float32(ldexp(Q, -s)): one rounding of an exact value (|Q| < 2^53).  s
    is one shift, or an array of per-era shifts for Q of shape [E, ...]."""
    Q = np.asarray(Q, dtype=np.int64)
    s = np.asarray(s, dtype=np.int64)
    if s.ndim == 1:
        s = s.reshape((-1,) + (1,) * (Q.ndim - 1))
    return np.ldexp(Q.astype(np.float64), -s).astype(F32)


def leaf_value(sq: int, count: int, s: int) -> np.float32:
    """Node mean of the quantised residuals: float32(ldexp(sq, -s) / count),
    float64 arithmetic (the reference's residual[node_indices].mean(),
    warpgbm/core.py:599 and :614)."""
    return F32(np.ldexp(np.float64(sq), -s) / np.float64(count))


# Leaf values and node totals use a second, wide quantisation: q63 =
# rint(r * 2^s63) with s63 = s + 62 - qbits (|q63| < 2^62), so every residual
# down to max|r| * 2^-38 keeps all 24 bits and a leaf's mean is exact to
# float64 precision relative to its own residuals, however small they are
# next to the tree's largest.  Sums of q63 are exact integers, carried on the
# device as two int64 words per sum: hi = q63 >> 32 (arithmetic) and
# lo = q63 & (2^32 - 1).
def shift63(s: int, qbits: int) -> int:
    return int(s) + 62 - int(qbits)


def leaf_value63(q63_rows, count: int, s63: int) -> np.float32:
    """float32 mean of a leaf from its rows' q63 values, in the device's exact
    steps: H = sum(hi) + (sum(lo) >> 32), L = sum(lo) & (2^32 - 1) (so that
    sum q63 = H * 2^32 + L), v = float64(H) * 2^32 + float64(L) (one rounding
    when |H| < 2^53), leaf = float32(ldexp(v, -s63) / float64(count))."""
    q = np.asarray(q63_rows, dtype=np.int64)
    hi = int((q >> 32).sum())
    lo = int((q & 0xFFFFFFFF).sum())
    H = hi + (lo >> 32)
    L = lo & 0xFFFFFFFF
    v = np.float64(H) * np.float64(4294967296.0) + np.float64(L)
    return F32(np.ldexp(v, -int(s63)) / np.float64(count))


# A node's histogram shift: the root takes the tree's shift s; a child keeps
# its parent's shift unless the shift of its own max|r| is at least
# NODE_SHIFT_STEP larger (its residuals are all below 2^-8 of the parent's
# scale), in which case it takes its own.  Every node's histogram is the exact
# integer histogram of its rows at its shift (so G is within count * max|r of
# the node| * 2^(NODE_SHIFT_STEP - 30) of the real sum); a sibling is taken
# as parent - child only when both children keep the parent's shift, where
# that subtraction is exact.
NODE_SHIFT_STEP = 8


def node_shift(max_abs, parent_shift: int, qbits: int) -> int:
    s_own = shift_from_absmax(max_abs, qbits)
    return s_own if s_own - int(parent_shift) >= NODE_SHIFT_STEP else int(parent_shift)


# Several eras (E > 1): the histogram of every (node, era) segment is
# quantised at the shift of its own largest |residual| (key_shift), so the
# sums of an era whose residuals are far smaller than another era's keep
# their precision (the reference sums each era's bins in float32 of their
# own scale, warpgbm/cuda/histogram_kernel.cu:38-45, and DES votes per era,
# warpgbm/core.py:580-583).  A sibling segment is parent - child only where
# the parent's and both children's shifts of that era are equal (the
# subtraction is then exact); otherwise both children's segments of that
# era are histogrammed directly.
def key_shift(max_abs, qbits: int) -> int:
    """Shift of one (node, era) segment from its largest |residual|: 0 for
    an empty segment, an all-zero one or a non-finite maximum."""
    m = F32(max_abs)
    if not np.isfinite(m):
        return 0
    return shift_from_absmax(m, qbits)


def era_absmax(r, rows, era, E: int) -> np.ndarray:
    """[E] largest |r| of the rows of each era among ``rows`` (0 for an era
    without rows; NaN when an era holds a NaN)."""
    rows = np.asarray(rows, dtype=np.int64)
    out = np.zeros(E, F32)
    a = np.abs(np.asarray(r, dtype=F32)[rows])
    e = np.asarray(era, np.int64)[rows]
    nan = np.isnan(a)
    np.maximum.at(out, e[~nan], a[~nan])
    out[np.unique(e[nan])] = F32(np.nan)
    return out


def quantise_by_era(r, rows, era, shifts) -> np.ndarray:
    """Full-length int64 q with q[s] = rint(r[s] * 2^shifts[era[s]]) for s in
    rows (0 elsewhere)."""
    rows = np.asarray(rows, dtype=np.int64)
    q = np.zeros(len(r), np.int64)
    if len(rows):
        sh = np.asarray(shifts, np.int64)[np.asarray(era, np.int64)[rows]]
        q[rows] = np.rint(np.ldexp(np.asarray(r, dtype=F32)[rows], sh)).astype(np.int64)
    return q


# --------------------------------------------------------------------------- histogram
def histogram_exact_q(codes, q, rows, feats, era, E: int, B: int):
    """Exact integer histogram (restates warpgbm/cuda/histogram_kernel.cu:33-59
    with integer sums): Q[e, f, b] = sum of q[s], C[e, f, b] = number of s,
    over s in rows with e = era[s] (all 0 when E == 1) and
    b = codes[s, feats[f]] in [0, B).  codes: int8 [N, >=max(feats)+1]."""
    rows = np.asarray(rows, dtype=np.int64)
    feats = np.asarray(feats, dtype=np.int64)
    F = len(feats)
    Q = np.zeros((E, F, B), dtype=np.int64)
    C = np.zeros((E, F, B), dtype=np.int64)
    if len(rows) == 0:
        return Q, C
    qs = np.asarray(q, dtype=np.int64)[rows]
    es = np.zeros(len(rows), np.int64) if E == 1 else np.asarray(era, np.int64)[rows]
    ok_e = (es >= 0) & (es < E)
    for fi, f in enumerate(feats):
        b = np.asarray(codes[rows, f], dtype=np.int64)
        ok = ok_e & (b >= 0) & (b < B)
        idx = es[ok] * B + b[ok]
        # float64 weights: every partial sum is an integer below 2^53, hence exact
        Q[:, fi, :] = np.rint(np.bincount(idx, weights=qs[ok].astype(np.float64),
                                          minlength=E * B)).astype(np.int64).reshape(E, B)
        C[:, fi, :] = np.bincount(idx, minlength=E * B).reshape(E, B)
    return Q, C


def histogram_exact(codes, resid, rows, feats, era, E: int, B: int, qbits=None):
    """float32 G, H of one compute_histogram3 call in the HIP library's
    arithmetic: exact sums of residuals quantised at one shift from
    max|resid| over ``rows`` (E == 1) or, with several eras, at each era's
    own shift from max|resid| over the call's rows of that era (key_shift),
    then one rounding.  qbits follows the call's row count.  Sums over a
    non-finite residual are NaN (the whole call, or the era's)."""
    rows = np.asarray(rows, dtype=np.int64)
    r = np.asarray(resid, dtype=F32)
    qb = qbits_for_rows(max(len(rows), 1)) if qbits is None else qbits
    if E == 1:
        m = np.max(np.abs(r[rows])) if len(rows) else F32(0)
        if not np.isfinite(m):
            Q, C = histogram_exact_q(codes, np.zeros(len(r), np.int64), rows, feats, era, E, B)
            return np.full(Q.shape, np.nan, F32), C.astype(F32)
        s = shift_from_absmax(m, qb)
        Q, C = histogram_exact_q(codes, quantise(r, s), rows, feats, era, E, B)
        return dequantise(Q, s), C.astype(F32)
    e = np.asarray(era, np.int64)
    ok = rows[(e[rows] >= 0) & (e[rows] < E)]
    mx = era_absmax(r, ok, e, E)
    S = np.array([key_shift(v, qb) for v in mx], np.int64)
    q = quantise_by_era(np.where(np.isfinite(r), r, F32(0)), ok, e, S)
    Q, C = histogram_exact_q(codes, q, rows, feats, era, E, B)
    G = dequantise(Q, S)
    G[~np.isfinite(mx)] = np.nan
    return G, C.astype(F32)


def histogram_segments_exact(codes, resid, order, seg, feats, B: int, n_pos=None):
    """G, H [S, F, B] of one wgbm_histogram_segments call: segment k holds
    positions seg[k] .. seg[k+1]-1, whose rows are order[p] (residual
    resid[order[p]]).  One segment: one shift from max|r| over the call's
    n_pos positions; several: each segment at its own shift (key_shift of
    its largest |r|).  qbits follows n_pos."""
    order = np.asarray(order, np.int64)
    seg = np.asarray(seg, np.int64)
    r = np.asarray(resid, dtype=F32)
    S = len(seg) - 1
    n_pos = int(seg[-1]) if n_pos is None else int(n_pos)
    qb = qbits_for_rows(max(n_pos, 1))
    F = len(feats)
    G = np.zeros((S, F, B), F32)
    H = np.zeros((S, F, B), F32)
    for k in range(S):
        rows = order[seg[k]:seg[k + 1]]
        pool = order[:n_pos] if S == 1 else rows
        m = np.max(np.abs(r[pool])) if len(pool) else F32(0)
        s = key_shift(m, qb)
        Q, C = histogram_exact_q(codes, quantise(np.where(np.isfinite(r), r, F32(0)), s), rows,
                                 feats, None, 1, B)
        G[k] = dequantise(Q[0], s) if np.isfinite(m) else np.nan
        H[k] = C[0]
    return G, H


def histogram_f32_seq(codes, resid, rows, feats, era, E: int, B: int):
    """Literal restatement of histogram_kernel.cu:33-59 with the float32
    atomics applied in ascending position order (one of the orders the
    reference's atomics can produce): G += residual, H += 1.0f."""
    rows = np.asarray(rows, dtype=np.int64)
    feats = np.asarray(feats, dtype=np.int64)
    F = len(feats)
    G = np.zeros((E, F, B), dtype=F32)
    H = np.zeros((E, F, B), dtype=F32)
    r = np.asarray(resid, dtype=F32)
    es = np.zeros(len(rows), np.int64) if E == 1 else np.asarray(era, np.int64)[rows]
    for fi, f in enumerate(feats):
        b = np.asarray(codes[rows, f], dtype=np.int64)
        ok = (b >= 0) & (b < B) & (es >= 0) & (es < E)
        # np.add.at is unbuffered and applies the adds in index order, in float32
        np.add.at(G[:, fi, :], (es[ok], b[ok]), r[rows[ok]])
        np.add.at(H[:, fi, :], (es[ok], b[ok]), F32(1.0))
    return G, H


# --------------------------------------------------------------------------- split
def split_scan(G, H, min_child_samples, eps):
    """Per-era gain and direction, warpgbm/cuda/best_split_kernel.cu:25-54:
    sequential float32 totals over bins, then a sequential float32 prefix over
    b < B-1.  Vectorised over (era, feature).  Returns gain, dir [E, F, B-1]."""
    G = np.asarray(G, dtype=F32)
    H = np.asarray(H, dtype=F32)
    E, F, B = G.shape
    mcw = F32(min_child_samples)
    eps = F32(eps)
    Gt = np.zeros((E, F), F32)
    Ht = np.zeros((E, F), F32)
    for b in range(B):
        Gt = Gt + G[:, :, b]
        Ht = Ht + H[:, :, b]
    tot = (Gt * Gt) / (Ht + eps)
    GL = np.zeros((E, F), F32)
    HL = np.zeros((E, F), F32)
    gain = np.zeros((E, F, B - 1), F32)
    dirn = np.zeros((E, F, B - 1), F32)
    for b in range(B - 1):
        GL = GL + G[:, :, b]
        HL = HL + H[:, :, b]
        GR = Gt - GL
        HR = Ht - HL
        ok = (HL >= mcw) & (HR >= mcw)
        with np.errstate(divide="ignore", invalid="ignore"):
            g = (GL * GL) / (HL + eps) + (GR * GR) / (HR + eps) - tot
            lv = GL / (HL + eps)
            rv = GR / (HR + eps)
        gain[:, :, b] = np.where(ok, g, F32(0))
        dirn[:, :, b] = np.where(ok, np.where(lv > rv, F32(1), F32(-1)), F32(0))
    return gain, dirn


DES_ERA_BLOCK = 32


def era_sum_f64(gain):
    """float64 sum over axis 0 of float32 per-era values in the DES order:
    each block of 32 consecutive eras summed in era order, then the block
    sums in block order."""
    gain = np.asarray(gain, dtype=F32)
    E = gain.shape[0]
    acc = np.zeros(gain.shape[1:], np.float64)
    for b0 in range(0, E, DES_ERA_BLOCK):
        blk = np.zeros(gain.shape[1:], np.float64)
        for e in range(b0, min(E, b0 + DES_ERA_BLOCK)):  # era order inside the block
            blk = blk + gain[e].astype(np.float64)
        acc = acc + blk  # block order
    return acc


def des_criterion(gain, dirn):
    """(crit, agree) over [F, B-1] from per-era arrays (warpgbm/core.py:577-583).
    E == 1: crit = gain[0].  E > 1: crit = float32(sum_e gain_e / E) with the
    era sum in float64 in two levels: the eras of each block of 32 consecutive
    eras summed in era order, then the block sums in block order (for E <= 32
    that is the plain sequential sum); agree = |sum_e dir_e|, an exact
    integer (the reference's |mean_e dir| is that integer over E)."""
    gain = np.asarray(gain, dtype=F32)
    E = gain.shape[0]
    if E == 1:
        return gain[0].copy(), None
    crit = (era_sum_f64(gain) / np.float64(E)).astype(F32)
    agree = np.abs(np.rint(np.asarray(dirn, dtype=np.float64)).astype(np.int64).sum(axis=0))
    return crit, agree


def des_select(gain, dirn, min_split_gain):
    """Best (local feature, bin) or (-1, -1), warpgbm/core.py:577-594:
    mask = crit > min_split_gain (and agree == max agree when E > 1);
    first flat index of the masked maximum (torch.argmax takes the first)."""
    crit, agree = des_criterion(gain, dirn)
    msg = F32(min_split_gain)
    mask = crit > msg
    if agree is not None:
        mask &= agree == agree.max()
    if not mask.any():
        return -1, -1
    masked = np.where(mask, crit, F32(-np.inf))
    idx = int(np.argmax(masked.reshape(-1)))  # first maximum
    nb = gain.shape[2]
    return idx // nb, idx % nb


# --------------------------------------------------------------------------- binning
def bin_column(x, edges):
    """warpgbm/cuda/binner.cu:17-23: bin = number of LEADING edges with
    x >= edge (the linear scan stops at the first failure; NaN x -> 0)."""
    x = np.asarray(x, dtype=F32)
    e = np.asarray(edges, dtype=F32)
    if e.size == 0:
        return np.zeros(x.shape, np.int8)
    ge = x[:, None] >= e[None, :]
    return np.cumprod(ge, axis=1).sum(axis=1).astype(np.int8)


def quantile_levels(num_bins: int) -> np.ndarray:
    """torch.linspace(0, 1, B + 1)[1:-1] in float32 (warpgbm/core.py:529-531),
    via torch's own CPU linspace."""
    import torch

    return torch.linspace(0, 1, num_bins + 1, dtype=torch.float32)[1:-1].numpy().copy()


def quantile_edges_sorted(s, q):
    """torch.quantile(x, q) (linear interpolation) from ascending-sorted x,
    float32: rank = q*(n-1); lo = floor, hi = ceil; w = rank - lo;
    d = b - a; edge = w < 0.5 ? fma(w, d, a) : fma(w - 1, d, b) (torch's lerp
    is evaluated with fused multiply-adds); NaN anywhere -> all NaN.  The
    fused multiply-add needs C (numpy has none): see csrc/oracle.c."""
    from . import clib

    return clib.quantile_sorted(s, q)


def quantile_edges(X, num_bins: int) -> np.ndarray:
    """[F, B-1] edges of every column of X (NaN sorts last, as in torch.sort)."""
    X = np.asarray(X, dtype=F32)
    q = quantile_levels(num_bins)
    out = np.empty((X.shape[1], num_bins - 1), F32)
    for f in range(X.shape[1]):
        out[f] = quantile_edges_sorted(np.sort(X[:, f]), q)
    return out


def bin_matrix(X, edges) -> np.ndarray:
    X = np.asarray(X, dtype=F32)
    out = np.empty(X.shape, np.int8)
    for f in range(X.shape[1]):
        out[:, f] = bin_column(X[:, f], edges[f])
    return out


# --------------------------------------------------------------------------- inference
def flatten_tree(tree, max_nodes: int) -> np.ndarray:
    """Pre-order table (feature, bin, left, right, is_leaf, leaf_value),
    NaN-filled (warpgbm/core.py:1215-1252)."""
    flat = np.full((max_nodes, 6), np.nan, dtype=F32)
    counter = [0]

    def walk(node):
        i = counter[0]
        counter[0] += 1
        if "leaf_value" in node:
            flat[i, 4] = 1.0
            flat[i, 5] = node["leaf_value"]
            return
        flat[i, 0] = node["feature"]
        flat[i, 1] = node["bin"]
        flat[i, 4] = 0.0
        flat[i, 2] = counter[0]
        walk(node["left"])
        flat[i, 3] = counter[0]
        walk(node["right"])

    walk(tree)
    return flat


def predict_table(codes, table, lr, out):
    """warpgbm/cuda/predict.cu:23-44 with the trees added in tree order:
    out[i] = out[i] + float32(lr * leaf_t), t = 0..T-1.  Returns a new array.
    A walk that would leave the table -- a split feature outside [0, F), a
    child index outside [0, M), or more than M steps -- contributes NaN (the
    reference reads out of bounds there; this build's kernels define NaN)."""
    codes = np.asarray(codes)
    table = np.asarray(table, dtype=F32)
    out = np.array(out, dtype=F32, copy=True)
    lr = F32(lr)
    N = codes.shape[0]
    T, M, _ = table.shape
    for t in range(T):
        node = np.zeros(N, np.int64)
        leafv = np.full(N, np.nan, F32)
        active = np.ones(N, bool)
        for _ in range(M + 1):
            nd = table[t, node]
            is_leaf = active & (nd[:, 4] > F32(0.5))
            leafv[is_leaf] = nd[is_leaf, 5]
            active &= ~is_leaf
            if not active.any():
                break
            # rows already at a leaf (or on NaN padding) read column 0 and
            # keep their node: only the active rows' fields are cast
            nd_act = np.where(active[:, None], nd, F32(0))
            feat = nd_act[:, 0].astype(np.int64)
            sb = nd_act[:, 1].astype(np.int64)
            active &= (feat >= 0) & (feat < codes.shape[1])  # leaves the row: NaN
            c = codes[np.arange(N), np.clip(feat, 0, codes.shape[1] - 1)].astype(np.int64)
            nxt = np.where(c <= sb, nd_act[:, 2], nd_act[:, 3]).astype(np.int64)
            active &= (nxt >= 0) & (nxt < M)  # leaves the table: NaN
            node = np.where(active, nxt, node)
        out = out + lr * leafv
    return out.astype(F32)


def predict_tree_dict(codes, tree) -> np.ndarray:
    """Leaf value reached by every row (recursive dict walk, code <= bin -> left)."""
    codes = np.asarray(codes)
    N = codes.shape[0]
    out = np.empty(N, F32)

    def walk(node, idx):
        if len(idx) == 0:
            return
        if "leaf_value" in node:
            out[idx] = F32(node["leaf_value"])
            return
        go = codes[idx, int(node["feature"])].astype(np.int64) <= int(node["bin"])
        walk(node["left"], idx[go])
        walk(node["right"], idx[~go])

    walk(tree, np.arange(N))
    return out
