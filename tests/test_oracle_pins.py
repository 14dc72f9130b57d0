"""Pins of the CPU oracle (oracle/) against things other than itself.

The reference ships no golden vectors or known-answer tests for this path
(its tests are statistical thresholds on a CUDA GPU), so each oracle function
is checked here against brute force on tiny inputs, a library routine the
reference itself calls (torch.quantile, torch.bucketize, torch.linspace),
closed forms, and invariants chosen so that a dropped term, wrong sign,
off-by-one bin or transposed index fails.

  ops.bin_column            brute-force linear scan; torch.bucketize(right=True)
  ops.quantile_edges_sorted torch.quantile (CPU) bit-exact
  ops.quantile_levels       k / B within 1 ulp; torch.linspace
  ops.quantise/dequantise   lossless for |r| >= max|r|*2^(24-qbits); error <= 2^-(s+1)
  ops.histogram_exact_q     brute-force integer dict; count invariants;
                            child + sibling == parent
  ops.histogram_exact       |G - fsum(r)| <= n 2^-(s+1) + ulp; vs f32 sequential;
                            several eras: within 1e-5 of sum|r| per bin next to
                            another era's outlier, equal to per-era calls
  ops.histogram_segments_exact  per segment equal to one-segment calls
  ops.era_absmax / key_shift  hand values, NaN / inf / empty eras
  ops.histogram_f32_seq     per-row float32 loop
  ops.split_scan            scalar float32 loop; hand KAT; gain >= 0 identity
  ops.des_select            hand-built DES cases; first-index ties
  ops.predict_table         recursive dict walk; stump closed form
  gbm.Forest / TreeGrower   planted split found; leaf = group mean; train
                            preds == predict; min_child respected
  clib.expf / softmax       numpy float64 exp within 2 ulp; rows sum to 1
  gbm.base_score            float32 nearest the exact rational mean; torch's
                            CPU float32 Y.mean() within 4 ulp
  gbm.class_prior_logits    torch CPU float32 log((y == k).float().mean()
                            + 1e-10) within 1 ulp; hand values; absent class 0
  gbm.uniform_prior_logits  torch evaluating core.py:1003-1007 literally
                            (float64 log, float32 store), bit-exact, K=2..3000
  gbm.era_ids_int32         torch .type(torch.int32) (test_api_validation.py)
  clib.quantile_edges_matrix / bin_matrix / predict_tables / split_scan_q
                            (the C loops of the full-size checks) equal to the
                            pinned numpy restatements above, bit for bit
"""
import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import clib, gbm, ops

F32 = np.float32


# --------------------------------------------------------------------------- binning
def _brute_bin(x, edges):
    out = []
    for v in x:
        b = 0
        while b < len(edges) and v >= edges[b]:
            b += 1
        out.append(b)
    return np.array(out, np.int8)


@pytest.mark.parametrize("seed", range(5))
def test_bin_column_brute_force(seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(300).astype(F32)
    x[::17] = np.nan
    e = np.sort(rng.standard_normal(rng.integers(1, 20)).astype(F32))
    e_unsorted = rng.standard_normal(9).astype(F32)
    e_nan = e.copy()
    e_nan[len(e) // 2] = np.nan
    x[5] = e[0]  # equality goes right (x >= edge)
    for edges in (e, e_unsorted, e_nan, np.full(4, np.nan, F32), np.array([1.0, 1.0, 1.0], F32)):
        assert np.array_equal(ops.bin_column(x, edges), _brute_bin(x, edges))


def test_bin_column_matches_bucketize_and_nan_rule():
    rng = np.random.default_rng(7)
    x = rng.standard_normal(10000).astype(F32)
    e = np.sort(rng.standard_normal(31).astype(F32))
    x[:31] = e  # exact hits
    ref = torch.bucketize(torch.from_numpy(x), torch.from_numpy(e), right=True).numpy()
    assert np.array_equal(ops.bin_column(x, e), ref.astype(np.int8))
    xn = np.array([np.nan], F32)
    assert ops.bin_column(xn, e)[0] == 0  # reference: NaN -> 0 (bucketize would say 31)


# --------------------------------------------------------------------------- quantile
@pytest.mark.parametrize("B", [2, 5, 10, 32, 127])
def test_quantile_edges_bit_exact_vs_torch_quantile(B):
    rng = np.random.default_rng(B)
    q = ops.quantile_levels(B)
    for n in (1, 2, 3, 7, 100, 999, 5000):
        for kind in ("normal", "ties", "tiny"):
            if kind == "normal":
                col = rng.standard_normal(n).astype(F32)
            elif kind == "ties":
                col = rng.integers(0, 4, n).astype(F32)
            else:
                col = (rng.standard_normal(n) * 1e-30).astype(F32)
            ref = torch.quantile(torch.from_numpy(col), torch.from_numpy(q)).numpy()
            got = ops.quantile_edges_sorted(np.sort(col), q)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (n, kind)


def test_quantile_edges_many_random_columns_bit_exact():
    rng = np.random.default_rng(123)
    q = ops.quantile_levels(32)
    X = (rng.standard_normal((4096, 64)) * rng.uniform(0.1, 100, 64)).astype(F32)
    ref = torch.quantile(torch.from_numpy(X), torch.from_numpy(q), dim=0).numpy().T
    got = ops.quantile_edges(X, 32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_quantile_nan_column_all_nan():
    col = np.array([0.5, np.nan, -1.0, 2.0], F32)
    q = ops.quantile_levels(4)
    ref = torch.quantile(torch.from_numpy(col), torch.from_numpy(q)).numpy()
    got = ops.quantile_edges_sorted(np.sort(col), q)
    assert np.isnan(ref).all() and np.isnan(got).all()


def test_quantile_levels():
    for B in (2, 3, 10, 32, 127):
        q = ops.quantile_levels(B)
        assert q.dtype == F32 and len(q) == B - 1
        k = np.arange(1, B, dtype=np.float64) / B
        assert np.all(np.abs(q.astype(np.float64) - k) <= np.spacing(F32(1.0)))


# --------------------------------------------------------------------------- quantisation
def test_quantise_lossless_and_bounded():
    rng = np.random.default_rng(0)
    r = (rng.standard_normal(100000) * 3).astype(F32)
    r[0] = 0.0
    r[1] = -np.max(np.abs(r)) * 1.0
    m = np.max(np.abs(r))
    for n in (10, 10**6, 2**24):
        qb = ops.qbits_for_rows(n)
        s = ops.shift_from_absmax(m, qb)
        q = ops.quantise(r, s)
        assert np.max(np.abs(q)) <= 2**qb
        back = np.ldexp(q.astype(np.float64), -s)
        assert np.all(np.abs(back - r.astype(np.float64)) <= 2.0 ** (-s - 1))
        # r * 2^s is an integer (lossless) once |r| >= max|r| * 2^(24 - qbits)
        big = np.abs(r) >= m * 2.0 ** (24 - qb)
        assert np.array_equal(back[big], r[big].astype(np.float64))
        assert n * 2**qb < 2**53
    assert ops.shift_from_absmax(0.0, 28) == 0
    assert ops.qbits_for_rows(10**6) == 28


# --------------------------------------------------------------------------- histograms
def _tiny_hist_case(seed, E=3, B=6, N=80, Fm=7):
    rng = np.random.default_rng(seed)
    codes = rng.integers(-2, B + 2, (N, Fm)).astype(np.int8)  # out-of-range both sides
    r = rng.standard_normal(N).astype(F32)
    rows = rng.choice(N, N // 2, replace=False)
    feats = rng.permutation(Fm)[:5]
    era = rng.integers(0, E, N).astype(np.int32)
    return codes, r, rows, feats, era, E, B


@pytest.mark.parametrize("seed", range(4))
def test_histogram_exact_q_brute_force(seed):
    codes, r, rows, feats, era, E, B = _tiny_hist_case(seed)
    q = ops.quantise(r, 20)
    Q, C = ops.histogram_exact_q(codes, q, rows, feats, era, E, B)
    Qb = np.zeros_like(Q)
    Cb = np.zeros_like(C)
    for s in rows:
        for fi, f in enumerate(feats):
            b = int(codes[s, f])
            if 0 <= b < B:
                Qb[era[s], fi, b] += int(q[s])
                Cb[era[s], fi, b] += 1
    assert np.array_equal(Q, Qb) and np.array_equal(C, Cb)
    # the C restatement agrees with the numpy one
    Q2, C2 = clib.hist_exact_q(codes, q, rows, feats, era, E, B)
    assert np.array_equal(Q, Q2) and np.array_equal(C, C2)


def test_histogram_invariants_and_subtraction():
    rng = np.random.default_rng(5)
    N, Fm, B, E = 2000, 9, 8, 4
    codes = rng.integers(0, B, (N, Fm)).astype(np.int8)
    r = rng.standard_normal(N).astype(F32)
    era = rng.integers(0, E, N).astype(np.int32)
    q = ops.quantise(r, 22)
    rows = np.arange(N)
    Q, C = ops.histogram_exact_q(codes, q, rows, np.arange(Fm), era, E, B)
    # every feature sees every row once: per-era totals equal across features
    for e in range(E):
        assert np.all(C[e].sum(axis=1) == np.count_nonzero(era == e))
        assert np.all(Q[e].sum(axis=1) == q[era == e].sum())
    left = rows[codes[:, 3] <= 4]
    right = rows[codes[:, 3] > 4]
    QL, CL = ops.histogram_exact_q(codes, q, left, np.arange(Fm), era, E, B)
    QR, CR = ops.histogram_exact_q(codes, q, right, np.arange(Fm), era, E, B)
    assert np.array_equal(QL + QR, Q) and np.array_equal(CL + CR, C)


def test_histogram_exact_vs_true_sum_and_f32_sequential():
    rng = np.random.default_rng(11)
    N, Fm, B = 5000, 6, 16
    codes = rng.integers(0, B, (N, Fm)).astype(np.int8)
    r = (rng.standard_normal(N) * np.exp(rng.uniform(-6, 3, N))).astype(F32)
    rows = rng.permutation(N)[:4000]
    G, H = ops.histogram_exact(codes, r, rows, np.arange(Fm), None, 1, B)
    Gs, Hs = ops.histogram_f32_seq(codes, r, rows, np.arange(Fm), np.zeros(N, np.int32), 1, B)
    assert np.array_equal(H, Hs)
    s = ops.shift_from_absmax(np.max(np.abs(r[rows])), ops.qbits_for_rows(len(rows)))
    for f in range(Fm):
        for b in range(B):
            sel = rows[codes[rows, f] == b]
            true = math.fsum(float(v) for v in r[sel])
            bound = len(sel) * 2.0 ** (-s - 1) + float(np.spacing(np.abs(G[0, f, b])))
            assert abs(float(G[0, f, b]) - true) <= bound
            # float32 sequential accumulation error bound ~ n * eps * sum|r|
            absum = math.fsum(abs(float(v)) for v in r[sel])
            assert abs(float(Gs[0, f, b]) - true) <= len(sel) * 2**-24 * absum + 1e-30


def _bin_true_sums(codes, r, rows, era, E, B, f):
    """float64 (fsum) sum and sum of |r| of every (era, bin) of feature f."""
    true = np.zeros((E, B))
    absum = np.zeros((E, B))
    for e in range(E):
        for b in range(B):
            sel = rows[(codes[rows, f] == b) & (era[rows] == e)]
            true[e, b] = math.fsum(float(v) for v in r[sel])
            absum[e, b] = math.fsum(abs(float(v)) for v in r[sel])
    return true, absum


def test_histogram_exact_eras_keep_their_own_scale():
    """Several eras: each era's sums are quantised at the shift of its own
    largest |r|, so an era of 1e-3 residuals next to an era holding a 1e6
    outlier is summed to within 1e-5 of its bins' sum of |r| (a single shift
    for the call would round every 1e-3 residual to 0: planted below)."""
    rng = np.random.default_rng(21)
    N, Fm, B, E = 4000, 3, 8, 4
    codes = rng.integers(0, B, (N, Fm)).astype(np.int8)
    era = np.repeat(np.arange(E), N // E).astype(np.int32)
    r = (1e-3 * rng.standard_normal(N)).astype(F32)
    r[5] = F32(1e6)  # era 0
    rows = np.arange(N)
    G, H = ops.histogram_exact(codes, r, rows, np.arange(Fm), era, E, B)
    for f in range(Fm):
        true, absum = _bin_true_sums(codes, r, rows, era, E, B, f)
        err = np.abs(G[1:, f, :].astype(np.float64) - true[1:])
        assert np.all(err <= 1e-5 * absum[1:])
    # the same eras through the one-era path, era by era, at the call's qbits
    qb = ops.qbits_for_rows(N)
    for e in range(E):
        Ge, He = ops.histogram_exact(codes, r, rows[era == e], np.arange(Fm), None, 1, B, qbits=qb)
        assert np.array_equal(Ge[0], G[e]) and np.array_equal(He[0], H[e])
    # planted: one shift for the whole call (step 2^-8 next to the outlier)
    # rounds the 1e-3 residuals of eras 1..3 away and fails the same bound
    s = ops.shift_from_absmax(np.max(np.abs(r)), qb)
    Q1, _ = ops.histogram_exact_q(codes, ops.quantise(r, s), rows, np.arange(Fm), era, E, B)
    G1 = ops.dequantise(Q1, s)
    true, absum = _bin_true_sums(codes, r, rows, era, E, B, 0)
    assert np.any(np.abs(G1[1:, 0, :].astype(np.float64) - true[1:]) > 1e-5 * absum[1:])


def test_histogram_segments_exact_per_segment_shift():
    """Several segments: each at the shift of its own largest |r|, equal to
    the one-segment histogram of its rows at the call's qbits; one segment:
    the shift of the call's positions."""
    rng = np.random.default_rng(22)
    N, Fm, B, S = 3000, 4, 6, 5
    codes = rng.integers(-1, B + 1, (N, Fm)).astype(np.int8)
    r = (rng.standard_normal(N) * 10.0 ** rng.integers(-4, 3, N)).astype(F32)
    order = rng.permutation(N).astype(np.int32)
    seg = np.array([0, 700, 700, 1500, 2900, 3000], np.int64)  # one empty segment
    G, H = ops.histogram_segments_exact(codes, r, order, seg, np.arange(Fm), B)
    qb = ops.qbits_for_rows(N)
    for k in range(S):
        rows = order[seg[k]:seg[k + 1]]
        Gk, Hk = ops.histogram_exact(codes, r, rows, np.arange(Fm), None, 1, B, qbits=qb)
        assert np.array_equal(G[k], Gk[0]) and np.array_equal(H[k], Hk[0])
    G1, H1 = ops.histogram_segments_exact(codes, r, order, np.array([0, 2000]), np.arange(Fm), B,
                                          n_pos=N)
    s = ops.shift_from_absmax(np.max(np.abs(r)), qb)  # over all N positions
    Q, C = ops.histogram_exact_q(codes, ops.quantise(r, s), order[:2000], np.arange(Fm), None, 1, B)
    assert np.array_equal(G1[0], ops.dequantise(Q[0], s)) and np.array_equal(H1[0], C[0])


def test_era_absmax_and_key_shift():
    r = np.array([1.0, -3.0, 2.0, np.nan, 5.0, -0.0], F32)
    era = np.array([0, 0, 1, 2, 1, 3])
    m = ops.era_absmax(r, np.arange(6), era, 5)
    assert m[0] == 3 and m[1] == 5 and np.isnan(m[2]) and m[3] == 0 and m[4] == 0
    assert np.array_equal(np.nan_to_num(clib.era_absmax(r, np.arange(6), era, 5), nan=-1),
                          np.nan_to_num(m, nan=-1))
    assert ops.key_shift(F32(0), 28) == 0 and ops.key_shift(F32(np.inf), 28) == 0
    assert ops.key_shift(F32(np.nan), 28) == 0
    assert ops.key_shift(F32(3.0), 28) == 26  # 3 = 0.75 * 2^2: 3 * 2^26 < 2^28


def test_histogram_f32_seq_matches_row_loop():
    codes, r, rows, feats, era, E, B = _tiny_hist_case(9)
    G, H = ops.histogram_f32_seq(codes, r, rows, feats, era, E, B)
    Gb = np.zeros_like(G)
    Hb = np.zeros_like(H)
    for fi, f in enumerate(feats):
        for s in rows:  # ascending position order
            b = int(codes[s, f])
            if 0 <= b < B:
                Gb[era[s], fi, b] = F32(Gb[era[s], fi, b] + r[s])
                Hb[era[s], fi, b] = F32(Hb[era[s], fi, b] + F32(1))
    assert np.array_equal(G, Gb) and np.array_equal(H, Hb)


# --------------------------------------------------------------------------- split
def _scalar_split(G, H, mcw, eps):
    E, F, B = G.shape
    gain = np.zeros((E, F, B - 1), F32)
    dirn = np.zeros((E, F, B - 1), F32)
    mcw, eps = F32(mcw), F32(eps)
    for e in range(E):
        for f in range(F):
            gt = F32(0)
            ht = F32(0)
            for b in range(B):
                gt = F32(gt + G[e, f, b])
                ht = F32(ht + H[e, f, b])
            gl = F32(0)
            hl = F32(0)
            for b in range(B - 1):
                gl = F32(gl + G[e, f, b])
                hl = F32(hl + H[e, f, b])
                gr = F32(gt - gl)
                hr = F32(ht - hl)
                if hl >= mcw and hr >= mcw:
                    a1 = F32(F32(gl * gl) / F32(hl + eps))
                    a2 = F32(F32(gr * gr) / F32(hr + eps))
                    a3 = F32(F32(gt * gt) / F32(ht + eps))
                    gain[e, f, b] = F32(F32(a1 + a2) - a3)
                    lv = F32(gl / F32(hl + eps))
                    rv = F32(gr / F32(hr + eps))
                    dirn[e, f, b] = 1.0 if lv > rv else -1.0
    return gain, dirn


@pytest.mark.parametrize("seed", range(3))
def test_split_scan_vs_scalar_loop(seed):
    rng = np.random.default_rng(seed)
    E, F, B = 3, 7, 9
    H = rng.integers(0, 30, (E, F, B)).astype(F32)
    G = (rng.standard_normal((E, F, B)) * H).astype(F32)
    gain, dirn = ops.split_scan(G, H, 20, 1e-6)
    g2, d2 = _scalar_split(G, H, 20, 1e-6)
    assert np.array_equal(gain.view(np.uint32), g2.view(np.uint32))
    assert np.array_equal(dirn, d2)


def test_split_scan_hand_kat():
    # one era, one feature, 3 bins: G = [3, -1, 4], H = [2, 1, 5], eps = 0, mcw = 1
    G = np.array([[[3.0, -1.0, 4.0]]], F32)
    H = np.array([[[2.0, 1.0, 5.0]]], F32)
    gain, dirn = ops.split_scan(G, H, 1, 0.0)
    # b=0: L=(3,2) R=(3,6): 9/2 + 9/6 - 36/8 = 1.5 ; left mean 1.5 > right 0.5 -> +1
    # b=1: L=(2,3) R=(4,5): 4/3 + 16/5 - 36/8 = 1/30 ; 0.667 < 0.8 -> -1
    exact = [Fraction(9, 2) + Fraction(9, 6) - Fraction(36, 8),
             Fraction(4, 3) + Fraction(16, 5) - Fraction(36, 8)]
    for b in range(2):
        assert abs(float(gain[0, 0, b]) - float(exact[b])) <= 4 * np.spacing(F32(4.5))
    assert dirn[0, 0].tolist() == [1.0, -1.0]
    # min_child masking: with mcw = 3 the first threshold (HL = 2) is masked
    gain, dirn = ops.split_scan(G, H, 3, 0.0)
    assert gain[0, 0, 0] == 0 and dirn[0, 0, 0] == 0 and gain[0, 0, 1] != 0


def test_split_gain_nonnegative_identity():
    # with eps = 0 the split gain GL^2/HL + GR^2/HR - G^2/H >= 0 (Cauchy-Schwarz)
    rng = np.random.default_rng(3)
    H = rng.integers(1, 50, (2, 40, 12)).astype(F32)
    G = (rng.standard_normal((2, 40, 12)) * 10).astype(F32)
    gain, _ = ops.split_scan(G, H, 1, 0.0)
    tot = np.abs(G.sum(axis=2)) ** 2 / H.sum(axis=2)
    assert np.all(gain >= -1e-4 * (1 + tot[:, :, None]))


# --------------------------------------------------------------------------- DES selection
def test_des_select_e1_argmax_first_index():
    gain = np.array([[[0.5, 2.0, 2.0], [2.0, 1.0, 0.0]]], F32)
    dirn = np.sign(gain)
    assert ops.des_select(gain, dirn, 0.0) == (0, 1)  # first of the three 2.0s
    assert ops.des_select(gain, dirn, 5.0) == (-1, -1)
    assert ops.des_select(np.zeros((1, 2, 3), F32), np.zeros((1, 2, 3), F32), 0.0) == (-1, -1)


def test_des_select_prefers_consistent_direction():
    # feature 0: large gains but directions disagree across eras;
    # feature 1: smaller gains, same direction in all eras -> feature 1 wins
    gain = np.array([[[9.0], [1.0]], [[9.0], [1.0]], [[9.0], [1.0]]], F32)
    dirn = np.array([[[1.0], [1.0]], [[-1.0], [1.0]], [[1.0], [1.0]]], F32)
    assert ops.des_select(gain, dirn, 0.0) == (1, 0)
    # the max-agreement candidates all fail min_split_gain -> leaf, even
    # though feature 0 passes it
    assert ops.des_select(gain, dirn, 2.0) == (-1, -1)
    # a masked era (dir 0, gain 0) dilutes both means equally
    dirn2 = dirn.copy()
    dirn2[0, 1, 0] = 0.0
    gain2 = gain.copy()
    gain2[0, 1, 0] = 0.0
    # agree: f0 |1-1+1| = 1, f1 |0+1+1| = 2 -> f1 still
    assert ops.des_select(gain2, dirn2, 0.0) == (1, 0)


def test_des_criterion_era_sum_order():
    """E <= 32: the plain sequential float64 sum.  E > 32: 32-era blocks, each
    summed in era order, then the block sums in order -- on values where the
    two orders round differently (sequentially every 2^-53 is lost against
    1.0; inside the second block they first add up exactly)."""
    gain = np.zeros((40, 1, 1), F32)
    gain[0] = 1.0
    gain[1:32] = F32(2.0**-53)
    gain[32] = F32(2.0**-50)
    gain[33:40] = F32(2.0**-53)
    seq = 0.0
    for e in range(40):
        seq = seq + float(gain[e, 0, 0])
    assert seq == 1.0 + 2.0**-50
    got = ops.era_sum_f64(gain)[0, 0]
    assert got == 1.0 + 2.0**-49  # (1.0) + (2^-50 + 7 * 2^-53) = 1 + 15 * 2^-53, rounded
    small = gain[:20]
    s20 = 0.0
    for e in range(20):
        s20 = s20 + float(small[e, 0, 0])
    assert ops.era_sum_f64(small)[0, 0] == s20
    crit, _ = ops.des_criterion(gain, np.zeros_like(gain))
    assert crit[0, 0] == np.float32(got / 40)


def test_des_criterion_mean_is_float64_sequential():
    rng = np.random.default_rng(1)
    gain = rng.standard_normal((500, 3, 4)).astype(F32)
    crit, agree = ops.des_criterion(gain, np.sign(gain))
    exact = np.array([[math.fsum(gain[:, f, b].astype(float)) / 500 for b in range(4)]
                      for f in range(3)])
    assert np.all(np.abs(crit - exact) <= 2 * np.spacing(np.abs(crit).astype(F32)) + 1e-12)
    assert agree.dtype == np.int64


# --------------------------------------------------------------------------- predict
def _random_tree(rng, depth, max_depth, F, B):
    if depth == max_depth or rng.random() < 0.25:
        return {"leaf_value": float(F32(rng.standard_normal())), "samples": 1}
    return {"feature": int(rng.integers(F)), "bin": int(rng.integers(-1, B)),
            "left": _random_tree(rng, depth + 1, max_depth, F, B),
            "right": _random_tree(rng, depth + 1, max_depth, F, B)}


def test_predict_table_vs_dict_walk():
    rng = np.random.default_rng(2)
    F, B, D = 6, 8, 4
    codes = rng.integers(-1, B, (500, F)).astype(np.int8)
    trees = [_random_tree(rng, 0, D, F, B) for _ in range(7)]
    table = np.stack([ops.flatten_tree(t, 2 ** (D + 1)) for t in trees])
    lr = 0.3
    base = np.full(500, F32(0.25), F32)
    got = ops.predict_table(codes, table, lr, base)
    exp = base.copy()
    for t in trees:
        exp = exp + F32(lr) * ops.predict_tree_dict(codes, t)
    assert np.array_equal(got, exp)


def test_predict_stump_closed_form():
    codes = np.array([[0], [3], [4], [9]], np.int8)
    stump = {"feature": 0, "bin": 3, "left": {"leaf_value": -2.0, "samples": 2},
             "right": {"leaf_value": 5.0, "samples": 2}}
    table = ops.flatten_tree(stump, 4)[None]
    assert table[0, 0, 2] == 1 and table[0, 0, 3] == 2  # pre-order ids
    got = ops.predict_table(codes, table, 0.5, np.zeros(4, F32))
    assert got.tolist() == [-1.0, -1.0, 2.5, 2.5]


def test_predict_table_malformed_walks_are_nan():
    """Known answers of the NaN rule: a split on a feature outside [0, F), an
    edge to a child outside [0, M), and a cycle (more than M steps) give NaN
    for the rows that take them and leave the other rows' values alone."""
    codes = np.array([[0, 0], [5, 0], [5, 9], [0, 9]], np.int8)
    nan = np.nan
    #        feature bin left right leaf value
    table = np.array([[[0, 3, 1, 2, 0, nan],      # node 0: code0 <= 3 -> 1 else 2
                       [7, 0, 3, 3, 0, nan],      # node 1: feature 7 >= F=2 -> NaN
                       [1, 4, 3, 9, 0, nan],      # node 2: code1 <= 4 -> 3 else child 9 >= M
                       [0, 0, 0, 0, 1, 1.5]],     # node 3: leaf 1.5
                      [[1, 4, 1, 2, 0, nan],      # tree 2, node 0: code1 <= 4 -> 1 else 2
                       [0, 9, 0, 0, 0, nan],      # node 1: back to 0 forever (cycle)
                       [0, 0, 0, 0, 1, -2.0],     # node 2: leaf -2
                       [0, 0, 0, 0, 1, 0.0]]], F32)
    got = ops.predict_table(codes, table, 1.0, np.zeros(4, F32))
    # row 0: tree 1 -> node 1 (NaN); row 1: node 2 -> node 3: 1.5, tree 2 cycle: NaN
    # row 2: node 2 -> child 9: NaN; row 3: tree 1 NaN (node 1), tree 2 -> leaf -2
    assert np.isnan(got).tolist() == [True, True, True, True]
    one = ops.predict_table(codes, table[:1], 1.0, np.zeros(4, F32))
    assert np.isnan(one).tolist() == [True, False, True, True] and one[1] == F32(1.5)
    two = ops.predict_table(codes, table[1:], 1.0, np.zeros(4, F32))
    assert np.isnan(two).tolist() == [True, True, False, False] and two[2] == F32(-2.0)


# --------------------------------------------------------------------------- tree growth
def test_gbm_finds_planted_split_and_group_means():
    rng = np.random.default_rng(4)
    N, F, B = 3000, 5, 16
    codes = rng.integers(0, B, (N, F)).astype(np.int8)
    y = np.where(codes[:, 2] <= 6, -3.0, 4.0).astype(F32) + F32(0.01) * rng.standard_normal(N).astype(F32)
    f = gbm.Forest(num_bins=B, max_depth=1, n_estimators=1, learning_rate=1.0,
                   min_child_weight=20).fit_codes(codes, y)
    t = f.forest[0]
    assert (t["feature"], t["bin"]) == (2, 6)
    r = y - f.base
    for side, sel in (("left", codes[:, 2] <= 6), ("right", codes[:, 2] > 6)):
        assert abs(t[side]["leaf_value"] - float(np.mean(r[sel], dtype=np.float64))) < 1e-5
        assert t[side]["samples"] == int(sel.sum())


def test_gbm_invariants_regression():
    rng = np.random.default_rng(8)
    N, F, B = 4000, 8, 12
    codes = rng.integers(0, B, (N, F)).astype(np.int8)
    y = (codes[:, 0] * 0.3 - codes[:, 5] * 0.2 + rng.standard_normal(N)).astype(F32)
    era = rng.integers(0, 3, N)
    f = gbm.Forest(num_bins=B, max_depth=4, n_estimators=5, learning_rate=0.2,
                   min_child_weight=30).fit_codes(codes, y, era_id=era)
    assert np.array_equal(f.predict_codes(codes), f.train_preds)

    def check(node, rows):
        if "leaf_value" in node:
            assert node["samples"] == len(rows)
            return 1
        go = codes[rows, node["feature"]] <= node["bin"]
        # every era with rows on both sides satisfies min_child (count >= 30)
        # for at least one era (the split had positive gain somewhere)
        okl = [np.count_nonzero(era[rows[go]] == e) >= 30 for e in range(3)]
        okr = [np.count_nonzero(era[rows[~go]] == e) >= 30 for e in range(3)]
        assert any(a and b for a, b in zip(okl, okr))
        return check(node["left"], rows[go]) + check(node["right"], rows[~go])

    for t in f.forest:
        assert check(t, np.arange(N)) <= 2 ** 4
    assert f.feature_importance[0] > 0 and f.feature_importance[5] > 0


def test_gbm_multiclass_invariants():
    rng = np.random.default_rng(6)
    N, F, B, K = 1500, 6, 10, 3
    codes = rng.integers(0, B, (N, F)).astype(np.int8)
    labels = (codes[:, 1] * K // B).astype(np.int32)
    f = gbm.Forest(objective="multiclass", num_bins=B, max_depth=3, n_estimators=4,
                   learning_rate=0.5, min_child_weight=10).fit_codes(codes, labels)
    p = f.predict_codes(codes)
    assert np.allclose(p.sum(axis=1), 1.0, atol=1e-6)
    assert (np.argmax(p, axis=1) == labels).mean() > 0.9
    res = clib.softmax_residual(f.train_scores, labels)
    assert np.allclose(res.sum(axis=0), 0.0, atol=1e-6)


# --------------------------------------------------------------------------- exp / softmax
def test_expf_accuracy():
    x = np.concatenate([np.linspace(-103, 88, 200001, dtype=F32),
                        np.array([0.0, -0.0, -1e-30, 1e-30, -87.3, -88.0, -100.0], F32)])
    got = clib.expf(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(F32)).astype(np.float64)
    norm = ref >= np.finfo(F32).tiny
    assert np.all(np.abs(got - ref)[norm] <= 2 * ulp[norm])
    assert np.all(np.abs(got - ref)[~norm] <= 2 * 2.0 ** -149)
    assert clib.expf(np.array([-200.0], F32))[0] == 0.0


def test_softmax_rows_sum_to_one():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((1000, 7)) * 20).astype(F32)
    p = clib.softmax_rows(x)
    ref = np.exp(x - x.max(axis=1, keepdims=True))
    ref /= ref.sum(axis=1, keepdims=True)
    assert np.allclose(p.sum(axis=1), 1.0, atol=1e-6)
    assert np.allclose(p, ref, rtol=1e-5, atol=1e-7)


# --------------------------------------------------------------------------- start values
def _f32_nearest(fr):
    """The float32 nearest the rational fr (ties to even), by exact comparison
    of the neighbours of a first guess."""
    x = F32(float(fr))
    cands = [np.nextafter(x, F32(-np.inf)), x, np.nextafter(x, F32(np.inf))]
    best = min(cands, key=lambda c: (abs(Fraction(float(c)) - fr),
                                     int(np.asarray(c, F32).view(np.uint32)) & 1))
    return F32(best)


def _ulps(a, b):
    ia = np.asarray(a, F32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, F32).view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


@pytest.mark.parametrize("n,loc,seed", [(1, 0.0, 0), (7, 3.0, 1), (1000, 1000.0, 2),
                                        (200_000, 0.0, 3), (200_000, 1000.0, 4)])
def test_base_score_is_nearest_float_to_exact_mean(n, loc, seed):
    """Y.mean() (core.py:387): the float32 nearest the exact mean.  A float32
    running sum -- a plausible slip -- is off by many ulps on the offset
    targets (loc = 1000), and a dropped row changes the mean."""
    rng = np.random.default_rng(seed)
    y = (loc + rng.standard_normal(n)).astype(F32)
    exact = sum((Fraction(float(v)) for v in y), Fraction(0)) / n
    want = _f32_nearest(exact)
    assert gbm.base_score(y) == want
    if n >= 1000 and loc != 0.0:
        run = F32(0)
        for v in y[:20000]:
            run = F32(run + v)
        sub_exact = _f32_nearest(sum((Fraction(float(v)) for v in y[:20000]), Fraction(0)) / 20000)
        assert run / F32(20000) != sub_exact  # the slip is caught by this check


def test_base_score_vs_torch_float32_mean():
    """torch's own float32 mean (the reference's call, on the CPU here) agrees
    within 4 ulp up to 2M rows; it reduces in float32 in its own order, so
    equality is not expected."""
    rng = np.random.default_rng(5)
    for n in (10, 1000, 123_457, 2_000_000):
        y = (rng.standard_normal(n) * 7.0 + 3.0).astype(F32)
        t = F32(torch.from_numpy(y).mean().item())
        assert _ulps(gbm.base_score(y), t) <= 4, n


def test_class_prior_logits_vs_torch():
    """log((y == k).float().mean() + 1e-10) per present class (core.py:450-456)
    against torch's CPU float32 evaluation: within 1 ulp everywhere (torch's
    float32 log is not correctly rounded) and identical almost everywhere.
    A uniform prior, a log10, or a log of an absent class (-23.03 instead of
    the 0 the reference leaves) would fail."""
    rng = np.random.default_rng(6)
    diff = total = 0
    for _ in range(300):
        n = int(rng.integers(2, 50_000))
        K = int(rng.integers(2, 12))
        p = rng.dirichlet(np.ones(K))
        lab = rng.choice(K, size=n, p=p).astype(np.int32)
        lab[lab == K - 1] = 0  # class K-1 absent
        got = gbm.class_prior_logits(lab, K)
        t = torch.from_numpy(lab)
        want = np.zeros(K, F32)
        for k in range(K):
            pk = (t == k).float().mean()
            if pk > 0:
                want[k] = F32(torch.log(pk + 1e-10).item())
        assert got[K - 1] == 0.0
        u = _ulps(got, want)
        assert u.max() <= 1
        diff += int(np.count_nonzero(u))
        total += K
    assert diff <= total // 500
    # hand values: a 3:1 split
    v = gbm.class_prior_logits(np.array([0, 0, 0, 1], np.int32), 2)
    assert v[0] == F32(math.log(0.75)) and v[1] == F32(math.log(0.25))


def test_uniform_prior_logits_vs_reference_expression():
    """predict_proba's start logits, evaluated as core.py:1003-1007 writes
    them (numpy 1/K, + 1e-10, torch.tensor -> float64 log, stored into a
    float32 tensor), bit-exact for K = 2..3000.  Rounding 1/K + 1e-10 to
    float32 before the log (a plausible slip) differs at K = 47."""
    for K in range(2, 3001):
        classes = np.arange(K)
        F = torch.zeros((1, K), dtype=torch.float32)
        for k in (0, K - 1):
            prior_k = (classes == classes[k]).sum() / len(classes)
            F[:, k] = torch.log(torch.tensor(prior_k + 1e-10))
        got = gbm.uniform_prior_logits(K)
        assert got[0] == F[0, 0].item() and got[-1] == F[0, K - 1].item(), K
    slip = F32(np.log(np.float64(F32(1.0 / 47 + 1e-10))))
    assert slip != gbm.uniform_prior_logits(47)[0]


# --------------------------------------------------------------------------- full-size C loops
def test_clib_edges_and_codes_equal_numpy_restatement():
    rng = np.random.default_rng(11)
    X = rng.standard_normal((3001, 23)).astype(F32)
    X[:, 2] = np.round(X[:, 2])            # heavy ties
    X[::50, 4] = np.nan                    # a NaN column: all edges NaN
    X[:, 5] = 7.0                          # constant column
    X[:, 6] = np.abs(X[:, 6]) + 1.0        # positive only
    for B in (2, 5, 32, 127):
        e_np = ops.quantile_edges(X, B)
        e_c = clib.quantile_edges_matrix(X, B)
        # bit-exact, except that an edge on a zero may carry either sign: a
        # comparison sort leaves -0.0 and +0.0 in input order, the radix key
        # (the GPU's) puts -0.0 first; the codes cannot differ
        same = (e_np.view(np.uint32) == e_c.view(np.uint32)) | ((e_np == 0) & (e_c == 0))
        assert same.all(), B
        assert np.array_equal(ops.bin_matrix(X, e_np), clib.bin_matrix(X, e_np)), B


def test_clib_split_scan_q_equals_numpy():
    rng = np.random.default_rng(12)
    for _ in range(25):
        E, F, B = int(rng.integers(1, 5)), int(rng.integers(1, 30)), int(rng.integers(2, 40))
        C = rng.integers(0, 60, (E, F, B))
        Q = rng.integers(-2**27, 2**27, (E, F, B)) * C
        s = int(rng.integers(8, 30))
        mcw = float(rng.integers(1, 40))
        g1, d1 = ops.split_scan(ops.dequantise(Q, s), C.astype(F32), mcw, 1e-6)
        g2, d2 = clib.split_scan_q(Q, C, s, mcw, 1e-6)
        assert np.array_equal(g1.view(np.uint32), g2.view(np.uint32))
        assert np.array_equal(d1, d2)


def test_clib_predict_tables_equals_numpy_and_dict_walk():
    rng = np.random.default_rng(13)
    N, F, B, K = 700, 9, 8, 3
    X = rng.standard_normal((N, F)).astype(F32)
    codes = ops.bin_matrix(X, ops.quantile_edges(X, B))
    y = rng.integers(0, K, N)
    f = gbm.Forest(objective="multiclass", num_bins=B, max_depth=3, n_estimators=3,
                   learning_rate=0.3, min_child_weight=5).fit_codes(codes, y)
    trees = [t for rnd in f.forest for t in rnd]
    tabs = np.stack([ops.flatten_tree(t, 16) for t in trees])
    cls = np.tile(np.arange(K, dtype=np.int32), 3)
    start = np.tile(gbm.uniform_prior_logits(K), (N, 1))
    got = clib.predict_tables(codes, tabs, 0.3, start, cls)
    want = start.copy()
    for t, k in zip(range(len(trees)), cls):
        want[:, k] = ops.predict_table(codes, tabs[t:t + 1], 0.3, want[:, k])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(clib.softmax_rows(got), f.predict_codes(codes))
    one = clib.predict_tables(codes, tabs[:1], 0.3, np.zeros(N, F32))
    assert np.array_equal(one, F32(0.3) * ops.predict_tree_dict(codes, trees[0]))
