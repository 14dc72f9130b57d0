"""The exact arithmetic against the reference's literal float32 arithmetic.

The oracle's exact mode (the HIP library's arithmetic: quantised residuals,
exact integer histogram sums, per-node histogram shifts with one era and
per-(node, era) shifts with several, wide leaf sums) and
its literal mode (gbm.LiteralF32Grower: float32 histograms accumulated in
position order, float32 sibling subtraction as warpgbm/core.py:638-643,
float32 leaf means as core.py:599) grow forests on the same data, and
gbm.compare_growth walks them node by node.  Differences must be near-ties
judged on float64 criteria of the node's rows; on heavy-tailed targets, where
the literal float32 sums lose the small residuals next to large ones, a
difference may also be one where the exact mode's pick is the better one in
float64.  Leaf values agree within 1e-5 of the leaf's mean |residual|.

CPU only: both modes are the oracle's.
"""
import numpy as np
import pytest

from oracle import gbm, ops
from tests.conftest import c1_data

F32 = np.float32


def test_c1_literal_f32_growth_identical():
    X, y = c1_data()
    codes = ops.bin_matrix(X, ops.quantile_edges(X, 32))
    kw = dict(num_bins=32, max_depth=5, n_estimators=20, learning_rate=0.1)
    exact = gbm.Forest(**kw).fit_codes(codes, y)
    literal = gbm.Forest(**kw).fit_codes(codes, y, literal_f32=True)
    assert gbm.compare_growth(exact, literal, codes) == (20, None)


def test_des_literal_f32_growth_identical():
    rng = np.random.default_rng(2)
    N, F, E = 6000, 30, 6
    X = rng.integers(0, 5, (N, F)).astype(np.int8)
    era = np.repeat(np.arange(E), N // E)
    sign = np.where(rng.random((E, 10)) < 0.5, -1.0, 1.0)
    sign[:, :5] = 1.0
    score = ((X[:, :10] - 2) * sign[era]).sum(axis=1) + rng.standard_normal(N)
    y = (np.digitize(score, np.quantile(score, [0.2, 0.4, 0.6, 0.8])) / 4.0).astype(F32)
    kw = dict(num_bins=5, max_depth=4, n_estimators=6, learning_rate=0.5)
    exact = gbm.Forest(**kw).fit_codes(X, y, era_id=era)
    literal = gbm.Forest(**kw).fit_codes(X, y, era_id=era, literal_f32=True)
    assert gbm.compare_growth(exact, literal, X) == (6, None)


def heavy_tailed(seed, n=2000):
    """+-1e-3 targets (sign of x1) on n - 2 rows, +1e6 and -1e6 on two rows."""
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, 4)).astype(F32)
    y = np.where(X[:, 1] > 0, 1e-3, -1e-3).astype(F32)
    y[0], y[1] = 1e6, -1e6
    return X, y


def heavy_kw(depth):
    return dict(num_bins=4, max_depth=depth, n_estimators=3, learning_rate=0.1,
                min_child_weight=5)


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("depth", [2, 3, 4])
def test_heavy_tailed_exact_vs_literal(seed, depth):
    X, y = heavy_tailed(seed)
    codes = ops.bin_matrix(X, ops.quantile_edges(X, 4))
    exact = gbm.Forest(**heavy_kw(depth)).fit_codes(codes, y)
    literal = gbm.Forest(**heavy_kw(depth)).fit_codes(codes, y, literal_f32=True)
    gbm.compare_growth(exact, literal, codes, exact_may_win=True)


def test_heavy_tailed_check_catches_one_shift_per_tree(monkeypatch):
    """Planted in the oracle: one 28-bit shift per tree for histograms and
    leaf sums (no node shifts, no wide leaf sums).  Residuals of 1e-3 next to
    1e6 then quantise to 0: leaves of the small rows become 0.0 and their
    splits vanish, which the comparison must reject."""
    monkeypatch.setattr(ops, "NODE_SHIFT_STEP", 10**6)

    def leaf_one_shift(self, rows):
        q = ops.quantise(self.r, self.s)[rows]
        v = ops.leaf_value(int(q.sum()), len(rows), self.s)
        self.leaf_rows.append((rows, v))
        return {"leaf_value": float(v), "samples": int(len(rows))}

    monkeypatch.setattr(gbm.TreeGrower, "_leaf", leaf_one_shift)
    failed = 0
    for seed in (0, 2, 3):
        X, y = heavy_tailed(seed)
        codes = ops.bin_matrix(X, ops.quantile_edges(X, 4))
        exact = gbm.Forest(**heavy_kw(3)).fit_codes(codes, y)
        literal = gbm.Forest(**heavy_kw(3)).fit_codes(codes, y, literal_f32=True)
        with pytest.raises(AssertionError):
            gbm.compare_growth(exact, literal, codes, exact_may_win=True)
        failed += 1
    assert failed == 3


def test_node_shift_rule():
    """A child keeps its parent's histogram shift unless its own is at least
    NODE_SHIFT_STEP finer; the wide leaf sum recovers means far below the
    tree's histogram resolution."""
    qb = 28
    s_parent = ops.shift_from_absmax(F32(1e6), qb)
    assert ops.node_shift(F32(5e5), s_parent, qb) == s_parent          # one bit finer
    assert ops.node_shift(F32(1e6 / 200), s_parent, qb) == s_parent    # 7.6 bits finer
    assert ops.node_shift(F32(1e-3), s_parent, qb) == ops.shift_from_absmax(F32(1e-3), qb)
    s63 = ops.shift63(s_parent, qb)
    r = np.full(1000, F32(1e-3))
    assert ops.quantise(r, s_parent).sum() == 0  # below the tree's histogram step
    v = ops.leaf_value63(ops.quantise(r, s63), len(r), s63)
    assert abs(float(v) - 1e-3) <= 1e-3 * 2**-23


def heavy_tailed_eras(seed, big, n=4000, E=4):
    """Eras whose residual scales differ: +-1e-3 targets (sign of x1) plus
    1e-4 noise on E equal eras, and +big, -big on two rows of era 0."""
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, 6)).astype(F32)
    y = (np.where(X[:, 1] > 0, 1e-3, -1e-3) + 1e-4 * rng.standard_normal(n)).astype(F32)
    y[0], y[1] = big, -big
    era = np.repeat(np.arange(E), n // E)
    return X, y, era


HEAVY_ERA_KW = dict(num_bins=8, max_depth=3, n_estimators=2, learning_rate=0.1,
                    min_child_weight=5)


@pytest.mark.parametrize("big", [1e4, 1e5, 1e6])
def test_heavy_tailed_eras_exact_vs_literal(big):
    """Every (node, era) segment is quantised at its own shift, so eras 1-3
    keep their sums and their direction votes next to era 0's outliers: the
    exact mode's picks are admissible under the float64 DES rule in every
    seed (one shift per node fails 2/8 seeds at 1e4 and all at 1e6)."""
    for seed in range(8):
        X, y, era = heavy_tailed_eras(seed, big)
        codes = ops.bin_matrix(X, ops.quantile_edges(X, 8))
        exact = gbm.Forest(**HEAVY_ERA_KW).fit_codes(codes, y, era_id=era)
        literal = gbm.Forest(**HEAVY_ERA_KW).fit_codes(codes, y, era_id=era, literal_f32=True)
        gbm.compare_growth(exact, literal, codes, exact_may_win=True)


def test_heavy_tailed_eras_check_catches_one_shift_per_node(monkeypatch):
    """Planted in the oracle: every era of a node quantised at the node's
    shift (from its largest |r| over all eras).  Eras 1-3 then round to zero
    next to era 0's 1e6 outliers and vote -1 everywhere; the comparison must
    reject the resulting picks."""
    def node_wide(self, rows):
        m = np.max(np.abs(self.r[rows])) if len(rows) else F32(0)
        return np.full(self.E, ops.key_shift(m, self.qbits), np.int64)

    monkeypatch.setattr(gbm.TreeGrower, "_key_shifts", node_wide)
    failed = 0
    for seed in range(8):
        X, y, era = heavy_tailed_eras(seed, 1e6)
        codes = ops.bin_matrix(X, ops.quantile_edges(X, 8))
        exact = gbm.Forest(**HEAVY_ERA_KW).fit_codes(codes, y, era_id=era)
        literal = gbm.Forest(**HEAVY_ERA_KW).fit_codes(codes, y, era_id=era, literal_f32=True)
        try:
            gbm.compare_growth(exact, literal, codes, exact_may_win=True)
        except AssertionError:
            failed += 1
    assert failed >= 6
