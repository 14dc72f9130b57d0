"""End-to-end parity of the estimator (level-wise native engine on the GPU)
with the oracle's restatement of the reference's recursive tree growth.

Bar: identical tree dicts (features, bins, leaf values as floats, sample
counts), identical predictions and importances (bit-exact), for regression
(config C1: 10k x 50, 32 bins, depth 5, 20 trees), softmax multiclass, era-aware DES, colsample subsets,
warm start and save/load."""
import numpy as np
import pytest
import torch

from oracle import gbm, ops
from tests.conftest import c1_data, print_case
from warpgbm_amd import WarpGBM

pytestmark = pytest.mark.gpu
F32 = np.float32


def bits(a):
    return np.asarray(a, dtype=F32).view(np.uint32)


def oracle_codes(model, X):
    """Codes the oracle bins X to, with edges the oracle computes itself."""
    edges = ops.quantile_edges(X, model.num_bins)
    got = torch.as_tensor(model.bin_edges).cpu().numpy()
    assert np.array_equal(bits(got), bits(edges)), "bin edges differ"
    return ops.bin_matrix(X, edges)


def test_c1_regression_bit_exact(gpu):
    print_case("estimator", "C1 regression")
    X, y = c1_data()
    m = WarpGBM(num_bins=32, max_depth=5, n_estimators=20, learning_rate=0.1)
    m.fit(X, y)
    codes = oracle_codes(m, X)
    ref = gbm.Forest(num_bins=32, max_depth=5, n_estimators=20, learning_rate=0.1,
                     min_child_weight=20, min_split_gain=0.0, L2_reg=1e-6).fit_codes(codes, y)
    assert m.base_prediction == float(ref.base)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
    p = m.predict(X)
    assert np.array_equal(bits(p), bits(ref.predict_codes(codes)))
    assert np.array_equal(bits(p), bits(ref.train_preds))
    # tables rebuilt from the tree dicts (what a loaded or edited forest uses)
    # predict exactly as the ones taken from the engine's records at fit
    m._heap = None
    assert np.array_equal(bits(m.predict(X)), bits(p))
    assert np.array_equal(bits(m.per_era_feature_importance_), bits(ref.imp))
    assert np.corrcoef(p, y)[0, 1] > 0.9


@pytest.mark.parametrize("B", [5, 8, 10, 16, 64])
def test_one_era_bin_counts_bit_exact(gpu, B):
    """The one-era split step's compile-time bin counts (10 is the
    estimator's default) grow the oracle's trees: regression on 6000 rows
    and a 3-class softmax, depth 4."""
    print_case("estimator", "one-era bin count", B)
    rng = np.random.default_rng(40 + B)
    N, F = 6000, 12
    X = rng.standard_normal((N, F)).astype(F32)
    y = (X[:, 0] - 0.5 * X[:, 3] ** 2 + 0.1 * rng.standard_normal(N)).astype(F32)
    kw = dict(num_bins=B, max_depth=4, n_estimators=3, learning_rate=0.3, min_child_weight=5)
    m = WarpGBM(**kw).fit(X, y)
    codes = oracle_codes(m, X)
    ref = gbm.Forest(**kw).fit_codes(codes, y)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
    assert np.array_equal(bits(m.predict(X)), bits(ref.predict_codes(codes)))
    labels = (X[:, 1] > 0).astype(np.int64) + (X[:, 2] > 0.5)
    kw = dict(objective="multiclass", num_bins=B, max_depth=4, n_estimators=2,
              learning_rate=0.3, min_child_weight=5)
    m = WarpGBM(**kw).fit(X, labels)
    codes = oracle_codes(m, X)
    ref = gbm.Forest(**kw).fit_codes(codes, labels)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"round {i} differs"


def test_multiclass_bit_exact(gpu):
    print_case("estimator", "multiclass K=4")
    rng = np.random.default_rng(1)
    N, F, K = 6000, 12, 4
    means = rng.standard_normal((K, F)) * 1.5
    labels = rng.integers(0, K, N)
    X = (means[labels] + rng.standard_normal((N, F))).astype(F32)
    y = np.array(["a", "b", "c", "d"])[labels]
    m = WarpGBM(objective="multiclass", num_bins=16, max_depth=4, n_estimators=8,
                learning_rate=0.3, min_child_weight=10)
    m.fit(X, y)
    codes = oracle_codes(m, X)
    ref = gbm.Forest(objective="multiclass", num_bins=16, max_depth=4, n_estimators=8,
                     learning_rate=0.3, min_child_weight=10).fit_codes(codes, labels)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"round {i} differs"
    proba = m.predict_proba(X)
    assert np.array_equal(bits(proba), bits(ref.predict_codes(codes)))
    m._heap = None
    assert np.array_equal(bits(m.predict_proba(X)), bits(proba))
    assert np.allclose(proba.sum(axis=1), 1.0, atol=1e-5)
    assert (m.predict(X) == y).mean() > 0.8


def test_multiclass_many_features_bit_exact(gpu):
    """Many features and K trees per round: the level histograms of the deeper
    levels have enough (tree, node) segments x feature planes for the plane
    finalize (exact int64 level sums, sibling = parent - child)."""
    print_case("estimator", "multiclass K=5, F=300")
    rng = np.random.default_rng(11)
    N, F, K = 8000, 300, 5
    means = rng.standard_normal((K, F)) * 0.4
    labels = rng.integers(0, K, N)
    X = (means[labels] + rng.standard_normal((N, F))).astype(F32)
    kw = dict(objective="multiclass", num_bins=32, max_depth=4, n_estimators=4,
              learning_rate=0.3, min_child_weight=10)
    m = WarpGBM(**kw).fit(X, labels)
    codes = oracle_codes(m, X)
    ref = gbm.Forest(**kw).fit_codes(codes, labels)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"round {i} differs"
    assert np.array_equal(bits(m.predict_proba(X)), bits(ref.predict_codes(codes)))


# era code layouts (engine tuning key 2): the int8 codes, or the pair-code
# copy (num_bins <= 7; the int8 codes above that)
LAYOUTS = [0, 1]


@pytest.mark.parametrize("layout", LAYOUTS)
def test_era_des_prebinned_bit_exact(gpu, layout):
    print_case("estimator", "DES E=6 prebinned layout", layout)
    rng = np.random.default_rng(2)
    N, F, E = 6000, 30, 6
    X = rng.integers(0, 5, (N, F)).astype(np.int8)
    era = np.repeat(np.arange(E), N // E)
    sign = np.where(rng.random((E, 10)) < 0.5, -1.0, 1.0)
    sign[:, :5] = 1.0  # features 0-4 consistent across eras, 5-9 flip
    score = ((X[:, :10] - 2) * sign[era]).sum(axis=1) + rng.standard_normal(N)
    y = np.digitize(score, np.quantile(score, [0.2, 0.4, 0.6, 0.8])) / 4.0
    m = WarpGBM(num_bins=5, max_depth=4, n_estimators=6, learning_rate=0.5)
    m._engine_tuning = {2: layout}
    m.fit(X, y.astype(F32), era_id=era)
    ref = gbm.Forest(num_bins=5, max_depth=4, n_estimators=6, learning_rate=0.5).fit_codes(
        X, y.astype(F32), era_id=era)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
    assert np.array_equal(bits(m.per_era_feature_importance_), bits(ref.imp))
    assert m.per_era_feature_importance_.shape == (E, F)
    assert np.array_equal(bits(m.predict(X)), bits(ref.predict_codes(X)))


@pytest.mark.parametrize("E,B", [(1, 10), (3, 10), (3, 5)])
def test_prebinned_negative_and_wrapped_codes_bit_exact(gpu, E, B):
    """Pre-binned integer input with negative values: every column max is
    < num_bins, so it is used as codes (warpgbm/core.py:499-505), cast to
    int8 (values below -128 wrap, e.g. -200 -> 56 >= num_bins).  Codes outside
    [0, num_bins) are skipped by the histograms (histogram_kernel.cu:41) and
    compared as signed int8 by the partition and predict (core.py:629,
    predict.cu:43): negative codes go left, wrapped ones >= num_bins right."""
    print_case("estimator", "pre-binned negative codes E B", E, B)
    rng = np.random.default_rng(8)
    N, F = 5000, 14
    X = rng.integers(-2, B, (N, F)).astype(np.int64)
    X[rng.random((N, F)) < 0.05] = -200           # wraps to int8 56
    era = np.repeat(np.arange(E), N // E + 1)[:N]
    score = np.clip(X[:, :4], -1, None).sum(axis=1) + rng.standard_normal(N)
    y = (score / 5.0).astype(F32)
    kw = dict(num_bins=B, max_depth=4, n_estimators=5, learning_rate=0.4, min_child_weight=5)
    m = WarpGBM(**kw).fit(X, y, era_id=era)
    codes = X.astype(np.int8)
    assert (codes >= B).any() and (codes < 0).any()
    ref = gbm.Forest(**kw).fit_codes(codes, y, era_id=era)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
    assert np.array_equal(bits(m.predict(X)), bits(ref.predict_codes(codes)))
    assert np.array_equal(bits(m.per_era_feature_importance_), bits(ref.imp))


def test_int8_input_over_num_bins_is_quantile_binned(gpu):
    """int8 input with a value >= num_bins fails the pre-binned test
    (warpgbm/core.py:501-503) and is quantile-binned as float32, at fit and
    at predict."""
    print_case("estimator", "int8 not pre-binned")
    rng = np.random.default_rng(5)
    N, F = 4000, 9
    X = rng.integers(-4, 5, (N, F)).astype(np.int8)
    X[N - 1, F - 1] = 7  # one value >= num_bins = 6
    y = (X[:, 0] * 0.5 + X[:, 1] - X[:, 2] + rng.standard_normal(N)).astype(F32)
    m = WarpGBM(num_bins=6, max_depth=3, n_estimators=5, learning_rate=0.3)
    m.fit(X, y)
    Xf = X.astype(F32)
    codes = oracle_codes(m, Xf)
    ref = gbm.Forest(num_bins=6, max_depth=3, n_estimators=5, learning_rate=0.3).fit_codes(codes, y)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
    assert np.array_equal(bits(m.predict(X)), bits(ref.predict_codes(codes)))


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("mcw,B", [(1, 12), (20, 12), (1, 7), (20, 3), (1, 2)])
def test_era_des_colsample_uneven_eras_bit_exact(gpu, mcw, B, layout):
    """Direct era path (every era fits one LDS tile): uneven era sizes, eras
    that are empty at deeper nodes, a feature subset per tree, generic bin
    counts (B <= 7 with layout 1: pair codes and pair tables); with
    min_child_weight 20 many
    (node, era) segments hold fewer than 2*20 rows (no candidate can split
    them) from the root down."""
    print_case("estimator", "DES E=7 uneven colsample mcw B layout", mcw, B, layout)
    rng = np.random.default_rng(5)
    sizes = np.array([900, 40, 1500, 7, 600, 1200, 253])
    E, N, F = len(sizes), int(sizes.sum()), 23
    era = np.repeat(np.arange(E), sizes)
    X = rng.integers(0, B, (N, F)).astype(np.int8)
    score = (X[:, :6] - (B - 1) / 2).sum(axis=1) * np.where(era % 2 == 0, 1.0, -0.5) + rng.standard_normal(N)
    y = (score / 10.0).astype(F32)
    kw = dict(num_bins=B, max_depth=5, n_estimators=5, learning_rate=0.3, min_child_weight=mcw)
    m = WarpGBM(colsample_bytree=0.6, random_state=11, **kw)
    m._engine_tuning = {2: layout}
    m.fit(X, y, era_id=era)
    ref = gbm.Forest(**kw).fit_codes(X, y, era_id=era, feat_sets=m.feature_subsets_)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
    assert np.array_equal(bits(m.per_era_feature_importance_), bits(ref.imp))


@pytest.mark.parametrize("E,B", [(3, 2), (70, 5), (40, 7), (33, 8), (5, 16)])
def test_era_des_bins_and_blocks_bit_exact(gpu, E, B):
    """The era path (pair codes for num_bins <= 7, int8 codes above) against
    the oracle: uneven era sizes (empty, tiny and dead eras, more than one
    32-era block), more than one feature chunk, a feature subset,
    min_split_gain > 0 and negative codes."""
    print_case("estimator", "DES bins / blocks E B", E, B)
    rng = np.random.default_rng(40 + E + B)
    F = 300 if B < 8 else 150
    sizes = rng.integers(0, 200, E)
    sizes[0] = 1
    N = int(sizes.sum())
    era = np.repeat(np.arange(E), sizes)
    X = rng.integers(0, B, (N, F)).astype(np.int8)
    X[rng.random((N, F)) < 0.01] = -1  # outside [0, num_bins): no bin (still pre-binned)
    flip = np.where(rng.random(E) < 0.5, -1.0, 1.0)
    score = ((X[:, :6].astype(np.float64) - B / 2).sum(axis=1)
             + flip[era] * (X[:, 6] - B / 2) + rng.standard_normal(N))
    y = (score / 4.0).astype(F32)
    kw = dict(num_bins=B, max_depth=5, n_estimators=3, learning_rate=0.4, min_child_weight=4,
              min_split_gain=0.01)
    m = WarpGBM(colsample_bytree=0.7, random_state=5, **kw).fit(X, y, era_id=era)
    ref = gbm.Forest(**kw).fit_codes(X, y, era_id=era, feat_sets=m.feature_subsets_)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs from the oracle"
    assert sum(str(t).count("'feature'") for t in m.forest) > 0
    assert np.array_equal(bits(m.per_era_feature_importance_), bits(ref.imp))
    assert np.array_equal(bits(m.predict(X)), bits(ref.predict_codes(X)))


def test_era_des_many_eras_blocks_bit_exact(gpu):
    """More eras than one 32-era block of the DES era sum (70 ids: two full
    blocks and a partial one), uneven sizes with tiny eras, an id with no
    rows and a feature subset: the oracle's trees, importances and
    predictions."""
    print_case("estimator", "DES E=70 era blocks")
    rng = np.random.default_rng(12)
    E, F, B = 70, 37, 5
    sizes = rng.integers(2, 160, E)
    sizes[[3, 40, 69]] = [1, 0, 300]
    N = int(sizes.sum())
    era = np.repeat(np.arange(E), sizes)
    X = rng.integers(0, B, (N, F)).astype(np.int8)
    flip = np.where(rng.random(E) < 0.5, -1.0, 1.0)
    score = (X[:, :4] - 2).sum(axis=1) + flip[era] * (X[:, 4] - 2) + rng.standard_normal(N)
    y = (score / 4.0).astype(F32)
    kw = dict(num_bins=B, max_depth=4, n_estimators=4, learning_rate=0.4, min_child_weight=6)
    m = WarpGBM(colsample_bytree=0.8, random_state=3, **kw)
    m.fit(X, y, era_id=era)
    ref = gbm.Forest(**kw).fit_codes(X, y, era_id=era, feat_sets=m.feature_subsets_)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
    assert np.array_equal(bits(m.per_era_feature_importance_), bits(ref.imp))
    assert np.array_equal(bits(m.predict(X)), bits(ref.predict_codes(X)))


@pytest.mark.parametrize("E,part", [(130, 1), (130, 0), (1100, 1)])
def test_era_level_partition_modes_bit_exact(gpu, E, part):
    """Era levels with the route reserving each segment's child ranges
    (engine tuning key 7 = 1: no block prefix; segments of 300-700 rows
    cross partition blocks) and with the block prefix (0) grow the oracle's
    trees; 1100 eras take the node scan's loop over more eras than a
    thread keeps in registers.  Heavy-tailed residuals move the children's
    per-era histogram shifts (the segment maxima)."""
    print_case("estimator", "era level partition", E, part)
    rng = np.random.default_rng(50 + E + part)
    F, B = 9, 5
    sizes = rng.integers(300, 700, E) if E < 1000 else rng.integers(5, 40, E)
    N = int(sizes.sum())
    era = np.repeat(np.arange(E), sizes)
    X = rng.integers(0, B, (N, F)).astype(np.int8)
    flip = np.where(rng.random(E) < 0.5, -1.0, 1.0)
    score = (X[:, :3] - 2).sum(axis=1) + flip[era] * (X[:, 3] - 2) + rng.standard_normal(N)
    y = (score / 4.0).astype(F32)
    y[rng.integers(0, N, 5)] *= 1e4
    kw = dict(num_bins=B, max_depth=5, n_estimators=2, learning_rate=0.4, min_child_weight=4)
    m = WarpGBM(**kw)
    m._engine_tuning = {7: part}
    m.fit(X, y, era_id=era)
    ref = gbm.Forest(**kw).fit_codes(X, y, era_id=era)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
    assert np.array_equal(bits(m.predict(X)), bits(ref.predict_codes(X)))


def test_era_des_large_eras_histogram_path_bit_exact(gpu):
    """Eras larger than one LDS tile (65536 rows) take the per-era histogram
    path (tile partials, exact sibling subtraction, era accumulation)."""
    print_case("estimator", "DES E=2 large eras")
    rng = np.random.default_rng(6)
    N, F, E = 140_000, 8, 2
    era = np.repeat(np.arange(E), N // E)
    X = rng.integers(0, 8, (N, F)).astype(np.int8)
    score = (X[:, 0] - 3.5) + np.where(era == 0, 1.0, -1.0) * (X[:, 1] - 3.5) + rng.standard_normal(N)
    y = (score / 4.0).astype(F32)
    kw = dict(num_bins=8, max_depth=3, n_estimators=3, learning_rate=0.5)
    m = WarpGBM(**kw).fit(X, y, era_id=era)
    ref = gbm.Forest(**kw).fit_codes(X, y, era_id=era)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
    assert np.array_equal(bits(m.per_era_feature_importance_), bits(ref.imp))


def test_colsample_subsets_bit_exact(gpu):
    print_case("estimator", "colsample 0.5")
    X, y = c1_data(n=5000, f=40, seed=3)
    m = WarpGBM(num_bins=16, max_depth=4, n_estimators=10, colsample_bytree=0.5,
                random_state=7)
    m.fit(X, y)
    assert len(m.feature_subsets_) == 10 and all(len(s) == 20 for s in m.feature_subsets_)
    codes = oracle_codes(m, X)
    ref = gbm.Forest(num_bins=16, max_depth=4, n_estimators=10).fit_codes(
        codes, y, feat_sets=m.feature_subsets_)
    for a, b in zip(m.forest, ref.forest):
        assert a == b
    m2 = WarpGBM(num_bins=16, max_depth=4, n_estimators=10, colsample_bytree=0.5,
                 random_state=7).fit(X, y)
    assert np.array_equal(m2.predict(X), m.predict(X))


def test_warm_start_and_save_load(gpu, tmp_path):
    print_case("estimator", "warm start / save-load")
    X, y = c1_data(n=4000, f=20, seed=4)
    full = WarpGBM(num_bins=16, max_depth=3, n_estimators=12).fit(X, y)
    part = WarpGBM(num_bins=16, max_depth=3, n_estimators=6, warm_start=True).fit(X, y)
    part.n_estimators = 12
    part.fit(X, y)
    assert part._trees_trained == 12
    assert np.array_equal(bits(part.predict(X)), bits(full.predict(X)))
    path = tmp_path / "m.pkl"
    full.save_model(str(path))
    loaded = WarpGBM().load_model(str(path))
    assert np.array_equal(bits(loaded.predict(X)), bits(full.predict(X)))


def test_eval_and_early_stopping(gpu):
    print_case("estimator", "eval set")
    X, y = c1_data(n=4000, f=20, seed=5)
    # 31 trees: evaluation runs at i = 0, 2, ..., 30, so the last one sees all trees
    m = WarpGBM(num_bins=16, max_depth=3, n_estimators=31, learning_rate=0.3)
    m.fit(X[:3000], y[:3000], X_eval=X[3000:], y_eval=y[3000:], eval_every_n_trees=2,
          early_stopping_rounds=2, eval_metric="mse")
    assert len(m.training_loss) == m._trees_trained
    assert m.training_loss[-1] < m.training_loss[0]
    if m._trees_trained == 31:
        # eval predictions tracked during training equal predict() on the eval set
        p = m.predict(X[3000:])
        assert abs(float(((y[3000:] - p) ** 2).mean()) - m.eval_loss[-1]) <= 1e-5 * m.eval_loss[-1]
    else:
        # stopped early: the last eval loss rose against the one esr evaluations before
        assert m.eval_loss[-3] < m.eval_loss[-1]
    # early stopping triggers on a metric that gets worse: 1 - corr on a shuffled target
    rng = np.random.default_rng(0)
    m2 = WarpGBM(num_bins=16, max_depth=3, n_estimators=60, learning_rate=1.0)
    m2.fit(X[:3000], y[:3000], X_eval=X[3000:], y_eval=rng.permutation(y[3000:]),
           eval_every_n_trees=1, early_stopping_rounds=3, eval_metric="corr")
    assert m2._trees_trained < 60


def test_binary_objective(gpu):
    print_case("estimator", "binary")
    rng = np.random.default_rng(6)
    X = rng.standard_normal((3000, 8)).astype(F32)
    y = (X[:, 0] + 0.5 * X[:, 1] > 0).astype(np.int64)
    m = WarpGBM(objective="binary", num_bins=16, max_depth=3, n_estimators=20,
                learning_rate=0.3).fit(X, y)
    assert m.predict_proba(X).shape == (3000, 2)
    assert (m.predict(X) == y).mean() > 0.9


def _heavy_targets(rng, n, signal):
    """+-1e-3 targets (sign of ``signal``) with +1e6 and -1e6 on two rows."""
    y = np.where(signal > 0, 1e-3, -1e-3).astype(F32)
    y[0], y[1] = 1e6, -1e6
    return y


def _small_leaves(tree, out):
    if "leaf_value" in tree:
        out.append(tree["leaf_value"])
    else:
        _small_leaves(tree["left"], out)
        _small_leaves(tree["right"], out)
    return out


@pytest.mark.parametrize("seed,depth", [(0, 3), (2, 4), (3, 3), (5, 4)])
def test_heavy_tailed_regression_bit_exact(gpu, seed, depth):
    """Residuals of 1e-3 next to +-1e6: nodes whose residuals are all small
    take their own histogram shift (both children histogrammed), leaves use
    the wide sums, so the small rows get their own means and splits -- bit
    for bit the oracle's arithmetic (whose agreement with the reference's
    float32 arithmetic is checked in test_literal_f32.py)."""
    print_case("estimator", "heavy-tailed regression seed depth", seed, depth)
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((2000, 4)).astype(F32)
    y = _heavy_targets(rng, 2000, X[:, 1])
    kw = dict(num_bins=4, max_depth=depth, n_estimators=3, learning_rate=0.1,
              min_child_weight=5)
    m = WarpGBM(**kw).fit(X, y)
    codes = oracle_codes(m, X)
    ref = gbm.Forest(**kw).fit_codes(codes, y)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
    assert np.array_equal(bits(m.predict(X)), bits(ref.predict_codes(codes)))
    small = [v for v in _small_leaves(m.forest[0], []) if abs(v) < 1e-2]
    assert small and all(v != 0.0 for v in small)  # the small rows' own means


@pytest.mark.parametrize("N,E", [(6000, 4), (140_000, 2)])
def test_heavy_tailed_eras_bit_exact(gpu, N, E):
    """The same targets through the era paths: direct per-(node, era) LDS
    histograms (eras <= 65536 rows) and the per-era histogram path with exact
    subtraction (larger eras)."""
    print_case("estimator", "heavy-tailed eras N E", N, E)
    rng = np.random.default_rng(9)
    X = rng.integers(0, 5, (N, 6)).astype(np.int8)
    era = np.repeat(np.arange(E), N // E)
    y = _heavy_targets(rng, N, X[:, 2].astype(np.float64) - 2 + 0.5 * (era % 2))
    kw = dict(num_bins=5, max_depth=4, n_estimators=2, learning_rate=0.1, min_child_weight=5)
    m = WarpGBM(**kw).fit(X, y, era_id=era)
    ref = gbm.Forest(**kw).fit_codes(X, y, era_id=era)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
    assert np.array_equal(bits(m.per_era_feature_importance_), bits(ref.imp))
    assert np.array_equal(bits(m.predict(X)), bits(ref.predict_codes(X)))


@pytest.mark.parametrize("N,E", [(4000, 4), (140_000, 2)])
@pytest.mark.parametrize("big", [1e4, 1e6])
def test_eras_of_different_scales_bit_exact(gpu, N, E, big):
    """Eras whose residual scales differ by up to 1e9 (+-1e-3 targets, two
    +-big rows in era 0): every (node, era) segment is quantised at its own
    shift, on the direct era path (eras <= 65536 rows) and on the per-era
    histogram path (larger eras, the sibling subtracted per era only where
    the shifts agree).  Trees, importances and predictions bit-exact against
    the oracle, whose agreement with the reference's float32 DES picks on
    this data is checked in test_literal_f32.py."""
    from tests.test_literal_f32 import HEAVY_ERA_KW, heavy_tailed_eras

    print_case("estimator", "eras of different scales N E big", N, E, big)
    X, y, era = heavy_tailed_eras(3, big, n=N, E=E)
    m = WarpGBM(**HEAVY_ERA_KW).fit(X, y, era_id=era)
    codes = oracle_codes(m, X)
    ref = gbm.Forest(**HEAVY_ERA_KW).fit_codes(codes, y, era_id=era)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
    assert np.array_equal(bits(m.per_era_feature_importance_), bits(ref.imp))
    assert np.array_equal(bits(m.predict(X)), bits(ref.predict_codes(codes)))


def _des_gate_data(N=8000, E=4, seed=12):
    """Four eras: feature 0 moves the target a little in the same direction
    in every era, feature 1 a lot but with opposite signs in eras {0, 1} and
    {2, 3}; features 2, 3 are noise."""
    rng = np.random.default_rng(seed)
    X = rng.integers(0, 5, (N, 4)).astype(np.int8)
    era = np.repeat(np.arange(E), N // E)
    sgn = np.where(era < E // 2, 1.0, -1.0)
    y = (0.01 * (X[:, 0] - 2) + sgn * (X[:, 1] - 2) + 0.001 * rng.standard_normal(N))
    return X, y.astype(F32), era


def test_des_leaf_when_max_agreement_candidates_fail_min_split_gain(gpu):
    """core.py:583-586: the DES mask is (agree == max agree) & (crit >
    min_split_gain); when every max-agreement candidate fails the gain
    threshold the node is a leaf, although lower-agreement candidates (here
    feature 1, whose sign flips between eras and whose criterion is some 500
    times larger) pass it.  min_split_gain is set between the two, from the
    oracle's root criteria; without it the root splits."""
    print_case("estimator", "DES leaf by min_split_gain")
    X, y, era = _des_gate_data()
    E, B = 4, 5
    r = y - gbm.base_score(y)
    qb = ops.qbits_for_rows(len(y))
    S = np.array([ops.key_shift(m, qb) for m in ops.era_absmax(r, np.arange(len(y)), era, E)])
    Q, C = ops.histogram_exact_q(X, ops.quantise_by_era(r, np.arange(len(y)), era, S),
                                 np.arange(len(y)), np.arange(4), era, E, B)
    gain, dirn = ops.split_scan(ops.dequantise(Q, S), C.astype(F32), 20, 1e-6)
    crit, agree = ops.des_criterion(gain, dirn)
    top = agree == agree.max()
    a, b = float(crit[top].max()), float(crit.max())
    assert b > 100 * a  # the gate lies between the two
    msg = float(np.sqrt(a * b))
    for gate, expect_leaf in ((0.0, False), (msg, True)):
        kw = dict(num_bins=B, max_depth=3, n_estimators=2, learning_rate=0.1,
                  min_split_gain=gate)
        m = WarpGBM(**kw).fit(X, y, era_id=era)
        ref = gbm.Forest(**kw).fit_codes(X, y, era_id=era)
        assert ("leaf_value" in ref.forest[0]) == expect_leaf
        for i, (ta, tb) in enumerate(zip(m.forest, ref.forest)):
            assert ta == tb, f"gate {gate}: tree {i} differs"
        assert np.array_equal(bits(m.predict(X)), bits(ref.predict_codes(X)))


@pytest.mark.parametrize("level_bytes", [0, 1])
def test_chunked_levels_regression_bit_exact(gpu, level_bytes):
    """A level budget of 1 byte leaves room for one (tree, node) at a time:
    every level below the root is processed node by node, each histogrammed
    directly.  The trees are the same as with the whole-level path."""
    print_case("estimator", "chunked levels regression, level_bytes", level_bytes)
    X, y = c1_data(4000, 12)
    kw = dict(num_bins=16, max_depth=6, n_estimators=3, learning_rate=0.3, min_child_weight=10)
    m = WarpGBM(**kw)
    m._engine_level_bytes = level_bytes
    m.fit(X, y)
    codes = oracle_codes(m, X)
    ref = gbm.Forest(**kw).fit_codes(codes, y)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
    assert np.array_equal(bits(m.predict(X)), bits(ref.predict_codes(codes)))


def test_chunked_levels_multiclass_and_eras_bit_exact(gpu):
    print_case("estimator", "chunked levels multiclass / DES direct / large eras")
    # softmax, 4 class trees per round: chunks of nodes across trees
    rng = np.random.default_rng(3)
    N, F, K = 3000, 8, 4
    labels = rng.integers(0, K, N)
    X = (rng.standard_normal((K, F))[labels] * 1.5 + rng.standard_normal((N, F))).astype(F32)
    kw = dict(objective="multiclass", num_bins=12, max_depth=4, n_estimators=2,
              learning_rate=0.3, min_child_weight=5)
    m = WarpGBM(**kw)
    m._engine_level_bytes = 40_000  # a few (tree, node)s per chunk
    m.fit(X, labels)
    codes = oracle_codes(m, X)
    ref = gbm.Forest(**kw).fit_codes(codes, labels)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"round {i} differs"
    # direct era path (every era <= 65536 rows) and the per-era histogram path
    for N, E, lb in ((6000, 6, 1), (140_000, 2, 1)):
        rng = np.random.default_rng(4)
        X = rng.integers(0, 5, (N, 10)).astype(np.int8)
        era = np.repeat(np.arange(E), N // E)
        score = (X[:, 0] - 2) + np.where(era % 2 == 0, 1.0, -1.0) * (X[:, 1] - 2)
        y = (score + rng.standard_normal(N)).astype(F32) / 4
        kw = dict(num_bins=5, max_depth=4, n_estimators=2, learning_rate=0.5)
        m = WarpGBM(**kw)
        m._engine_level_bytes = lb
        m.fit(X, y, era_id=era)
        ref = gbm.Forest(**kw).fit_codes(X, y, era_id=era)
        for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
            assert a == b, f"E={E} tree {i} differs"
        assert np.array_equal(bits(m.per_era_feature_importance_), bits(ref.imp))


def test_127_bins_depth_10_bit_exact(gpu):
    """The reference demo's shape (127 bins, depth 10): the one-feature-per-
    lane histogram variant, deep heaps in the predictor."""
    print_case("estimator", "127 bins depth 10")
    rng = np.random.default_rng(5)
    N = 30_000
    t = rng.uniform(0, 4 * np.pi, N)
    X = np.stack([t * np.cos(t), t * np.sin(t), rng.standard_normal(N),
                  rng.standard_normal(N)], axis=1).astype(F32) + 0.3 * rng.standard_normal((N, 4)).astype(F32)
    y = (np.sin(t) + 0.1 * rng.standard_normal(N)).astype(F32)
    kw = dict(num_bins=127, max_depth=10, n_estimators=4, learning_rate=0.3, min_child_weight=5)
    m = WarpGBM(**kw).fit(X, y)
    codes = oracle_codes(m, X)
    ref = gbm.Forest(**kw).fit_codes(codes, y)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
    assert np.array_equal(bits(m.predict(X)), bits(ref.predict_codes(codes)))
    assert max(_depth(t) for t in m.forest) == 10


def _depth(node):
    if "leaf_value" in node:
        return 0
    return 1 + max(_depth(node["left"]), _depth(node["right"]))


def test_depth_beyond_twenty_bit_exact(gpu):
    """max_depth 22 (the engine used to stop at 20): with min_child_weight 1
    the trees reach their full depth on a small set."""
    print_case("estimator", "max_depth 22")
    rng = np.random.default_rng(6)
    N = 3000
    X = rng.standard_normal((N, 5)).astype(F32)
    y = (X[:, 0] * 3 + np.sin(5 * X[:, 1]) + rng.standard_normal(N)).astype(F32)
    kw = dict(num_bins=64, max_depth=22, n_estimators=2, learning_rate=0.5, min_child_weight=1)
    m = WarpGBM(**kw).fit(X, y)
    codes = oracle_codes(m, X)
    ref = gbm.Forest(**kw).fit_codes(codes, y)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
    assert np.array_equal(bits(m.predict(X)), bits(ref.predict_codes(codes)))
    assert max(_depth(t) for t in m.forest) > 12


@pytest.mark.parametrize("scan,fuse,root,part", [(1, 1, 1, 1), (1, 1, 1, 0), (0, 0, 1, 1),
                                                  (1, 0, 1, 1), (1, 1, 0, 1)])
def test_one_era_level_scans_bit_exact(gpu, scan, fuse, root, part):
    """The per-level kernels of one-era fits in each setting (engine tuning
    key 3: node scan with a thread or a wave per node; key 4: split search
    and leaf step fused or not; key 5: the root's positions and totals in one
    launch with a root tile plan made once, or the root partition pass and a
    plan per round; key 6: split levels of up to 1024 nodes partitioned
    in one pass with reserved child ranges, or route + block prefix + stable
    scatter) grow the oracle's trees.  Heavy tails on
    60000 rows: nodes spanning many partition blocks whose child maxima move
    their histogram shift (both children histogrammed); depth 12 (2048 nodes
    at the last split level, past the 1024 planned from registers); softmax
    with 5 class trees and 640 nodes at depth 7; 300 features (two split
    workgroups per node, the fused step's last-arrival path)."""
    print_case("estimator", "one-era level scan, fused finish, root path, one-pass partition",
               scan, fuse, root, part)
    tuning = {3: scan, 4: fuse, 5: root, 6: part}
    rng = np.random.default_rng(12)
    N = 60_000
    X = rng.standard_normal((N, 5)).astype(F32)
    y = _heavy_targets(rng, N, X[:, 1])
    y[2:200] *= 1e4  # a band of mid-sized residuals
    kw = dict(num_bins=8, max_depth=12, n_estimators=2, learning_rate=0.3, min_child_weight=1)
    m = WarpGBM(**kw)
    m._engine_tuning = tuning
    m.fit(X, y)
    codes = oracle_codes(m, X)
    ref = gbm.Forest(**kw).fit_codes(codes, y)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
    assert np.array_equal(bits(m.predict(X)), bits(ref.predict_codes(codes)))
    assert max(_depth(t) for t in m.forest) == 12
    # softmax: 5 trees per round, 640 (tree, node)s at depth 7
    N, F, K = 30_000, 6, 5
    labels = rng.integers(0, K, N)
    X = (rng.standard_normal((K, F))[labels] + rng.standard_normal((N, F))).astype(F32)
    kw = dict(objective="multiclass", num_bins=16, max_depth=8, n_estimators=2,
              learning_rate=0.3, min_child_weight=2)
    m = WarpGBM(**kw)
    m._engine_tuning = tuning
    m.fit(X, labels)
    codes = oracle_codes(m, X)
    ref = gbm.Forest(**kw).fit_codes(codes, labels)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"round {i} differs"
    assert np.array_equal(bits(m.predict_proba(X)), bits(ref.predict_codes(codes)))
    # 300 features: n_sel > 256, several split workgroups per node
    N, F = 20_000, 300
    X = rng.standard_normal((N, F)).astype(F32)
    y = (X[:, 7] + 0.5 * (X[:, 280] > 0) + 0.3 * rng.standard_normal(N)).astype(F32)
    kw = dict(num_bins=16, max_depth=5, n_estimators=3, learning_rate=0.3, min_child_weight=5)
    m = WarpGBM(**kw)
    m._engine_tuning = tuning
    m.fit(X, y)
    codes = oracle_codes(m, X)
    ref = gbm.Forest(**kw).fit_codes(codes, y)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"300-feature tree {i} differs"
    assert "'feature': 280" in str(m.forest[0]) or "'feature': 7" in str(m.forest[0])


def test_predict_reads_split_columns_only(gpu):
    """Inputs of >= 65536 rows are binned only in the columns the forest
    splits on (gathered on the host, uploaded and binned as a narrow code
    matrix): the predictions equal the full binning path and the oracle's,
    bit for bit, for float32, float64 and non-contiguous input, regression
    and multiclass."""
    print_case("estimator", "predict from split columns")
    rng = np.random.default_rng(11)
    N, F = 20000, 300
    X = rng.standard_normal((N, F)).astype(F32)
    y = (2.0 * X[:, 7] - X[:, 150] + 0.5 * X[:, 299] + 0.1 * rng.standard_normal(N)).astype(F32)
    m = WarpGBM(num_bins=32, max_depth=4, n_estimators=10, learning_rate=0.1)
    m.fit(X, y)
    cols, _ = m._used_features()
    assert 2 * len(cols) <= F and {7, 150} <= set(cols.tolist())
    Xt = rng.standard_normal((70_001, F)).astype(F32)
    p = m.predict(Xt)
    full = m.predict_binned(m.bin_inference_data(Xt)).cpu().numpy()
    assert np.array_equal(bits(p), bits(full))
    ref = gbm.Forest(num_bins=32, max_depth=4, n_estimators=10, learning_rate=0.1,
                     min_child_weight=20, min_split_gain=0.0, L2_reg=1e-6)
    ref.forest, ref.base = m.forest, F32(m.base_prediction)
    codes_t = ops.bin_matrix(Xt, torch.as_tensor(m.bin_edges).cpu().numpy())
    assert np.array_equal(bits(p), bits(ref.predict_codes(codes_t)))
    assert np.array_equal(bits(m.predict(Xt.astype(np.float64))), bits(p))
    assert np.array_equal(bits(m.predict(np.asfortranarray(Xt))), bits(p))

    K = 3
    lab = rng.integers(0, K, N)
    Xc = rng.standard_normal((N, F)).astype(F32)
    Xc[:, 11] += 2.0 * lab
    Xc[:, 201] -= 1.5 * lab
    mc = WarpGBM(objective="multiclass", num_bins=16, max_depth=3, n_estimators=6,
                 learning_rate=0.2)
    mc.fit(Xc, lab)
    cols, _ = mc._used_features()
    assert 2 * len(cols) <= F
    Xct = rng.standard_normal((66_000, F)).astype(F32)
    Xct[:, 11] += 2.0 * rng.integers(0, K, len(Xct))
    pr = mc.predict_proba(Xct)
    full = mc.predict_proba_binned(mc.bin_inference_data(Xct)).cpu().numpy()
    assert np.array_equal(bits(pr), bits(full))
    assert np.array_equal(mc.predict(Xct), mc.classes_[np.argmax(full, axis=1)])
