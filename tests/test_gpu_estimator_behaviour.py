"""Estimator behaviours the reference's own test suite checks (warm start,
save / load, random_state, eras, importances, a small real dataset), run on
the GPU engine.  Where the reference asserts closeness, these assert bit
equality: the engine is deterministic and its sums are exact.

Reference tests followed: tests/test_warm_start.py, tests/test_random_state.py,
tests/test_feature_importance.py, tests/test_multiclass.py,
tests/test_comparison_lightgbm.py (the LightGBM side of that comparison is
not installed here; the accuracy bar and the oracle's trees stand in)."""
import numpy as np
import pytest

from oracle import gbm
from tests.conftest import c1_data, print_case
from warpgbm_amd import WarpGBM

pytestmark = pytest.mark.gpu
F32 = np.float32


def bits(a):
    return np.asarray(a, dtype=F32).view(np.uint32)


def blobs(n, f, k, seed):
    rng = np.random.default_rng(seed)
    means = rng.standard_normal((k, f)) * 1.5
    labels = rng.integers(0, k, n)
    return (means[labels] + rng.standard_normal((n, f))).astype(F32), labels


def test_warm_start_false_refits_from_scratch(gpu):
    """warm_start=False: a second fit() starts over and reproduces the first
    model (tests/test_warm_start.py:58-80)."""
    print_case("behaviour", "warm_start False refit")
    X, y = c1_data(n=3000, f=10, seed=21)
    m = WarpGBM(num_bins=16, max_depth=3, n_estimators=15, learning_rate=0.2, random_state=42)
    p1 = m.fit(X, y).predict(X)
    forest1 = list(m.forest)
    p2 = m.fit(X, y).predict(X)
    assert m._trees_trained == 15 and len(m.forest) == 15
    assert m.forest == forest1
    assert np.array_equal(bits(p1), bits(p2))


def test_warm_start_already_complete_adds_nothing(gpu):
    """warm_start=True with n_estimators trees already grown: fit() grows no
    more (tests/test_warm_start.py:83-104)."""
    print_case("behaviour", "warm_start complete")
    X, y = c1_data(n=2000, f=10, seed=22)
    m = WarpGBM(num_bins=16, max_depth=3, n_estimators=10, warm_start=True, random_state=42)
    m.fit(X, y)
    forest1, p1 = list(m.forest), m.predict(X)
    m.fit(X, y)
    assert m._trees_trained == 10 and m.forest == forest1
    assert np.array_equal(bits(m.predict(X)), bits(p1))


@pytest.mark.parametrize("objective,k", [("multiclass", 4), ("binary", 2)])
def test_classification_warm_start_equals_full_fit(gpu, objective, k):
    """Rounds grown in two warm-started fits equal the same rounds grown at
    once: trees, probabilities and importances (tests/test_warm_start.py:107-199)."""
    print_case("behaviour", "warm start", objective)
    X, labels = blobs(3000, 9, k, seed=23)
    kw = dict(objective=objective, num_bins=16, max_depth=3, learning_rate=0.3,
              min_child_weight=5)
    full = WarpGBM(n_estimators=12, **kw).fit(X, labels)
    part = WarpGBM(n_estimators=5, warm_start=True, **kw).fit(X, labels)
    part.n_estimators = 12
    part.fit(X, labels)
    assert part._trees_trained == 12
    assert part.forest == full.forest
    assert np.array_equal(bits(part.predict_proba(X)), bits(full.predict_proba(X)))
    assert np.array_equal(bits(part.per_era_feature_importance_),
                          bits(full.per_era_feature_importance_))


def test_save_load_multiclass_then_resume(gpu, tmp_path):
    """A saved multiclass model predicts identically after loading and, with
    warm_start, resumes to the same model as one uninterrupted fit
    (tests/test_warm_start.py:243-413)."""
    print_case("behaviour", "save/load multiclass resume")
    X, labels = blobs(2500, 7, 3, seed=24)
    y = np.array(["cat", "dog", "bird"])[labels]
    kw = dict(objective="multiclass", num_bins=16, max_depth=3, learning_rate=0.3,
              min_child_weight=5)
    full = WarpGBM(n_estimators=10, **kw).fit(X, y)
    part = WarpGBM(n_estimators=4, warm_start=True, **kw).fit(X, y)
    path = tmp_path / "mc.pkl"
    part.save_model(str(path))
    loaded = WarpGBM().load_model(str(path))
    assert np.array_equal(bits(loaded.predict_proba(X)), bits(part.predict_proba(X)))
    assert (loaded.predict(X) == part.predict(X)).all()
    loaded.warm_start = True
    loaded.n_estimators = 10
    loaded.fit(X, y)
    assert loaded.forest == full.forest
    assert np.array_equal(bits(loaded.predict_proba(X)), bits(full.predict_proba(X)))


def test_importance_accumulates_over_warm_start(gpu):
    """Importances of a warm-started model only grow, and end equal to the
    uninterrupted fit's (tests/test_warm_start.py:416-440)."""
    print_case("behaviour", "importance over warm start")
    X, y = c1_data(n=3000, f=10, seed=25)
    kw = dict(num_bins=16, max_depth=3, learning_rate=0.2)
    m = WarpGBM(n_estimators=8, warm_start=True, **kw).fit(X, y)
    imp8 = m.get_feature_importance(normalize=False).copy()
    m.n_estimators = 16
    m.fit(X, y)
    imp16 = m.get_feature_importance(normalize=False)
    assert np.all(imp16 >= imp8) and imp16.sum() > imp8.sum()
    full = WarpGBM(n_estimators=16, **kw).fit(X, y)
    assert np.array_equal(bits(imp16), bits(full.get_feature_importance(normalize=False)))


def test_random_state_reproducible_with_colsample(gpu):
    """The same random_state draws the same feature subsets and grows the same
    model; another seed draws other subsets; no seed still trains
    (tests/test_random_state.py)."""
    print_case("behaviour", "random_state")
    X, y = c1_data(n=3000, f=20, seed=26)
    kw = dict(num_bins=16, max_depth=3, n_estimators=10, learning_rate=0.2,
              colsample_bytree=0.5)
    a = WarpGBM(random_state=7, **kw).fit(X, y)
    b = WarpGBM(random_state=7, **kw).fit(X, y)
    c = WarpGBM(random_state=8, **kw).fit(X, y)
    assert a.forest == b.forest
    assert np.array_equal(bits(a.predict(X)), bits(b.predict(X)))
    assert any(not np.array_equal(s, t) for s, t in zip(a.feature_subsets_, c.feature_subsets_))
    assert all(len(s) == 10 for s in a.feature_subsets_)
    d = WarpGBM(**kw).fit(X, y)
    assert d._trees_trained == 10


def test_no_era_equals_single_era(gpu):
    """Without era_id the model is the one-era model (era ids all equal):
    trees, predictions, importances (tests/test_feature_importance.py:265)."""
    print_case("behaviour", "no era == one era")
    X, y = c1_data(n=3000, f=10, seed=27)
    kw = dict(num_bins=16, max_depth=4, n_estimators=8, learning_rate=0.2)
    a = WarpGBM(**kw).fit(X, y)
    b = WarpGBM(**kw).fit(X, y, era_id=np.full(len(y), 3))
    assert a.forest == b.forest
    assert np.array_equal(bits(a.predict(X)), bits(b.predict(X)))
    assert np.array_equal(bits(a.per_era_feature_importance_), bits(b.per_era_feature_importance_))
    assert a.per_era_feature_importance_.shape == (1, 10)


def test_per_era_importance_ranks_the_stable_feature(gpu):
    """Per-era importances: one row per era, their sum is the feature
    importance, and the feature whose effect holds in every era ranks first in
    every era (tests/test_feature_importance.py:190-262)."""
    print_case("behaviour", "per-era importance")
    rng = np.random.default_rng(28)
    E, n_era, F = 4, 1500, 6
    era = np.repeat(np.arange(E), n_era)
    X = rng.integers(0, 5, (E * n_era, F)).astype(np.int8)
    flip = np.where(np.arange(E) % 2 == 0, 1.0, -1.0)
    y = (2.0 * (X[:, 0] - 2) + flip[era] * 0.5 * (X[:, 1] - 2)
         + 0.3 * rng.standard_normal(E * n_era)).astype(F32)
    m = WarpGBM(num_bins=5, max_depth=3, n_estimators=10, learning_rate=0.3)
    m.fit(X, y, era_id=era)
    per = m.get_per_era_feature_importance(normalize=False)
    assert per.shape == (E, F)
    assert np.allclose(per.sum(axis=0), m.get_feature_importance(normalize=False), rtol=1e-6)
    assert (np.argmax(per, axis=1) == 0).all()
    ref = gbm.Forest(num_bins=5, max_depth=3, n_estimators=10, learning_rate=0.3).fit_codes(
        X, y, era_id=era)
    assert m.forest == ref.forest
    assert np.array_equal(bits(m.per_era_feature_importance_), bits(ref.imp))


def test_iris_multiclass(gpu):
    """Iris (150 rows, 4 features, 3 classes; bundled with scikit-learn):
    training accuracy and the oracle's trees
    (tests/test_comparison_lightgbm.py:52-116)."""
    datasets = pytest.importorskip("sklearn.datasets")
    print_case("behaviour", "iris")
    iris = datasets.load_iris()
    X, labels = iris.data.astype(F32), iris.target
    kw = dict(objective="multiclass", num_bins=16, max_depth=3, n_estimators=30,
              learning_rate=0.2, min_child_weight=2)
    m = WarpGBM(**kw).fit(X, labels)
    assert (m.predict(X) == labels).mean() >= 0.95
    from oracle import ops

    codes = ops.bin_matrix(X, ops.quantile_edges(X, 16))
    ref = gbm.Forest(**kw).fit_codes(codes, labels)
    assert m.forest == ref.forest
    assert np.array_equal(bits(m.predict_proba(X)), bits(ref.predict_codes(codes)))


def test_predict_zero_rows(gpu):
    """A prediction over no rows returns empty arrays of the right shapes
    (regression values, class labels, class probabilities) and leaves the
    model usable: the next prediction matches one made before it."""
    print_case("behaviour", "predict on zero rows")
    X, y = c1_data(n=2000, f=12, seed=5)
    m = WarpGBM(num_bins=16, max_depth=3, n_estimators=5, learning_rate=0.2)
    m.fit(X, y)
    p = m.predict(X)
    z = m.predict(X[:0])
    assert z.shape == (0,)
    assert np.array_equal(bits(m.predict(X)), bits(p))
    Xc, labels = blobs(1500, 6, 3, seed=8)
    c = WarpGBM(objective="multiclass", num_bins=16, max_depth=3, n_estimators=4,
                learning_rate=0.3)
    c.fit(Xc, labels)
    pr = c.predict_proba(Xc)
    assert c.predict(Xc[:0]).shape == (0,)
    assert c.predict_proba(Xc[:0]).shape == (0, 3)
    assert np.array_equal(bits(c.predict_proba(Xc)), bits(pr))


@pytest.mark.parametrize("value", [0.0, 2.5, -1024.0])
def test_constant_target_grows_no_splits(gpu, value):
    """A constant target (values whose running sums are exact in float32, so
    the base prediction, warpgbm/core.py:387, is the value itself) leaves every
    residual exactly zero: every candidate's gain is 0, which does not pass
    the strict gain > min_split_gain test (warpgbm/core.py:579-583), so no tree
    splits, every leaf value is 0 and every prediction is the target."""
    print_case("behaviour", f"constant target {value}")
    X, _ = c1_data(n=3000, f=12, seed=9)
    y = np.full(len(X), value, F32)
    m = WarpGBM(num_bins=16, max_depth=4, n_estimators=6, learning_rate=0.3)
    m.fit(X, y)
    assert np.float32(m.base_prediction) == np.float32(value)
    assert np.array_equal(bits(m.predict(X)), bits(np.full(len(X), value, F32)))
    assert float(np.sum(m.get_feature_importance(normalize=False))) == 0.0


def _as_reference_forest(forest, dev):
    """The forest as the reference's fit leaves it: a split's "feature" is
    feat_indices_tree[local_feature], a 0-d int64 tensor on the device
    (warpgbm/core.py:653-654); "bin" and the leaf values are Python numbers
    (.item(), core.py:590-594, 606)."""
    import torch

    def conv(node):
        if "leaf_value" in node:
            return dict(node)
        return {"feature": torch.tensor(int(node["feature"]), dtype=torch.int64, device=dev),
                "bin": node["bin"], "left": conv(node["left"]), "right": conv(node["right"])}

    return [[conv(t) for t in r] if isinstance(r, list) else conv(r) for r in forest]


@pytest.mark.parametrize("objective", ["regression", "multiclass"])
def test_load_reference_written_pickle(gpu, tmp_path, objective):
    """A pickle in the reference's save_model layout (warpgbm/core.py:1122-1153)
    whose trees hold device-tensor features and whose bin_edges is a device
    tensor loads through load_model and predicts exactly as the model it was
    made from."""
    import pickle

    import torch

    print_case("behaviour", "reference-written pickle", objective)
    dev = torch.device("cuda:0")
    if objective == "regression":
        X, y = c1_data(n=3000, f=12, seed=31)
        m = WarpGBM(num_bins=16, max_depth=3, n_estimators=8).fit(X, y)
    else:
        X, labels = blobs(2000, 6, 3, seed=32)
        m = WarpGBM(objective="multiclass", num_bins=16, max_depth=3, n_estimators=5,
                    learning_rate=0.3, min_child_weight=5).fit(X, labels)
    path = tmp_path / "ref.pkl"
    m.save_model(str(path))
    with open(path, "rb") as f:
        state = pickle.load(f)  # written by this test just above
    state["forest"] = _as_reference_forest(m.forest, dev)
    state["bin_edges"] = torch.as_tensor(m.bin_edges).to(dev)
    with open(path, "wb") as f:
        pickle.dump(state, f)
    loaded = WarpGBM().load_model(str(path))
    if objective == "regression":
        assert np.array_equal(bits(loaded.predict(X)), bits(m.predict(X)))
    else:
        assert np.array_equal(bits(loaded.predict_proba(X)), bits(m.predict_proba(X)))
        assert (loaded.predict(X) == m.predict(X)).all()
    # the reference's flat predict table of a loaded tree equals the original's
    first = (lambda mm: mm.forest[0][0] if objective == "multiclass" else mm.forest[0])
    a, b = loaded.flatten_tree(first(loaded), 64), m.flatten_tree(first(m), 64)
    assert torch.allclose(a, b, rtol=0, atol=0, equal_nan=True)
