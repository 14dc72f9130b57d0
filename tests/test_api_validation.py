"""Host-side error behaviour of the estimator, mirroring the reference's
host-forceable checks (warpgbm/core.py:83-143, 216-291, 353-356, 983-984,
1054-1055, 1118-1119).  CPU only: every check fires before device work."""
import numpy as np
import pytest

from warpgbm_amd import WarpGBM
from warpgbm_amd.core import _dict_to_heap, _heaps_to_dicts, _preorder_heap


@pytest.mark.parametrize("kw,exc", [
    ({"objective": "ranking"}, ValueError),
    ({"num_bins": 1}, ValueError),
    ({"num_bins": 128}, ValueError),
    ({"num_bins": 10.0}, TypeError),
    ({"max_depth": 0}, ValueError),
    ({"learning_rate": 0.0}, ValueError),
    ({"learning_rate": 1.5}, ValueError),
    ({"learning_rate": "0.1"}, TypeError),
    ({"n_estimators": 0}, ValueError),
    ({"min_child_weight": 0}, ValueError),
    ({"min_split_gain": -1.0}, ValueError),
    ({"threads_per_block": 48}, ValueError),
    ({"rows_per_thread": 17}, ValueError),
    ({"L2_reg": -1e-3}, ValueError),
    ({"colsample_bytree": 0.0}, ValueError),
    ({"colsample_bytree": 1.01}, ValueError),
])
def test_hyperparameter_validation(kw, exc):
    with pytest.raises(exc):
        WarpGBM(**kw)


def test_constructor_needs_no_gpu():
    m = WarpGBM(num_bins=32, max_depth=5)
    assert m.forest == [{} for _ in range(100)] and not m._is_fitted


@pytest.mark.parametrize("args,exc,msg", [
    (([[1.0]], np.zeros(1)), TypeError, "numpy arrays"),
    ((np.zeros(3), np.zeros(3)), ValueError, "2-dimensional"),
    ((np.zeros((3, 2)), np.zeros((3, 1))), ValueError, "1-dimensional"),
    ((np.zeros((3, 2)), np.zeros(4)), ValueError, "same number of rows"),
])
def test_fit_argument_validation(args, exc, msg):
    with pytest.raises(exc, match=msg):
        WarpGBM().fit(*args)


def test_fit_era_and_eval_validation():
    X, y = np.zeros((4, 2)), np.zeros(4)
    with pytest.raises(TypeError, match="era_id must be a numpy array"):
        WarpGBM().fit(X, y, era_id=[0, 0, 1, 1])
    with pytest.raises(ValueError, match="same length"):
        WarpGBM().fit(X, y, era_id=np.zeros(3))
    with pytest.raises(ValueError, match="must all be defined"):
        WarpGBM().fit(X, y, X_eval=X)
    with pytest.raises(ValueError, match="eval_every_n_trees"):
        WarpGBM().fit(X, y, X_eval=X, y_eval=y, eval_every_n_trees=0)
    with pytest.raises(ValueError, match="early_stopping_rounds"):
        WarpGBM().fit(X, y, X_eval=X, y_eval=y, eval_every_n_trees=1, early_stopping_rounds=-2)
    with pytest.raises(ValueError, match="Invalid eval_metric"):
        WarpGBM().fit(X, y, X_eval=X, y_eval=y, eval_every_n_trees=1, eval_metric="auc")


def test_binary_requires_two_classes():
    with pytest.raises(ValueError, match="exactly 2 classes"):
        WarpGBM(objective="binary").fit(np.zeros((6, 2)), np.array([0, 1, 2, 0, 1, 2]))


def test_unfitted_errors():
    m = WarpGBM()
    with pytest.raises(ValueError, match="predict_proba only available"):
        m.predict_proba(np.zeros((2, 2)))
    with pytest.raises(ValueError, match="Cannot save unfitted"):
        m.save_model("/tmp/never.pkl")
    with pytest.raises(ValueError, match="not been fitted"):
        m.get_feature_importance()
    with pytest.raises(ValueError, match="not been fitted"):
        m.get_per_era_feature_importance()


def test_heap_dict_round_trip_and_preorder():
    tree = {"feature": 3, "bin": 5,
            "left": {"feature": 1, "bin": 0, "left": {"leaf_value": 1.5, "samples": 2},
                     "right": {"leaf_value": -0.25, "samples": 3}},
            "right": {"leaf_value": 2.0, "samples": 7}}
    H = 7
    f, b, v = _dict_to_heap(tree, H)
    assert f.tolist() == [3, 1, -1, -1, -1, -1, -1]
    cnt = np.array([12, 5, 7, 2, 3, 0, 0])
    back = _heaps_to_dicts(np.asarray(f)[None], np.asarray(b)[None], np.asarray(v)[None],
                           cnt[None])
    assert back == [tree]
    assert _preorder_heap(7).tolist() == [0, 1, 3, 4, 2, 5, 6]

    # complete heaps (computed level by level) against a depth-first walk,
    # and heaps that are not complete
    def walk(H):
        out, stack = [], [0]
        while stack:
            h = stack.pop()
            if h < H:
                out.append(h)
                stack += [2 * h + 2, 2 * h + 1]
        return out

    for H in [1, 3, 15, 63, 1023, 4095, 2, 6, 100]:
        assert _preorder_heap(H).tolist() == walk(H), H

    def internal(feat):
        return [int(h) for h in _preorder_heap(len(feat)) if feat[h] >= 0]

    assert internal([3, 1, 2, -1, -1, -1, -1]) == [0, 1, 2]
    # engine records mark nodes below a leaf as absent (-2)
    feat = [0, -1, 4, -2, -2, -1, -1]
    assert internal(feat) == [0, 2]
    second = {"feature": 0, "bin": 2, "left": {"leaf_value": 1.0, "samples": 4},
              "right": {"feature": 4, "bin": 1, "left": {"leaf_value": -3.5, "samples": 4},
                        "right": {"leaf_value": 2.0, "samples": 1}}}
    # several records in one call ([rounds, trees, H]), an all-absent one included
    fs = np.array([[f, feat], [[-2] * 7, f]], np.int32)
    bs = np.array([[b, [2, 0, 1, 0, 0, 0, 0]], [[0] * 7, b]], np.int32)
    vs = np.array([[v, [0.0, 1.0, 0.0, 0.0, 0.0, -3.5, 2.0]], [[0.0] * 7, v]], np.float32)
    cs = np.array([[cnt, [9, 4, 5, 0, 0, 4, 1]], [[0] * 7, cnt]], np.int64)
    assert _heaps_to_dicts(fs, bs, vs, cs) == [tree, second, None, tree]


def test_heap_of_tensor_features():
    """Trees the reference's fit wrote hold a split's feature as a 0-d int64
    tensor (warpgbm/core.py:653-654): the heap tables and the flat predict
    table take them as the integers they hold."""
    import torch

    plain = {"feature": 7, "bin": 2,
             "left": {"leaf_value": 0.5, "samples": 3},
             "right": {"feature": 1, "bin": 0, "left": {"leaf_value": -1.0, "samples": 2},
                       "right": {"leaf_value": 2.5, "samples": 1}}}
    tens = {"feature": torch.tensor(7), "bin": 2,
            "left": {"leaf_value": 0.5, "samples": 3},
            "right": {"feature": torch.tensor(1), "bin": 0,
                      "left": {"leaf_value": -1.0, "samples": 2},
                      "right": {"leaf_value": 2.5, "samples": 1}}}
    for a, b in zip(_dict_to_heap(tens, 7), _dict_to_heap(plain, 7)):
        assert np.array_equal(a, b)
    fa, fb = WarpGBM().flatten_tree(tens, 8), WarpGBM().flatten_tree(plain, 8)
    assert torch.allclose(fa, fb, rtol=0, atol=0, equal_nan=True)


def test_flatten_tree_matches_reference_layout():
    tree = {"feature": 3, "bin": 5, "left": {"leaf_value": 1.5, "samples": 2},
            "right": {"feature": 0, "bin": 1, "left": {"leaf_value": 0.5, "samples": 1},
                      "right": {"leaf_value": -1.0, "samples": 1}}}
    flat = WarpGBM().flatten_tree(tree, 8).numpy()
    assert flat[0, :5].tolist() == [3, 5, 1, 2, 0]
    assert flat[1, 4:].tolist() == [1.0, 1.5]
    assert flat[2, :5].tolist() == [0, 1, 3, 4, 0]
    assert np.isnan(flat[5:]).all()


def test_era_layout_matches_unique_sort():
    """The era bookkeeping (warpgbm/core.py:493 and :540: era ids cast to
    int32, then sorted unique eras, inverse indices, stable era order,
    offsets) equals torch's own cast + torch.unique followed by a stable
    argsort, including the linear path for non-decreasing era ids."""
    import torch

    from warpgbm_amd import device as D

    def by_sort(era):
        t = torch.from_numpy(np.asarray(era)).type(torch.int32)
        uniq, inv = torch.unique(t, sorted=True, return_inverse=True)
        uniq = uniq.numpy()
        inv = inv.numpy().astype(np.int32).reshape(-1)
        order = np.argsort(inv, kind="stable").astype(np.int32)
        counts = np.bincount(inv, minlength=len(uniq)).astype(np.int64)
        start = np.zeros(len(uniq) + 1, dtype=np.int64)
        np.cumsum(counts, out=start[1:])
        return uniq, inv, order, start

    rng = np.random.default_rng(0)
    cases = [np.ones(10, np.int32), np.repeat(np.arange(5), 7), np.array([3]),
             np.repeat([-2, 0, 5, 9], [1, 4, 2, 3]), rng.integers(0, 4, 50),
             np.sort(rng.integers(0, 9, 100)), np.array([1.5, 1.5, 2.0]), np.array([2, 2, 1, 1]),
             np.array([1.2, 1.7, 0.4, -0.6, 2.9]), np.array([2**32 + 5, 5, -1], np.int64),
             np.array([True, False, True]), rng.integers(0, 3, 40).astype(np.uint8)]
    for era in cases:
        got, ref = D.era_layout(era), by_sort(era)
        for a, b in zip(got, ref):
            assert np.array_equal(a, b) and a.dtype == b.dtype, era
    # the reference's float -> int32 truncation: 1.2 and 1.7 are one era
    assert len(D.era_layout(np.array([1.2, 1.7]))[0]) == 1
    # int64 ids wrap to 32 bits as in torch: 2^32 + 5 and 5 are one era
    assert len(D.era_layout(np.array([2**32 + 5, 5], np.int64))[0]) == 1
    # torch.from_numpy refuses strings, as the reference's fit does
    with pytest.raises(TypeError):
        D.era_layout(np.array(["a", "b"]))


def test_oracle_era_cast_matches_torch():
    """The oracle's era cast (numpy C cast) equals torch's .type(torch.int32)
    (warpgbm/core.py:493) on floats, wide and unsigned integers and bools."""
    import torch

    from oracle import gbm

    rng = np.random.default_rng(1)
    for era in (rng.standard_normal(200) * 50, np.array([1.2, 1.7, -0.5, -1.9]),
                rng.integers(-2**40, 2**40, 100), rng.integers(0, 200, 64).astype(np.uint8),
                np.array([True, False]), rng.integers(0, 9, 30).astype(np.int16)):
        want = torch.from_numpy(np.asarray(era)).type(torch.int32).numpy()
        assert np.array_equal(gbm.era_ids_int32(era), want), era.dtype


def test_heaps_to_dicts_random_records():
    """The C tree builder against a recursive walk of the heap records on
    random trees of depth 1-8: absent roots (None), absent children of a
    split (None), NaN leaves, counts beyond 32 bits, and leaves below a leaf
    (ignored)."""
    rng = np.random.default_rng(3)

    def walk(f, b, v, c, h):
        if h >= len(f) or f[h] < -1:
            return None
        if f[h] == -1:
            return {"leaf_value": float(v[h]), "samples": int(c[h])}
        return {"feature": int(f[h]), "bin": int(b[h]), "left": walk(f, b, v, c, 2 * h + 1),
                "right": walk(f, b, v, c, 2 * h + 2)}

    for D in (1, 3, 6, 8):
        H = (1 << (D + 1)) - 1
        M = 60
        feat = rng.choice([-2, -1, 0, 5, 77], size=(M, H), p=[0.2, 0.3, 0.2, 0.2, 0.1])
        feat = feat.astype(np.int32)
        feat[:, (H - 1) // 2:] = np.minimum(feat[:, (H - 1) // 2:], -1)  # no split at depth D
        bin_ = rng.integers(-5, 127, (M, H)).astype(np.int32)
        leaf = rng.standard_normal((M, H)).astype(np.float32)
        leaf[rng.random((M, H)) < 0.05] = np.nan
        cnt = rng.integers(0, 2**40, (M, H)).astype(np.int64)
        got = _heaps_to_dicts(feat.reshape(3, M // 3, H), bin_.reshape(3, M // 3, H),
                              leaf.reshape(3, M // 3, H), cnt.reshape(3, M // 3, H))
        want = [walk(feat[t], bin_[t], leaf[t], cnt[t], 0) for t in range(M)]
        # repr: NaN leaves compare equal as text; key order is the reference's
        assert repr(got) == repr(want), D
    with pytest.raises(ValueError, match="no child slots"):
        _heaps_to_dicts(np.array([[-1, 2, -1]], np.int32), np.zeros((1, 3), np.int32),
                        np.zeros((1, 3), np.float32), np.zeros((1, 3), np.int64))
    from warpgbm_amd import _trees
    with pytest.raises(ValueError, match="different lengths"):
        _trees.heaps_to_dicts(np.zeros(7, np.int32), np.zeros(7, np.int32),
                              np.zeros(6, np.float32), np.zeros(7, np.int64), 7)
    with pytest.raises(TypeError):
        _trees.heaps_to_dicts(np.zeros(7, np.int64), np.zeros(7, np.int32),
                              np.zeros(7, np.float32), np.zeros(7, np.int64), 7)
