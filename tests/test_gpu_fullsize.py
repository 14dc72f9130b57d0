"""Parity at the benchmark's full sizes, against the oracle's C loops.

C2: root and 16-node histograms of 1,000,000 x 1,000 int8 codes, bit-exact
(exact integer sums, one float32 rounding), plus size-independent invariants:
every feature counts every row, and the 16 nodes add up to the root exactly.
C3 (1M x 1000 float32, 32 bins, depth 5, 100 trees, lr 0.01): quantile edges
and codes bit-exact, all 100 trees identical to the oracle's recursive growth
(in four chunks of 25 trees: a chunk starts from the training scores of the
trees before it, which equal the oracle's when those trees are identical),
and the predictions of all 100 trees on the training rows and on 1M held-out
rows bit-exact against the oracle's traversal of the fitted forest.
C4 (500k x 2000 pre-binned, 500 eras, depth 8): two trees grown by the oracle
here, and all 100 trees, the per-era importance and the training predictions
against the digests of the oracle's forest committed in
tests/golden/c4_forest_digest.json (made by tests/golden/make_c4_digest.py).
C5 (200k x 100, 10 classes, depth 6, 200 rounds): edges, codes and all 200
rounds (2000 trees, four chunks of 50 rounds) identical; predict_proba of all
2000 trees on 1M rows bit-exact against the oracle's traversal + uniform
prior + softmax.
"""
import numpy as np
import pytest
import torch

from bench import c2_inputs, c3_inputs, c4_inputs, c5_inputs
from oracle import clib, gbm, ops
from tests.conftest import print_case
from warpgbm_amd import WarpGBM, _lib
from warpgbm_amd import device as D

pytestmark = pytest.mark.gpu
F32 = np.float32


def bits(a):
    return np.asarray(a, dtype=F32).view(np.uint32)


def test_c2_full_size_histograms_bit_exact(gpu):
    """Both code layouts: raw int8 codes (flags 0, padding -1) and the native
    layout the benchmark and the engine use (flags WGBM_CODES_NATIVE, made by
    the pre-binned copy)."""
    print_case("fullsize", "C2 root + 16 nodes, 1M x 1000")
    N, F, B = 1_000_000, 1000, 32
    dev = torch.device("cuda:0")
    codes_h, grad, node = c2_inputs(N, F)
    S = D.codes_stride(F)
    raw = torch.full((N, S), -1, dtype=torch.int8, device=dev)
    raw[:, :F] = torch.from_numpy(codes_h).to(dev)
    native = D.codes_from_int8(torch.from_numpy(codes_h).to(dev), False, B)[0]
    assert native.stride == S
    grad_d = torch.from_numpy(grad).to(dev)
    order = np.argsort(node, kind="stable").astype(np.int32)
    seg = np.zeros(17, np.int64)
    seg[1:] = np.cumsum(np.bincount(node, minlength=16))
    order_d, seg_d = torch.from_numpy(order).to(dev), torch.from_numpy(seg).to(dev)
    seg1 = torch.tensor([0, N], dtype=torch.int64, device=dev)
    s = ops.shift_from_absmax(np.max(np.abs(grad)), ops.qbits_for_rows(N))
    q = ops.quantise(grad, s)
    feats = np.arange(F)
    Q, C = clib.hist_exact_q(codes_h, q, None, feats, None, 1, B)
    assert np.all(C[0].sum(axis=1) == N)  # every feature counts every row
    node_ref = [clib.hist_exact_q(codes_h, q, order[seg[k]:seg[k + 1]], feats, None, 1, B)
                for k in range(16)]
    lib = _lib.load()
    st = _lib.current_stream_ptr(dev)
    for name, codes, flags in (("raw", raw, 0), ("native", native.rm, _lib.CODES_NATIVE)):
        print_case("fullsize", "C2", name)
        G1 = torch.zeros((1, F, B), device=dev)
        H1 = torch.zeros_like(G1)
        G16 = torch.zeros((16, F, B), device=dev)
        H16 = torch.zeros_like(G16)
        _lib.check(lib.wgbm_histogram_segments(codes.data_ptr(), N, S, F, grad_d.data_ptr(), None,
                                               seg1.data_ptr(), 1, N, B, flags, G1.data_ptr(),
                                               H1.data_ptr(), st), "root")
        _lib.check(lib.wgbm_histogram_segments(codes.data_ptr(), N, S, F, grad_d.data_ptr(),
                                               order_d.data_ptr(), seg_d.data_ptr(), 16, N, B,
                                               flags, G16.data_ptr(), H16.data_ptr(), st),
                   "16 nodes")
        torch.cuda.synchronize()
        assert np.array_equal(H1.cpu().numpy()[0], C[0].astype(F32)), name
        assert np.array_equal(bits(G1.cpu().numpy()[0]), bits(ops.dequantise(Q[0], s))), name
        H16c, G16c = H16.cpu().numpy(), G16.cpu().numpy()
        Qsum = np.zeros_like(Q[0])
        Csum = np.zeros_like(C[0])
        for k in range(16):
            Qk, Ck = node_ref[k]
            assert np.array_equal(H16c[k], Ck[0].astype(F32)), f"{name} node {k} counts"
            assert np.array_equal(bits(G16c[k]), bits(ops.dequantise(Qk[0], s))), \
                f"{name} node {k} sums"
            Qsum += Qk[0]
            Csum += Ck[0]
        # nodes add up to the root
        assert np.array_equal(Qsum, Q[0]) and np.array_equal(Csum, C[0])
    del raw, native, grad_d, order_d, seg_d
    torch.cuda.empty_cache()


def _leaf_rows(node):
    if "leaf_value" in node:
        return node["samples"]
    return _leaf_rows(node["left"]) + _leaf_rows(node["right"])


def _gpu_codes(m, X):
    """The codes fit bins X to: the library's binner with the model's edges."""
    Xd = D.upload_float(X, torch.device("cuda:0"))
    c = D.bin_matrix(Xd, torch.as_tensor(m.bin_edges), with_cm=False)
    out = c.rm[:, :X.shape[1]].cpu().numpy()
    del Xd, c
    return out


def _tables(trees, max_depth):
    return np.stack([ops.flatten_tree(t, 2 ** (max_depth + 1)) for t in trees])


@pytest.fixture(scope="module")
def c3_fit(gpu):
    print_case("fullsize", "C3 fit 1M x 1000, 100 trees depth 5")
    X, y = c3_inputs(1_000_000, 1000, 0)
    m = WarpGBM(num_bins=32, max_depth=5, n_estimators=100, learning_rate=0.01)
    m.fit(X, y)
    edges = clib.quantile_edges_matrix(X, 32)
    codes = clib.bin_matrix(X, edges)
    return X, y, m, edges, codes


def test_c3_full_size_edges_and_codes(c3_fit):
    X, y, m, edges, codes = c3_fit
    print_case("fullsize", "C3 edges, codes")
    assert np.array_equal(bits(torch.as_tensor(m.bin_edges).cpu().numpy()), bits(edges))
    assert np.array_equal(_gpu_codes(m, X), codes)
    assert m.base_prediction == float(gbm.base_score(y))


def _grow_chunk(codes, targets, start, era, E, kw, n, on_tree):
    """Grow n trees (or rounds) with the oracle from the scores `start`:
    regression (targets = y, start [N]) or softmax (targets = labels, start
    [N, K]), in the arithmetic of gbm.Forest.fit_codes; on_tree(i, trees)
    after each."""
    N, F = codes.shape
    qbits = ops.qbits_for_rows(N)
    rows = np.arange(N)
    scores = np.array(start, dtype=F32, copy=True)

    def grower():
        return gbm.TreeGrower(codes, era, E, kw["num_bins"], kw["max_depth"],
                              kw.get("min_child_weight", 20), kw.get("min_split_gain", 0.0),
                              kw.get("L2_reg", 1e-6), np.arange(F), qbits,
                              clib.hist_exact_q, clib.split_scan_q)

    lr = F32(kw["learning_rate"])
    for i in range(n):
        if scores.ndim == 1:
            g = grower()
            tree = g.grow(np.asarray(targets, F32) - scores, rows)
            for rws, v in g.leaf_rows:
                scores[rws] = scores[rws] + lr * v
            on_tree(i, tree)
        else:
            res = gbm.softmax_residuals(scores, targets)
            trees = []
            for k in range(scores.shape[1]):
                g = grower()
                trees.append(g.grow(res[k], rows))
                for rws, v in g.leaf_rows:
                    scores[rws, k] = scores[rws, k] + lr * v
            on_tree(i, trees)
    return scores


C3_KW = dict(num_bins=32, max_depth=5, learning_rate=0.01)


@pytest.mark.parametrize("chunk", range(4))
def test_c3_full_size_all_trees_identical(c3_fit, chunk):
    """Trees 25*chunk .. 25*chunk + 24 against the oracle, grown from the
    training scores of the GPU's trees before them."""
    X, y, m, edges, codes = c3_fit
    t0 = 25 * chunk
    print_case("fullsize", "C3 trees", t0, "to", t0 + 24)
    base = np.full(len(y), F32(m.base_prediction), F32)
    start = base if t0 == 0 else clib.predict_tables(codes, _tables(m.forest[:t0], 5), 0.01, base)

    def check(i, tree):
        assert m.forest[t0 + i] == tree, f"tree {t0 + i} differs"
        assert _leaf_rows(tree) == len(y)

    _grow_chunk(codes, y, start, np.zeros(len(y), np.int64), 1, C3_KW, 25, check)


def test_c3_full_size_predictions_bit_exact(c3_fit):
    X, y, m, edges, codes = c3_fit
    print_case("fullsize", "C3 predictions, training rows and 1M held-out rows")
    tabs = _tables(m.forest, 5)
    base = np.full(len(y), np.float32(m.base_prediction), F32)
    want = clib.predict_tables(codes, tabs, 0.01, base)
    assert np.array_equal(bits(m.predict(X)), bits(want))
    Xt, yt = c3_inputs(1_000_000, 1000, 1)
    got = m.predict(Xt)
    want_t = clib.predict_tables(clib.bin_matrix(Xt, edges), tabs, 0.01, base)
    assert np.array_equal(bits(got), bits(want_t))
    assert np.corrcoef(got, yt)[0, 1] > 0.7


def test_c4_full_size_depth8_bit_exact(gpu):
    print_case("fullsize", "C4 500k x 2000, 500 eras, 2 trees depth 8")
    X, y, era = c4_inputs()
    kw = dict(num_bins=5, max_depth=8, n_estimators=2, learning_rate=0.1)
    m = WarpGBM(**kw).fit(X, y, era_id=era)
    ref = gbm.Forest(**kw).fit_codes(X, y, era_id=era, hist=clib.hist_exact_q,
                                     scan=clib.split_scan_q)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
        assert _leaf_rows(a) == len(y)  # every row in one leaf
    assert np.array_equal(bits(m.per_era_feature_importance_), bits(ref.imp))


def test_c4_full_size_100_trees_against_digests(gpu):
    """The benchmark's whole C4 forest: every tree's digest (structure,
    features, bins, leaf counts, leaf value bits), the per-era importance and
    the training predictions against the oracle's, committed as a fixture."""
    import json
    from pathlib import Path

    from tests.golden.forest_digest import array_digest, tree_digest

    print_case("fullsize", "C4 100 trees depth 8 against the oracle's digests")
    fixture = Path(__file__).parent / "golden" / "c4_forest_digest.json"
    if not fixture.exists():
        pytest.skip("tests/golden/c4_forest_digest.json not generated "
                    "(python tests/golden/make_c4_digest.py)")
    ref = json.loads(fixture.read_text())
    X, y, era = c4_inputs()
    m = WarpGBM(num_bins=5, max_depth=8, n_estimators=100, learning_rate=0.1)
    m.fit(X, y, era_id=era)
    got = [tree_digest(t) for t in m.forest]
    bad = [i for i, (a, b) in enumerate(zip(got, ref["trees"])) if a != b]
    assert len(got) == len(ref["trees"]) == 100 and not bad, f"trees differ: {bad[:10]}"
    assert array_digest(m.per_era_feature_importance_) == ref["per_era_importance"]
    assert array_digest(m.predict(X)) == ref["train_preds"]


def test_native_codes_beyond_2gib_bit_exact(gpu):
    """2.2M x 1000 pre-binned codes: the native matrix (2.2M x 1024 bytes)
    is past 2^31 bytes, so the histogram tile kernel loads codes with 64-bit
    global addresses (kLoadGlobalAligned, 4 codes per lane) instead of 32-bit
    buffer offsets; one tree of depth 3 against the oracle, and its training
    predictions."""
    print_case("fullsize", "2.2M x 1000 pre-binned, native codes beyond 2 GiB")
    rng = np.random.default_rng(7)
    N, F, B = 2_200_000, 1000, 32
    X = rng.integers(0, B, (N, F), dtype=np.int8)
    y = ((X[:, 3] > 15) + 0.5 * (X[:, 700] > 20) + 0.1 * rng.standard_normal(N)).astype(F32)
    assert N * D.codes_stride(F) >= 2**31
    kw = dict(num_bins=B, max_depth=3, n_estimators=1, learning_rate=0.5)
    m = WarpGBM(**kw).fit(X, y)
    ref = gbm.Forest(**kw).fit_codes(X, y, hist=clib.hist_exact_q, scan=clib.split_scan_q)
    assert m.forest[0] == ref.forest[0]
    assert str(ref.forest[0]).count("'feature'") == 7  # a full tree of depth 3
    assert np.array_equal(bits(m.predict(X)), bits(ref.predict_codes(X)))
    del X
    torch.cuda.empty_cache()


C5_KW = dict(objective="multiclass", num_bins=32, max_depth=6, learning_rate=0.1)


@pytest.fixture(scope="module")
def c5_fit(gpu):
    print_case("fullsize", "C5 fit 200k x 100, K=10, depth 6, 200 rounds")
    X, lab = c5_inputs()
    m = WarpGBM(n_estimators=200, **C5_KW).fit(X, lab)
    edges = clib.quantile_edges_matrix(X, 32)
    codes = clib.bin_matrix(X, edges)
    return X, lab, m, edges, codes


def test_c5_full_size_edges_and_codes(c5_fit):
    X, lab, m, edges, codes = c5_fit
    print_case("fullsize", "C5 edges, codes")
    assert np.array_equal(bits(torch.as_tensor(m.bin_edges).cpu().numpy()), bits(edges))
    assert np.array_equal(_gpu_codes(m, X), codes)


def _class_tables(rounds):
    trees = [t for rnd in rounds for t in rnd]
    cls = np.tile(np.arange(10, dtype=np.int32), len(rounds))
    return _tables(trees, 6), cls


@pytest.mark.parametrize("chunk", range(4))
def test_c5_full_size_all_rounds_identical(c5_fit, chunk):
    """Rounds 50*chunk .. 50*chunk + 49 (10 class trees each) against the
    oracle, grown from the training scores of the GPU's rounds before them
    (the training priors, then every earlier tree in round and class order)."""
    X, lab, m, edges, codes = c5_fit
    r0 = 50 * chunk
    print_case("fullsize", "C5 rounds", r0, "to", r0 + 49)
    start = np.tile(gbm.class_prior_logits(lab, 10), (len(lab), 1)).astype(F32)
    if r0:
        tabs, cls = _class_tables(m.forest[:r0])
        start = clib.predict_tables(codes, tabs, 0.1, start, cls)

    def check(i, trees):
        assert m.forest[r0 + i] == trees, f"round {r0 + i} differs"

    _grow_chunk(codes, lab, start, np.zeros(len(lab), np.int64), 1, C5_KW, 50, check)


def test_c5_full_size_predict_proba_bit_exact(c5_fit):
    X, lab, m, edges, codes = c5_fit
    print_case("fullsize", "C5 predict_proba on 1M rows")
    Xt, lt = c5_inputs(rows_per_class=100_000, seed=1)
    got = m.predict_proba(Xt)
    tabs, cls = _class_tables(m.forest)
    start = np.tile(gbm.uniform_prior_logits(10), (len(lt), 1))
    logits = clib.predict_tables(clib.bin_matrix(Xt, edges), tabs, 0.1, start, cls)
    assert np.array_equal(bits(got), bits(clib.softmax_rows(logits)))
    assert (got.argmax(axis=1) == lt).mean() > 0.95
