"""GPU parity of the reference-compatible ops (warpgbm_amd.node_kernel, i.e.
the C ABI) and the batched entry points against the CPU oracle.

Bar: bit-exact for codes, counts, histogram sums (the oracle reproduces the
library's exact-sum arithmetic), split gains/directions and predictions; the
literal float32 restatement of the reference histogram (sequential atomics)
agrees within the float32 accumulation bound, stated in the test."""
import math
import zlib

import numpy as np
import pytest
import torch

from oracle import clib, ops
from tests.conftest import print_case
from warpgbm_amd import _lib
from warpgbm_amd import device as D
from warpgbm_amd import node_kernel

pytestmark = pytest.mark.gpu
F32 = np.float32
dev = torch.device("cuda:0")


def t(a, dtype=None):
    x = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        x = x.to(dtype)
    return x.to(dev)


def bits(a):
    return np.asarray(a, dtype=F32).view(np.uint32)


HIST_CASES = [
    # name, N, Fm, B, E, n_rows_used, n_feats_used, code range
    ("c1_like_unaligned_stride", 10000, 50, 32, 1, None, None, (0, 32)),
    ("gathered_subset_negative_codes", 20000, 64, 32, 1, 7000, 40, (-3, 36)),
    ("eras_3", 12000, 48, 16, 3, 9000, 48, (0, 16)),
    ("eras_500_small_bins", 30000, 40, 5, 500, None, None, (0, 5)),
    ("b2", 5000, 33, 2, 1, None, None, (-1, 3)),
    ("b33_v16_edge", 6000, 100, 33, 2, 4000, 100, (0, 33)),
    ("b34_v8", 6000, 100, 34, 1, None, None, (0, 34)),
    ("b67_v8_edge", 4000, 70, 67, 1, None, 55, (0, 67)),
    ("b68_v4", 4000, 70, 68, 1, None, None, (-5, 70)),
    ("b127", 8000, 130, 127, 2, None, None, (-128, 127)),
    ("wide_1000", 60000, 1000, 32, 1, 50000, 1000, (0, 32)),
]


@pytest.mark.parametrize("case", HIST_CASES, ids=[c[0] for c in HIST_CASES])
def test_compute_histogram3_bit_exact(gpu, case):
    name, N, Fm, B, E, nr, nf, (lo, hi) = case
    print_case("compute_histogram3", name)
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    codes = rng.integers(lo, hi, (N, Fm)).astype(np.int8)
    resid = (rng.standard_normal(N) * np.exp(rng.uniform(-3, 2, N))).astype(F32)
    rows = np.arange(N) if nr is None else np.sort(rng.choice(N, nr, replace=False))
    feats = np.arange(Fm) if nf is None else rng.permutation(Fm)[:nf]
    era = rng.integers(0, E, N).astype(np.int32)
    G = torch.zeros((E, len(feats), B), device=dev)
    H = torch.zeros_like(G)
    node_kernel.compute_histogram3(t(codes), t(resid), t(rows, torch.int32),
                                   t(feats, torch.int32), t(era), G, H, B, 64, 4)
    Gr, Hr = ops.histogram_exact(codes, resid, rows, feats, era, E, B)
    assert np.array_equal(H.cpu().numpy(), Hr)
    assert np.array_equal(bits(G.cpu().numpy()), bits(Gr))
    if N * len(feats) <= 2_000_000:
        # the literal reference restatement (float32 atomics in row order)
        Gs, Hs = ops.histogram_f32_seq(codes, resid, rows, feats, era, E, B)
        assert np.array_equal(Hs, Hr)
        absum = np.zeros_like(Gs, dtype=np.float64)
        rws = rows
        es = era[rws] if E > 1 else np.zeros(len(rws), np.int64)
        for fi, f in enumerate(feats):
            b = codes[rws, f].astype(np.int64)
            ok = (b >= 0) & (b < B)
            np.add.at(absum[:, fi, :], (es[ok], b[ok]), np.abs(resid[rws[ok]]).astype(np.float64))
        # |float32 sequential sum - true sum| <= count * 2^-24 * sum|r| (bound used
        # with 2^-23); the library's sum is the true sum of residuals rounded to
        # multiples of 2^-s (error <= count * 2^-(s+1), s from max|r| of the call)
        # plus one final float32 rounding
        # (s from max|r| of the call, or of the era's rows with several eras)
        qb = ops.qbits_for_rows(len(rows))
        if E == 1:
            s = np.array([ops.shift_from_absmax(np.max(np.abs(resid[rows])), qb)])
        else:
            s = np.array([ops.key_shift(m, qb)
                          for m in ops.era_absmax(resid, rows, era, E)])
        s = s.reshape(-1, 1, 1).astype(np.float64)
        Gc = G.cpu().numpy()
        tol = (Hs.astype(np.float64) * 2.0**-23 * absum + Hs.astype(np.float64) * 2.0**(-s - 1)
               + np.spacing(np.abs(Gc)).astype(np.float64))
        assert np.all(np.abs(Gc.astype(np.float64) - Gs) <= tol)


def _feats(kind, Fm, rng):
    if kind == "sorted_run":          # aligned run: one V-byte load per row
        return np.arange(100, 612)
    if kind == "unaligned_run":       # consecutive but not V-aligned: byte loads
        return np.arange(101, 613)
    if kind == "reversed":
        return np.arange(Fm)[::-1].copy()
    if kind == "dups":                # repeated indices: each output gets the column
        f = rng.permutation(Fm)[:60]
        return np.concatenate([f, f[:17], f[5:9]])
    if kind == "identity":
        return np.arange(Fm)
    return rng.permutation(Fm)[:int(kind)]


FMAP_CASES = [
    # name, N, Fm, B, E, feature choice
    ("sorted_run", 20000, 1000, 32, 1, "sorted_run"),
    ("unaligned_run", 20000, 1000, 32, 1, "unaligned_run"),
    ("half_random_c2_like", 30000, 1000, 32, 1, "500"),
    ("reversed", 12000, 203, 32, 1, "reversed"),
    ("dups", 12000, 203, 17, 2, "dups"),
    ("bytes_mode_identity", 9000, 131, 32, 1, "identity"),
    ("bytes_mode_subset", 9000, 131, 32, 1, "100"),
    ("eras_40_subset", 20000, 64, 16, 40, "30"),
    ("eras_9000_two_windows", 30000, 8, 4, 9000, "identity"),
]


@pytest.mark.parametrize("case", FMAP_CASES, ids=[c[0] for c in FMAP_CASES])
def test_compute_histogram3_feature_maps(gpu, case):
    """Feature indices in any order, with repeats, runs and random subsets:
    only the selected columns are histogrammed and every output o receives
    column feature_indices[o]; eras regrouped in LDS windows (E > 8192 takes
    two).  Bit-exact against the oracle."""
    name, N, Fm, B, E, kind = case
    print_case("compute_histogram3 feature map", name)
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    codes = rng.integers(-2, B + 2, (N, Fm)).astype(np.int8)
    resid = rng.standard_normal(N).astype(F32)
    rows = np.sort(rng.choice(N, N * 3 // 4, replace=False))
    feats = _feats(kind, Fm, rng)
    era = rng.integers(0, E, N).astype(np.int32)
    G = torch.zeros((E, len(feats), B), device=dev)
    H = torch.zeros_like(G)
    node_kernel.compute_histogram3(t(codes), t(resid), t(rows, torch.int32),
                                   t(feats, torch.int32), t(era), G, H, B)
    Gr, Hr = ops.histogram_exact(codes, resid, rows, feats, era, E, B)
    assert np.array_equal(H.cpu().numpy(), Hr)
    assert np.array_equal(bits(G.cpu().numpy()), bits(Gr))


def test_compute_histogram3_out_of_range_features(gpu):
    """Feature indices outside [0, n_feats) (which the reference would read
    out of bounds) contribute nothing: those outputs keep their values; the
    others are exact."""
    print_case("compute_histogram3", "out-of-range feature indices")
    rng = np.random.default_rng(11)
    N, Fm, B = 6000, 70, 8
    codes = rng.integers(0, B, (N, Fm)).astype(np.int8)
    resid = rng.standard_normal(N).astype(F32)
    feats = np.array([3, -1, 69, 70, 5, 1 << 20, 3, -(1 << 30)], np.int64)
    valid = (feats >= 0) & (feats < Fm)
    era = np.zeros(N, np.int32)
    G = torch.full((1, len(feats), B), 7.0, device=dev)
    H = torch.full((1, len(feats), B), 7.0, device=dev)
    node_kernel.compute_histogram3(t(codes), t(resid), t(np.arange(N), torch.int32),
                                   t(feats, torch.int32), t(era), G, H, B)
    Gr, Hr = ops.histogram_exact(codes, resid, np.arange(N), feats[valid], era, 1, B)
    Gc, Hc = G.cpu().numpy(), H.cpu().numpy()
    assert np.all(Gc[:, ~valid] == 7.0) and np.all(Hc[:, ~valid] == 7.0)
    assert np.array_equal(Hc[:, valid], Hr + F32(7.0))
    assert np.array_equal(bits(Gc[:, valid]), bits(Gr + F32(7.0)))


@pytest.mark.parametrize("scale", [1e9, 1e12, 1e30])
def test_compute_histogram3_huge_residuals(gpu, scale):
    """Residuals of magnitude 2^qbits and above give a negative shift (the
    sums are kept in units of 2^-s > 1); the tile kernel must quantise with
    that shift, not clamp it to 0."""
    print_case("compute_histogram3", "huge residuals", scale)
    rng = np.random.default_rng(int(math.log10(scale)))
    N, Fm, B, E = 9000, 40, 16, 2
    codes = rng.integers(-1, B + 1, (N, Fm)).astype(np.int8)
    resid = (rng.standard_normal(N) * scale).astype(F32)
    rows = np.sort(rng.choice(N, 7000, replace=False))
    feats = rng.permutation(Fm)[:31]
    era = rng.integers(0, E, N).astype(np.int32)
    s = ops.shift_from_absmax(np.max(np.abs(resid[rows])), ops.qbits_for_rows(len(rows)))
    assert s < 0
    G = torch.zeros((E, len(feats), B), device=dev)
    H = torch.zeros_like(G)
    node_kernel.compute_histogram3(t(codes), t(resid), t(rows, torch.int32),
                                   t(feats, torch.int32), t(era), G, H, B)
    Gr, Hr = ops.histogram_exact(codes, resid, rows, feats, era, E, B)
    assert np.array_equal(H.cpu().numpy(), Hr)
    assert np.array_equal(bits(G.cpu().numpy()), bits(Gr))


def test_compute_histogram3_accumulates_and_handles_empty(gpu):
    print_case("compute_histogram3", "accumulate/empty")
    rng = np.random.default_rng(1)
    N, Fm, B = 3000, 20, 8
    codes = rng.integers(0, B, (N, Fm)).astype(np.int8)
    resid = rng.standard_normal(N).astype(F32)
    era = np.zeros(N, np.int32)
    feats = np.arange(Fm)
    G = torch.full((1, Fm, B), 2.5, device=dev)
    H = torch.full((1, Fm, B), 1.0, device=dev)
    node_kernel.compute_histogram3(t(codes), t(resid), t(np.arange(0), torch.int32),
                                   t(feats, torch.int32), t(era), G, H, B)
    assert torch.all(G == 2.5) and torch.all(H == 1.0)
    node_kernel.compute_histogram3(t(codes), t(resid), t(np.arange(N), torch.int32),
                                   t(feats, torch.int32), t(era), G, H, B)
    Gr, Hr = ops.histogram_exact(codes, resid, np.arange(N), feats, era, 1, B)
    assert np.array_equal(bits(G.cpu().numpy()), bits(Gr + F32(2.5)))
    assert np.array_equal(H.cpu().numpy(), Hr + F32(1.0))


def test_compute_histogram3_rejects_bad_input(gpu):
    codes = torch.zeros((10, 4), dtype=torch.int8, device=dev)
    r = torch.zeros(10, device=dev)
    rows = torch.arange(10, dtype=torch.int32, device=dev)
    feats = torch.arange(4, dtype=torch.int32, device=dev)
    era = torch.zeros(10, dtype=torch.int32, device=dev)
    G = torch.zeros((1, 4, 8), device=dev)
    with pytest.raises(RuntimeError, match="dtype"):
        node_kernel.compute_histogram3(codes, r.double(), rows, feats, era, G, G.clone(), 8)
    with pytest.raises(RuntimeError, match="num_bins"):
        node_kernel.compute_histogram3(codes, r, rows, feats, era, G, G.clone(), 9)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        node_kernel.compute_histogram3(codes.cpu(), r, rows, feats, era, G, G.clone(), 8)


@pytest.mark.parametrize("E,F,B", [(1, 300, 32), (4, 50, 2), (7, 33, 17), (13, 157, 5),
                                   (1, 5, 127), (2, 70, 33)])
def test_compute_split_bit_exact(gpu, E, F, B):
    """Per-era gains and directions of best_split_kernel.cu:61-88 for 2 to
    127 bins, including pair counts that leave the last workgroup partly
    empty (300, 200, 231, 2041, 140 pairs)."""
    print_case("compute_split", E, F, B)
    rng = np.random.default_rng(E * 1000 + F)
    H = rng.integers(0, 60, (E, F, B)).astype(F32)
    H[:, ::7, :] = 0  # masked features
    G = (rng.standard_normal((E, F, B)) * np.sqrt(H + 1)).astype(F32)
    ge = torch.empty((E, F, B - 1), device=dev)
    de = torch.empty_like(ge)
    node_kernel.compute_split(t(G), t(H), 0.0, 20, 1e-6, ge, de, 128)
    gr, dr = ops.split_scan(G, H, 20, 1e-6)
    assert np.array_equal(bits(ge.cpu().numpy()), bits(gr))
    assert np.array_equal(de.cpu().numpy(), dr)


def test_custom_cuda_binner_bit_exact(gpu):
    print_case("custom_cuda_binner")
    rng = np.random.default_rng(3)
    x = rng.standard_normal(100003).astype(F32)
    x[::101] = np.nan
    x[7::997] = np.inf
    x[11::991] = -np.inf
    for edges in (np.sort(rng.standard_normal(31)).astype(F32), rng.standard_normal(9).astype(F32),
                  np.full(5, np.nan, F32), np.zeros(0, F32),
                  np.sort(rng.standard_normal(126)).astype(F32)):
        x[:len(edges)] = edges
        out = torch.empty(len(x), dtype=torch.int8, device=dev)
        node_kernel.custom_cuda_binner(t(x), t(edges), out)
        assert np.array_equal(out.cpu().numpy(), ops.bin_column(x, edges))


def _random_tree(rng, depth, max_depth, F, B):
    if depth == max_depth or rng.random() < 0.2:
        return {"leaf_value": float(F32(rng.standard_normal())), "samples": 1}
    return {"feature": int(rng.integers(F)), "bin": int(rng.integers(-1, B)),
            "left": _random_tree(rng, depth + 1, max_depth, F, B),
            "right": _random_tree(rng, depth + 1, max_depth, F, B)}


def test_predict_forest_bit_exact(gpu):
    print_case("predict_forest")
    rng = np.random.default_rng(4)
    N, F, B, D_ = 20000, 37, 16, 6
    codes = rng.integers(-2, B, (N, F)).astype(np.int8)
    trees = [_random_tree(rng, 0, D_, F, B) for _ in range(25)]
    table = np.stack([ops.flatten_tree(tr, 2 ** (D_ + 1)) for tr in trees])
    out = torch.full((N,), 0.75, device=dev)
    node_kernel.predict_forest(t(codes), t(table), 0.1, out)
    ref = ops.predict_table(codes, table, 0.1, np.full(N, F32(0.75)))
    assert np.array_equal(bits(out.cpu().numpy()), bits(ref))


def _chain_tree(rng, depth, F, B):
    """A split at every level down one side: depth `depth` in 2*depth + 1 nodes."""
    if depth == 0:
        return {"leaf_value": float(F32(rng.standard_normal())), "samples": 1}
    return {"feature": int(rng.integers(F)), "bin": int(rng.integers(0, B)),
            "left": {"leaf_value": float(F32(rng.standard_normal())), "samples": 1},
            "right": _chain_tree(rng, depth - 1, F, B)}


@pytest.mark.parametrize("F", [296, 300])
@pytest.mark.parametrize("case", ["plain", "big_bins", "bad_nodes", "deep", "neg_bin", "few"])
def test_predict_forest_heap_path_bit_exact(gpu, case, F):
    """predict_forest with enough trees and rows takes the heap path (flat
    tables -> heap tables, then the LDS predictor over the raw codes when
    rows are a multiple of 8 bytes (F = 296), or over a native copy of the
    codes (F = 300)); tables it cannot hold fall back to the flat walk on the
    device.  Every case against the oracle's flat walk
    (warpgbm/cuda/predict.cu:13-44):
    * plain: depth-5 trees in 64-slot tables, codes -128..127 (negative codes
      go left at every split, 127 right at every bin <= 126);
    * big_bins: split bins 127..300 (every int8 code goes left);
    * bad_nodes: features outside [0, F) and child indices outside [0, M)
      (the flat walk's NaN), which the heap holds as NaN leaves;
    * deep: one tree deeper than its table's heap (fallback);
    * neg_bin: a negative split bin (fallback);
    * few: fewer trees than the heap path takes (the flat walk alone)."""
    print_case("predict_forest heap path", case, F)
    rng = np.random.default_rng(20 + len(case) + F)
    N, B, D_ = 9000, 32, 5
    M = 2 ** (D_ + 1)
    codes = rng.integers(-3, B + 2, (N, F)).astype(np.int8)
    codes[rng.random((N, F)) < 0.01] = 127
    codes[rng.random((N, F)) < 0.01] = -128
    T = 3 if case == "few" else 40
    trees = [_random_tree(rng, 0, D_, F, B) for _ in range(T)]
    for tr in trees:  # bins in [0, B): _random_tree draws -1 too
        stack = [tr]
        while stack:
            nd = stack.pop()
            if "feature" in nd:
                nd["bin"] = max(nd["bin"], 0)
                stack += [nd["left"], nd["right"]]
    if case == "deep":
        trees[7] = _chain_tree(rng, D_ + 3, F, B)
    table = np.stack([ops.flatten_tree(tr, M) for tr in trees])
    splits = np.argwhere(table[:, :, 4] == 0)
    if case == "big_bins":
        pick = splits[rng.random(len(splits)) < 0.2]
        table[pick[:, 0], pick[:, 1], 1] = rng.integers(127, 301, len(pick))
    if case == "bad_nodes":
        pick = splits[rng.random(len(splits)) < 0.05]
        table[pick[:, 0], pick[:, 1], 0] = F + 5
        pick = splits[rng.random(len(splits)) < 0.05]
        table[pick[:, 0], pick[:, 1], 2] = M + 3
        pick = splits[rng.random(len(splits)) < 0.05]
        table[pick[:, 0], pick[:, 1], 3] = -1
    if case == "neg_bin":
        table[splits[0][0], splits[0][1], 1] = -1
    out = torch.full((N,), 0.25, device=dev)
    node_kernel.predict_forest(t(codes), t(table), 0.1, out)
    ref = ops.predict_table(codes, table, 0.1, np.full(N, F32(0.25)))
    got = out.cpu().numpy()
    assert np.array_equal(bits(got), bits(ref))
    if case == "bad_nodes":
        assert np.isnan(ref).any()
    if case == "plain":
        # the same codes at an address that is not 8-byte aligned: the raw
        # read does not apply, the native copy does
        buf = torch.empty(N * F + 4, dtype=torch.int8, device=dev)
        cod = buf[4:].view(N, F)
        cod.copy_(t(codes))
        assert cod.data_ptr() % 8 == 4 and cod.is_contiguous()
        out2 = torch.full((N,), 0.25, device=dev)
        node_kernel.predict_forest(cod, t(table), 0.1, out2)
        assert np.array_equal(bits(out2.cpu().numpy()), bits(ref))


def _random_heap(rng, R, K, depth, F, B):
    """R rounds x K heap-ordered trees (node h: children 2h+1, 2h+2; feat -1
    = leaf) of depth <= ``depth``, with garbage below every leaf (the
    predictors must never read it) and the reference table of each tree."""
    H = (1 << (depth + 1)) - 1
    feat = rng.integers(-1, F, (R, K, H)).astype(np.int32)   # garbage everywhere first
    binv = rng.integers(0, B - 1, (R, K, H)).astype(np.int32)
    leaf = rng.standard_normal((R, K, H)).astype(F32)
    tables = np.zeros((R * K, H, 6), F32)
    for r in range(R):
        for k in range(K):
            f, b, lv, tb = feat[r, k], binv[r, k], leaf[r, k], tables[r * K + k]
            stack = [(0, 0)]
            while stack:
                h, d = stack.pop()
                if d == depth or rng.random() < 0.25:
                    f[h] = -1
                    tb[h] = (0, 0, 0, 0, 1, lv[h])
                else:
                    f[h] = rng.integers(F)
                    tb[h] = (f[h], b[h], 2 * h + 1, 2 * h + 2, 0, 0)
                    stack += [(2 * h + 1, d + 1), (2 * h + 2, d + 1)]
    return feat, binv, leaf, tables


# name, rows, features, bins, classes, rounds, depth: the LDS-resident
# predictor (also with single-leaf trees and blocks of 9 rows), the row-block
# predictor (partial last tree chunk and row block, deep trees, one round
# per tree chunk) and the heap walker
PRED_CASES = [
    ("resident", 5000, 40, 16, 1, 30, 5),
    ("rows_partial_chunk", 7001, 100, 32, 10, 23, 6),
    ("rows_deep", 3000, 20, 8, 1, 50, 9),
    ("rows_one_round_per_chunk", 2000, 30, 8, 3, 4, 10),
    ("resident_depth0", 500, 10, 4, 10, 200, 0),
    ("heap", 3000, 30, 8, 10, 3, 10),
    ("heap_depth0", 500, 10, 4, 10, 2000, 0),
]


@pytest.mark.parametrize("case", PRED_CASES, ids=[c[0] for c in PRED_CASES])
def test_predict_heap_paths_bit_exact(gpu, case):
    """wgbm_predict_heap (the estimator's predictor) on raw codes with values
    outside [0, B) equals the reference-table walk (warpgbm/cuda/predict.cu:
    23-44, trees added in (round, class) order) bit for bit, whichever of its
    three kernels the shape selects."""
    name, N, F, B, K, R, depth = case
    print_case("predict_heap", name)
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    raw = rng.integers(-2, B + 3, (N, F)).astype(np.int8)
    feat, binv, leaf, tables = _random_heap(rng, R, K, depth, F, B)
    out0 = rng.standard_normal((N, K)).astype(F32)
    codes = D.codes_from_int8(D.upload_int8(raw, dev), False, B)[0]
    out = t(out0)
    D.predict_heap(codes, t(feat), t(binv), t(leaf), R, K, depth, 0.1, out)
    cls = np.tile(np.arange(K, dtype=np.int32), R)
    ref = clib.predict_tables(raw, tables, F32(0.1), out0, cls)
    assert np.array_equal(bits(out.cpu().numpy()), bits(ref))


def native_layout(raw, num_bins, stride):
    """The library's native row-major code layout (include/warpgbm_amd.h):
    codes in [0, B) as is, negative codes B, codes >= B and padding B + 1."""
    n, F = raw.shape
    out = np.full((n, stride), num_bins + 1, np.int16)
    r = raw.astype(np.int16)
    out[:, :F] = np.where(r < 0, num_bins, np.where(r >= num_bins, num_bins + 1, r))
    return out.astype(np.uint8).view(np.int8)


@pytest.mark.parametrize("B,F", [(32, 203), (5, 203), (50, 203), (126, 203), (127, 203),
                                 (32, 1000), (50, 700), (32, 100), (5, 60)])
@pytest.mark.parametrize("native", [False, True])
def test_histogram_segments_bit_exact(gpu, native, B, F):
    """16 node segments of raw codes with values outside [0, B) (negative and
    >= B: skipped, histogram_kernel.cu:41), through the raw-code kernel and
    through the native layout made by the pre-binned copy; both equal the
    oracle on the raw codes.  B = 127 has no native-layout kernel (its rows
    would not fit a byte) and takes the clamping one.  The wide cases (16
    segments x 16 or more feature planes) take the plane finalize; 100 and 60
    features take two and one feature per lane."""
    print_case("histogram_segments", "16 nodes", "native" if native else "raw", B, F)
    rng = np.random.default_rng(5 + B + F)
    N, S = 40000, 16
    stride = D.codes_stride(F)
    raw = rng.integers(-3, B + 3, (N, F)).astype(np.int8)
    resid = rng.standard_normal(N).astype(F32)
    node = rng.integers(0, S, N)
    order = np.argsort(node, kind="stable").astype(np.int32)
    seg = np.zeros(S + 1, np.int64)
    seg[1:] = np.cumsum(np.bincount(node, minlength=S))
    G = torch.zeros((S, F, B), device=dev)
    H = torch.zeros_like(G)
    from warpgbm_amd import _lib

    lib = _lib.load()
    if native:
        c = D.codes_from_int8(t(raw), False, B)[0]
        assert np.array_equal(c.rm.cpu().numpy(), native_layout(raw, B, stride))
        codes_d, flags = c.rm, _lib.CODES_NATIVE
    else:
        padded = np.full((N, stride), -1, np.int8)
        padded[:, :F] = raw
        codes_d, flags = t(padded), 0
    # keep the device tensors alive until the asynchronous call has run
    resid_d, order_d, seg_d = t(resid), t(order), t(seg)
    rc = lib.wgbm_histogram_segments(codes_d.data_ptr(), N, stride, F, resid_d.data_ptr(),
                                     order_d.data_ptr(), seg_d.data_ptr(), S, N, B, flags,
                                     G.data_ptr(), H.data_ptr(),
                                     _lib.current_stream_ptr(dev))
    _lib.check(rc, "histogram_segments")
    torch.cuda.synchronize()
    Gr, Hr = ops.histogram_segments_exact(raw, resid, order, seg, np.arange(F), B)
    Gc, Hc = G.cpu().numpy(), H.cpu().numpy()
    assert np.array_equal(Hc, Hr)
    assert np.array_equal(bits(Gc), bits(Gr))


def _rel_ok(G, codes, r, rows, key_of_row, n_keys, feats, B, skip_key):
    """|G - float64 sum| <= 1e-5 * sum|r| for every (key, feature, bin) but
    skip_key's (the key of the outlier)."""
    kr = key_of_row[rows]
    for fi, f in enumerate(feats):
        b = codes[rows, f].astype(np.int64)
        ok = (b >= 0) & (b < B)
        idx = kr[ok] * B + b[ok]
        true = np.bincount(idx, weights=r[rows[ok]].astype(np.float64), minlength=n_keys * B)
        absum = np.bincount(idx, weights=np.abs(r[rows[ok]]).astype(np.float64),
                            minlength=n_keys * B)
        err = np.abs(G[:, fi, :].reshape(-1).astype(np.float64) - true)
        keep = np.repeat(np.arange(n_keys) != skip_key, B)
        assert np.all(err[keep] <= 1e-5 * absum[keep])


def test_compute_histogram3_era_outlier(gpu):
    """A 1e6 residual in era 0 next to eras of 1e-3 residuals: each era is
    quantised at the shift of its own largest |r|, so the small eras' sums
    hold to 1e-5 of their bins' sum of |r| (bit-exact against the oracle)."""
    print_case("compute_histogram3", "era outlier")
    rng = np.random.default_rng(31)
    N, Fm, B, E = 30000, 64, 16, 5
    codes = rng.integers(-1, B + 1, (N, Fm)).astype(np.int8)
    era = rng.integers(0, E, N).astype(np.int32)
    resid = (1e-3 * rng.standard_normal(N)).astype(F32)
    big = np.flatnonzero(era == 0)[:3]
    resid[big] = F32(1e6) * np.array([1, -1, 0.5], F32)
    rows = np.sort(rng.choice(N, 25000, replace=False))
    rows = np.union1d(rows, big)
    feats = rng.permutation(Fm)[:50]
    G = torch.zeros((E, len(feats), B), device=dev)
    H = torch.zeros_like(G)
    node_kernel.compute_histogram3(t(codes), t(resid), t(rows, torch.int32),
                                   t(feats, torch.int32), t(era), G, H, B)
    Gr, Hr = ops.histogram_exact(codes, resid, rows, feats, era, E, B)
    Gc = G.cpu().numpy()
    assert np.array_equal(H.cpu().numpy(), Hr)
    assert np.array_equal(bits(Gc), bits(Gr))
    _rel_ok(Gc, codes, resid, rows, era.astype(np.int64), E, feats, B, skip_key=0)


def test_histogram_segments_segment_outlier(gpu):
    """Segments: a 1e6 residual in segment 2 leaves the other segments'
    sums of 1e-3 residuals at their own scale (1e-5 of sum|r| per bin), and
    the no-allocation entry point gives the same bits."""
    print_case("histogram_segments", "segment outlier")
    rng = np.random.default_rng(32)
    N, F, B, S = 40000, 203, 32, 16
    stride = D.codes_stride(F)
    raw = rng.integers(-2, B + 2, (N, F)).astype(np.int8)
    resid = (1e-3 * rng.standard_normal(N)).astype(F32)
    node = rng.integers(0, S, N)
    resid[np.flatnonzero(node == 2)[:2]] = F32(1e6)
    order = np.argsort(node, kind="stable").astype(np.int32)
    seg = np.zeros(S + 1, np.int64)
    seg[1:] = np.cumsum(np.bincount(node, minlength=S))
    padded = np.full((N, stride), -1, np.int8)
    padded[:, :F] = raw
    lib = _lib.load()
    codes_d, resid_d, order_d, seg_d = t(padded), t(resid), t(order), t(seg)
    out = []
    for fn in (lib.wgbm_histogram_segments, lib.wgbm_histogram_segments_noalloc):
        G = torch.zeros((S, F, B), device=dev)
        H = torch.zeros_like(G)
        rc = fn(codes_d.data_ptr(), N, stride, F, resid_d.data_ptr(), order_d.data_ptr(),
                seg_d.data_ptr(), S, N, B, 0, G.data_ptr(), H.data_ptr(),
                _lib.current_stream_ptr(dev))
        _lib.check(rc, "histogram_segments")
        torch.cuda.synchronize()
        out.append((G.cpu().numpy(), H.cpu().numpy()))
    Gr, Hr = ops.histogram_segments_exact(raw, resid, order, seg, np.arange(F), B)
    for Gc, Hc in out:
        assert np.array_equal(Hc, Hr)
        assert np.array_equal(bits(Gc), bits(Gr))
    _rel_ok(out[0][0], raw, resid, order.astype(np.int64), node, S, np.arange(F), B,
            skip_key=2)


@pytest.mark.parametrize("B", [32, 2, 127, 5, 100])
def test_quantile_edges_and_bin_matrix(gpu, B):
    print_case("quantile_edges/bin_matrix B", B)
    rng = np.random.default_rng(6)
    N, F = 20001, 70
    X = (rng.standard_normal((N, F)) * rng.uniform(0.01, 50, F)).astype(F32)
    # ties; + 0.0 turns the -0.0 of rounded small negatives into +0.0: the
    # radix selection orders -0.0 before +0.0 (as a radix sort does), while
    # torch's CPU comparison sort may leave them either way (equal keys), so
    # the torch cross-check below would see a zero of the other sign
    X[:, 3] = np.round(X[:, 3]) + F32(0.0)
    X[::997, 5] = np.nan          # NaN column -> all edges NaN -> all codes 0
    X[17, 9], X[18, 9] = np.inf, -np.inf  # +inf counts every edge (past the search's padding)
    Xd = D.upload_float(X, dev)
    edges = D.quantile_edges(Xd, B).cpu().numpy()
    ref_edges = ops.quantile_edges(X, B)
    assert np.array_equal(bits(edges), bits(ref_edges))
    ref_torch = torch.quantile(torch.from_numpy(X[:, :4]), torch.from_numpy(ops.quantile_levels(B)),
                               dim=0).numpy().T
    assert np.array_equal(bits(edges[:4]), bits(ref_torch))
    codes = D.bin_matrix(Xd, torch.from_numpy(edges), with_cm=True)
    rm = codes.rm.cpu().numpy()
    cm = codes.cm.cpu().numpy()
    ref = ops.bin_matrix(X, edges)
    assert np.array_equal(rm[:, :F], ref)
    assert np.all(rm[:, F:].view(np.uint8) == B + 1)  # native layout padding (byte B + 1)
    assert np.array_equal(cm, ref.T)
    assert np.all(ref[:, 5] == 0)


def test_copy_prebinned(gpu):
    print_case("copy_prebinned")
    rng = np.random.default_rng(7)
    X = rng.integers(-3, 5, (5000, 300)).astype(np.int64)
    c = D.upload_prebinned(X, dev, with_cm=True, num_bins=5)
    assert np.array_equal(c.rm.cpu().numpy(), native_layout(X.astype(np.int8), 5, c.stride))
    assert np.array_equal(c.cm.cpu().numpy(), X.astype(np.int8).T)  # raw codes
    # the in-pass "every value < num_bins" test, at and around the boundary,
    # against the host's column maxima (warpgbm/core.py:501-503)
    X8 = rng.integers(-128, 5, (70_001, 129)).astype(np.int8)
    x8 = D.upload_int8(X8, dev)
    for thr in (4, 5, 6, 127):
        c, over = D.codes_from_int8(x8, False, thr, check=True)
        assert over == (not np.all(X8.max(axis=0) < thr)), thr
        assert np.array_equal(c.rm.cpu().numpy(), native_layout(X8, thr, c.stride))
    X8[69_999, 128] = 17
    c, over = D.codes_from_int8(D.upload_int8(X8, dev), True, 17, check=True)
    assert over and np.array_equal(c.cm.cpu().numpy(), X8.T)
    c, over = D.codes_from_int8(D.upload_int8(X8, dev), True, 18, check=True)
    assert not over


@pytest.mark.parametrize("B", [2, 5, 32, 127])
def test_native_quantile_selection_bit_exact(gpu, B):
    """Radix-selection edges equal torch.quantile / the oracle for tiny columns,
    heavy ties, constant columns, NaN columns and many targets."""
    print_case("quantile_edges_matrix", B)
    rng = np.random.default_rng(B)
    cols = []
    for n in (1, 2, 3, 7, 64, 1000, 20011):
        X = np.empty((n, 6), F32)
        X[:, 0] = rng.standard_normal(n)
        X[:, 1] = rng.integers(-2, 3, n)                       # heavy ties
        X[:, 2] = 3.5                                          # constant
        X[:, 3] = (rng.standard_normal(n) * 1e-35)             # subnormal range
        X[:, 4] = np.abs(rng.standard_normal(n)) * 1e30        # large
        X[:, 5] = rng.standard_normal(n)
        if n > 5:
            X[n // 2, 5] = np.nan                              # NaN column -> all NaN
        Xd = D.upload_float(X, dev)
        got = D.quantile_edges(Xd, B).cpu().numpy()
        ref = ops.quantile_edges(X, B)
        assert np.array_equal(bits(got), bits(ref)), n
        tq = torch.quantile(torch.from_numpy(X[:, :5]), torch.from_numpy(ops.quantile_levels(B)),
                            dim=0).numpy().T
        assert np.array_equal(bits(got[:5]), bits(tq)), n
        # sorted-input entry point agrees too
        srt = torch.sort(Xd.t().contiguous(), dim=1).values
        got2 = D.quantile_edges_sorted(srt, B).cpu().numpy()
        assert np.array_equal(bits(got2[:5]), bits(ref[:5])), n


@pytest.mark.parametrize("B", [5, 32, 127])
def test_quantile_selection_value_buckets_bit_exact(gpu, B):
    """Columns large enough for the value-bucket first pass: smooth data (the
    target buckets go to the buffer), heavy ties and outliers that stretch
    the range (the buffer would overflow: radix over the whole column),
    infinities, a constant -0.0 column and a NaN column; all equal the
    oracle, and torch.quantile where no signed zero is involved."""
    print_case("quantile_edges value buckets", B)
    rng = np.random.default_rng(100 + B)
    n = 300_001
    X = np.empty((n, 9), F32)
    X[:, 0] = rng.standard_normal(n)
    X[:, 1] = rng.uniform(1.0, 2.0, n)
    X[:, 2] = rng.integers(0, 4, n)                  # heavy ties
    X[:, 3] = rng.standard_normal(n)
    X[7, 3] = 1e30                                   # outlier stretches the range
    X[:, 4] = rng.standard_normal(n)
    X[11, 4] = np.inf
    X[:, 5] = rng.standard_normal(n)
    X[13, 5] = -np.inf
    X[:, 6] = rng.exponential(1.0, n) ** 3           # heavy tail
    X[:, 7] = -0.0                                   # constant negative zero
    X[:, 8] = rng.standard_normal(n)
    X[n // 3, 8] = np.nan
    Xd = D.upload_float(X, dev)
    got = D.quantile_edges(Xd, B).cpu().numpy()
    ref = ops.quantile_edges(X, B)
    assert np.array_equal(bits(got), bits(ref))
    cols = [0, 1, 3, 4, 5, 6]
    tq = torch.quantile(torch.from_numpy(X[:, cols]), torch.from_numpy(ops.quantile_levels(B)),
                        dim=0).numpy().T
    assert np.array_equal(bits(got[cols]), bits(tq))


@pytest.mark.parametrize("B", [5, 32, 127])
def test_staged_quantile_edges_bit_exact(gpu, B):
    """Edges taken from columns staged block by block during the upload
    (upload_float_with_edges: several blocks, a ragged last one, float64
    input rounded while staging) equal those of the whole resident matrix and
    the oracle, with ties, outliers, infinities, a constant column and a NaN
    column; the device copy is X itself."""
    print_case("upload_float_with_edges", B)
    rng = np.random.default_rng(200 + B)
    n, F = 300_001, 12
    X = rng.standard_normal((n, F))                  # float64: rounded while staging
    X[:, 1] = rng.integers(0, 4, n)                  # heavy ties
    X[7, 2] = 1e30                                   # outlier stretches the range
    X[11, 3] = np.inf
    X[13, 4] = -np.inf
    X[:, 5] = 2.5                                    # constant
    X[n // 3, 6] = np.nan                            # NaN column -> NaN edges
    X[:, 7] = rng.exponential(1.0, n) ** 3           # heavy tail
    saved = D._STAGE_BYTES
    # the pinned staging buffers are allocated once at the current size:
    # dropped before and after, so that they are re-made at each size
    with D._stage_lock:
        D._stage_bufs.clear()
    try:
        D._STAGE_BYTES = 1 << 20                     # ~22 blocks of 21,824 rows
        assert D._streams(X, 4)
        Xd, got = D.upload_float_with_edges(X, dev, B)
    finally:
        D._STAGE_BYTES = saved
        torch.cuda.synchronize()
        with D._stage_lock:
            D._stage_bufs.clear()
    X32 = X.astype(F32)
    assert np.array_equal(bits(Xd.cpu().numpy()), bits(X32))  # NaN included
    whole = D.quantile_edges(D.upload_float(X32, dev), B).cpu().numpy()
    got = got.cpu().numpy()
    assert np.array_equal(bits(got), bits(whole))
    assert np.array_equal(bits(got), bits(ops.quantile_edges(X32, B)))


def test_staged_quantile_rows_validation(gpu):
    """The staging entry point refuses rows that do not start on a multiple
    of 4 or that run past the column stride (host checks, no launch)."""
    lib = _lib.load()
    X = torch.zeros((64, 3), dtype=torch.float32, device=dev)
    cols = torch.zeros((3, 64), dtype=torch.int32, device=dev)
    km = torch.zeros(6, dtype=torch.int32, device=dev)
    args = (X.data_ptr(), 8, 3, 3)
    tail = (cols.data_ptr(), 64, km.data_ptr(), km[3:].data_ptr(), None)
    assert lib.wgbm_quantile_stage_rows(*args, 2, *tail) != 0
    assert lib.wgbm_quantile_stage_rows(*args, 60, *tail) != 0
    assert lib.wgbm_quantile_stage_rows(*args, 56, *tail) == 0
    torch.cuda.synchronize()


def test_staged_upload_exact(gpu):
    """The pinned, multi-threaded upload reproduces X (float64 input rounded
    to float32) exactly, including a ragged last chunk."""
    print_case("upload_float")
    rng = np.random.default_rng(9)
    X = rng.standard_normal((300_001, 230))           # float64: converted while staging
    Xd = D.upload_float(X, dev)
    assert torch.equal(Xd.cpu(), torch.from_numpy(X.astype(np.float32)))
    X32 = rng.standard_normal((250_000, 300), dtype=np.float32)
    assert torch.equal(D.upload_float(X32, dev).cpu(), torch.from_numpy(X32))


def test_streamed_binning_exact(gpu):
    """Predict-time binning that bins each uploaded chunk as it lands
    (upload_and_bin) writes the same native codes as binning the whole
    uploaded matrix, over several chunks and a ragged last one, float64 input
    and NaN included."""
    print_case("upload_and_bin")
    rng = np.random.default_rng(10)
    n, F, B = 300_001, 230, 32
    X = rng.standard_normal((n, F))                   # float64: rounded while staging
    X[rng.random((n, F)) < 1e-4] = np.nan
    Xd = D.upload_float(X, dev)
    edges = D.quantile_edges(Xd, B)
    want = D.bin_matrix(Xd, edges, with_cm=False)
    got = D.upload_and_bin(X, edges, dev)
    assert got.stride == want.stride and got.num_bins == want.num_bins
    assert torch.equal(got.rm, want.rm)


def test_importance_add_in_node_order(gpu):
    """wgbm_importance_add equals np.add.at's one-by-one float32 adds (the
    reference's sequential per-node += at warpgbm/core.py:624-627), bit for
    bit, for repeated, single and absent features and values of mixed scale
    (large then tiny adds expose any reordering)."""
    print_case("importance_add")
    rng = np.random.default_rng(0)
    for trial in range(40):
        F, E, M = int(rng.integers(1, 30)), int(rng.integers(1, 7)), int(rng.integers(0, 300))
        idx = rng.integers(0, F, M) if trial % 3 else np.full(M, F - 1)
        val = (rng.standard_normal((M, E)) * 10.0 ** rng.integers(-8, 8, (M, 1))).astype(F32)
        acc0 = rng.standard_normal((E, F)).astype(F32)
        want = acc0.copy()
        np.add.at(want.T, idx, val)
        # gain rows stored shuffled; node lists the rows in add order by feature
        perm = rng.permutation(M)
        rows = np.empty((max(M, 1), E), F32)
        rows[perm] = val
        by_f = np.argsort(idx, kind="stable")
        fstart = np.searchsorted(idx[by_f], np.arange(F + 1)).astype(np.int64)
        acc = t(acc0)
        D.importance_add(acc, t(rows), t(perm[by_f].astype(np.int64)), t(fstart))
        assert np.array_equal(bits(acc.cpu().numpy()), bits(want)), trial


def test_lds_atomic_probe(gpu):
    """The instrumentation probe runs and reports a plausible whole-GPU rate
    of 64-bit LDS atomic adds (between 1e11 and 1e14 per second)."""
    import ctypes

    print_case("probe", "lds atomics")
    rate = ctypes.c_double(0.0)
    _lib.check(gpu.wgbm_probe_lds_atomics(64, 50, ctypes.byref(rate), _lib.current_stream_ptr()),
               "probe")
    assert 1e11 < rate.value < 1e14
