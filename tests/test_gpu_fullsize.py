"""Parity at the benchmark's full sizes, against the oracle's C loops.

C2: root and 16-node histograms of 1,000,000 x 1,000 int8 codes, bit-exact
(exact integer sums, one float32 rounding), plus size-independent invariants:
every feature counts every row, and the 16 nodes add up to the root exactly.
C4: 500,000 x 2,000 pre-binned codes with 500 eras (the benchmark's own
inputs), two trees of depth 2 grown by the direct era path, tree for tree and
importance bit for bit equal to the oracle's recursive growth."""
import numpy as np
import pytest
import torch

from bench import c2_inputs, c4_inputs
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


def test_c4_full_size_first_levels_bit_exact(gpu):
    print_case("fullsize", "C4 500k x 2000, 500 eras, 2 trees depth 2")
    X, y, era = c4_inputs()
    kw = dict(num_bins=5, max_depth=2, n_estimators=2, learning_rate=0.5)
    m = WarpGBM(**kw).fit(X, y, era_id=era)
    ref = gbm.Forest(**kw).fit_codes(X, y, era_id=era, hist=clib.hist_exact_q)
    for i, (a, b) in enumerate(zip(m.forest, ref.forest)):
        assert a == b, f"tree {i} differs"
    assert np.array_equal(bits(m.per_era_feature_importance_), bits(ref.imp))

    def leaf_rows(node):
        if "leaf_value" in node:
            return node["samples"]
        return leaf_rows(node["left"]) + leaf_rows(node["right"])

    assert all(leaf_rows(tree) == len(y) for tree in m.forest)  # every row in one leaf
