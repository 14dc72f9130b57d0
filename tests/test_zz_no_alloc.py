"""wgbm_histogram_segments_noalloc against wgbm_histogram_segments through the
C ABI: two calls in a row, the second with a smaller input, each bit-exact
against the allocating entry point on the same input; a call needing more
than the fixed scratch is rejected with the sizes in the error."""
import ctypes as C

import numpy as np
import pytest
import torch

from tests.conftest import print_case
from warpgbm_amd import _lib
from warpgbm_amd import device as D

pytestmark = pytest.mark.gpu
F32 = np.float32


def _case(seed, N, F, B, n_seg, native, dev):
    rng = np.random.default_rng(seed)
    codes_h = rng.integers(-1, B + 2, (N, F), dtype=np.int8)  # out-of-range codes too
    grad = torch.from_numpy(rng.standard_normal(N).astype(F32)).to(dev)
    node = rng.integers(0, n_seg, N)
    order = torch.from_numpy(np.argsort(node, kind="stable").astype(np.int32)).to(dev)
    seg = np.zeros(n_seg + 1, np.int64)
    seg[1:] = np.cumsum(np.bincount(node, minlength=n_seg))
    seg = torch.from_numpy(seg).to(dev)
    if native:
        c = D.codes_from_int8(torch.from_numpy(np.clip(codes_h, 0, B - 1)).to(dev), False, B)[0]
        codes, S, flags = c.rm, c.stride, _lib.CODES_NATIVE
    else:
        codes, S, flags = torch.from_numpy(codes_h).to(dev), F, 0
    return codes, S, flags, grad, order, seg


def _run(fn, lib, codes, N, S, F, grad, order, seg, n_seg, B, flags, st, dev):
    G = torch.zeros((n_seg, F, B), device=dev)
    H = torch.zeros_like(G)
    rc = fn(codes.data_ptr(), N, S, F, grad.data_ptr(), order.data_ptr(), seg.data_ptr(), n_seg,
            N, B, flags, G.data_ptr(), H.data_ptr(), st)
    _lib.check(rc, "histogram")
    torch.cuda.synchronize()
    return G.cpu().numpy(), H.cpu().numpy()


def test_noalloc_matches_allocating_entry_point(gpu):
    dev = torch.device("cuda:0")
    lib = _lib.load()
    st = _lib.current_stream_ptr(dev)
    # two calls in a row on the shared array, the second smaller
    for seed, N, F, B, n_seg, native in ((0, 300_000, 700, 32, 16, True),
                                         (1, 40_000, 90, 16, 5, False)):
        print_case("noalloc", "N F B segments native", N, F, B, n_seg, native)
        codes, S, flags, grad, order, seg = _case(seed, N, F, B, n_seg, native, dev)
        args = (codes, N, S, F, grad, order, seg, n_seg, B, flags, st, dev)
        Ga, Ha = _run(lib.wgbm_histogram_segments_noalloc, lib, *args)
        Gr, Hr = _run(lib.wgbm_histogram_segments, lib, *args)
        assert np.array_equal(Ga.view(np.uint32), Gr.view(np.uint32))
        assert np.array_equal(Ha, Hr)
        assert Ha.sum() > 0


def test_noalloc_rejects_calls_beyond_its_scratch(gpu):
    """300 segments of 1000 features need a tile of partials each (256 KiB
    at 32 bins), 75 MiB in all, more than the fixed array: the call is
    refused before any work, with both sizes in the message.  Every pointer
    is a real device buffer of the call's shape, so a size check that ran
    late would compute a histogram (and fail the return code check) rather
    than touch memory outside the buffers."""
    dev = torch.device("cuda:0")
    lib = _lib.load()
    st = _lib.current_stream_ptr(dev)
    N, F, B, n_seg = 600, 1000, 32, 300
    rng = np.random.default_rng(3)
    codes = torch.from_numpy(rng.integers(0, B, (N, F), dtype=np.int8)).to(dev)
    grad = torch.from_numpy(rng.standard_normal(N).astype(F32)).to(dev)
    order = torch.arange(N, dtype=torch.int32, device=dev)
    seg = torch.from_numpy(np.arange(n_seg + 1, dtype=np.int64) * 2).to(dev)
    G = torch.zeros((n_seg, F, B), device=dev)
    H = torch.zeros_like(G)
    rc = lib.wgbm_histogram_segments_noalloc(codes.data_ptr(), N, F, F, grad.data_ptr(),
                                             order.data_ptr(), seg.data_ptr(), n_seg, N, B, 0,
                                             G.data_ptr(), H.data_ptr(), st)
    torch.cuda.synchronize()
    assert rc == 1000
    msg = lib.wgbm_last_error().decode()
    assert "needs" in msg and str(64 * 1024 * 1024) in msg
    assert float(H.sum()) == 0.0  # nothing ran
