"""warpgbm.cuda.node_kernel served by warpgbm_amd.node_kernel, so the
reference's `from warpgbm.cuda import node_kernel` (warpgbm/core.py:7)
resolves to this library.  A stand-in package layout (empty __init__ files
in a temporary directory) plays the reference's package; nothing of the
reference is read."""
import importlib
import sys

import pytest


@pytest.fixture
def fake_reference_package(tmp_path, monkeypatch):
    pkg = tmp_path / "warpgbm"
    (pkg / "cuda").mkdir(parents=True)
    (pkg / "__init__.py").write_text("")
    (pkg / "cuda" / "__init__.py").write_text("")
    monkeypatch.syspath_prepend(str(tmp_path))
    saved = {k: v for k, v in sys.modules.items() if k == "warpgbm" or k.startswith("warpgbm.")}
    for k in saved:
        del sys.modules[k]
    yield
    for k in [k for k in sys.modules if k == "warpgbm" or k.startswith("warpgbm.")]:
        del sys.modules[k]
    sys.modules.update(saved)


@pytest.mark.parametrize("parent_first", [False, True])
def test_reference_import_resolves_to_library(fake_reference_package, parent_first):
    from warpgbm_amd import node_kernel

    if parent_first:
        importlib.import_module("warpgbm.cuda")
    node_kernel.install_as_reference_module()
    ns = {}
    exec("from warpgbm.cuda import node_kernel as nk", ns)
    assert ns["nk"] is node_kernel
    for name in ("compute_histogram3", "compute_split", "custom_cuda_binner", "predict_forest"):
        assert callable(getattr(ns["nk"], name))
