"""warpgbm_amd: WarpGBM's histogram / DES split / binning / inference hot path
as hand-written HIP kernels for AMD Instinct MI355X (gfx950).

``from warpgbm_amd import WarpGBM`` gives the reference's estimator API;
``warpgbm_amd.node_kernel`` mirrors the reference's native op module.
"""
from .core import WarpGBM

__all__ = ["WarpGBM"]
__version__ = "0.1.0"
