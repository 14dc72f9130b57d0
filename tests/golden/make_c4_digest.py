"""Writes tests/golden/c4_forest_digest.json: the oracle's 100-tree C4 forest
(benchmark config C4: 500,000 x 2,000 pre-binned int8 codes in {0..4}, 500
eras, num_bins 5, depth 8, lr 0.1; inputs from bench.c4_inputs, numpy
default_rng(0)), grown by oracle.gbm.Forest with the C loops, as per-tree
digests (forest_digest.tree_digest) plus digests of the per-era importance
and the training predictions.  tests/test_gpu_fullsize.py fits the same
forest on the GPU and compares every digest.

Runs on the CPU in this repository (about 30 minutes on 8 cores):
    python tests/golden/make_c4_digest.py
"""
from __future__ import annotations

import json
import sys
import time
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

from bench import c4_inputs  # noqa: E402
from oracle import clib, gbm  # noqa: E402
from tests.golden.forest_digest import array_digest, tree_digest  # noqa: E402

OUT = HERE / "c4_forest_digest.json"
C4_KW = dict(num_bins=5, max_depth=8, n_estimators=100, learning_rate=0.1)


def main():
    X, y, era = c4_inputs()
    t0 = time.time()

    def progress(i):
        print(f"tree {i + 1}/100 at {time.time() - t0:.0f} s", flush=True)

    f = gbm.Forest(**C4_KW).fit_codes(X, y, era_id=era, hist=clib.hist_exact_q,
                                      scan=clib.split_scan_q, progress=progress)
    out = {
        "config": "C4: bench.c4_inputs(), " + json.dumps(C4_KW),
        "trees": [tree_digest(t) for t in f.forest],
        "per_era_importance": array_digest(f.imp),
        "train_preds": array_digest(f.train_preds),
    }
    OUT.write_text(json.dumps(out, indent=1) + "\n")
    print("wrote", OUT, f"in {time.time() - t0:.0f} s")


if __name__ == "__main__":
    main()
