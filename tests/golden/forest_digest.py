"""Canonical digests of fitted trees, for comparing a forest with a committed
fixture (tests/golden/c4_forest_digest.json) instead of regrowing it.

A tree's digest is the SHA-256 of its nested dict written in pre-order as
text: a split as ``S<feature>,<bin>(<left><right>)``, a leaf as
``L<float32 bits of leaf_value in hex>,<samples>``.  Two trees have equal
digests exactly when their structure, split features and bins, leaf sample
counts and leaf values (bit for bit) are equal.
"""
from __future__ import annotations

import hashlib

import numpy as np


def tree_text(node) -> str:
    if "leaf_value" in node:
        bits = np.float32(node["leaf_value"]).view(np.uint32)
        return f"L{int(bits):08x},{int(node['samples'])}"
    return (f"S{int(node['feature'])},{int(node['bin'])}("
            + tree_text(node["left"]) + tree_text(node["right"]) + ")")


def tree_digest(node) -> str:
    return hashlib.sha256(tree_text(node).encode()).hexdigest()


def array_digest(a) -> str:
    """SHA-256 of a float32 array's bits (C order)."""
    return hashlib.sha256(np.ascontiguousarray(a, dtype=np.float32).tobytes()).hexdigest()
