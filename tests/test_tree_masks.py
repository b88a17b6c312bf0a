"""Draft-tree ancestor masks (kernels.ancestor_masks), on the CPU.

The masks are the tree attention's input format (bit j of node i set when j
is i or one of i's ancestors; engine/kernels/attention.py:245-254).  They are
checked against the transitive closure of the parent relation computed as a
boolean matrix power, on random trees up to the full 64 nodes (node 63 sets
the int64 sign bit), a chain and the verify template the benchmark uses.
"""

from __future__ import annotations

import numpy as np
import pytest

from starter_amd import kernels as K


def _closure_masks(parent: list[int]) -> list[int]:
    n = len(parent)
    a = np.eye(n, dtype=bool)                 # reflexive
    for i, p in enumerate(parent):
        if p >= 0:
            a[i, p] = True                    # i -> its parent
    for _ in range(7):                        # paths of up to 2^7 > 64 steps
        a = (a.astype(np.int64) @ a.astype(np.int64)) > 0
    out = []
    for i in range(n):
        m = sum(1 << j for j in range(n) if a[i, j])
        out.append(m - (1 << 64) if m >= 1 << 63 else m)
    return out


@pytest.mark.parametrize("seed", range(12))
def test_masks_equal_the_closure_of_the_parent_relation(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 65)) if seed < 10 else 64
    parent = [-1] + [int(rng.integers(-1, i)) if seed % 3 == 0 else int(rng.integers(0, i)) for i in range(1, n)]
    assert K.ancestor_masks(parent) == _closure_masks(parent)


def test_chain_and_template():
    chain = [t - 1 for t in range(64)]
    m = K.ancestor_masks(chain)
    assert m[0] == 1 and m[5] == 0b111111 and m[63] == -1     # all 64 bits: -1 as int64
    assert K.ancestor_masks([-1, 0, 0, 1, 0, 2, 1, 0]) == [1, 3, 5, 11, 17, 37, 67, 129]


@pytest.mark.parametrize("parent", [[0], [-1, 1], [-1, 2, 0], [-2]])
def test_rejects_parents_after_their_children(parent):
    with pytest.raises(ValueError):
        K.ancestor_masks(parent)


def test_rejects_more_than_64_nodes():
    with pytest.raises(ValueError):
        K.ancestor_masks([t - 1 for t in range(65)])
