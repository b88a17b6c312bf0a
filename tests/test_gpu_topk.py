"""GPU parity of fast_topk (engine/kernels/topk.py:17-46) against the CPU
oracle, which restates the same lane-sweep algorithm: values and indices must
be identical (integer/selection work: bit-exact)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from starter_amd import kernels as K
from tests._util import BF16, bits, randn_bf16

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("N,V,k", [(16, 151936, 8), (64, 151936, 4), (128, 151936, 8), (3, 1000, 8), (5, 2048, 1),
                                   (2, 7, 7), (4, 151935, 16)])
def test_topk_matches_oracle(N, V, k):
    g = torch.Generator().manual_seed(N * V + k)
    L = randn_bf16((N, V), 2.0, g)
    if V > 5000:   # collisions, ties and a -inf column
        L[0, 5000] = 40.0
        L[0, 5000 + 2048] = 39.0
        L[1, 10] = L[1, 4000] = 41.0
        L[2, 3] = float("-inf")
    vals, idxs = K.fast_topk(L.to(DEV), k)
    ov, oi = oracle.topk(bits(L), k)
    assert np.array_equal(idxs.cpu().numpy(), oi)
    assert np.array_equal(vals.cpu().numpy(), ov)
    assert torch.equal(idxs[:, 0].cpu().long(), torch.argmax(L, -1))


def test_topk_odd_stride_rows():
    """Unaligned rows take the scalar load path and give the same result."""
    g = torch.Generator().manual_seed(3)
    big = randn_bf16((6, 3001), 1.0, g)
    L = big[:, 1:2990]        # row stride 3001, first column unaligned
    vals, idxs = K.fast_topk(big.to(DEV)[:, 1:2990], 6)
    ov, oi = oracle.topk(bits(L.contiguous()), 6)
    assert np.array_equal(idxs.cpu().numpy(), oi) and np.array_equal(vals.cpu().numpy(), ov)
