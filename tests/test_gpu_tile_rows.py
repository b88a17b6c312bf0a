"""GPU parity of ring-path tiles whose height is not a multiple of 16 (needs an MI355X).

A tile of the LDS-fed ring path covers ``rows`` weight rows (gate/up: that
many gate rows and as many up rows); slab rows past it load the zero line and
their MFMA rows are never read.  The host picks heights such as N / 256 so
every CU gets one tile (o_proj 10 rows, gate_up 38), and five 256-column chunks
per wave (ku 40) run K = 9728 without a global split.  Each epilogue is
checked against the CPU oracle with such tiles: plain store, split-K partials
and their finish, SwiGLU (with 2 and 3 slabs per half), gate/up partials and
the fused argmax, on the Qwen3-4B shapes and on a ragged N whose last tile is
partial.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from starter_amd import kernels as K
from starter_amd._lib import SK_PATH_MFMA_LDS, SkConfig
from tests._util import assert_gateup_parity, assert_parity, bits, check_argmax_rows, from_bits, randn_bf16

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _w(N, Kd, seed):
    return randn_bf16((N, Kd), 0.02, torch.Generator().manual_seed(seed))


def _x(M, Kd, seed):
    return randn_bf16((M, Kd), 1.0, torch.Generator().manual_seed(50_000 + seed + M))


def ring(waves, ku, rows, split=1, grid=0):
    return SkConfig.make(SK_PATH_MFMA_LDS, waves=waves, ku=ku, rows=rows, split=split, grid=grid)


GEMM_CASES = [
    # (N, K, config)
    (2560, 4096, ring(16, 8, 10)),           # o_proj: 256 tiles of 10 rows
    (2560, 4096, ring(16, 8, 12)),
    (2560, 4096, ring(16, 8, 11)),           # 2560 = 232 * 11 + 8: a partial last tile
    (2560, 4096, ring(4, 32, 12)),           # four chunks per wave
    (2560, 4096, ring(8, 8, 20, split=2)),   # two 16-row slabs, 4 rows of the second, split-K finish
    (6144, 2560, ring(10, 8, 24)),           # qkv: 256 tiles of 24 rows
    (6144, 2560, ring(10, 8, 26)),
    (2560, 9728, ring(8, 40, 12)),           # down: five chunks per wave, no global split
    (2560, 9728, ring(8, 40, 16)),
    (2560, 9728, ring(4, 40, 10, split=2)),  # five chunks per wave with a split
    (777, 2560, ring(10, 8, 7)),             # ragged N, 7-row tiles
    (777, 2560, ring(10, 8, 30, grid=9)),    # several tiles per workgroup
]


@pytest.mark.parametrize("case", GEMM_CASES, ids=lambda c: f"{c[0]}x{c[1]}-" + "-".join(
    f"{k}{v}" for k, v in c[2].as_dict().items()))
@pytest.mark.parametrize("M", [1, 5, 8, 16])
def test_gemm_tile_rows(case, M):
    N, Kd, cfg = case
    w, x = _w(N, Kd, N + Kd), _x(M, Kd, N)
    out = K.gemm(x.to(DEV), w.to(DEV), config=cfg)
    torch.cuda.synchronize()
    assert_parity(out, from_bits(oracle.gemm(bits(x), bits(w))), f"N={N} K={Kd} {cfg} M={M}")


GATEUP_CASES = [
    (9728, ring(10, 8, 38)),            # three slabs per half, 6 rows in the last
    (9728, ring(10, 8, 40)),
    (9728, ring(10, 8, 19)),            # two slabs per half
    (9728, ring(10, 8, 24)),
    (9728, ring(5, 8, 19, split=2)),    # gate and up partials, split-K finish
    (1000, ring(10, 8, 38, grid=8)),    # ragged I, several tiles per workgroup
]


@pytest.mark.parametrize("case", GATEUP_CASES, ids=lambda c: f"I{c[0]}-" + "-".join(
    f"{k}{v}" for k, v in c[1].as_dict().items()))
@pytest.mark.parametrize("M", [1, 8, 16])
def test_gateup_tile_rows(case, M):
    I, cfg = case
    Kd = 2560
    wgu, x = _w(2 * I, Kd, 17 + I), _x(M, Kd, 17)
    wd = wgu.to(DEV)
    out = K.gateup_swiglu(x.to(DEV), wd[:I], wd[I:], config=cfg)
    torch.cuda.synchronize()
    assert_gateup_parity(out, bits(x), bits(wgu[:I]), bits(wgu[I:]), f"I={I} {cfg} M={M}")


@pytest.mark.parametrize("cfg", [ring(10, 8, 24), ring(10, 8, 10), ring(10, 8, 13, grid=64)],
                         ids=["rows24", "rows10", "rows13-grid64"])
@pytest.mark.parametrize("M", [1, 8])
def test_lm_argmax_tile_rows(cfg, M):
    """Fused argmax with tiles of 24, 10 and 13 rows over a 20000-token vocabulary."""
    V, Kd = 20000, 2560
    w, x = _w(V, Kd, 7), _x(M, Kd, 7)
    ids, maxv = K.lm_argmax(x.to(DEV), w.to(DEV), config=cfg)
    torch.cuda.synchronize()
    logits = oracle.gemm(bits(x), bits(w))
    o_ids, o_maxv = oracle.argmax(logits)
    check_argmax_rows(ids, maxv, logits, o_ids, o_maxv, f"lm_argmax {cfg} M={M}")
