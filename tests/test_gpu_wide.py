"""GPU parity of the wide-M path (SK_PATH_WIDE, csrc/sk_wide.hpp) against the CPU oracle (needs an MI355X).

Up to 128 activation rows run in one workgroup: four or eight waves split
the 16-row activation tiles and every wave multiplies the whole weight tile,
staged once per 256-column step in LDS (groups = 4: weight tile and
activation rows both staged in LDS per 128-column step, csrc/sk_wide2.hpp).  Checked with every epilogue (bf16
store, SwiGLU, fused argmax, split-K partials and their in-kernel finish for
the plain and the gate/up GEMM), at the verify row counts of the reference
(B x R = 64 and 128; engine/engine.py:451) and ragged ones, with tile heights
that are not multiples of 16 and a ragged N.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from starter_amd import kernels as K
from starter_amd._lib import SK_PATH_WIDE, SkConfig
from tests._util import assert_gateup_parity, assert_parity, bits, check_argmax_rows, from_bits, randn_bf16

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _w(N, Kd, seed):
    return randn_bf16((N, Kd), 0.02, torch.Generator().manual_seed(seed))


def _x(M, Kd, seed):
    return randn_bf16((M, Kd), 1.0, torch.Generator().manual_seed(70_000 + seed + M))


def wide(waves, rows, split=1, grid=0, wn=1):
    """A wide configuration; ``wn`` (the ``groups`` field) = wave groups along the tile's slabs."""
    return SkConfig.make(SK_PATH_WIDE, waves=waves, ku=8, rows=rows, split=split, grid=grid, groups=wn)


def _ids(c):
    return "-".join(f"{k}{v}" for k, v in c.as_dict().items())


GEMM_CASES = [
    (6144, 2560, wide(4, 32)),
    (6144, 2560, wide(8, 24)),
    (6144, 2560, wide(4, 48, split=2)),     # split-K partials, finished in-kernel
    (2560, 4096, wide(8, 40, split=3)),     # 16 chunks in three slices of 6, 6, 4
    (2560, 9728, wide(4, 80, split=4)),     # five slabs per tile
    (777, 2560, wide(4, 13)),               # ragged N, 13-row tiles (two slabs, 3 rows of the second unused)
    (777, 2560, wide(8, 96, grid=4)),       # six slabs, several tiles per workgroup
    (1000, 2336, wide(4, 20, split=2)),     # K = 9 * 256 + 32: the last step is partial
    (6144, 2560, wide(8, 48, wn=2)),        # waves in two groups of slabs x four of activation tiles
    (2560, 9728, wide(8, 96, split=4, wn=2)),
    (777, 2560, wide(8, 20, wn=2, grid=16)),
    # groups = 4: activation rows staged in LDS too (four waves, 32 rows each)
    (6144, 2560, wide(4, 48, wn=4)),
    (6144, 2560, wide(4, 64, split=2, wn=4)),
    (2560, 4096, wide(4, 40, split=3, wn=4)),   # K slices of 6, 6, 4 chunks
    (2560, 9728, wide(4, 80, split=4, wn=4)),
    (777, 2560, wide(4, 13, wn=4)),             # one slab, ragged N
    (777, 2560, wide(4, 128, grid=4, wn=4)),    # eight slabs, several tiles per workgroup
    (1000, 2336, wide(4, 20, split=2, wn=4)),   # K = 18 * 128 + 32: the last step is partial
    (6144, 2560, wide(8, 48, wn=4)),            # eight waves: each step's K units split in two
    (2560, 9728, wide(8, 32, split=3, wn=4)),
    (777, 2560, wide(8, 90, grid=4, wn=4)),
    (1000, 2336, wide(8, 20, split=2, wn=4)),
    (777, 2560, wide(8, 128, grid=3, wn=4)),    # eight slabs at eight waves
]


@pytest.mark.parametrize("case", GEMM_CASES, ids=lambda c: f"{c[0]}x{c[1]}-{_ids(c[2])}")
@pytest.mark.parametrize("M", [1, 33, 64, 100, 128])
def test_wide_gemm(case, M):
    N, Kd, cfg = case
    w, x = _w(N, Kd, N + Kd), _x(M, Kd, N)
    out = K.gemm(x.to(DEV), w.to(DEV), config=cfg)
    torch.cuda.synchronize()
    assert_parity(out, from_bits(oracle.gemm(bits(x), bits(w))), f"N={N} K={Kd} {cfg} M={M}")


GATEUP_CASES = [
    (9728, wide(4, 32)),
    (9728, wide(8, 40)),                    # three slabs per half
    (9728, wide(4, 16, split=2)),           # gate and up partials
    (1000, wide(8, 24, grid=8)),            # ragged I, several tiles per workgroup
    (9728, wide(8, 32, wn=2)),              # two groups of slabs: gate and up slab of each group
    (9728, wide(8, 24, split=2, wn=2)),
    (9728, wide(4, 38, wn=4)),                  # 256 tiles of 38 gate + 38 up rows
    (9728, wide(4, 64, wn=4)),
    (9728, wide(4, 24, split=2, wn=4)),
    (1000, wide(4, 40, grid=8, wn=4)),
    (9728, wide(8, 38, wn=4)),
    (9728, wide(8, 24, split=2, wn=4)),
]


@pytest.mark.parametrize("case", GATEUP_CASES, ids=lambda c: f"I{c[0]}-{_ids(c[1])}")
@pytest.mark.parametrize("M", [8, 64, 128])
def test_wide_gateup(case, M):
    I, cfg = case
    Kd = 2560
    wgu, x = _w(2 * I, Kd, 19 + I), _x(M, Kd, 19)
    wd = wgu.to(DEV)
    out = K.gateup_swiglu(x.to(DEV), wd[:I], wd[I:], config=cfg)
    torch.cuda.synchronize()
    assert_gateup_parity(out, bits(x), bits(wgu[:I]), bits(wgu[I:]), f"I={I} {cfg} M={M}")


@pytest.mark.parametrize("cfg", [wide(4, 64), wide(8, 96), wide(4, 27, grid=64), wide(8, 96, wn=2), wide(4, 128, wn=4),
                                 wide(4, 27, grid=64, wn=4), wide(8, 96, wn=4), wide(8, 128, wn=4),
                                 wide(8, 128, grid=40, wn=4)], ids=_ids)
@pytest.mark.parametrize("M", [1, 64, 128])
def test_wide_lm_argmax(cfg, M):
    """Fused argmax over a 30000-token vocabulary (many tiles per workgroup)."""
    V, Kd = 30000, 2560
    w, x = _w(V, Kd, 9), _x(M, Kd, 9)
    ids, maxv = K.lm_argmax(x.to(DEV), w.to(DEV), config=cfg)
    torch.cuda.synchronize()
    logits = oracle.gemm(bits(x), bits(w))
    o_ids, o_maxv = oracle.argmax(logits)
    check_argmax_rows(ids, maxv, logits, o_ids, o_maxv, f"lm_argmax {cfg} M={M}")


@pytest.mark.parametrize("cfg", [wide(4, 128, wn=4), wide(8, 96, wn=4), wide(8, 128, wn=4),
                                 wide(8, 128, grid=40, wn=4)], ids=_ids)
def test_wide_lm_argmax_exact_ties(cfg):
    """Duplicate weight rows give bit-identical logits; the lowest column must
    win when the copies share a lane's columns, sit in different quarters or
    slabs of one tile, in adjacent tiles, or in different workgroups."""
    V, Kd, M = 40_000, 2560, 8
    w, x = _w(V, Kd, 5), _x(M, Kd, 5)
    pairs = [(100, 39_000), (7, 8), (20_000, 30_000), (0, V - 1), (45, 110), (130, 131), (31, 33), (255, 256)]
    for m, (lo, hi) in enumerate(pairs):
        hot = (x[m].float() * 0.05).to(torch.bfloat16)   # strongly aligned with row m's activations
        w[lo] = hot
        w[hi] = hot
    ids, maxv = K.lm_argmax(x.to(DEV), w.to(DEV), config=cfg)
    torch.cuda.synchronize()
    assert ids.cpu().tolist() == [lo for lo, _ in pairs]
    o_ids, o_maxv = oracle.lm_argmax(bits(x), bits(w))
    assert (ids.cpu().numpy() == o_ids).all()
    assert (maxv.cpu().numpy() == o_maxv).all()
