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


# ---------------------------------------------------------------------------
# Residual hand-off on the two-operand wide path (groups = 4): the producer
# after split-K partials, the consumers normalising rows while staging them.
# ---------------------------------------------------------------------------

HID, EPS = 2560, 1e-6


def _sums16(ro: torch.Tensor) -> torch.Tensor:
    """fp64 sums of squares over 16-column groups of an [M, N] bf16 tensor."""
    M, N = ro.shape
    G = (N + 15) // 16
    f = torch.zeros((M, G * 16), dtype=torch.float64)
    f[:, :N] = ro.double()
    return f.pow(2).view(M, G, 16).sum(-1)


def _exact(shape, seed):
    """Values in {0, +-0.5, ..., +-2}: every partial sum of squares is exact in
    fp32, so a row's rstd does not depend on the summation order."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randint(-4, 5, shape, generator=g).float() * 0.5).to(torch.bfloat16)


def _gain(seed):
    g = torch.Generator().manual_seed(seed)
    return (1 + 0.1 * torch.randn(HID, generator=g)).to(torch.bfloat16)


@pytest.mark.parametrize("N,Kd,cfg", [
    (2560, 4096, wide(8, 32, split=3, wn=4)),   # o_proj
    (2560, 9728, wide(8, 32, split=3, wn=4)),   # down
    (2560, 4096, wide(8, 64, split=2, wn=4)),   # four slabs per tile
    (200, 512, wide(8, 32, split=2, wn=4)),     # ragged N: the last tile's columns past N
], ids=lambda v: v if isinstance(v, int) else _ids(v))
@pytest.mark.parametrize("M", [128, 100, 33])
def test_wide_gemm_residual_bit_exact_against_gemm_plus_add(N, Kd, cfg, M):
    """r_out = bf16(r + y) bit for bit with y the plain wide GEMM of the same
    configuration (same split-K sum order), sums of squares against fp64."""
    a, w, r = _x(M, Kd, 80), _w(N, Kd, 81), _x(M, N, 82)
    ad, wd, rd = a.to(DEV), w.to(DEV), r.to(DEV)
    y = K.gemm(ad, wd, config=cfg)
    ro = torch.empty_like(rd)
    sq = torch.full((M, K.sumsq_groups(M, N)), float("nan"), dtype=torch.float32, device=DEV)
    K.gemm_residual(ad, wd, rd, ro, sq, config=cfg)
    torch.cuda.synchronize()
    assert_parity(y, from_bits(oracle.gemm(bits(a), bits(w))), f"projection N={N} M={M} {cfg}")
    want = (r.float() + y.cpu().float()).to(torch.bfloat16)
    assert torch.equal(ro.cpu().view(torch.int16), want.view(torch.int16)), f"residual N={N} M={M}"
    got, ref = sq.cpu().double(), _sums16(want)
    assert torch.all(torch.isfinite(got))
    assert torch.allclose(got, ref, rtol=2e-6, atol=0), (got - ref).abs().max().item()


PRE_CASES = [
    ("qkv", wide(8, 48, wn=4)),       # 48-row tiles in four slabs (two waves per 32 rows)
    ("qkv", wide(8, 24, wn=4)),
    ("gate_up", wide(8, 40, wn=4)),
    ("gate_up", wide(8, 24, wn=4)),
    ("lm_argmax", wide(8, 128, wn=4)),
    ("lm_argmax", wide(8, 96, grid=64, wn=4)),
]


def _consume(kind, xd, sq, wnd, wd, cfg, pre: bool):
    """The consumer (pre=True) or the unfused pipeline: add + RMSNorm launch,
    then the projection with the same configuration."""
    if kind == "qkv":
        if pre:
            return K.rmsnorm_pre_gemm(xd, sq, wnd, EPS, wd, config=cfg)
        return K.rmsnorm_gemm(xd, torch.zeros_like(xd), wnd, EPS, torch.empty_like(xd), wd, config=cfg)
    if kind == "gate_up":
        I = wd.shape[0] // 2
        if pre:
            return K.rmsnorm_pre_gateup_swiglu(xd, sq, wnd, EPS, wd[:I], wd[I:], config=cfg)
        return K.rmsnorm_gateup_swiglu(xd, torch.zeros_like(xd), wnd, EPS, torch.empty_like(xd), wd[:I], wd[I:],
                                       config=cfg)
    if pre:
        return K.rmsnorm_pre_lm_argmax(xd, sq, wnd, EPS, wd, config=cfg)
    return K.rmsnorm_lm_argmax(xd, torch.zeros_like(xd), wnd, EPS, torch.empty_like(xd), wd, config=cfg)


_PRE_N = {"qkv": 6144, "gate_up": 2 * 9728, "lm_argmax": 30000}


@pytest.mark.parametrize("kind,cfg", PRE_CASES, ids=lambda v: v if isinstance(v, str) else _ids(v))
@pytest.mark.parametrize("M", [128, 77])
def test_wide_pre_exact_stats_equals_unfused_pipeline(kind, cfg, M):
    x, wn, w = _exact((M, HID), 90 + M), _gain(91), _w(_PRE_N[kind], HID, 92)
    xd, wnd, wd = x.to(DEV), wn.to(DEV), w.to(DEV)
    got = _consume(kind, xd, _sums16(x).float().to(DEV), wnd, wd, cfg, pre=True)
    ref = _consume(kind, xd, None, wnd, wd, cfg, pre=False)
    torch.cuda.synchronize()
    if kind == "lm_argmax":
        assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])
    else:
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("kind,cfg", PRE_CASES, ids=lambda v: v if isinstance(v, str) else _ids(v))
@pytest.mark.parametrize("M", [128, 50])
def test_wide_pre_random_against_oracle(kind, cfg, M):
    import numpy as np

    x, wn, w = _x(M, HID, 95), _gain(96), _w(_PRE_N[kind], HID, 97)
    got = _consume(kind, x.to(DEV), _sums16(x).float().to(DEV), wn.to(DEV), w.to(DEV), cfg, pre=True)
    torch.cuda.synchronize()
    _, h = oracle.add_rmsnorm(bits(x), np.zeros_like(bits(x)), bits(wn), EPS)
    what = f"pre {kind} M={M} {cfg}"
    if kind == "qkv":
        assert_parity(got, from_bits(oracle.gemm(h, bits(w))), what)
    elif kind == "gate_up":
        I = w.shape[0] // 2
        assert_gateup_parity(got, h, bits(w[:I]), bits(w[I:]), what)
    else:
        o_ids, o_max = oracle.lm_argmax(h, bits(w))
        check_argmax_rows(got[0], got[1], oracle.gemm(h, bits(w)), o_ids, o_max, what)
