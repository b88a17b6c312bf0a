"""GPU parity of the HIP hot path against the CPU oracle (needs an MI355X).

Inputs are drawn on a seeded CPU generator, copied to the GPU, and the same
bits go through the oracle.  Parity rule (north star): every output element
within 1e-2 * max(|ref|, 1e-3 * rms(ref row)) of the oracle; the residual
stream ``xout`` and SwiGLU of given inputs bit-exact; argmax ids bit-exact
wherever the oracle's bf16 top-2 logits differ (margin > 1e-2), maxv exact.

Shape grid: the five Qwen3-4B decode weights at M in {1,2,4,8,16,32,40,48,64}
(and M = 48, the last tuned row count below 64) plus the
reference test grid (tests/test_kernels.py:
111-124, 147-161, 170-224): N=777 ragged, M in {1,4,16,48,96,128}.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from starter_amd import kernels as K
from starter_amd._lib import (SK_ERR_ALIGN, SK_ERR_CONFIG, SK_ERR_SHAPE, SK_ERR_WORKSPACE, SK_OP_GATEUP, SK_OP_GEMM,
                              SK_PATH_GEMV, SK_PATH_MFMA, SK_PATH_MFMA_LDS, SkConfig, SkError)
from tests._util import (BF16, assert_gateup_parity, assert_parity, bits, check_argmax_rows, from_bits, randn_bf16,
                         reference_tolerance_ok)

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
QKV, O, GU, D, LM = (6144, 2560), (2560, 4096), (19456, 2560), (2560, 9728), (151936, 2560)
M_SWEEP = [1, 2, 4, 8, 16, 32, 40, 48, 64]

_cache: dict = {}


def _weights(N: int, Kd: int, seed: int, scale: float = 0.02) -> torch.Tensor:
    key = ("w", N, Kd, seed, scale)
    if key not in _cache:
        g = torch.Generator().manual_seed(seed)
        _cache[key] = randn_bf16((N, Kd), scale, g)
    return _cache[key]


def _acts(M: int, Kd: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(10_000 + seed * 131 + M)
    return randn_bf16((M, Kd), 1.0, g)


def _gpu(t: torch.Tensor) -> torch.Tensor:
    key = ("gpu", t.data_ptr(), tuple(t.shape))
    if t.numel() > 50_000_000:
        if key not in _cache:
            _cache[key] = t.to(DEV)
        return _cache[key]
    return t.to(DEV)


def _oracle_gemm(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return from_bits(oracle.gemm(bits(x), bits(w)))


# ---------------------------------------------------------------------------
# Plain GEMM (qkv / o / d / lm logits)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape", [QKV, O, D], ids=["qkv", "o_proj", "down"])
@pytest.mark.parametrize("M", M_SWEEP)
def test_gemm_qwen_shapes_default_config(shape, M):
    N, Kd = shape
    w = _weights(N, Kd, seed=N + Kd)
    x = _acts(M, Kd, seed=N)
    out = K.gemm(x.to(DEV), _gpu(w))
    torch.cuda.synchronize()
    assert_parity(out, _oracle_gemm(x, w), f"gemm N={N} K={Kd} M={M}")


@pytest.mark.parametrize("M", M_SWEEP)
def test_gemm_lm_head_logits(M):
    N, Kd = LM
    w = _weights(N, Kd, seed=7)
    x = _acts(M, Kd, seed=7)
    out = K.gemm(x.to(DEV), _gpu(w))
    torch.cuda.synchronize()
    assert_parity(out, _oracle_gemm(x, w), f"lm logits M={M}")


@pytest.mark.parametrize("M", [1, 4, 16, 48, 96, 128])
@pytest.mark.parametrize("shape", [(6144, 2560), (2560, 9728), (777, 2560)], ids=["6144x2560", "2560x9728", "777x2560"])
def test_gemm_reference_grid(shape, M):
    """The reference's own GEMM test grid (tests/test_kernels.py:111-124),
    including M > 64 (row groups in one launch where the table has them, else
    64-row launches) and the ragged N = 777."""
    N, Kd = shape
    w = _weights(N, Kd, seed=3 * N)
    x = _acts(M, Kd, seed=5)
    out = K.gemm(x.to(DEV), _gpu(w))
    ref = _oracle_gemm(x, w)
    assert_parity(out, ref, f"ref grid N={N} K={Kd} M={M}")
    assert reference_tolerance_ok(out, ref)


M_WIDE = [65, 100, 128, 129, 200]


@pytest.mark.parametrize("M", M_WIDE)
@pytest.mark.parametrize("name", ["qkv", "o_proj", "gate_up", "down"])
def test_wide_calls_default_config(name, M):
    """More than 64 rows, as in the reference's verify forward at batch 16
    (B x R = 128 rows): up to 128 rows run as one launch of row groups, more
    as 128-row launches plus the remainder, default configuration."""
    if name == "gate_up":
        I2, Kd = GU
        I = I2 // 2
        wgu = _weights(I2, Kd, seed=17)
        x = _acts(M, Kd, seed=17)
        wd = _gpu(wgu)
        out = K.gateup_swiglu(x.to(DEV), wd[:I], wd[I:])
        assert_gateup_parity(out, bits(x), bits(wgu[:I]), bits(wgu[I:]), f"gateup M={M}")
        return
    N, Kd = {"qkv": QKV, "o_proj": O, "down": D}[name]
    w = _weights(N, Kd, seed=N + Kd)
    x = _acts(M, Kd, seed=N)
    out = K.gemm(x.to(DEV), _gpu(w))
    torch.cuda.synchronize()
    assert_parity(out, _oracle_gemm(x, w), f"gemm {name} M={M}")


@pytest.mark.parametrize("M", [129, 130])
@pytest.mark.parametrize("name", ["qkv", "gate_up", "lm_argmax"])
def test_wide_calls_with_the_default_config_passed_explicitly(name, M):
    """default_config(op, M) passed back explicitly: the 128-row launch runs
    its row groups, the one- or two-row remainder as many groups as hold a row."""
    from starter_amd._lib import SK_OP_LM_ARGMAX, default_config

    if name == "gate_up":
        I2, Kd = GU
        I = I2 // 2
        wgu = _weights(I2, Kd, seed=17)
        x = _acts(M, Kd, seed=23)
        wd = _gpu(wgu)
        cfg = default_config(SK_OP_GATEUP, M, I, Kd)
        out = K.gateup_swiglu(x.to(DEV), wd[:I], wd[I:], config=cfg)
        assert_gateup_parity(out, bits(x), bits(wgu[:I]), bits(wgu[I:]), f"gateup M={M} {cfg}")
        return
    if name == "lm_argmax":
        V, Kd = LM
        w = _weights(V, Kd, seed=7)
        x = _acts(M, Kd, seed=29)
        cfg = default_config(SK_OP_LM_ARGMAX, M, V, Kd)
        ids, maxv = K.lm_argmax(x.to(DEV), _gpu(w), config=cfg)
        logits = oracle.gemm(bits(x), bits(w))
        o_ids, o_maxv = oracle.argmax(logits)
        check_argmax_rows(ids, maxv, logits, o_ids, o_maxv, f"lm_argmax M={M} {cfg}")
        return
    N, Kd = QKV
    w = _weights(N, Kd, seed=N + Kd)
    x = _acts(M, Kd, seed=31)
    cfg = default_config(SK_OP_GEMM, M, N, Kd)
    out = K.gemm(x.to(DEV), _gpu(w), config=cfg)
    torch.cuda.synchronize()
    assert_parity(out, _oracle_gemm(x, w), f"qkv M={M} {cfg}")


@pytest.mark.parametrize("M", [100, 128, 129])
def test_wide_lm_head(M):
    """lm_head at up to 128 rows in one launch, more as a second launch: the
    fused argmax (default configuration; each launch's last workgroup clears
    the candidate table for the next) and the logits GEMM."""
    V, Kd = LM
    w = _weights(V, Kd, seed=7)
    x = _acts(M, Kd, seed=11)
    wd = _gpu(w)
    ids, maxv = K.lm_argmax(x.to(DEV), wd)
    logits = oracle.gemm(bits(x), bits(w))
    o_ids, o_maxv = oracle.argmax(logits)
    check_argmax_rows(ids, maxv, logits, o_ids, o_maxv, f"lm_argmax M={M}")
    out = K.gemm(x.to(DEV), wd)
    torch.cuda.synchronize()
    assert_parity(out, from_bits(logits), f"lm logits M={M}")


GEMM_CONFIGS = [
    SkConfig.make(SK_PATH_MFMA, waves=4, ku=20, rows=16),
    SkConfig.make(SK_PATH_MFMA, waves=8, ku=10, rows=16),
    SkConfig.make(SK_PATH_MFMA, waves=16, ku=5, rows=16),
    SkConfig.make(SK_PATH_MFMA, waves=8, ku=10, rows=32),
    SkConfig.make(SK_PATH_MFMA, waves=2, ku=20, rows=16, split=2),
    SkConfig.make(SK_PATH_MFMA, waves=4, ku=5, rows=16, split=4),
    SkConfig.make(SK_PATH_MFMA, waves=4, ku=20, rows=16, grid=64),
    SkConfig.make(SK_PATH_GEMV, waves=1, ku=5, rows=4),
    SkConfig.make(SK_PATH_GEMV, waves=3, ku=2, rows=8),
    SkConfig.make(SK_PATH_GEMV, waves=2, ku=3, rows=2),
    SkConfig.make(SK_PATH_GEMV, waves=1, ku=2, rows=4, split=3),
    SkConfig.make(SK_PATH_MFMA_LDS, waves=5, ku=16, rows=16),
    SkConfig.make(SK_PATH_MFMA_LDS, waves=3, ku=16, rows=32, split=2),
    SkConfig.make(SK_PATH_MFMA_LDS, waves=10, ku=8, rows=16),
    SkConfig.make(SK_PATH_MFMA_LDS, waves=3, ku=16, rows=16, split=2),
    SkConfig.make(SK_PATH_MFMA_LDS, waves=5, ku=16, rows=16, grid=40),
]


@pytest.mark.parametrize("cfg", GEMM_CONFIGS, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.as_dict().items()))
@pytest.mark.parametrize("M", [1, 3, 8])
def test_gemm_every_config(cfg, M):
    """Each candidate configuration, like the reference's per-config test loop."""
    N, Kd = 1536, 2560
    w = _weights(N, Kd, seed=99)
    x = _acts(M, Kd, seed=99)
    out = K.gemm(x.to(DEV), w.to(DEV), config=cfg)
    assert_parity(out, _oracle_gemm(x, w), f"config {cfg} M={M}")


def test_gemm_deterministic_and_config_independent_bounds():
    N, Kd, M = 2560, 9728, 8
    w = _weights(N, Kd, seed=N + Kd)
    x = _acts(M, Kd, seed=1).to(DEV)
    a = K.gemm(x, _gpu(w))
    b = K.gemm(x, _gpu(w))
    assert torch.equal(a, b)   # no atomics: bitwise reproducible
    c = K.gemm(x, _gpu(w), config=SkConfig.make(SK_PATH_MFMA, waves=8, ku=10, rows=16, split=4))
    ref = _oracle_gemm(x.cpu(), w)
    assert_parity(c, ref, "split 4")


def test_epilogue_rounding_is_round_to_nearest_even():
    """One-hot pair weights make C = a_i + a_j exactly in fp32; the bf16
    store must round it like torch (ties to even)."""
    M, Kd, N = 16, 64, 32
    rng = np.random.default_rng(0)
    base = rng.standard_normal((M, Kd)).astype(np.float32)
    a = torch.from_numpy(base).to(BF16)
    af = a.float()
    w = torch.zeros(N, Kd, dtype=BF16)
    for n in range(N):
        w[n, n % Kd] = 1.0
        w[n, (n * 7 + 3) % Kd] = 2.0 ** -(n % 12)
    exact = af @ w.float().T            # exact in fp32 for these operands
    out = K.gemm(a.to(DEV), w.to(DEV))
    assert torch.equal(out.cpu(), exact.to(BF16))


# ---------------------------------------------------------------------------
# gate/up + SwiGLU
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["qkv", "o_proj", "gate_up", "down", "lm_head"])
def test_strict_rule_counts(name):
    """The plain north-star rule, |out - ref| <= 1e-2 * max(|ref|, 1e-3 * rms(row)),
    counted on every element at every C4 row count and at 128 rows (one launch
    of row groups) with the default configuration (seeded inputs as above).  The plain GEMMs must meet it
    everywhere.  gate_up's SwiGLU output rounds g and u to bf16 first, so a
    strict violation is allowed only where the midpoint-aware rule explains it
    (assert_gateup_parity), and the count is reported.  One line per point is
    printed (run with -s to collect them)."""
    from tests._util import gateup_violations, rel_violations

    for M in M_SWEEP + [128]:
        if name == "gate_up":
            I2, Kd = GU
            I = I2 // 2
            wgu = _weights(I2, Kd, seed=17)
            x = _acts(M, Kd, seed=17)
            wd = _gpu(wgu)
            out = K.gateup_swiglu(x.to(DEV), wd[:I], wd[I:])
            torch.cuda.synchronize()
            ref = from_bits(oracle.gateup_swiglu(bits(x), bits(wgu[:I]), bits(wgu[I:])))
            bad, worst = rel_violations(out, ref)
            viol, amb, exact = gateup_violations(out, bits(x), bits(wgu[:I]), bits(wgu[I:]))
            print(f"strict {name} M={M}: {bad} of {out.numel()} outside the plain rule (worst ratio {worst:.3g}); "
                  f"midpoint-aware rule: {viol} violations, {amb} ambiguous, {exact:.5f} of the rest bit-exact")
            assert viol == 0 and exact >= 0.999
            continue
        N, Kd = {"qkv": QKV, "o_proj": O, "down": D, "lm_head": LM}[name]
        seed = 7 if name == "lm_head" else N + Kd
        w = _weights(N, Kd, seed=seed)
        x = _acts(M, Kd, seed=seed if name == "lm_head" else N)
        out = K.gemm(x.to(DEV), _gpu(w))
        torch.cuda.synchronize()
        bad, worst = rel_violations(out, _oracle_gemm(x, w))
        print(f"strict {name} M={M}: {bad} of {out.numel()} outside the plain rule (worst ratio {worst:.3g})")
        assert bad == 0


@pytest.mark.parametrize("M", M_SWEEP)
def test_gateup_qwen_default_config(M):
    I2, Kd = GU
    I = I2 // 2
    wgu = _weights(I2, Kd, seed=17)
    x = _acts(M, Kd, seed=17)
    wd = _gpu(wgu)
    out = K.gateup_swiglu(x.to(DEV), wd[:I], wd[I:])
    assert_gateup_parity(out, bits(x), bits(wgu[:I]), bits(wgu[I:]), f"gateup M={M}")


@pytest.mark.parametrize("M", [17, 24, 32])
@pytest.mark.parametrize("grid", [0, 96])
def test_ring_one_partial_buffer(M, grid):
    """10 waves of 32 rows on the ring path need one partial-tile buffer in LDS
    (two do not fit): one more barrier per tile, several tiles per workgroup
    (grid 96: six or seven tiles each).  gate/up+SwiGLU and a ragged GEMM."""
    I2, Kd = GU
    I = I2 // 2
    cfg = SkConfig.make(SK_PATH_MFMA_LDS, waves=10, ku=8, rows=16, grid=grid)
    wgu = _weights(I2, Kd, seed=29)
    x = _acts(M, Kd, seed=29)
    wd = _gpu(wgu)
    out = K.gateup_swiglu(x.to(DEV), wd[:I], wd[I:], config=cfg)
    assert_gateup_parity(out, bits(x), bits(wgu[:I]), bits(wgu[I:]), f"gateup one buffer M={M} grid={grid}")
    N = 6144 - 48
    w = _weights(N, Kd, seed=31)
    cfg = SkConfig.make(SK_PATH_MFMA_LDS, waves=10, ku=8, rows=32, grid=grid)
    out = K.gemm(x.to(DEV), _gpu(w), config=cfg)
    assert_parity(out, _oracle_gemm(x, w), f"gemm one buffer M={M} grid={grid}")


@pytest.mark.parametrize("M", [33, 40, 48])
@pytest.mark.parametrize("grid", [0, 64])
def test_ring_half_slab_in_flight(M, grid):
    """48-row activation tiles keep half a weight slab in flight per wave (four
    ring registers, each refilled with the load four ahead, across slab and
    tile boundaries), ten waves of one 256-column chunk each, no K split;
    several tiles per workgroup at grid 64.  gate/up+SwiGLU and a ragged GEMM."""
    I2, Kd = GU
    I = I2 // 2
    cfg = SkConfig.make(SK_PATH_MFMA_LDS, waves=10, ku=8, rows=16, grid=grid)
    wgu = _weights(I2, Kd, seed=37)
    x = _acts(M, Kd, seed=37)
    wd = _gpu(wgu)
    out = K.gateup_swiglu(x.to(DEV), wd[:I], wd[I:], config=cfg)
    assert_gateup_parity(out, bits(x), bits(wgu[:I]), bits(wgu[I:]), f"gateup half ring M={M} grid={grid}")
    N = 6144 - 40
    w = _weights(N, Kd, seed=41)
    out = K.gemm(x.to(DEV), _gpu(w), config=cfg)
    assert_parity(out, _oracle_gemm(x, w), f"gemm half ring M={M} grid={grid}")


@pytest.mark.parametrize("M,groups", [(33, 2), (50, 3), (61, 4), (64, 2), (100, 4), (128, 4), (128, 8)])
@pytest.mark.parametrize("split", [1, 2])
def test_ring_row_groups(M, groups, split):
    """Row groups: the rows split into `groups` independent GEMMs launched side
    by side (groups of ceil(M / groups) rows, the last one shorter), each with
    its own counters and split-K partials.  gate/up+SwiGLU and a ragged GEMM at
    one and two K splits, several tiles per workgroup (grid 64 or 32 per
    group), and bit-identity with the ungrouped launch, whose per-element
    summation order is the same (one chunk per wave, waves summed in order)."""
    I2, Kd = GU
    I = I2 // 2
    waves = 10 if split == 1 else 5
    cfg = SkConfig.make(SK_PATH_MFMA_LDS, waves=waves, ku=8, rows=16, split=split, grid=64 * split // 2 * 2,
                        groups=groups)
    wgu = _weights(I2, Kd, seed=43)
    x = _acts(M, Kd, seed=43)
    wd = _gpu(wgu)
    xd = x.to(DEV)
    out = K.gateup_swiglu(xd, wd[:I], wd[I:], config=cfg)
    what = f"M={M} groups={groups} split={split}"
    assert_gateup_parity(out, bits(x), bits(wgu[:I]), bits(wgu[I:]), f"gateup row groups {what}")
    N = 6144 - 56
    w = _weights(N, Kd, seed=47)
    cfg_g = SkConfig.make(SK_PATH_MFMA_LDS, waves=waves, ku=8, rows=32, split=split, grid=32 * split, groups=groups)
    out = K.gemm(xd, _gpu(w), config=cfg_g)
    assert_parity(out, _oracle_gemm(x, w), f"gemm row groups {what}")
    # the same rows one group at a time through the plain launch, where its
    # registers allow: identical bits
    for g0 in range(0, M, -(-M // groups)):
        rows = xd[g0:g0 + -(-M // groups)]
        plain = SkConfig.make(SK_PATH_MFMA_LDS, waves=waves, ku=8, rows=32, split=split, grid=32 * split)
        assert torch.equal(K.gemm(rows, _gpu(w), config=plain), out[g0:g0 + rows.shape[0]]), f"{what} rows {g0}+"


@pytest.mark.parametrize("M,groups,grid", [(64, 2, 640), (49, 3, 96), (40, 2, 8), (128, 4, 256), (97, 4, 8)])
def test_lm_argmax_row_groups(M, groups, grid):
    """The fused argmax with row groups: one arrival counter per group, every
    row's candidate in one table; a ragged vocabulary at one grid."""
    V, Kd = LM
    if grid == 8:
        V = 40_000 - 13
    w = _weights(V, Kd, seed=53)
    x = _acts(M, Kd, seed=53)
    cfg = SkConfig.make(SK_PATH_MFMA_LDS, waves=10, ku=8, rows=16, grid=grid, groups=groups)
    ids, maxv = K.lm_argmax(x.to(DEV), _gpu(w), config=cfg)
    logits = oracle.gemm(bits(x), bits(w))
    o_ids, o_maxv = oracle.argmax(logits)
    check_argmax_rows(ids, maxv, logits, o_ids, o_maxv, f"lm_argmax row groups M={M} groups={groups}")
    ids2, maxv2 = K.lm_argmax(x.to(DEV), _gpu(w), config=cfg)   # the counters were returned to zero
    assert torch.equal(ids, ids2) and torch.equal(maxv, maxv2)


GATEUP_CONFIGS = [
    SkConfig.make(SK_PATH_MFMA, waves=8, ku=10, rows=16),
    SkConfig.make(SK_PATH_MFMA, waves=16, ku=5, rows=16),
    SkConfig.make(SK_PATH_MFMA, waves=4, ku=10, rows=16, split=2),
    SkConfig.make(SK_PATH_GEMV, waves=1, ku=5, rows=4),
    SkConfig.make(SK_PATH_GEMV, waves=2, ku=3, rows=2),
    SkConfig.make(SK_PATH_MFMA_LDS, waves=5, ku=16, rows=16),
    SkConfig.make(SK_PATH_MFMA_LDS, waves=5, ku=8, rows=16, split=2),
    SkConfig.make(SK_PATH_MFMA_LDS, waves=3, ku=16, rows=16, split=2),
]


@pytest.mark.parametrize("cfg", GATEUP_CONFIGS, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.as_dict().items()))
@pytest.mark.parametrize("M", [1, 4])
def test_gateup_every_config(cfg, M):
    I, Kd = 1024, 2560
    wgu = _weights(2 * I, Kd, seed=23)
    x = _acts(M, Kd, seed=23)
    wd = wgu.to(DEV)
    out = K.gateup_swiglu(x.to(DEV), wd[:I], wd[I:], config=cfg)
    assert_gateup_parity(out, bits(x), bits(wgu[:I]), bits(wgu[I:]), f"gateup config {cfg}")


def test_gateup_reference_grid_m16():
    """tests/test_kernels.py:147-161 at M = 16 against F.silu(F.linear) * F.linear."""
    I, Kd, M = 9728, 2560, 16
    wgu = _weights(2 * I, Kd, seed=17)
    x = _acts(M, Kd, seed=3)
    wd = _gpu(wgu)
    out = K.gateup_swiglu(x.to(DEV), wd[:I], wd[I:])
    ref = F.silu(F.linear(x, wgu[:I])) * F.linear(x, wgu[I:])
    assert reference_tolerance_ok(out, ref)
    assert_gateup_parity(out, bits(x), bits(wgu[:I]), bits(wgu[I:]), "gateup M=16")


# ---------------------------------------------------------------------------
# lm_head + fused argmax, standalone argmax
# ---------------------------------------------------------------------------

LM_CONFIGS = {"default": None, "mfma_lds": SkConfig.make(SK_PATH_MFMA_LDS, waves=5, ku=16, rows=16),
              "gemv": SkConfig.make(SK_PATH_GEMV, waves=1, ku=5, rows=4)}


@pytest.mark.parametrize("cfg,M", [("default", M) for M in M_SWEEP] +
                         [("mfma_lds", M) for M in (1, 8, 32)] + [("gemv", M) for M in (1, 8)])
def test_lm_argmax_full_vocab(M, cfg):
    """Every C4 row count with the default (tuned) configuration, plus the two
    alternative paths where they apply (GEMV: M <= 8; one unsplit LDS-path
    instance: M <= 32, the argmax cannot split K)."""
    V, Kd = LM
    w = _weights(V, Kd, seed=7)
    x = _acts(M, Kd, seed=11)
    ids, maxv = K.lm_argmax(x.to(DEV), _gpu(w), config=LM_CONFIGS[cfg])
    logits = oracle.gemm(bits(x), bits(w))
    o_ids, o_maxv = oracle.argmax(logits)
    check_argmax_rows(ids, maxv, logits, o_ids, o_maxv, f"lm_argmax M={M} {cfg}")


def test_lm_argmax_exact_ties_across_workgroups():
    """Duplicate weight rows far apart produce bit-identical logits; the lowest
    index must win even when the copies land in different workgroups."""
    V, Kd, M = 40_000, 2560, 4
    g = torch.Generator().manual_seed(5)
    w = randn_bf16((V, Kd), 0.02, g)
    x = _acts(M, Kd, seed=5)
    for m, (lo, hi) in enumerate([(100, 39_000), (7, 8), (20_000, 30_000), (0, V - 1)]):
        hot = (x[m].float() * 0.05).to(BF16)      # strongly aligned with row m's activations
        w[lo] = hot
        w[hi] = hot
    ids, maxv = K.lm_argmax(x.to(DEV), w.to(DEV))
    assert ids.cpu().tolist() == [100, 7, 20_000, 0]
    o_ids, o_maxv = oracle.lm_argmax(bits(x), bits(w))
    assert np.array_equal(ids.cpu().numpy(), o_ids)
    assert np.array_equal(maxv.cpu().numpy(), o_maxv)


def test_lm_argmax_golden():
    d = np.load(oracle.HERE.parent / "tests" / "golden" / "lm_argmax_m4_v777_k128.npz", allow_pickle=False)
    # K = 128 is a multiple of 32: runs unchanged through the HIP path.
    ids, maxv = K.lm_argmax(from_bits(d["x"]).to(DEV), from_bits(d["w"]).to(DEV))
    o_ids, o_maxv = oracle.lm_argmax(d["x"], d["w"])
    assert np.array_equal(ids.cpu().numpy(), o_ids)
    assert np.array_equal(maxv.cpu().numpy(), o_maxv)


@pytest.mark.parametrize("M,V", [(3, 151936), (64, 151936), (5, 1024), (2, 1), (3, 1001)])
def test_argmax_standalone(M, V):
    g = torch.Generator().manual_seed(V + M)
    L = (torch.randn(M, V, generator=g) * 4).to(BF16)
    if V > 300:
        L[0, 7] = L[0].max() + 1
        L[1, 100] = L[1, 200] = L[1].max() + 2
    ids, maxv = K.argmax(L.to(DEV))
    assert torch.equal(ids.cpu(), torch.argmax(L, -1))
    assert torch.equal(maxv.cpu(), L.max(-1).values.float())


def test_argmax_golden_nan_signed_zero_ties():
    d = np.load(oracle.HERE.parent / "tests" / "golden" / "argmax_m7_v1000.npz", allow_pickle=False)
    ids, maxv = K.argmax(from_bits(d["logits"]).to(DEV))
    assert np.array_equal(ids.cpu().numpy(), d["ids"])
    assert np.array_equal(maxv.cpu().numpy(), d["maxv"], equal_nan=True)


# ---------------------------------------------------------------------------
# Elementwise pieces: residual add + RMSNorm, SwiGLU
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("M", [1, 5, 16, 64, 96])
def test_add_rmsnorm(M):
    Kd = 2560
    g = torch.Generator().manual_seed(M)
    x = randn_bf16((M, Kd), 1.0, g)
    y = randn_bf16((M, Kd), 1.0, g)
    w = (1 + 0.1 * torch.randn(Kd, generator=g)).to(BF16)
    xo = torch.empty(M, Kd, dtype=BF16, device=DEV)
    out = K.add_rms_norm(x.to(DEV), y.to(DEV), w.to(DEV), 1e-6, xo)
    o_xout, o_out = oracle.add_rmsnorm(bits(x), bits(y), bits(w), 1e-6)
    assert np.array_equal(bits(xo), o_xout)                      # bit-exact residual
    diff = (out.cpu().float() - from_bits(o_out).float()).abs()
    assert bool((diff <= from_bits(o_out).float().abs() * 2.0 ** -6).all())
    assert (bits(out) != o_out).mean() < 1e-3


def test_add_rmsnorm_in_place_into_x():
    """``xout=None`` writes the residual back into x (engine/kernels/add_rmsnorm.py:67)."""
    M, Kd = 9, 2560
    g = torch.Generator().manual_seed(9)
    x = randn_bf16((M, Kd), 1.0, g)
    y = randn_bf16((M, Kd), 1.0, g)
    w = (1 + 0.1 * torch.randn(Kd, generator=g)).to(BF16)
    xd = x.to(DEV)
    out = K.add_rms_norm(xd, y.to(DEV), w.to(DEV), 1e-6)
    o_xout, o_out = oracle.add_rmsnorm(bits(x), bits(y), bits(w), 1e-6)
    assert np.array_equal(bits(xd), o_xout)
    assert (bits(out) != o_out).mean() < 1e-3


def test_swiglu_standalone_bitexact():
    g = torch.Generator().manual_seed(37)
    gu = randn_bf16((37, 2 * 9728), 3.0, g)
    out = K.swiglu(gu.to(DEV))
    assert np.array_equal(bits(out), oracle.swiglu(bits(gu)))
    assert torch.equal(out.cpu(), F.silu(gu[:, :9728]) * gu[:, 9728:])


# ---------------------------------------------------------------------------
# Boundary behaviour: errors, empty input, graph capture
# ---------------------------------------------------------------------------

def test_errors_are_raised_before_launch():
    a = torch.randn(4, 2560, device=DEV).to(BF16)
    w = torch.randn(64, 2560, device=DEV).to(BF16)
    with pytest.raises(SkError) as e:
        K.gemm(torch.randn(4, 2600, device=DEV).to(BF16)[:, :2568], torch.randn(64, 2568, device=DEV).to(BF16))
    assert e.value.status == SK_ERR_SHAPE        # K not a multiple of 32
    big = torch.randn(4, 2568, device=DEV).to(BF16)
    with pytest.raises(SkError) as e:
        K.gemm(big[:, 8:].contiguous()[:, :2560] if False else big[:, 1:2561], w)
    assert e.value.status == SK_ERR_ALIGN        # activation pointer off by 2 bytes
    with pytest.raises(SkError) as e:
        K.gemm(a, w, config=SkConfig.make(SK_PATH_MFMA, waves=1, ku=5, rows=16))
    assert e.value.status == SK_ERR_CONFIG       # K slice not covered
    cfg = SkConfig.make(SK_PATH_MFMA, waves=4, ku=10, rows=16, split=2)
    with pytest.raises(SkError) as e:
        K.gemm(a, w, config=cfg, ws=torch.empty(16, dtype=torch.uint8, device=DEV))
    assert e.value.status == SK_ERR_WORKSPACE
    with pytest.raises(ValueError):
        K.gemm(a.float(), w)


def test_empty_batch_is_a_noop():
    w = torch.randn(64, 2560, device=DEV).to(BF16)
    a = torch.empty(0, 2560, device=DEV, dtype=BF16)
    assert K.gemm(a, w).shape == (0, 64)


def test_graph_capture_replays_match_eager():
    """All entry points under one captured graph, replayed several times with
    eager work in between; every replay must equal the eager result."""
    M = 8
    x = _acts(M, 2560, seed=77).to(DEV)
    wq = _gpu(_weights(*QKV, seed=QKV[0] + QKV[1]))
    wgu = _gpu(_weights(*GU, seed=17))
    wl = _gpu(_weights(*LM, seed=7))
    I = GU[0] // 2
    mm = K.SkinnyMatmul(M, QKV[0], QKV[1], DEV)
    gu = K.SkinnyGateUp(M, I, GU[1], DEV, config=SkConfig.make(SK_PATH_MFMA, waves=4, ku=10, rows=16, split=2))
    lm = K.LmArgmax(M, LM[0], LM[1], DEV)
    eager = (mm(x, wq).clone(), gu(x, wgu[:I], wgu[I:]).clone(), *[t.clone() for t in lm(x, wl)])
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            mm(x, wq); gu(x, wgu[:I], wgu[I:]); lm(x, wl)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = (mm(x, wq), gu(x, wgu[:I], wgu[I:]), *lm(x, wl))
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, eager):
            assert torch.equal(a, b)
        K.gemm(x, wq)   # eager work between replays
        torch.cuda.synchronize()


def test_workspace_counters_reset_between_calls():
    """Split-K and argmax finish in the last-arriving workgroup using arrival
    counters in the workspace; every call must leave them at zero, so repeated
    calls on one workspace (and calls with smaller inputs) stay correct."""
    N, Kd = 2560, 9728
    w = _gpu(_weights(N, Kd, seed=N + Kd))
    cfg = SkConfig.make(SK_PATH_MFMA, waves=8, ku=10, rows=16, split=4)
    mm = K.SkinnyMatmul(8, N, Kd, DEV, config=cfg)
    x = _acts(8, Kd, seed=4)
    ref = _oracle_gemm(x, w.cpu())
    outs = [mm(x.to(DEV), w) for _ in range(3)]
    for o in outs:
        assert torch.equal(o, outs[0])
    assert_parity(outs[0], ref, "split-K repeated")
    lm = K.LmArgmax(8, LM[0], LM[1], DEV)
    wl = _gpu(_weights(*LM, seed=7))
    xs = _acts(8, LM[1], seed=12).to(DEV)
    first = [t.clone() for t in lm(xs, wl)]
    for _ in range(2):
        again = lm(xs, wl)
        assert torch.equal(again[0], first[0]) and torch.equal(again[1], first[1])
    L = (torch.randn(4, 5000) * 3).to(BF16).to(DEV)
    ws = torch.zeros(K._lib.workspace_bytes(K.SK_OP_ARGMAX, 4, 5000, 0), dtype=torch.uint8, device=DEV)
    for _ in range(3):
        ids, _ = K.argmax(L, ws=ws)
        assert torch.equal(ids.cpu(), torch.argmax(L.cpu(), -1))


MFMT_CASES = {  # shape, 32-column units per wave (8: 256, 16: 512, 32: 1024), rows, global split
    "qkv": (QKV, 16, 16, 1),
    "o_proj": (O, 16, 16, 1),
    "down": (D, 16, 16, 3),
    "qkv_kw256_rows32": (QKV, 8, 32, 2),
    # four 256-column chunks per wave: down's last wave covers 1.5 chunks past K
    "down_kw1024": (D, 32, 16, 1),
    "down_kw1024_rows32": (D, 32, 32, 1),
    "o_proj_kw1024_split2": (O, 32, 16, 2),
}


def mfmt_config(Kd: int, ku: int, rows: int, split: int, M: int) -> SkConfig:
    """One K chunk per wave; above 32 rows use 256-column chunks and enough
    splits that at most 8 waves share a tile.  Four chunks per wave (ku=32)
    allow 8 waves per workgroup up to 16 rows and 4 above (registers)."""
    if M > 32:
        ku, rows = 8, 16
        split = max(split, 1)
        while -(-(Kd // 256) // split) > 8:
            split += 1
    chunks = -(-Kd // (32 * ku))
    if ku == 32:
        while -(-chunks // split) > (8 if M <= 16 else 4):
            split += 1
    return SkConfig.make(SK_PATH_MFMA_LDS, waves=-(-chunks // split), ku=ku, rows=rows, split=split)


@pytest.mark.parametrize("case", list(MFMT_CASES))
@pytest.mark.parametrize("M", [1, 8, 16, 40, 64])
def test_mfma_lds_path_qwen_shapes(case, M):
    (N, Kd), ku, rows, split = MFMT_CASES[case]
    cfg = mfmt_config(Kd, ku, rows, split, M)
    w = _weights(N, Kd, seed=N + Kd)
    x = _acts(M, Kd, seed=N)
    out = K.gemm(x.to(DEV), _gpu(w), config=cfg)
    assert_parity(out, _oracle_gemm(x, w), f"mfma_lds {case} M={M} {cfg}")


@pytest.mark.parametrize("Kd", [2592, 1056, 4096 + 288])
@pytest.mark.parametrize("M", [3, 16])
def test_mfma_lds_multi_chunk_ragged_k(Kd, M):
    """Waves of four 256-column chunks where K ends inside a chunk (per-lane
    zero columns) and inside a wave (chunks past K load zeros)."""
    N = 200
    units = -(-Kd // 1024)
    cfg = SkConfig.make(SK_PATH_MFMA_LDS, waves=units, ku=32, rows=16, split=1)
    w = _weights(N, Kd, seed=Kd)
    x = _acts(M, Kd, seed=Kd + 1)
    out = K.gemm(x.to(DEV), _gpu(w), config=cfg)
    assert_parity(out, _oracle_gemm(x, w), f"mfma_lds ragged K={Kd} M={M} {cfg}")


@pytest.mark.parametrize("M", [1, 8, 40])
def test_mfma_lds_path_gateup(M):
    I2, Kd = GU
    I = I2 // 2
    wgu = _weights(I2, Kd, seed=17)
    x = _acts(M, Kd, seed=17)
    wd = _gpu(wgu)
    cfg = mfmt_config(Kd, 16, 16, 1, M)
    out = K.gateup_swiglu(x.to(DEV), wd[:I], wd[I:], config=cfg)
    assert_gateup_parity(out, bits(x), bits(wgu[:I]), bits(wgu[I:]), f"mfma_lds gateup M={M}")
