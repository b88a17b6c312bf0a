"""GPU parity of the residual-add + RMSNorm prologue ops (needs an MI355X).

Call sites mm["qkv"], mm["gu"] and mm["lm"] (engine/model.py:202-210): xout =
x + y is written bit-exact and the projection consumes rms_norm(xout, w_norm)
(prologue engine/kernels/gemm.py:28-56 / 184-208, casts rmsnorm.py:34-45).

Two input families:
  * random N(0, 1) activations: xout bit-exact, outputs under the parity rule
    against the oracle's projection of the oracle's normalised rows (the
    kernel's fp32 row sum of squares may differ from the oracle's in the last
    bits, moving a few normalised values by one bf16 ulp);
  * "exact-stats" activations from {0, +-0.5, ..., +-2}: x + y and every partial
    sum of squares are exact in fp32 whatever the order, so rstd and the
    normalised rows are bit-identical everywhere; then the fused kernel must
    equal the unfused HIP pipeline (add_rms_norm, then the projection with the
    same configuration) bit for bit, and gate/up meets the full gate/up rule.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from starter_amd import kernels as K
from starter_amd._lib import SK_ERR_ALIAS, SK_PATH_GEMV, SK_PATH_MFMA, SK_PATH_MFMA_LDS, SkConfig, SkError
from tests._util import (BF16, assert_gateup_parity, assert_parity, bits, check_argmax_rows, from_bits, randn_bf16,
                         rel_violations)

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
EPS = 1e-6
H = 2560
QKV, GU, LM = 6144, 19456, 151936
M_SWEEP = [1, 2, 4, 8, 16, 32, 40, 64]

_cache: dict = {}


def _w(N: int, seed: int) -> torch.Tensor:
    """Weights [N, H] on the GPU (cached) and their CPU copy."""
    key = (N, seed)
    if key not in _cache:
        g = torch.Generator().manual_seed(seed)
        cpu = randn_bf16((N, H), 0.02, g)
        _cache[key] = (cpu, cpu.to(DEV))
    return _cache[key]


def _inputs(M: int, seed: int, exact: bool = False):
    g = torch.Generator().manual_seed(1000 + seed * 7 + M)
    if exact:
        x = (torch.randint(-4, 5, (M, H), generator=g).float() * 0.5).to(BF16)
        y = (torch.randint(-4, 5, (M, H), generator=g).float() * 0.25).to(BF16)
    else:
        x = randn_bf16((M, H), 1.0, g)
        y = randn_bf16((M, H), 1.0, g)
    wn = (1 + 0.1 * torch.randn(H, generator=g)).to(BF16)
    return x, y, wn


def _oracle_norm(x, y, wn):
    return oracle.add_rmsnorm(bits(x), bits(y), bits(wn), EPS)   # (xout bits, normalised bits)


def _dev(*ts):
    return [t.to(DEV) for t in ts]


# ---------------------------------------------------------------------------
# mm["qkv"] / mm["lm"] logits: add + RMSNorm + GEMM
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("M", M_SWEEP + [96])
def test_rmsnorm_gemm_qkv_default_config(M):
    wc, wd = _w(QKV, 1)
    x, y, wn = _inputs(M, 1)
    xd, yd, wnd = _dev(x, y, wn)
    xo = torch.empty_like(xd)
    out = K.rmsnorm_gemm(xd, yd, wnd, EPS, xo, wd)
    o_xout, o_h = _oracle_norm(x, y, wn)
    assert np.array_equal(bits(xo), o_xout), "xout must be bit-exact"
    assert_parity(out, from_bits(oracle.gemm(o_h, bits(wc))), f"rmsnorm qkv M={M}")
    assert np.array_equal(bits(xd), bits(x)) and np.array_equal(bits(yd), bits(y)), "inputs must be untouched"


@pytest.mark.parametrize("M", [1, 8, 32])
def test_rmsnorm_gemm_lm_logits(M):
    wc, wd = _w(LM, 2)
    x, y, wn = _inputs(M, 2)
    xd, yd, wnd = _dev(x, y, wn)
    xo = torch.empty_like(xd)
    out = K.rmsnorm_gemm(xd, yd, wnd, EPS, xo, wd)
    o_xout, o_h = _oracle_norm(x, y, wn)
    assert np.array_equal(bits(xo), o_xout)
    assert_parity(out, from_bits(oracle.gemm(o_h, bits(wc))), f"rmsnorm lm logits M={M}")


NORM_CONFIGS = {   # fused (GEMV, one split) and unfused (MFMA paths, global split)
    "gemv": SkConfig.make(SK_PATH_GEMV, waves=1, ku=5, rows=2),
    "gemv_4w": SkConfig.make(SK_PATH_GEMV, waves=4, ku=2, rows=2),
    "mfma_lds_256": SkConfig.make(SK_PATH_MFMA_LDS, waves=10, ku=8, rows=16),
    "mfma_lds_512": SkConfig.make(SK_PATH_MFMA_LDS, waves=5, ku=16, rows=16),
    "split2": SkConfig.make(SK_PATH_MFMA_LDS, waves=5, ku=8, rows=16, split=2),
    "mfma_regs": SkConfig.make(SK_PATH_MFMA, waves=8, ku=10, rows=16),
}


@pytest.mark.parametrize("name", list(NORM_CONFIGS))
@pytest.mark.parametrize("M", [1, 3, 8, 16])
def test_rmsnorm_gemm_exact_stats_equals_unfused_pipeline(name, M):
    cfg = NORM_CONFIGS[name]
    if cfg.path == SK_PATH_GEMV and M > 8:
        pytest.skip("the GEMV path takes at most 8 rows")
    wc, wd = _w(QKV, 3)
    x, y, wn = _inputs(M, 3, exact=True)
    xd, yd, wnd = _dev(x, y, wn)
    xo = torch.empty_like(xd)
    fused = K.rmsnorm_gemm(xd, yd, wnd, EPS, xo, wd, config=cfg)
    xo2 = torch.empty_like(xd)
    h = K.add_rms_norm(xd, yd, wnd, EPS, xo2)
    unfused = K.gemm(h, wd, config=cfg)
    o_xout, o_h = _oracle_norm(x, y, wn)
    assert np.array_equal(bits(h), o_h), "exact-stats rows: HIP add_rms_norm equals the oracle"
    assert np.array_equal(bits(xo), o_xout) and np.array_equal(bits(xo2), o_xout)
    assert torch.equal(fused, unfused), f"fused prologue differs from add_rms_norm + gemm ({name})"
    assert_parity(fused, from_bits(oracle.gemm(o_h, bits(wc))), f"exact-stats {name} M={M}")


# ---------------------------------------------------------------------------
# mm["gu"]: add + RMSNorm + gate/up + SwiGLU
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("M", M_SWEEP)
def test_rmsnorm_gateup_exact_stats(M):
    wc, wd = _w(GU, 4)
    I = GU // 2
    x, y, wn = _inputs(M, 4, exact=True)
    xd, yd, wnd = _dev(x, y, wn)
    xo = torch.empty_like(xd)
    out = K.rmsnorm_gateup_swiglu(xd, yd, wnd, EPS, xo, wd[:I], wd[I:])
    o_xout, o_h = _oracle_norm(x, y, wn)
    assert np.array_equal(bits(xo), o_xout)
    wb = bits(wc)
    assert_gateup_parity(out, o_h, wb[:I], wb[I:], f"rmsnorm gateup exact-stats M={M}")


@pytest.mark.parametrize("M", [1, 8, 16])
def test_rmsnorm_gateup_random(M):
    """Random rows: xout bit-exact; outputs within 1e-2 of the oracle's
    pipeline except where one bf16 ulp of a normalised value moves g or u
    across a rounding midpoint (bounded here to 1% of the elements)."""
    wc, wd = _w(GU, 4)
    I = GU // 2
    x, y, wn = _inputs(M, 5)
    xd, yd, wnd = _dev(x, y, wn)
    xo = torch.empty_like(xd)
    out = K.rmsnorm_gateup_swiglu(xd, yd, wnd, EPS, xo, wd[:I], wd[I:])
    o_xout, o_h = _oracle_norm(x, y, wn)
    assert np.array_equal(bits(xo), o_xout)
    wb = bits(wc)
    ref = oracle.gateup_swiglu(o_h, wb[:I], wb[I:])
    bad, worst = rel_violations(out, from_bits(ref), rtol=3e-2)
    assert bad <= out.numel() // 100, f"{bad} elements beyond 3e-2, worst ratio {worst:.3g}"


# ---------------------------------------------------------------------------
# mm["lm"] + argmax: add + RMSNorm + lm_head + greedy argmax
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("M", [1, 8, 32, 64])
def test_rmsnorm_lm_argmax(M):
    wc, wd = _w(LM, 2)
    x, y, wn = _inputs(M, 6)
    xd, yd, wnd = _dev(x, y, wn)
    xo = torch.empty_like(xd)
    ids, maxv = K.rmsnorm_lm_argmax(xd, yd, wnd, EPS, xo, wd)
    o_xout, o_h = _oracle_norm(x, y, wn)
    assert np.array_equal(bits(xo), o_xout)
    logits = oracle.gemm(o_h, bits(wc))
    o_ids, o_maxv = oracle.argmax(logits)
    check_argmax_rows(ids, maxv, logits, o_ids, o_maxv, f"rmsnorm lm_argmax M={M}")


# ---------------------------------------------------------------------------
# Drop-in pickers and graph capture
# ---------------------------------------------------------------------------

def test_pick_normed_signatures_and_graph_replay():
    """pick_normed / pick_lm_argmax return callables with the reference's
    (x, y, w_norm, xout, w) signature; captured into one graph and replayed
    they reproduce the eager results (workspace counters self-reset)."""
    M = 8
    wq = _w(QKV, 1)[1]
    wgu = _w(GU, 4)[1]
    wl = _w(LM, 2)[1]
    x, y, wn = _dev(*_inputs(M, 8))
    qkv = K.pick_normed("matmul", x, y, wn, wq, EPS)
    gu = K.pick_normed("gateup", x, y, wn, wgu, EPS)
    lm = K.pick_lm_argmax(x, wl, EPS)
    xa, xb, xc = (torch.empty_like(x) for _ in range(3))

    def step():
        return qkv(x, y, wn, xa, wq), gu(xa, y, wn, xb, wgu), *lm(xb, y, wn, xc, wl)

    eager = [t.clone() for t in step()]
    ref_x = [t.clone() for t in (xa, xb, xc)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = step()
    for _ in range(3):
        for t in (xa, xb, xc):
            t.zero_()
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, eager):
            assert torch.equal(a, b)
        for a, b in zip((xa, xb, xc), ref_x):
            assert torch.equal(a, b)
        K.rmsnorm_gemm(x, y, wn, EPS, torch.empty_like(x), wq)   # eager work between replays
        torch.cuda.synchronize()


def test_rmsnorm_alias_rejected():
    x, y, wn = _dev(*_inputs(4, 9))
    wq = _w(QKV, 1)[1]
    with pytest.raises(SkError) as e:
        K.rmsnorm_gemm(x, y, wn, EPS, x, wq)     # xout must not be x
    assert e.value.status == SK_ERR_ALIAS


def test_rmsnorm_empty_batch():
    wq = _w(QKV, 1)[1]
    x = torch.empty(0, H, dtype=BF16, device=DEV)
    assert K.rmsnorm_gemm(x, x.clone(), torch.ones(H, dtype=BF16, device=DEV), EPS, x.clone(), wq).shape == (0, QKV)
