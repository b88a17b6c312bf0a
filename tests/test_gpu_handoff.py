"""GPU parity of the residual hand-off ops (needs an MI355X).

The add + RMSNorm between two projections of a decoder layer
(engine/model.py:202-210) split across the two kernels:

  * producer sk_gemm_residual_bf16: r_out = bf16(r + y) with y the projection
    that sk_gemm_bf16 computes with the same configuration, bit for bit, and
    the fp32 sums of r_out^2 over each 16-column group (checked against an
    fp64 sum);
  * consumers sk_rmsnorm_pre_*: on "exact-stats" inputs (values in
    {0, +-0.5, ..., +-2}, whose squares and every partial sum are exact in fp32
    in any order) rstd is order-independent, so they must equal the unfused
    HIP pipeline (add + RMSNorm kernel, then the projection with the same
    configuration) bit for bit; on random inputs they meet the parity rule
    against the oracle's projection of the oracle's normalised rows.

At M = 49-64 both run as row groups (producers: two or three groups of up to
32 rows; consumers: four groups of 16 rows).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from starter_amd import kernels as K
from starter_amd._lib import SK_ERR_ALIAS, SK_ERR_SHAPE, SK_OP_RESID_GEMM, SkError, default_config
from tests._util import BF16, assert_gateup_parity, assert_parity, bits, check_argmax_rows, from_bits, randn_bf16

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
EPS = 1e-6
H = 2560


def _sums16(ro: torch.Tensor) -> torch.Tensor:
    """fp64 sums of squares over 16-column groups of a [M, N] bf16 tensor."""
    M, N = ro.shape
    G = (N + 15) // 16
    f = torch.zeros((M, G * 16), dtype=torch.float64)
    f[:, :N] = ro.double()
    return f.pow(2).view(M, G, 16).sum(-1)


def _rand(shape, seed, scale=1.0):
    return randn_bf16(shape, scale, torch.Generator().manual_seed(seed))


def _gain(seed):
    g = torch.Generator().manual_seed(seed)
    return (1 + 0.1 * torch.randn(H, generator=g)).to(BF16)


def _exact(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randint(-4, 5, shape, generator=g).float() * 0.5).to(BF16)


# ---------------------------------------------------------------------------
# producer
# ---------------------------------------------------------------------------

PRODUCER_CASES = {   # (N, K): o_proj, down (split-K with fixup at M >= 2), ragged N
    "o_proj": (2560, 4096),
    "down": (2560, 9728),
    "ragged": (200, 512),
}


@pytest.mark.parametrize("case", list(PRODUCER_CASES))
@pytest.mark.parametrize("M", [1, 5, 16, 32, 50, 64, 100, 128])
def test_gemm_residual_bit_exact_against_gemm_plus_add(case, M):
    N, Kd = PRODUCER_CASES[case]
    a, w, r = _rand((M, Kd), 1 + M), _rand((N, Kd), 2, 0.02), _rand((M, N), 3 + M)
    cfg = default_config(SK_OP_RESID_GEMM, M, N, Kd)
    ad, wd, rd = a.to(DEV), w.to(DEV), r.to(DEV)
    y = K.gemm(ad, wd, config=cfg)   # the projection the producer adds (same configuration)
    ro = torch.empty_like(rd)
    sq = torch.full((M, K.sumsq_groups(M, N)), float("nan"), dtype=torch.float32, device=DEV)
    K.gemm_residual(ad, wd, rd, ro, sq, config=cfg)
    torch.cuda.synchronize()
    assert_parity(y, from_bits(oracle.gemm(bits(a), bits(w))), f"projection {case} M={M} {cfg}")
    want = (r.float() + y.cpu().float()).to(BF16)
    assert torch.equal(ro.cpu().view(torch.int16), want.view(torch.int16)), f"residual {case} M={M}"
    ref = _sums16(want)
    got = sq.cpu().double()
    assert torch.all(torch.isfinite(got))
    assert torch.allclose(got, ref, rtol=2e-6, atol=0), (got - ref).abs().max().item()


def test_gemm_residual_in_place():
    """r_out may be r: each element is read and then written by one thread."""
    M, N, Kd = 8, 2560, 4096
    a, w, r = _rand((M, Kd), 11), _rand((N, Kd), 12, 0.02), _rand((M, N), 13)
    ad, wd = a.to(DEV), w.to(DEV)
    y = K.gemm(ad, wd, config=default_config(SK_OP_RESID_GEMM, M, N, Kd))
    rd = r.to(DEV)
    sq = torch.empty((M, N // 16), dtype=torch.float32, device=DEV)
    K.gemm_residual(ad, wd, rd, rd, sq)
    want = (r.float() + y.cpu().float()).to(BF16)
    assert torch.equal(rd.cpu().view(torch.int16), want.view(torch.int16))


def test_gemm_residual_rejects_aliasing_and_large_m():
    M, N, Kd = 4, 512, 512
    a = torch.zeros((M, Kd), dtype=BF16, device=DEV)
    w = torch.zeros((N, Kd), dtype=BF16, device=DEV)
    sq = torch.zeros((M, N // 16), dtype=torch.float32, device=DEV)
    with pytest.raises(SkError) as e:
        K.gemm_residual(a, w, a, a, sq)   # r_out overlaps the projection's input
    assert e.value.status == SK_ERR_ALIAS
    big = torch.zeros((129, Kd), dtype=BF16, device=DEV)   # more rows than one launch
    rr = torch.zeros((129, N), dtype=BF16, device=DEV)
    with pytest.raises(SkError) as e:
        K.gemm_residual(big, w, rr, torch.empty_like(rr), torch.zeros((129, N // 16), dtype=torch.float32,
                                                                       device=DEV))
    assert e.value.status == SK_ERR_SHAPE


# ---------------------------------------------------------------------------
# consumers
# ---------------------------------------------------------------------------

def _sq_of(x: torch.Tensor) -> torch.Tensor:
    return _sums16(x).float().to(DEV)


@pytest.mark.parametrize("M", [1, 3, 8, 16, 64, 128])
def test_rmsnorm_pre_gemm_exact_stats_equals_unfused_pipeline(M):
    x, wn, w = _exact((M, H), 20 + M), _gain(120), _rand((6144, H), 21, 0.02)
    xd, wnd, wd = x.to(DEV), wn.to(DEV), w.to(DEV)
    cfg = default_config(8, M, 6144, H)   # SK_OP_PRE_GEMM
    got = K.rmsnorm_pre_gemm(xd, _sq_of(x), wnd, EPS, wd, config=cfg)
    ref = K.rmsnorm_gemm(xd, torch.zeros_like(xd), wnd, EPS, torch.empty_like(xd), wd, config=cfg)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("M", [1, 8, 16, 64, 128])
def test_rmsnorm_pre_gateup_exact_stats_equals_unfused_pipeline(M):
    I = 9728
    x, wn, wgu = _exact((M, H), 30 + M), _gain(130), _rand((2 * I, H), 31, 0.02)
    xd, wnd, wgud = x.to(DEV), wn.to(DEV), wgu.to(DEV)
    cfg = default_config(9, M, I, H)   # SK_OP_PRE_GATEUP
    got = K.rmsnorm_pre_gateup_swiglu(xd, _sq_of(x), wnd, EPS, wgud[:I], wgud[I:], config=cfg)
    ref = K.rmsnorm_gateup_swiglu(xd, torch.zeros_like(xd), wnd, EPS, torch.empty_like(xd), wgud[:I], wgud[I:],
                                  config=cfg)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("M", [1, 8, 16, 64, 128])
def test_rmsnorm_pre_lm_argmax_exact_stats_equals_unfused_pipeline(M):
    V = 151936
    x, wn, w = _exact((M, H), 40 + M), _gain(140), _rand((V, H), 41, 0.02)
    xd, wnd, wd = x.to(DEV), wn.to(DEV), w.to(DEV)
    cfg = default_config(10, M, V, H)   # SK_OP_PRE_LM_ARGMAX
    ids, mv = K.rmsnorm_pre_lm_argmax(xd, _sq_of(x), wnd, EPS, wd, config=cfg)
    rids, rmv = K.rmsnorm_lm_argmax(xd, torch.zeros_like(xd), wnd, EPS, torch.empty_like(xd), wd, config=cfg)
    torch.cuda.synchronize()
    assert torch.equal(ids, rids) and torch.equal(mv, rmv)


@pytest.mark.parametrize("M", [1, 16, 50, 64, 100])
def test_rmsnorm_pre_gemm_random_against_oracle(M):
    x, wn, w = _rand((M, H), 50 + M), _gain(150), _rand((6144, H), 51, 0.02)
    got = K.rmsnorm_pre_gemm(x.to(DEV), _sq_of(x), wn.to(DEV), EPS, w.to(DEV))
    _, h = oracle.add_rmsnorm(bits(x), np.zeros_like(bits(x)), bits(wn), EPS)
    assert_parity(got, from_bits(oracle.gemm(h, bits(w))), f"pre gemm M={M}")


@pytest.mark.parametrize("M", [1, 5, 16, 64, 128])
def test_rmsnorm_pre_gateup_random_against_oracle(M):
    """The gate/up consumer on random residual rows (M = 16 is the decode
    step's batch) against the oracle's add_rmsnorm + gate/up + SwiGLU."""
    I = 9728
    x, wn, wgu = _rand((M, H), 55 + M), _gain(155), _rand((2 * I, H), 56, 0.02)
    wgud = wgu.to(DEV)
    got = K.rmsnorm_pre_gateup_swiglu(x.to(DEV), _sq_of(x), wn.to(DEV), EPS, wgud[:I], wgud[I:])
    torch.cuda.synchronize()
    _, h = oracle.add_rmsnorm(bits(x), np.zeros_like(bits(x)), bits(wn), EPS)
    assert_gateup_parity(got, h, bits(wgu[:I]), bits(wgu[I:]), f"pre gateup M={M}")


@pytest.mark.parametrize("M", [1, 8, 16])
def test_rmsnorm_pre_lm_argmax_random_against_oracle(M):
    V = 151936
    x, wn, w = _rand((M, H), 60 + M), _gain(61), _rand((V, H), 62, 0.02)
    ids, mv = K.rmsnorm_pre_lm_argmax(x.to(DEV), _sq_of(x), wn.to(DEV), EPS, w.to(DEV))
    _, h = oracle.add_rmsnorm(bits(x), np.zeros_like(bits(x)), bits(wn), EPS)
    o_ids, o_max = oracle.lm_argmax(h, bits(w))
    check_argmax_rows(ids, mv, oracle.gemm(h, bits(w)), o_ids, o_max, "pre lm_argmax")


# ---------------------------------------------------------------------------
# producer -> consumer, against the reference's normed projection
# ---------------------------------------------------------------------------

def test_handoff_chain_matches_normed_projection_and_replays_in_a_graph():
    """o_proj producer then gate/up consumer == mm["gu"](xa, o, post_norm, xb, wgu)
    (xout bit-exact, output within the parity rule); the pair captured in a HIP
    graph and replayed with eager work in between gives the eager result."""
    M, I = 16, 9728
    a, wo, xa = _rand((M, 4096), 70), _rand((H, 4096), 71, 0.02), _rand((M, H), 72)
    wn, wgu = _gain(173), _rand((2 * I, H), 73, 0.02)
    ad, wod, xad, wnd, wgud = a.to(DEV), wo.to(DEV), xa.to(DEV), wn.to(DEV), wgu.to(DEV)
    xb = torch.empty_like(xad)
    sq = torch.empty((M, H // 16), dtype=torch.float32, device=DEV)
    ws_o = K._workspace(SK_OP_RESID_GEMM, M, H, 4096, None, DEV)
    ws_gu = K._workspace(9, M, I, H, None, DEV)
    out = torch.empty((M, I), dtype=BF16, device=DEV)

    def step():
        K.gemm_residual(ad, wod, xad, xb, sq, ws=ws_o)
        K.rmsnorm_pre_gateup_swiglu(xb, sq, wnd, EPS, wgud[:I], wgud[I:], out=out, ws=ws_gu)

    step()
    torch.cuda.synchronize()
    eager_xb, eager_out = xb.clone(), out.clone()
    o = K.gemm(ad, wod)   # the reference call shape: mm["o"] then mm["gu"] with the prologue
    xref = torch.empty_like(xad)
    ref = K.rmsnorm_gateup_swiglu(xad, o, wnd, EPS, xref, wgud[:I], wgud[I:])
    torch.cuda.synchronize()
    assert torch.equal(eager_xb.view(torch.int16), xref.view(torch.int16))
    diff = (eager_out.float() - ref.float()).abs()
    scale = ref.float().abs().clamp_min(1e-3 * ref.float().pow(2).mean().sqrt())
    assert (diff > 2e-2 * scale).float().mean() < 1e-3, "hand-off gate/up far from the normed projection"

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for _ in range(3):
        xb.zero_()
        out.zero_()
        sq.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(xb, eager_xb) and torch.equal(out, eager_out)
