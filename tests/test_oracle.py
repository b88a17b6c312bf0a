"""Pin the CPU oracle before trusting it (CPU only).

Every oracle function is checked against (a) torch's CPU library routine for
the same reference function, (b) a closed form or exact special case that the
mathematics fixes, and (c) the committed golden fixtures.  The
``test_pins_reject_planted_mistakes`` cases feed deliberately broken oracles
(dropped term, transposed operand, wrong cast order, wrong tie rule) through
the same checks and require each to be caught.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from tests._util import BF16, assert_parity, bits, from_bits, randn_bf16, rel_violations

GOLDEN = Path(__file__).resolve().parent / "golden"


def _golden(name: str):
    return np.load(GOLDEN / f"{name}.npz", allow_pickle=False)


# --------------------------------------------------------------------------
# checks shared by the real oracle and the planted-mistake variants
# --------------------------------------------------------------------------

def _check_gemm_vs_torch(gemm_fn, M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = randn_bf16((M, K), 1.0, g)
    w = randn_bf16((N, K), 0.02, g)
    out = from_bits(gemm_fn(bits(x), bits(w)))
    ref = F.linear(x, w)
    bad, _ = rel_violations(out, ref)
    return bad == 0 and (out != ref).float().mean().item() < 0.01


def _check_gemm_exact_integers(gemm_fn):
    """Small integers: every product and partial sum is exact in fp32, so the
    only correct answer is the exact one.  M != N pins operand orientation."""
    rng = np.random.default_rng(7)
    M, N, K = 5, 11, 96
    a = rng.integers(-3, 4, size=(M, K)).astype(np.float32)
    w = rng.integers(-3, 4, size=(N, K)).astype(np.float32)
    exact = a @ w.T
    out = oracle.bf16_to_f32(gemm_fn(oracle.f32_to_bf16(a), oracle.f32_to_bf16(w)))
    return np.array_equal(out, oracle.bf16_to_f32(oracle.f32_to_bf16(exact)))


def _check_swiglu(swiglu_fn):
    g = torch.Generator().manual_seed(3)
    gu = randn_bf16((4, 2 * 700), 3.0, g)
    ref = F.silu(gu[:, :700]) * gu[:, 700:]
    return torch.equal(from_bits(swiglu_fn(bits(gu))), ref)


def _check_argmax(argmax_fn):
    d = _golden("argmax_m7_v1000")
    ids, maxv = argmax_fn(d["logits"])
    return np.array_equal(ids, d["ids"]) and np.array_equal(maxv, d["maxv"], equal_nan=True)


# --------------------------------------------------------------------------
# GEMM
# --------------------------------------------------------------------------

@pytest.mark.parametrize("M,N,K", [(1, 6144, 2560), (8, 6144, 2560), (8, 2560, 4096), (4, 2560, 9728),
                                   (16, 777, 2560), (40, 512, 2560), (64, 256, 2560), (3, 40, 96)])
def test_oracle_gemm_matches_torch_linear(M, N, K):
    assert _check_gemm_vs_torch(oracle.gemm, M, N, K, seed=M * 1000 + N)


def test_oracle_gemm_exact_integer_products():
    assert _check_gemm_exact_integers(oracle.gemm)


def test_oracle_gemm_one_hot_weights_gather_columns():
    """W row n = e_{p(n)}: C[:, n] must be A[:, p(n)] bit for bit."""
    g = torch.Generator().manual_seed(11)
    M, K, N = 6, 2560, 300
    x = randn_bf16((M, K), 1.0, g)
    perm = torch.randperm(K, generator=g)[:N]
    w = torch.zeros(N, K, dtype=BF16)
    w[torch.arange(N), perm] = 1.0
    out = from_bits(oracle.gemm(bits(x), bits(w)))
    assert torch.equal(out, x[:, perm])


def test_oracle_gemm_f32_close_to_fp64():
    """The fp32 sums stay within the fp32 accumulation bound K*u*sum|a*w| of fp64."""
    g = torch.Generator().manual_seed(5)
    M, N, K = 8, 1024, 9728
    x = randn_bf16((M, K), 1.0, g)
    w = randn_bf16((N, K), 0.02, g)
    f32 = torch.from_numpy(oracle.gemm_f32(bits(x), bits(w))).double()
    exact = x.double() @ w.double().T
    bound = K * 2.0 ** -24 * (x.double().abs() @ w.double().abs().T)
    assert bool(((f32 - exact).abs() <= bound).all())
    # The bf16 result is the rounding of the fp32 sum.
    out = oracle.gemm(bits(x), bits(w))
    assert np.array_equal(out, oracle.f32_to_bf16(f32.float().numpy()))


@pytest.mark.parametrize("name", ["gemm_m3_n40_k96", "gemm_m1_n48_k2560", "gemm_m19_n33_k256"])
def test_oracle_gemm_golden(name):
    d = _golden(name)
    out = from_bits(oracle.gemm(d["x"], d["w"]))
    assert_parity(out, from_bits(d["y"]), name)


# --------------------------------------------------------------------------
# SwiGLU and gate/up
# --------------------------------------------------------------------------

def test_oracle_swiglu_bitexact_vs_torch():
    assert _check_swiglu(oracle.swiglu)


def test_oracle_swiglu_every_bf16_gate_value():
    """All 65536 bf16 gate values against F.silu(g) * u (torch CPU)."""
    gvals = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(BF16)
    finite = torch.isfinite(gvals.float())
    gvals = gvals[finite]
    u = torch.full_like(gvals, 1.5)
    gu = torch.stack([gvals, u]).T.contiguous().view(-1, 2)   # M rows of [g | u] with I = 1
    out = from_bits(oracle.swiglu(bits(gu)))[:, 0]
    ref = F.silu(gvals) * u
    assert torch.equal(out, ref)


def test_oracle_swiglu_golden():
    d = _golden("swiglu_m3_i512")
    assert np.array_equal(oracle.swiglu(d["gu"]), d["y"])


@pytest.mark.parametrize("M,I,K", [(1, 9728, 2560), (8, 2048, 2560), (16, 512, 2560), (3, 24, 256)])
def test_oracle_gateup_matches_torch(M, I, K):
    g = torch.Generator().manual_seed(M + I)
    x = randn_bf16((M, K), 1.0, g)
    wgu = randn_bf16((2 * I, K), 0.02, g)
    out = from_bits(oracle.gateup_swiglu(bits(x), bits(wgu[:I]), bits(wgu[I:])))
    ref = F.silu(F.linear(x, wgu[:I])) * F.linear(x, wgu[I:])
    # F.linear's own summation order differs from the oracle's; the epilogue
    # then amplifies a 1-ulp difference of g or u by at most one more rounding.
    assert_parity(out, ref, f"gateup M={M}")
    # Same arithmetic composed from the oracle's own pieces is bit-exact.
    g32 = oracle.gemm(bits(x), bits(wgu[:I]))
    u32 = oracle.gemm(bits(x), bits(wgu[I:]))
    assert np.array_equal(out.view(torch.int16).numpy().view(np.uint16),
                          oracle.swiglu(np.concatenate([g32, u32], axis=1)))


def test_oracle_gateup_golden():
    d = _golden("gateup_m2_i24_k256")
    I = d["wgu"].shape[0] // 2
    out = from_bits(oracle.gateup_swiglu(d["x"], d["wgu"][:I], d["wgu"][I:]))
    assert_parity(out, from_bits(d["y"]), "gateup golden")


# --------------------------------------------------------------------------
# Residual add + RMSNorm
# --------------------------------------------------------------------------

def _ref_rmsnorm(x, w, eps):
    h = x.float()
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return w * h.to(x.dtype)


@pytest.mark.parametrize("M,K", [(1, 2560), (9, 2560), (5, 4096), (3, 128)])
def test_oracle_add_rmsnorm_matches_closed_form(M, K):
    g = torch.Generator().manual_seed(M * K)
    x = randn_bf16((M, K), 1.0, g)
    y = randn_bf16((M, K), 1.0, g)
    w = (1 + 0.1 * torch.randn(K, generator=g)).to(BF16)
    xout, out = oracle.add_rmsnorm(bits(x), bits(y), bits(w), 1e-6)
    assert torch.equal(from_bits(xout), x + y)          # bit-exact residual stream
    ref = _ref_rmsnorm(x + y, w, 1e-6)
    o = from_bits(out)
    # rstd can differ from torch's by the fp32 summation order of sum(s^2):
    # then bf16(s * r) moves by one ulp and the weight product by at most two.
    diff = (o.float() - ref.float()).abs()
    two_ulp = ref.float().abs() * 2.0 ** -6 + 1e-30
    assert bool((diff <= two_ulp).all())
    assert (o != ref).float().mean().item() < 1e-3


def test_oracle_add_rmsnorm_golden():
    d = _golden("add_rmsnorm_m4_k2560")
    xout, out = oracle.add_rmsnorm(d["x"], d["y"], d["w"], float(d["eps"]))
    assert np.array_equal(xout, d["xout"])
    assert (out != d["out"]).mean() < 1e-3


# --------------------------------------------------------------------------
# Argmax and lm_head + argmax
# --------------------------------------------------------------------------

def test_oracle_argmax_golden_ties_nan_signed_zero():
    assert _check_argmax(oracle.argmax)


@pytest.mark.parametrize("M,V", [(3, 151936), (64, 1024), (5, 1)])
def test_oracle_argmax_matches_torch(M, V):
    g = torch.Generator().manual_seed(V)
    L = (torch.randn(M, V, generator=g) * 4).to(BF16)
    if V > 300:
        L[0, 7] = L[0].max() + 1
        L[1, 100] = L[1, 200] = L[1].max() + 2
    ids, maxv = oracle.argmax(bits(L))
    assert np.array_equal(ids, torch.argmax(L, -1).numpy())
    assert np.array_equal(maxv, L.max(-1).values.float().numpy())


def test_oracle_lm_argmax_golden_and_consistency():
    d = _golden("lm_argmax_m4_v777_k128")
    ids, maxv = oracle.lm_argmax(d["x"], d["w"])
    # Against torch's logits: wherever the bf16 top-2 differ, the pick must agree.
    L = from_bits(d["logits"]).float()
    top2 = torch.topk(L, 2, dim=-1).values
    for m in range(L.shape[0]):
        if top2[m, 0] - top2[m, 1] > 1e-2:
            assert ids[m] == d["ids"][m]
    # Against the oracle's own gemm + argmax: identical arithmetic, identical answer.
    gi, gv = oracle.argmax(oracle.gemm(d["x"], d["w"]))
    assert np.array_equal(ids, gi) and np.array_equal(maxv, gv)


def test_f32_to_bf16_rounding_matches_torch():
    vals = np.array([1.0, 1.00390625, 1.01171875, 1.0039062, 1.0039063, -2.5, 3.4028235e38, 3.39e38,
                     1e-40, -1e-45, 0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 1.9921875, 0.1],
                    dtype=np.float32)
    rng = np.random.default_rng(0)
    vals = np.concatenate([vals, rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000)])
    ref = torch.from_numpy(vals).to(BF16).view(torch.int16).numpy().view(np.uint16)
    # NaN payloads are not part of the contract (torch's own scalar and
    # vectorised conversions disagree on them): compare NaN-ness only there.
    nan = np.isnan(vals)
    out = oracle.f32_to_bf16(vals)
    assert np.array_equal(out[~nan], ref[~nan])
    assert bool(np.isnan(oracle.bf16_to_f32(out[nan])).all())
    assert all(oracle.f32_to_bf16_c(float(v)) == int(r) for v, r, n in zip(vals[:200], ref[:200], nan[:200]) if not n)


# --------------------------------------------------------------------------
# The pins catch plausible mistakes (planted in CPU-side variants)
# --------------------------------------------------------------------------

def _dropped_tail(a, w):
    return oracle.gemm(np.ascontiguousarray(a[:, :-32]), np.ascontiguousarray(w[:, :-32]))


def _transposed(a, w):
    # Interprets W as [K, N] (column-major weight): rows become columns.
    K = a.shape[1]
    wt = np.ascontiguousarray(w.reshape(-1)[: w.size].reshape(K, -1).T) if w.shape[0] != K else w.T.copy()
    return oracle.gemm(a, np.ascontiguousarray(wt[: w.shape[0]]))


def _sign_flip(a, w):
    return oracle.gemm(a, w ^ np.uint16(0x8000))


def _swiglu_one_rounding(gu):
    # silu product rounded once instead of twice (a wrong cast placement).
    f = oracle.bf16_to_f32(gu)
    I = f.shape[1] // 2
    g, u = f[:, :I], f[:, I:]
    return oracle.f32_to_bf16((g / (1 + np.exp(-g))) * u)


def _argmax_last_tie(L):
    f = oracle.bf16_to_f32(L)
    ids = f.shape[1] - 1 - np.argmax(f[:, ::-1], axis=1)
    return ids.astype(np.int64), np.nanmax(f, axis=1).astype(np.float32)


@pytest.mark.parametrize("variant", ["dropped_tail", "transposed", "sign_flip"])
def test_pins_reject_planted_gemm_mistakes(variant):
    fn = {"dropped_tail": _dropped_tail, "transposed": _transposed, "sign_flip": _sign_flip}[variant]
    caught = (not _check_gemm_exact_integers(fn)) or (not _check_gemm_vs_torch(fn, 8, 96, 96, seed=1))
    assert caught


def test_pins_reject_planted_swiglu_and_argmax_mistakes():
    assert not _check_swiglu(_swiglu_one_rounding)
    assert not _check_argmax(_argmax_last_tie)


def test_gateup_parity_rule_accepts_reference_pipeline_and_rejects_wrong_epilogue():
    """The gate/up rule used by the GPU tests: torch's own pipeline (another
    fp32 summation order) passes; a one-rounding epilogue does not."""
    from tests._util import gateup_violations

    g = torch.Generator().manual_seed(4)
    x = randn_bf16((4, 2560), 1.0, g)
    w = randn_bf16((2 * 9728, 2560), 0.02, g)
    xb, wg, wu = bits(x), bits(w[:9728]), bits(w[9728:])
    good = F.silu(F.linear(x, w[:9728])) * F.linear(x, w[9728:])
    bad, _, exact = gateup_violations(good, xb, wg, wu)
    assert bad == 0 and exact == 1.0
    wrong = (F.silu(F.linear(x, w[:9728]).float()) * F.linear(x, w[9728:]).float()).to(BF16)
    _, _, exact = gateup_violations(wrong, xb, wg, wu)
    assert exact < 0.9


# --------------------------------------------------------------------------
# q/k RMSNorm + RoPE + KV-cache write (engine/kernels/rope.py)
# --------------------------------------------------------------------------

def rope_tables_cpu(D: int, theta: float, max_pos: int):
    """cos/sin bf16 tables built the way the reference builds them
    (engine/model.py:85-100): fp32 inv_freq, fp32 outer product, cat, cos/sin, bf16."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.int64).float() / D))
    positions = torch.arange(max_pos, dtype=torch.float32)
    freqs = (inv_freq[:, None].float() @ positions[None, :].float()).transpose(0, 1)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(BF16).contiguous(), emb.sin().to(BF16).contiguous()


def _torch_rope_reference(qkv, qw, kw, cos, sin, start, B, T, HQ, HKV, D, eps, positions=None):
    """The reference test's composition (tests/test_kernels.py:11-19, 45-53) on the CPU.
    ``positions`` [T]: the rotary position of each row (default start + t)."""
    def ref_rmsnorm(x, w):
        h = x.float()
        h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
        return w * h.to(x.dtype)

    def rotate_half(x):
        x1, x2 = x[..., : x.shape[-1] // 2], x[..., x.shape[-1] // 2:]
        return torch.cat((-x2, x1), dim=-1)

    q = qkv[:, : HQ * D].view(B, T, HQ, D)
    k = qkv[:, HQ * D:(HQ + HKV) * D].view(B, T, HKV, D)
    v = qkv[:, (HQ + HKV) * D:].view(B, T, HKV, D)
    if positions is None:
        positions = torch.arange(start, start + T)
    c = cos[positions][None, :, None, :]
    s = sin[positions][None, :, None, :]
    qn, kn = ref_rmsnorm(q, qw), ref_rmsnorm(k, kw)
    q_ref = ((qn * c) + (rotate_half(qn) * s)).transpose(1, 2)
    k_ref = ((kn * c) + (rotate_half(kn) * s)).transpose(1, 2)
    return q_ref, k_ref, v.transpose(1, 2)


@pytest.mark.parametrize("B,T,HQ,HKV,start", [(2, 5, 8, 2, 3), (3, 1, 32, 8, 700), (1, 16, 4, 4, 0)])
def test_oracle_rope_matches_reference_composition(B, T, HQ, HKV, start):
    D, CAP, eps = 128, start + T + 4, 1e-6
    g = torch.Generator().manual_seed(B * 100 + T)
    cos, sin = rope_tables_cpu(D, 5e6, CAP)
    qkv = randn_bf16((B * T, (HQ + 2 * HKV) * D), 1.0, g)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(BF16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(BF16)
    q_out = np.zeros((B, HQ, T, D), np.uint16)
    kc = np.zeros((B, HKV, CAP, D), np.uint16)
    vc = np.zeros((B, HKV, CAP, D), np.uint16)
    pos = np.full(B, start, np.int32)
    oracle.qk_norm_rope_cache(bits(qkv), bits(qw), bits(kw), bits(cos), bits(sin), pos, q_out, kc, vc, T, eps)
    q_ref, k_ref, v_ref = _torch_rope_reference(qkv, qw, kw, cos, sin, start, B, T, HQ, HKV, D, eps)
    # torch's CPU rsqrt and the oracle's 1/sqrt may differ in the last fp32
    # bit, which moves a normalised value by one bf16 ulp on rare elements
    qd = np.abs(q_out.astype(np.int32) - bits(q_ref).astype(np.int32))
    kd = np.abs(kc[:, :, start:start + T].astype(np.int32) - bits(k_ref).astype(np.int32))
    assert qd.max() <= 2 and (qd != 0).mean() < 2e-3, (qd.max(), (qd != 0).mean())
    assert kd.max() <= 2 and (kd != 0).mean() < 2e-3
    assert np.array_equal(vc[:, :, start:start + T], bits(v_ref))
    untouched = np.ones(CAP, bool)
    untouched[start:start + T] = False
    assert not kc[:, :, untouched].any() and not vc[:, :, untouched].any()


def test_oracle_rope_position_zero_is_norm_only():
    """At position 0, cos = 1 and sin = 0: the rotation is the identity, so the
    output is the per-head RMSNorm of the row, y = bf16(w * bf16(x * r))."""
    D, eps = 128, 1e-6
    g = torch.Generator().manual_seed(3)
    cos, sin = rope_tables_cpu(D, 1e6, 4)
    assert torch.all(cos[0] == 1) and torch.all(sin[0] == 0)
    qkv = randn_bf16((1, 3 * D), 2.0, g)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(BF16)
    q_out = np.zeros((1, 1, 1, D), np.uint16)
    kc = np.zeros((1, 1, 2, D), np.uint16)
    vc = np.zeros_like(kc)
    oracle.qk_norm_rope_cache(bits(qkv), bits(qw), bits(qw), bits(cos), bits(sin), np.zeros(1, np.int32), q_out, kc,
                              vc, 1, eps)
    x = qkv[0, :D].double()
    r = 1.0 / torch.sqrt((x * x).mean() + eps)
    y = (qw.float() * (x * r).float().to(BF16).float()).to(BF16)
    assert np.array_equal(q_out[0, 0, 0], bits(y))


def _rope_inputs(B, T, HQ, HKV, cap, seed, theta=1e6):
    g = torch.Generator().manual_seed(seed)
    cos, sin = rope_tables_cpu(128, theta, cap)
    qkv = randn_bf16((B * T, (HQ + 2 * HKV) * 128), 1.0, g)
    qw = (1 + 0.1 * torch.randn(128, generator=g)).to(BF16)
    kw = (1 + 0.1 * torch.randn(128, generator=g)).to(BF16)
    return qkv, qw, kw, cos, sin


def _oracle_rope(qkv, qw, kw, cos, sin, pos, B, T, HQ, HKV, cap, eps=1e-6, depth=None):
    q_out = np.zeros((B, HQ, T, 128), np.uint16)
    kc = np.zeros((B, HKV, cap, 128), np.uint16)
    vc = np.zeros((B, HKV, cap, 128), np.uint16)
    oracle.qk_norm_rope_cache(bits(qkv), bits(qw), bits(kw), bits(cos), bits(sin), np.asarray(pos, np.int32), q_out,
                              kc, vc, T, eps, depth=depth)
    return q_out, kc, vc


def test_oracle_rope_tree_depth_matches_reference_composition():
    """Draft-tree rows (engine/kernels/rope.py:94-122, DEPTH): row t goes to
    cache slot pos + t but rotates by position pos + depth[t]; siblings share a
    depth.  Against the reference test's composition with per-row positions."""
    B, T, HQ, HKV, start, eps = 2, 6, 8, 2, 40, 1e-6
    depth = np.array([0, 1, 1, 2, 2, 3], np.int32)   # root, two children, two grandchildren, ...
    cap = start + T + 4
    qkv, qw, kw, cos, sin = _rope_inputs(B, T, HQ, HKV, cap, seed=21)
    q_out, kc, vc = _oracle_rope(qkv, qw, kw, cos, sin, [start] * B, B, T, HQ, HKV, cap, eps, depth)
    q_ref, k_ref, v_ref = _torch_rope_reference(qkv, qw, kw, cos, sin, start, B, T, HQ, HKV, 128, eps,
                                                positions=torch.from_numpy(start + depth).long())
    qd = np.abs(q_out.astype(np.int32) - bits(q_ref).astype(np.int32))
    kd = np.abs(kc[:, :, start:start + T].astype(np.int32) - bits(k_ref).astype(np.int32))
    assert qd.max() <= 2 and (qd != 0).mean() < 2e-3, (qd.max(), (qd != 0).mean())
    assert kd.max() <= 2 and (kd != 0).mean() < 2e-3
    assert np.array_equal(vc[:, :, start:start + T], bits(v_ref))   # slots pos + t, raw values
    # the chain angles (pos + t) would give a different result for the rows whose depth != t
    q_chain, _, _ = _oracle_rope(qkv, qw, kw, cos, sin, [start] * B, B, T, HQ, HKV, cap, eps)
    assert not np.array_equal(q_chain[:, :, 2], q_out[:, :, 2])


def test_oracle_rope_depth_identities():
    """depth = 0..T-1 is the chain, bit for bit; a row rotated at depth d equals
    the same row alone in a chain at position pos + d; depth = -pos rotates by
    position 0, i.e. the per-head RMSNorm alone."""
    B, T, HQ, HKV, start = 1, 5, 4, 2, 9
    cap = start + T + 2
    qkv, qw, kw, cos, sin = _rope_inputs(B, T, HQ, HKV, cap, seed=22)
    chain = _oracle_rope(qkv, qw, kw, cos, sin, [start], B, T, HQ, HKV, cap)
    same = _oracle_rope(qkv, qw, kw, cos, sin, [start], B, T, HQ, HKV, cap, depth=np.arange(T, dtype=np.int32))
    for a, b in zip(chain, same):
        assert np.array_equal(a, b)
    depth = np.array([0, 3, 1, 1, 2], np.int32)
    q_t, k_t, _ = _oracle_rope(qkv, qw, kw, cos, sin, [start], B, T, HQ, HKV, cap, depth=depth)
    for t in range(T):
        q1, k1, _ = _oracle_rope(qkv[t:t + 1], qw, kw, cos, sin, [start + int(depth[t])], 1, 1, HQ, HKV, cap)
        assert np.array_equal(q_t[0, :, t], q1[0, :, 0])
        assert np.array_equal(k_t[0, :, start + t], k1[0, :, start + int(depth[t])])
    q0, _, _ = _oracle_rope(qkv, qw, kw, cos, sin, [start], B, T, HQ, HKV, cap, depth=np.full(T, -start, np.int32))
    x = qkv[0, :128].double()
    r = 1.0 / torch.sqrt((x * x).mean() + 1e-6)
    assert np.array_equal(q0[0, 0, 0], bits((qw.float() * (x * r).float().to(BF16).float()).to(BF16)))


def test_oracle_rope_rejects_positions_outside_the_table():
    B, T, HQ, HKV, start = 1, 3, 4, 2, 5
    cap = start + T
    qkv, qw, kw, cos, sin = _rope_inputs(B, T, HQ, HKV, cap, seed=23)
    with pytest.raises(ValueError):
        _oracle_rope(qkv, qw, kw, cos, sin, [start], B, T, HQ, HKV, cap, depth=np.array([0, 1, cap], np.int32))
    with pytest.raises(ValueError):
        _oracle_rope(qkv, qw, kw, cos, sin, [start], B, T, HQ, HKV, cap, depth=np.array([0, 1], np.int32))


# --------------------------------------------------------------------------
# decode attention (engine/kernels/attention.py:221-242)
# --------------------------------------------------------------------------

def _attn_inputs(B, HQ, HKV, R, CAP, seed):
    g = torch.Generator().manual_seed(seed)
    q = randn_bf16((B, HQ, R, 128), 1.0, g)
    kc = randn_bf16((B, HKV, CAP, 128), 1.0, g)
    vc = randn_bf16((B, HKV, CAP, 128), 1.0, g)
    return q, kc, vc


@pytest.mark.parametrize("R", [1, 2])
def test_oracle_attention_matches_sdpa(R):
    B, HQ, HKV, CAP = 3, 8, 2, 200
    q, kc, vc = _attn_inputs(B, HQ, HKV, R, CAP, seed=R)
    pos = np.array([200 - R, 0, 76], np.int32)
    scale = 128 ** -0.5
    out = oracle.decode_attention(bits(q), bits(kc), bits(vc), pos, scale)
    for b in range(B):
        L = int(pos[b]) + R
        k = kc[b, :, :L].double().repeat_interleave(HQ // HKV, dim=0)
        v = vc[b, :, :L].double().repeat_interleave(HQ // HKV, dim=0)
        mask = torch.arange(L)[None, :] <= (int(pos[b]) + torch.arange(R))[:, None]
        ref = F.scaled_dot_product_attention(q[b].double(), k, v, attn_mask=mask[None], scale=scale)
        got = torch.from_numpy(out[b]).transpose(0, 1).double()     # [HQ, R, D]
        assert (got - ref).abs().max().item() < 1e-5


def test_oracle_attention_special_cases():
    """One visible key: the output is that key's value row.  Zero query: every
    visible key has the same score, so the output is the mean of their values."""
    B, HQ, HKV, CAP = 2, 4, 1, 50
    q, kc, vc = _attn_inputs(B, HQ, HKV, 1, CAP, seed=9)
    out = oracle.decode_attention(bits(q), bits(kc), bits(vc), np.array([0, 0], np.int32), 0.1)
    for b in range(B):
        for h in range(HQ):
            assert np.array_equal(out[b, 0, h], vc[b, 0, 0].float().numpy())
    zq = torch.zeros_like(q)
    pos = np.array([9, 30], np.int32)
    out = oracle.decode_attention(bits(zq), bits(kc), bits(vc), pos, 0.1)
    for b in range(B):
        mean = vc[b, 0, : int(pos[b]) + 1].double().mean(0).numpy()
        assert np.abs(out[b, 0, 0] - mean).max() < 1e-6


# --------------------------------------------------------------------------
# fast_topk (engine/kernels/topk.py)
# --------------------------------------------------------------------------

def _exact_topk(L: torch.Tensor, k: int):
    """Exact top-k with the lowest column first among equal values (stable sort)."""
    s = torch.sort(L.float(), dim=-1, descending=True, stable=True)
    return s.values[:, :k].numpy(), s.indices[:, :k].to(torch.int32).numpy()


@pytest.mark.parametrize("V", [5, 1500, 2048])
def test_oracle_topk_is_exact_when_every_column_has_its_own_lane(V):
    """V <= 2048: each lane sees one column, so the lane sweep is an exact
    top-k with the lowest-index tie rule (values drawn coarse to force ties)."""
    g = torch.Generator().manual_seed(V)
    L = (torch.randint(-40, 40, (4, V), generator=g).float() / 8).to(BF16)
    k = min(8, V)
    v, i = oracle.topk(bits(L), k)
    ev, ei = _exact_topk(L, k)
    assert np.array_equal(v, ev) and np.array_equal(i, ei)


def test_oracle_topk_rank0_is_torch_argmax_and_lane_collisions_are_missed():
    V = 151936
    g = torch.Generator().manual_seed(1)
    L = randn_bf16((3, V), 1.0, g)
    L[0, 5000] = 20.0
    L[0, 5000 + 2048] = 19.0      # same lane as column 5000: the documented miss
    L[0, 77] = 18.0
    L[1, 100] = L[1, 9000] = 30.0  # exact tie in different lanes: lowest index first
    v, i = oracle.topk(bits(L), 4)
    assert np.array_equal(i[:, 0], torch.argmax(L, -1).numpy())
    assert list(i[0, :2]) == [5000, 77] and 5000 + 2048 not in i[0]
    assert list(i[1, :2]) == [100, 9000] and v[1, 0] == v[1, 1] == 30.0


def test_oracle_attention_tree_mask_matches_sdpa():
    """Draft-tree masks (engine/kernels/attention.py:229-236): row t sees every
    key before pos and the draft keys on its ancestor path."""
    B, HQ, HKV, R, CAP = 2, 8, 2, 5, 120
    q, kc, vc = _attn_inputs(B, HQ, HKV, R, CAP, seed=21)
    parent = [-1, 0, 0, 1, 2]
    masks = []
    for i in range(R):
        m, n = 0, i
        while n >= 0:
            m |= 1 << n
            n = parent[n]
        masks.append(m)
    tree = np.array(masks, np.int64)
    pos = np.array([50, 100], np.int32)
    scale = 128 ** -0.5
    out = oracle.decode_attention(bits(q), bits(kc), bits(vc), pos, scale, tree=tree)
    for b in range(B):
        p = int(pos[b])
        L = p + R
        k = kc[b, :, :L].double().repeat_interleave(HQ // HKV, dim=0)
        v = vc[b, :, :L].double().repeat_interleave(HQ // HKV, dim=0)
        draft = torch.tensor([[(masks[t] >> j) & 1 for j in range(R)] for t in range(R)], dtype=torch.bool)
        mask = torch.cat([torch.ones(R, p, dtype=torch.bool), draft], dim=1)
        ref = F.scaled_dot_product_attention(q[b].double(), k, v, attn_mask=mask[None], scale=scale)
        got = torch.from_numpy(out[b]).transpose(0, 1).double()
        assert (got - ref).abs().max().item() < 1e-5
