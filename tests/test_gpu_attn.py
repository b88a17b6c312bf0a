"""GPU parity of the attention side of the decode step (needs an MI355X):
q/k RMSNorm + RoPE + KV-cache write and split-K GQA decode attention, through
the C ABI, against the CPU oracle (pinned in tests/test_oracle.py against the
reference's own torch composition and SDPA).

Tolerances: RoPE outputs equal the oracle's except on at most 0.2% of the
elements, and there within one bf16 ulp at the head's scale (the GPU forms the
head's sum of squares in fp32, the oracle exactly; see _check_rope); value
rows bit-exact.  Attention: the reference test's bound
max |out - SDPA| < 2e-2 (tests/test_kernels.py:60-80) and, per element,
|out - exact| <= 2^-8 * (sum p|v| / sum p + |exact|): the error that bf16
probabilities (attention.py:9-11) and the bf16 output can cause, doubled.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from starter_amd import kernels as K
from tests._util import BF16, bits, from_bits, randn_bf16
from tests.test_oracle import rope_tables_cpu

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
D = 128


def _check_rope(out: torch.Tensor, ref_bits: np.ndarray, what: str) -> None:
    """Bit-exact except on rare elements where the fp32 sum of squares of the
    head differs in its last bit: there a normalised value moves by one bf16
    ulp, and the rotation sum bf16(a + b) can cancel, so the bound is one ulp
    at the scale of the head (1/128 of max(|ref|, rms(head)))."""
    o = oracle.bf16_to_f32(bits(out)).astype(np.float64)
    r = oracle.bf16_to_f32(ref_bits).astype(np.float64)
    rms = np.sqrt((r ** 2).mean(-1, keepdims=True))
    err = np.abs(o - r)
    assert (err <= np.maximum(np.abs(r), rms) / 128).all(), f"{what}: max err {err.max()}"
    assert (err != 0).mean() <= 2e-3, f"{what}: {(err != 0).mean():.2e} of elements differ"


@pytest.mark.parametrize("B,T,HQ,HKV,starts", [
    (2, 5, 8, 2, (3, 3)),                 # the reference test's shape (tests/test_kernels.py:30-56)
    (16, 1, 32, 8, tuple(range(1000, 1016))),   # Qwen3-4B decode step, per-sequence positions
    (2, 64, 32, 8, (0, 200)),             # prefill-like rows
])
def test_qk_norm_rope_cache_matches_oracle(B, T, HQ, HKV, starts):
    CAP = max(starts) + T + 3
    eps = 1e-6
    g = torch.Generator().manual_seed(B * T + HQ)
    cos, sin = rope_tables_cpu(D, 1e6, CAP)
    qkv = randn_bf16((B * T, (HQ + 2 * HKV) * D), 1.0, g)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(BF16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(BF16)
    pos = np.array(starts, np.int32)
    q_o = np.zeros((B, HQ, T, D), np.uint16)
    kc_o = np.zeros((B, HKV, CAP, D), np.uint16)
    vc_o = np.zeros_like(kc_o)
    oracle.qk_norm_rope_cache(bits(qkv), bits(qw), bits(kw), bits(cos), bits(sin), pos, q_o, kc_o, vc_o, T, eps)

    q_out = torch.empty(B, HQ, T, D, dtype=BF16, device=DEV)
    kc = torch.zeros(B, HKV, CAP, D, dtype=BF16, device=DEV)
    vc = torch.zeros_like(kc)
    K.qk_norm_rope_cache(qkv.to(DEV), qw.to(DEV), kw.to(DEV), cos.to(DEV), sin.to(DEV),
                         torch.from_numpy(pos).to(DEV), q_out, kc, vc, T, eps)
    torch.cuda.synchronize()
    _check_rope(q_out, q_o, "q")
    _check_rope(kc, kc_o, "k")
    assert np.array_equal(bits(vc), vc_o), "value rows are copied raw; untouched slots stay zero"


@pytest.mark.parametrize("B,depth", [
    (4, (0, 1, 1, 2, 2)),                 # root, two children, two grandchildren (draft tree, R = 5)
    (16, (0, 1, 2, 3)),                   # a chain given as depths: equals the chain call
    (3, (0, 1, 1, 1, 2, 3, 2, 4)),        # R = 8 rows, siblings at several depths
])
def test_qk_norm_rope_cache_tree_depth_matches_oracle(B, depth):
    """Draft-tree rows (engine/kernels/rope.py:94-122, the depth= argument of
    engine/model.py:204, 369-370): row t goes to cache slot pos + t and rotates
    by position pos + depth[t]; Qwen3-4B heads, per-sequence positions."""
    T, HQ, HKV, eps = len(depth), 32, 8, 1e-6
    starts = np.array([700 + 37 * b for b in range(B)], np.int32)
    CAP = int(starts.max()) + T + 3
    g = torch.Generator().manual_seed(B * 7 + T)
    cos, sin = rope_tables_cpu(D, 1e6, CAP)
    qkv = randn_bf16((B * T, (HQ + 2 * HKV) * D), 1.0, g)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(BF16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(BF16)
    dep = np.array(depth, np.int32)
    q_o = np.zeros((B, HQ, T, D), np.uint16)
    kc_o = np.zeros((B, HKV, CAP, D), np.uint16)
    vc_o = np.zeros_like(kc_o)
    oracle.qk_norm_rope_cache(bits(qkv), bits(qw), bits(kw), bits(cos), bits(sin), starts, q_o, kc_o, vc_o, T, eps,
                              depth=dep)
    q_out = torch.empty(B, HQ, T, D, dtype=BF16, device=DEV)
    kc = torch.zeros(B, HKV, CAP, D, dtype=BF16, device=DEV)
    vc = torch.zeros_like(kc)
    args = (qkv.to(DEV), qw.to(DEV), kw.to(DEV), cos.to(DEV), sin.to(DEV), torch.from_numpy(starts).to(DEV))
    K.qk_norm_rope_cache(*args, q_out, kc, vc, T, eps, depth=torch.from_numpy(dep).to(DEV))
    torch.cuda.synchronize()
    _check_rope(q_out, q_o, "q (tree depth)")
    _check_rope(kc, kc_o, "k (tree depth)")
    assert np.array_equal(bits(vc), vc_o), "value rows go to slots pos + t"
    if tuple(depth) == tuple(range(T)):   # the chain given as depths: bit for bit the chain call
        q2, kc2, vc2 = torch.empty_like(q_out), torch.zeros_like(kc), torch.zeros_like(vc)
        K.qk_norm_rope_cache(*args, q2, kc2, vc2, T, eps)
        torch.cuda.synchronize()
        assert torch.equal(q2, q_out) and torch.equal(kc2, kc) and torch.equal(vc2, vc)


def test_tree_verify_rope_then_tree_attention_matches_oracle():
    """The reference's draft-tree verify pair (engine/model.py:203-205 with
    depth= and tree masks): rotary step with per-row depths, then attention
    with the ancestor masks of the same tree, against the oracle's pair."""
    B, HQ, HKV, eps = 4, 32, 8, 1e-6
    parent = [-1, 0, 0, 1, 2]
    depth = np.array([0, 1, 1, 2, 2], np.int32)
    R = len(parent)
    starts = np.array([500, 517, 640, 901], np.int32)
    CAP = 1024
    g = torch.Generator().manual_seed(77)
    cos, sin = rope_tables_cpu(D, 1e6, CAP)
    qkv = randn_bf16((B * R, (HQ + 2 * HKV) * D), 1.0, g)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(BF16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(BF16)
    k0 = randn_bf16((B, HKV, CAP, D), 1.0, g)
    v0 = randn_bf16((B, HKV, CAP, D), 1.0, g)
    tree = np.array(K.ancestor_masks(parent), np.int64)
    q_o = np.zeros((B, HQ, R, D), np.uint16)
    kc_o, vc_o = bits(k0).copy(), bits(v0).copy()
    oracle.qk_norm_rope_cache(bits(qkv), bits(qw), bits(kw), bits(cos), bits(sin), starts, q_o, kc_o, vc_o, R, eps,
                              depth=depth)
    ref = oracle.decode_attention(q_o, kc_o, vc_o, starts, 1.0 / np.sqrt(D), with_abs=True, tree=tree)

    q = torch.empty(B, HQ, R, D, dtype=BF16, device=DEV)
    kc, vc = k0.to(DEV), v0.to(DEV)
    posd = torch.from_numpy(starts).to(DEV)
    K.qk_norm_rope_cache(qkv.to(DEV), qw.to(DEV), kw.to(DEV), cos.to(DEV), sin.to(DEV), posd, q, kc, vc, R, eps,
                         depth=torch.from_numpy(depth).to(DEV))
    attn = K.DecodeAttention(B, HQ, HKV, D, CAP, DEV, R=R, tree=True)
    out = torch.empty(B, R, HQ, D, dtype=BF16, device=DEV)
    attn(q, kc, vc, posd, out, torch.from_numpy(tree).to(DEV))
    torch.cuda.synchronize()
    _check_rope(q, q_o, "tree q")
    _check_rope(kc, kc_o, "tree k cache")
    # attention against the oracle's attention over the oracle's own rotated rows
    # (at most 0.2% of q/k elements may differ by one bf16 ulp, see _check_rope)
    _check_attention(out, ref, "tree verify attention")


def test_qk_norm_rope_cache_skips_slots_outside_the_cache():
    """pos is device data: a slot beyond the cache or the rotary table is
    skipped (no write, no fault), the in-range rows are still written."""
    B, T, HQ, HKV, CAP = 2, 4, 4, 2, 10
    g = torch.Generator().manual_seed(1)
    cos, sin = rope_tables_cpu(D, 1e6, CAP)
    qkv = randn_bf16((B * T, (HQ + 2 * HKV) * D), 1.0, g).to(DEV)
    w = torch.ones(D, dtype=BF16, device=DEV)
    pos = torch.tensor([8, 3], dtype=torch.int32, device=DEV)      # rows 2, 3 of sequence 0 fall outside
    q_out = torch.zeros(B, HQ, T, D, dtype=BF16, device=DEV)
    kc = torch.zeros(B, HKV, CAP, D, dtype=BF16, device=DEV)
    vc = torch.zeros_like(kc)
    K.qk_norm_rope_cache(qkv, w, w, cos.to(DEV), sin.to(DEV), pos, q_out, kc, vc, T, 1e-6)
    torch.cuda.synchronize()
    assert bool((kc[0, :, 8:10] != 0).any()) and bool((kc[1, :, 3:7] != 0).any())
    assert not bool((kc[0, :, :8] != 0).any()) and not bool((q_out[0, :, 2:] != 0).any())


def _check_attention(out: torch.Tensor, ref, what: str) -> None:
    """ref = (exact attention, softmax-weighted mean of |v|) from the oracle."""
    ref, wabs = ref
    o = out.float().cpu().numpy()
    err = np.abs(o - ref)
    assert err.max() < 2e-2, f"{what}: max |err| {err.max()}"
    # bf16 probabilities move the sum by at most 2^-9 * sum p|v| / sum p, the
    # bf16 output by 2^-9 * |out|; a factor 2 covers fp32 accumulation.
    bound = 2.0 ** -8 * (wabs + np.abs(ref)) + 1e-6
    bad = err > bound
    assert not bad.any(), f"{what}: {int(bad.sum())} elements outside 2^-8*(wabs + |ref|), worst {err.max()}"


@pytest.mark.parametrize("nsplit", [1, 4, None])
def test_decode_attention_reference_case(nsplit):
    """tests/test_kernels.py:60-80: lengths 200, 1 and 77 in a cache of 200."""
    B, HQ, HKV, CAP = 3, 8, 2, 200
    g = torch.Generator().manual_seed(0)
    q = randn_bf16((B, HQ, 1, D), 1.0, g)
    kc = randn_bf16((B, HKV, CAP, D), 1.0, g)
    vc = randn_bf16((B, HKV, CAP, D), 1.0, g)
    pos = np.array([199, 0, 76], np.int32)
    attn = K.DecodeAttention(B, HQ, HKV, D, CAP, DEV, nsplit=nsplit)
    out = torch.empty(B, 1, HQ, D, dtype=BF16, device=DEV)
    attn(q.to(DEV), kc.to(DEV), vc.to(DEV), torch.from_numpy(pos).to(DEV), out)
    ref = oracle.decode_attention(bits(q), bits(kc), bits(vc), pos, D ** -0.5, with_abs=True)
    _check_attention(out, ref, f"reference case nsplit={nsplit}")


@pytest.mark.parametrize("R", [1, 2])
def test_decode_attention_qwen_shape(R):
    """Qwen3-4B at batch 16: 32 query / 8 KV heads, cap 1408, ~1024 keys."""
    B, HQ, HKV, CAP = 16, 32, 8, 1408
    g = torch.Generator().manual_seed(R)
    q = randn_bf16((B, HQ, R, D), 1.0, g)
    kc = randn_bf16((B, HKV, CAP, D), 1.0, g)
    vc = randn_bf16((B, HKV, CAP, D), 1.0, g)
    pos = (1024 + torch.randint(0, 128, (B,), generator=g)).to(torch.int32).numpy()
    attn = K.DecodeAttention(B, HQ, HKV, D, CAP, DEV, R=R)
    out = torch.empty(B, R, HQ, D, dtype=BF16, device=DEV)
    attn(q.to(DEV), kc.to(DEV), vc.to(DEV), torch.from_numpy(pos).to(DEV), out)
    ref = oracle.decode_attention(bits(q), bits(kc), bits(vc), pos, D ** -0.5, with_abs=True)
    _check_attention(out, ref, f"qwen R={R}")


def test_decode_attention_graph_replay_with_growing_length():
    """The length comes from pos on the device: one captured graph replayed
    while pos advances matches eager calls at every length, and the split
    counters reset (several replays)."""
    B, HQ, HKV, CAP = 4, 32, 8, 512
    g = torch.Generator().manual_seed(5)
    q = randn_bf16((B, HQ, 1, D), 1.0, g).to(DEV)
    kc = randn_bf16((B, HKV, CAP, D), 1.0, g).to(DEV)
    vc = randn_bf16((B, HKV, CAP, D), 1.0, g).to(DEV)
    pos = torch.tensor([100, 7, 300, 450], dtype=torch.int32, device=DEV)
    attn = K.DecodeAttention(B, HQ, HKV, D, CAP, DEV, nsplit=6)
    out = torch.empty(B, 1, HQ, D, dtype=BF16, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        attn(q, kc, vc, pos, out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        attn(q, kc, vc, pos, out)
    for step in range(4):
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        eager = torch.empty_like(out)
        attn(q, kc, vc, pos, eager)
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay {step}"
        ref = oracle.decode_attention(bits(q), bits(kc), bits(vc), pos.cpu().numpy(), D ** -0.5, with_abs=True)
        _check_attention(got, ref, f"replay {step}")
        pos += 13


@pytest.mark.parametrize("nsplit", [1, 3])
def test_decode_attention_visible_key_boundary(nsplit):
    """Key pos[b] (the newest) is visible and key pos[b] + 1 is not: make the
    invisible key's score huge and the newest key's large, so any off-by-one in
    the length, the split ranges or the mask shows up as a wrong output row."""
    B, HQ, HKV, CAP = 4, 8, 2, 300
    g = torch.Generator().manual_seed(8)
    q = randn_bf16((B, HQ, 1, D), 1.0, g)
    kc = randn_bf16((B, HKV, CAP, D), 0.1, g)
    vc = randn_bf16((B, HKV, CAP, D), 1.0, g)
    pos = np.array([0, 63, 64, 250], np.int32)
    for b in range(B):
        for kh in range(HKV):
            lead = q[b, kh * (HQ // HKV), 0].float()
            kc[b, kh, pos[b] + 1] = (lead * 4).to(BF16)      # masked: would dominate
            kc[b, kh, pos[b]] = (lead * 2).to(BF16)          # visible: dominates head kh*G
    attn = K.DecodeAttention(B, HQ, HKV, D, CAP, DEV, nsplit=nsplit)
    out = torch.empty(B, 1, HQ, D, dtype=BF16, device=DEV)
    attn(q.to(DEV), kc.to(DEV), vc.to(DEV), torch.from_numpy(pos).to(DEV), out)
    ref = oracle.decode_attention(bits(q), bits(kc), bits(vc), pos, D ** -0.5, with_abs=True)
    _check_attention(out, ref, f"boundary nsplit={nsplit}")
    for b in range(B):   # the dominant newest key: the lead head's output is ~ its value row
        for kh in range(HKV):
            o = out[b, 0, kh * (HQ // HKV)].float().cpu()
            assert torch.allclose(o, vc[b, kh, pos[b]].float(), atol=0.05), (b, kh)


@pytest.mark.parametrize("R,nsplit", [(5, None), (8, 3), (3, 1), (2, None), (4, 2), (16, None), (16, 2)])
def test_decode_attention_verify_rows_chain(R, nsplit):
    """Speculative verify: R query rows per sequence (G*R = 8 .. 64 here: the
    8-row instance, one full or partial 16-row block, or two to four blocks,
    which run side by side on one XCD), chain mask (row t sees keys <= pos + t)."""
    B, HQ, HKV, CAP = 4, 32, 8, 700
    g = torch.Generator().manual_seed(R * 10 + (nsplit or 0))
    q = randn_bf16((B, HQ, R, D), 1.0, g)
    kc = randn_bf16((B, HKV, CAP, D), 1.0, g)
    vc = randn_bf16((B, HKV, CAP, D), 1.0, g)
    pos = np.array([0, 100, 511, 690 - R], np.int32)
    attn = K.DecodeAttention(B, HQ, HKV, D, CAP, DEV, R=R, nsplit=nsplit)
    out = torch.empty(B, R, HQ, D, dtype=BF16, device=DEV)
    attn(q.to(DEV), kc.to(DEV), vc.to(DEV), torch.from_numpy(pos).to(DEV), out)
    ref = oracle.decode_attention(bits(q), bits(kc), bits(vc), pos, D ** -0.5, with_abs=True)
    _check_attention(out, ref, f"verify chain R={R} nsplit={nsplit}")


@pytest.mark.parametrize("nsplit", [None, 2])
def test_decode_attention_draft_tree(nsplit):
    """Draft tree (attention.py:229-236): row t sees keys < pos and the draft
    keys on its ancestor path (masks from kernels.ancestor_masks)."""
    B, HQ, HKV, CAP, R = 3, 32, 8, 400, 6
    parent = [-1, 0, 0, 1, 1, 2]
    tree = torch.tensor(K.ancestor_masks(parent), dtype=torch.int64)
    g = torch.Generator().manual_seed(17)
    q = randn_bf16((B, HQ, R, D), 1.0, g)
    kc = randn_bf16((B, HKV, CAP, D), 1.0, g)
    vc = randn_bf16((B, HKV, CAP, D), 1.0, g)
    pos = np.array([10, 200, 393], np.int32)
    attn = K.DecodeAttention(B, HQ, HKV, D, CAP, DEV, R=R, tree=True, nsplit=nsplit)
    out = torch.empty(B, R, HQ, D, dtype=BF16, device=DEV)
    attn(q.to(DEV), kc.to(DEV), vc.to(DEV), torch.from_numpy(pos).to(DEV), out, tree.to(DEV))
    ref = oracle.decode_attention(bits(q), bits(kc), bits(vc), pos, D ** -0.5, with_abs=True, tree=tree.numpy())
    _check_attention(out, ref, f"tree nsplit={nsplit}")
