"""GPU tests of the fused q/k norm + RoPE + cache write + decode attention
launch (sk_decode_attention_rope_bf16, and sk_decode_attention_rope_tree_bf16
for draft trees; needs an MI355X).

The fused launch must equal the two launches it replaces,
sk_qk_norm_rope_cache_bf16 then sk_decode_attention_bf16 (each pinned against
the oracle in test_gpu_attn.py), bit for bit: the attention output and both
caches.  Cases: the Qwen3-4B decode shape at several split counts, verify rows
(up to 16 query rows per workgroup, and two row blocks), a slot past the planned
length, graph replays with a growing length, draft trees (rotated by pos +
depth, tree-masked) against qk_norm_rope_cache(depth) then the tree attention,
and argument checks.
"""

from __future__ import annotations

import pytest
import torch

from starter_amd import kernels as K
from starter_amd._lib import SK_ERR_ALIAS, SkError
from tests._util import BF16, randn_bf16
from tests.test_oracle import rope_tables_cpu

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
D = 128


def _setup(B, HQ, HKV, R, cap, starts, seed):
    g = torch.Generator().manual_seed(seed)
    cos, sin = rope_tables_cpu(D, 1e6, cap + 8)
    qkv = randn_bf16((B * R, (HQ + 2 * HKV) * D), 1.0, g).to(DEV)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(BF16).to(DEV)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(BF16).to(DEV)
    kc = randn_bf16((B, HKV, cap, D), 1.0, g).to(DEV)   # earlier positions' keys
    vc = randn_bf16((B, HKV, cap, D), 1.0, g).to(DEV)
    pos = torch.tensor(starts, dtype=torch.int32, device=DEV)
    return qkv, qw, kw, cos.to(DEV), sin.to(DEV), kc, vc, pos


def _unfused(attn, qkv, qw, kw, cos, sin, pos, kc, vc, eps):
    B, HQ, R = attn.B, attn.HQ, attn.R
    q = torch.empty(B, HQ, R, D, dtype=BF16, device=DEV)
    out = torch.empty(B, R, HQ, D, dtype=BF16, device=DEV)
    K.qk_norm_rope_cache(qkv, qw, kw, cos, sin, pos, q, kc, vc, R, eps)
    attn(q, kc, vc, pos, out)
    return out


def _fused(attn, qkv, qw, kw, cos, sin, pos, kc, vc, eps):
    out = torch.empty(attn.B, attn.R, attn.HQ, D, dtype=BF16, device=DEV)
    attn.rope_attend(qkv, qw, kw, cos, sin, pos, kc, vc, out, eps)
    return out


def _assert_same(a: torch.Tensor, b: torch.Tensor, what: str) -> None:
    assert torch.equal(a.view(torch.int16), b.view(torch.int16)), f"{what}: fused and unfused differ"


@pytest.mark.parametrize("B,HQ,HKV,R,cap,starts,maxlen,nsplit", [
    (16, 32, 8, 1, 1100, tuple(range(1000, 1016)), 1100, None),   # Qwen3-4B decode step
    (16, 32, 8, 1, 1100, tuple(range(1000, 1016)), 1100, 1),
    (16, 32, 8, 1, 1100, tuple(range(1000, 1016)), 1100, 3),
    (4, 32, 8, 1, 300, (0, 1, 63, 64), 300, 2),                   # first positions, split boundary
    (2, 8, 2, 2, 200, (50, 127), 200, 2),                         # verify rows: 8 rows per workgroup
    (2, 8, 2, 3, 200, (50, 126), 200, 3),                         # 12 rows in one row block of 16
    (2, 8, 2, 5, 200, (50, 124), 200, 2),                         # 20 rows: two row blocks of 16
    (3, 8, 2, 1, 300, (10, 150, 250), 128, None),                 # slots past the planned length
])
def test_fused_equals_rope_then_attention(B, HQ, HKV, R, cap, starts, maxlen, nsplit):
    eps = 1e-6
    qkv, qw, kw, cos, sin, kc, vc, pos = _setup(B, HQ, HKV, R, cap, starts, seed=B * 7 + R)
    attn = K.DecodeAttention(B, HQ, HKV, D, cap, DEV, nsplit=nsplit, R=R, maxlen=maxlen)
    kc1, vc1, kc2, vc2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    out1 = _unfused(attn, qkv, qw, kw, cos, sin, pos, kc1, vc1, eps)
    out2 = _fused(attn, qkv, qw, kw, cos, sin, pos, kc2, vc2, eps)
    torch.cuda.synchronize()
    _assert_same(kc2, kc1, "k cache")
    _assert_same(vc2, vc1, "v cache")
    _assert_same(out2, out1, "attention output")
    assert not torch.equal(kc2, kc), "the new key rows were written"


def test_fused_graph_replay_with_growing_length():
    """One captured fused launch replayed while pos grows (device-side
    length): every replay equals the eager unfused pair on its own copy."""
    B, HQ, HKV, cap, eps = 16, 32, 8, 1200, 1e-6
    qkv, qw, kw, cos, sin, kc, vc, pos = _setup(B, HQ, HKV, 1, cap, tuple(range(900, 916)), seed=5)
    attn = K.DecodeAttention(B, HQ, HKV, D, cap, DEV, maxlen=cap)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    out = torch.empty(B, 1, HQ, D, dtype=BF16, device=DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        attn.rope_attend(qkv, qw, kw, cos, sin, pos, kc, vc, out, eps)   # warm-up (pos 900..)
    torch.cuda.current_stream().wait_stream(s)
    ref = _unfused(attn, qkv, qw, kw, cos, sin, pos, kc_ref, vc_ref, eps)
    torch.cuda.synchronize()
    _assert_same(out, ref, "eager step")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        attn.rope_attend(qkv, qw, kw, cos, sin, pos, kc, vc, out, eps)
    for step in range(4):
        pos.add_(1)
        g.replay()
        ref = _unfused(attn, qkv, qw, kw, cos, sin, pos, kc_ref, vc_ref, eps)
        torch.cuda.synchronize()
        _assert_same(out, ref, f"replay {step}")
        _assert_same(kc, kc_ref, f"k cache after replay {step}")


@pytest.mark.parametrize("B,HQ,HKV,R,cap,starts,parents,nsplit", [
    (16, 32, 8, 4, 1300, tuple(range(1100, 1116)), (-1, 0, 0, 1), None),   # the bench's 4-row verify tree
    (16, 32, 8, 8, 1300, tuple(range(1100, 1116)), (-1, 0, 0, 1, 0, 2, 1, 0), None),   # batch-16 verify: 32 rows
    (2, 8, 2, 5, 200, (50, 124), (-1, 0, 1, 1, 0), 2),                       # 20 rows: two row blocks
    (3, 8, 2, 3, 300, (0, 150, 250), (-1, 0, 0), 3),                         # first positions, splits
])
def test_fused_tree_equals_rope_with_depth_then_tree_attention(B, HQ, HKV, R, cap, starts, parents, nsplit):
    """sk_decode_attention_rope_tree_bf16 against qk_norm_rope_cache(..., depth)
    then the tree-masked attention: output and both caches bit for bit; the
    same captured launch follows a new tree written into the masks/depths."""
    eps = 1e-6
    qkv, qw, kw, cos, sin, kc, vc, pos = _setup(B, HQ, HKV, R, cap, starts, seed=B * 11 + R)
    attn = K.DecodeAttention(B, HQ, HKV, D, cap, DEV, nsplit=nsplit, R=R, tree=True, maxlen=cap)

    def tree_of(par):
        depth = [0] * R
        for t in range(1, R):
            depth[t] = depth[par[t]] + 1
        return (torch.tensor(K.ancestor_masks(list(par)), dtype=torch.int64, device=DEV),
                torch.tensor(depth, dtype=torch.int32, device=DEV))

    masks, depth = tree_of(parents)
    kc1, vc1, kc2, vc2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    q = torch.empty(B, HQ, R, D, dtype=BF16, device=DEV)
    out1 = torch.empty(B, R, HQ, D, dtype=BF16, device=DEV)
    K.qk_norm_rope_cache(qkv, qw, kw, cos, sin, pos, q, kc1, vc1, R, eps, depth=depth)
    attn(q, kc1, vc1, pos, out1, masks)
    out2 = torch.empty_like(out1)
    attn.rope_attend(qkv, qw, kw, cos, sin, pos, kc2, vc2, out2, eps, tree=masks, depth=depth)
    torch.cuda.synchronize()
    _assert_same(kc2, kc1, "k cache")
    _assert_same(vc2, vc1, "v cache")
    _assert_same(out2, out1, "attention output")
    # a chain through the same captured launch: masks and depths are read at every call
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        attn.rope_attend(qkv, qw, kw, cos, sin, pos, kc2, vc2, out2, eps, tree=masks, depth=depth)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        attn.rope_attend(qkv, qw, kw, cos, sin, pos, kc2, vc2, out2, eps, tree=masks, depth=depth)
    chain_masks, chain_depth = tree_of(tuple([-1] + list(range(R - 1))))
    masks.copy_(chain_masks)
    depth.copy_(chain_depth)
    g.replay()
    K.qk_norm_rope_cache(qkv, qw, kw, cos, sin, pos, q, kc1, vc1, R, eps, depth=depth)
    attn(q, kc1, vc1, pos, out1, masks)
    torch.cuda.synchronize()
    _assert_same(kc2, kc1, "k cache (chain replay)")
    _assert_same(out2, out1, "attention output (chain replay)")


def test_fused_tree_argument_checks():
    B, HQ, HKV, R, cap = 2, 8, 2, 2, 64
    qkv, qw, kw, cos, sin, kc, vc, pos = _setup(B, HQ, HKV, R, cap, (3, 4), seed=13)
    out = torch.empty(B, R, HQ, D, dtype=BF16, device=DEV)
    tree_attn = K.DecodeAttention(B, HQ, HKV, D, cap, DEV, R=R, tree=True)
    with pytest.raises(Exception):   # a tree instance needs masks and depths
        tree_attn.rope_attend(qkv, qw, kw, cos, sin, pos, kc, vc, out, 1e-6)
    chain = K.DecodeAttention(B, HQ, HKV, D, cap, DEV, R=R)
    masks = torch.tensor(K.ancestor_masks([-1, 0]), dtype=torch.int64, device=DEV)
    depth = torch.tensor([0, 1], dtype=torch.int32, device=DEV)
    with pytest.raises(Exception):   # and a chain instance takes neither
        chain.rope_attend(qkv, qw, kw, cos, sin, pos, kc, vc, out, 1e-6, tree=masks, depth=depth)


def test_fused_rejects_aliasing_and_tree_instances():
    B, HQ, HKV, cap = 2, 8, 2, 64
    qkv, qw, kw, cos, sin, kc, vc, pos = _setup(B, HQ, HKV, 1, cap, (3, 4), seed=9)
    attn = K.DecodeAttention(B, HQ, HKV, D, cap, DEV)
    alias = kc.view(-1)[: B * HQ * D].view(B, 1, HQ, D)      # output inside the key cache
    with pytest.raises(SkError) as e:
        attn.rope_attend(qkv, qw, kw, cos, sin, pos, kc, vc, alias, 1e-6)
    assert e.value.status == SK_ERR_ALIAS
    tree_attn = K.DecodeAttention(B, HQ, HKV, D, cap, DEV, R=1, tree=True)
    out = torch.empty(B, 1, HQ, D, dtype=BF16, device=DEV)
    with pytest.raises(Exception):   # without its masks and depths
        tree_attn.rope_attend(qkv, qw, kw, cos, sin, pos, kc, vc, out, 1e-6)
