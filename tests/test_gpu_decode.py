"""End-to-end greedy decode on the HIP hot path (needs an MI355X).

A small Qwen3-shaped model (head width 128, GQA, 2 layers), and once the full
Qwen3-4B shape, decode through starter_amd.decode.DecodePlan: prefill, then
decode steps captured into one HIP graph.  Checks:
  * graph replays produce exactly the tokens of eager decode steps;
  * every step's token equals the argmax of an independent torch fp32
    restatement of the reference forward (engine/model.py:182-210,
    rope.py / rmsnorm.py casts) run on the same token sequence, wherever that
    reference's top-2 logit margin exceeds 0.05 (two valid fp32 summation
    orders can swap closer candidates).
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from starter_amd.decode import DecodePlan, Qwen3Config, SyntheticModel

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
CFG = Qwen3Config(hidden=512, intermediate=1024, layers=2, heads=4, kv_heads=2, head_dim=128, vocab=4096)


_DT = torch.float32   # accumulation type of the restatement (_reference_logits sets it per call)


def _bf(t):
    return t.to(torch.bfloat16).to(_DT)


def _rms(x, w, eps):
    r = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return _bf(w.to(_DT) * _bf(x * r))


def _reference_logits(model: SyntheticModel, ids: torch.Tensor, cos, sin, first: int = 0,
                      dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """torch restatement of the decode forward with the reference's bf16 casts,
    accumulated in ``dtype`` (fp32, or fp64 to measure the restatement's own
    sensitivity), over the whole sequence (causal); returns bf16-rounded logits
    [B, S - first, V] of positions first..S-1 (the lm_head runs on those only)."""
    global _DT
    _DT = dtype
    try:
        return _reference_logits_impl(model, ids, cos, sin, first)
    finally:
        _DT = torch.float32


def _reference_logits_impl(model: SyntheticModel, ids: torch.Tensor, cos, sin, first: int) -> torch.Tensor:
    cfg = model.cfg
    B, S = ids.shape
    HQ, HKV, D = cfg.heads, cfg.kv_heads, cfg.head_dim
    x = model.embed[ids].to(_DT)
    y = torch.zeros_like(x)
    pos = torch.arange(S, device=ids.device)
    c, s_ = cos[pos].to(_DT)[None, :, None, :], sin[pos].to(_DT)[None, :, None, :]

    def rot(t):
        t1, t2 = t[..., : D // 2], t[..., D // 2:]
        return torch.cat((-t2, t1), dim=-1)

    for layer in model.layers:
        xo = _bf(x + y)
        h = _rms(xo, layer.in_norm, cfg.eps)
        qkv = _bf(h @ layer.wqkv.to(_DT).t())
        q = qkv[..., : HQ * D].view(B, S, HQ, D)
        k = qkv[..., HQ * D:(HQ + HKV) * D].view(B, S, HKV, D)
        v = qkv[..., (HQ + HKV) * D:].view(B, S, HKV, D)
        qn, kn = _rms(q, layer.q_norm, cfg.eps), _rms(k, layer.k_norm, cfg.eps)
        q = _bf(_bf(qn * c) + _bf(rot(qn) * s_)).transpose(1, 2)
        k = _bf(_bf(kn * c) + _bf(rot(kn) * s_)).transpose(1, 2).repeat_interleave(HQ // HKV, dim=1)
        v = v.transpose(1, 2).repeat_interleave(HQ // HKV, dim=1)
        a = F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=model.scale)
        a = _bf(a).transpose(1, 2).reshape(B, S, HQ * D)
        o = _bf(a @ layer.wo.to(_DT).t())
        xo2 = _bf(xo + o)
        h2 = _rms(xo2, layer.post_norm, cfg.eps)
        I = cfg.intermediate
        g = _bf(h2 @ layer.wgu[:I].to(_DT).t())
        u = _bf(h2 @ layer.wgu[I:].to(_DT).t())
        act = _bf(_bf(F.silu(g)) * u)
        y = _bf(act @ layer.wd.to(_DT).t())
        x = xo2
    hf = _rms(_bf(x[:, first:] + y[:, first:]), model.final_norm, cfg.eps)
    return _bf(hf @ model.lm_head.to(_DT).t())


@pytest.mark.parametrize("handoff", [True, False])
def test_graph_replay_matches_eager_decode(handoff):
    torch.manual_seed(0)
    model = SyntheticModel(CFG, DEV, seed=1, norm_noise=0.1)
    B, T, N = 3, 40, 6
    ids = torch.randint(0, CFG.vocab, (B, T), device=DEV)
    eager = DecodePlan(model, B, T, N, handoff=handoff).generate(ids, N)
    plan = DecodePlan(model, B, T, N, handoff=handoff)
    plan.ids.copy_(ids)
    plan.prefill()
    plan.capture()
    toks = [plan.tok.clone()]
    for _ in range(N - 1):
        plan.step()
        toks.append(plan.tok.clone())
    torch.cuda.synchronize()
    assert torch.equal(torch.stack(toks, 1), eager)


@pytest.mark.parametrize("depth", [1, 3])
def test_pipelined_host_delivery_yields_the_decoded_tokens(depth):
    """DecodePlan.run (engine/engine.py:388-419): one host list per position,
    the GPU kept up to `depth` steps ahead through pinned slots and events;
    the lists equal generate()'s tokens, also when run twice on one plan (the
    captured step graph replays for the second run)."""
    model = SyntheticModel(CFG, DEV, seed=5, norm_noise=0.1)
    B, T, N = 3, 37, 9
    ids = torch.randint(0, CFG.vocab, (B, T), device=DEV, generator=torch.Generator(device=DEV).manual_seed(6))
    ref = DecodePlan(model, B, T, N).generate(ids, N).cpu()
    plan = DecodePlan(model, B, T, N)
    for _ in range(2):
        rows = list(plan.run(ids, N, depth=depth))
        assert len(rows) == N and all(isinstance(r, list) and len(r) == B for r in rows)
        assert torch.equal(torch.tensor(rows).t(), ref)
    with pytest.raises(ValueError):
        next(plan.run(ids, N + 1))
    plan.step()                         # step N of N planned: attends over T + N keys, still covered
    with pytest.raises(RuntimeError):   # a step past the planned length is refused, not silently truncated
        plan.step()


@pytest.mark.parametrize("handoff", [True, False])
def test_decode_tokens_match_torch_reference(handoff):
    """Both decode steps: the reference's normed projections, and the residual
    hand-off (norms finished inside the projection kernels)."""
    torch.backends.cuda.matmul.allow_tf32 = False
    model = SyntheticModel(CFG, DEV, seed=2, norm_noise=0.1)
    B, T, N = 2, 33, 8
    ids = torch.randint(0, CFG.vocab, (B, T), device=DEV, generator=torch.Generator(device=DEV).manual_seed(3))
    plan = DecodePlan(model, B, T, N, handoff=handoff)
    out = plan.generate(ids, N)                           # [B, N]: token after position T-1, T, ...
    seq = torch.cat([ids, out[:, :-1]], dim=1)            # the sequence the engine actually consumed
    logits = _reference_logits(model, seq, plan.cos, plan.sin)[:, T - 1:]      # [B, N, V]
    top2 = logits.topk(2, dim=-1)
    margin = top2.values[..., 0] - top2.values[..., 1]
    ref_tok = top2.indices[..., 0]
    decided = margin > 0.05
    assert decided.float().mean() > 0.5, "too few decided steps to be a meaningful check"
    assert torch.equal(out[decided], ref_tok[decided]), (out, ref_tok, margin)


def test_decode_tokens_match_torch_reference_qwen3_4b_shape():
    """The bench's decode step (residual hand-off) at the full Qwen3-4B shape
    (36 layers, hidden 2560, GQA 32/8, vocabulary 151936).  Over 36 layers the
    bf16 roundings of valid summation orders drift the logits (the same
    restatement accumulated in fp64 instead of fp32 moves them by up to 0.2),
    so each greedy token must score within 0.125 of the fp32 restatement's
    maximum: it equals the restatement's token wherever that token leads by
    more than 0.125, and is a near-tie candidate elsewhere."""
    torch.backends.cuda.matmul.allow_tf32 = False
    cfg = Qwen3Config()
    model = SyntheticModel(cfg, DEV, seed=4, norm_noise=0.1)
    B, T, N = 8, 64, 8
    ids = torch.randint(0, cfg.vocab, (B, T), device=DEV, generator=torch.Generator(device=DEV).manual_seed(5))
    plan = DecodePlan(model, B, T, N, handoff=True)
    out = plan.generate(ids, N)
    seq = torch.cat([ids, out[:, :-1]], dim=1)
    logits = _reference_logits(model, seq, plan.cos, plan.sin)[:, T - 1:]
    top2 = logits.topk(2, dim=-1)
    margin = top2.values[..., 0] - top2.values[..., 1]
    gap = top2.values[..., 0] - logits.gather(-1, out[..., None])[..., 0]
    tol = 0.125
    assert (margin > tol).float().mean() > 0.3, "too few decided steps to be a meaningful check"
    assert (gap <= tol).all(), (out, top2.indices[..., 0], margin, gap)


def test_decode_c5_size_graph_replay_matches_eager_and_reference():
    """BASELINE configuration 5 at its own size, the workload bench.py times:
    the same synthetic Qwen3-4B (seed 7), 16 prompts of 1024 uniform token ids
    (seed 11), prefill, then all 127 decode steps replayed from the captured
    graph (M = 16 hand-off consumers, one-split attention over ~1100 keys).
    The replayed tokens equal eager decode token for token, and each token
    scores within max(0.125, D) of the maximum logit at its position of both
    the fp32 and the fp64 restatement, D being how far those two restatements
    themselves differ there (the restatements run over the sequence the engine
    consumed; their lm_head only at the 128 decoded positions)."""
    torch.backends.cuda.matmul.allow_tf32 = False
    cfg = Qwen3Config()
    model = SyntheticModel(cfg, DEV, seed=7)
    B, T, N = 16, 1024, 128
    ids = torch.randint(0, cfg.vocab, (B, T), device=DEV, generator=torch.Generator(device=DEV).manual_seed(11))
    plan = DecodePlan(model, B, T, N, handoff=True)
    plan.ids.copy_(ids)
    plan.prefill()
    plan.capture()
    toks = [plan.tok.clone()]
    for _ in range(N - 1):
        plan.step()
        toks.append(plan.tok.clone())
    out = torch.stack(toks, 1)
    eager = DecodePlan(model, B, T, N, handoff=True).generate(ids, N)
    torch.cuda.synchronize()
    assert torch.equal(out, eager), (out != eager).nonzero()[:8].tolist()
    seq = torch.cat([ids, out[:, :-1]], dim=1)                                  # [16, 1151]
    l32 = _reference_logits(model, seq, plan.cos, plan.sin, first=T - 1)        # [16, 128, V]
    l64 = _reference_logits(model, seq, plan.cos, plan.sin, first=T - 1, dtype=torch.float64)
    # The restatement's own sensitivity at these positions: accumulating in fp64
    # instead of fp32 moves its logits by up to D (about 0.23 here, 36 layers
    # over ~1100 keys).  The engine is another valid accumulation order: each
    # of its tokens must trail either restatement's maximum by at most
    # max(0.125, D), equal the restatement's token wherever that one leads by
    # more, and agree with the fp64 restatement about as often as the fp32
    # restatement does (within 5 points).
    D = float((l32.double() - l64).abs().max())
    tol = max(0.125, D)
    ref64 = l64.argmax(-1)
    agree32 = float((l32.argmax(-1) == ref64).float().mean())
    report = {"D": round(D, 4), "tol": round(tol, 4), "fp32_vs_fp64_agree": agree32}
    for name, logits in (("fp32", l32), ("fp64", l64)):
        top2 = logits.topk(2, dim=-1)
        margin = top2.values[..., 0] - top2.values[..., 1]
        gap = top2.values[..., 0] - logits.gather(-1, out[..., None])[..., 0]
        decided = margin > tol
        report[name] = {"max_gap": float(gap.max()), "agree": float((out == top2.indices[..., 0]).float().mean()),
                        "decided": float(decided.float().mean())}
        assert (gap <= tol).all(), (report, (gap > tol).nonzero()[:8].tolist())
        assert torch.equal(out[decided], top2.indices[..., 0][decided]), report
    assert report["fp64"]["agree"] >= agree32 - 0.05, report
    print("C5 decode parity:", report)


@pytest.mark.parametrize("M", [1, 16])
def test_decode_matmuls_callables(M):
    """decode_matmuls (engine/model.py:137-179): each callable returns what the
    library call it wraps returns for the same inputs, bit for bit, and writes
    the same residual; "lm_argmax" picks the argmax of "lm"'s logits."""
    from starter_amd import kernels as K
    from starter_amd.decode import decode_matmuls

    m = SyntheticModel(CFG, DEV, seed=5, norm_noise=0.1)
    mm = decode_matmuls(m, M)
    g = torch.Generator(device=DEV).manual_seed(M)
    H, I = CFG.hidden, CFG.intermediate
    x = torch.randn(M, H, generator=g, device=DEV).to(torch.bfloat16)
    y = torch.randn(M, H, generator=g, device=DEV).to(torch.bfloat16)
    a = torch.randn(M, CFG.heads * CFG.head_dim, generator=g, device=DEV).to(torch.bfloat16)
    act = torch.randn(M, I, generator=g, device=DEV).to(torch.bfloat16)
    layer, eps = m.layers[0], CFG.eps
    xo1, xo2 = torch.empty_like(x), torch.empty_like(x)

    out = mm["qkv"](x, y, layer.in_norm, xo1, layer.wqkv)
    ref = K.rmsnorm_gemm(x, y, layer.in_norm, eps, xo2, layer.wqkv)
    assert torch.equal(out, ref) and torch.equal(xo1, xo2) and torch.equal(xo1, (x.float() + y.float()).bfloat16())
    assert torch.equal(mm["o"](a, layer.wo), K.gemm(a, layer.wo))
    out = mm["gu"](x, y, layer.post_norm, xo1, layer.wgu)
    ref = K.rmsnorm_gateup_swiglu(x, y, layer.post_norm, eps, xo2, layer.wgu[:I], layer.wgu[I:])
    assert torch.equal(out, ref) and torch.equal(xo1, xo2)
    assert torch.equal(mm["d"](act, layer.wd), K.gemm(act, layer.wd))
    logits = mm["lm"](x, y, m.final_norm, xo1, m.lm_head)
    assert torch.equal(logits, K.rmsnorm_gemm(x, y, m.final_norm, eps, xo2, m.lm_head))
    ids, maxv = mm["lm_argmax"](x, y, m.final_norm, xo2, m.lm_head)
    torch.cuda.synchronize()
    # the fused argmax may sum in another order than the logits GEMM's config:
    # ids must agree wherever the top-2 margin exceeds 1e-2 of the max
    top2 = logits.float().topk(2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > 1e-2 * top2[:, 0].abs()
    assert clear.sum() >= M // 2
    assert torch.equal(ids[clear], logits.float().argmax(-1)[clear])
    assert torch.allclose(maxv, top2[:, 0], rtol=1e-2, atol=0)


def _path(parents: list[int], t: int) -> list[int]:
    path = [t]
    while parents[path[-1]] >= 0:
        path.append(parents[path[-1]])
    return path[::-1]


@pytest.mark.parametrize("tree,B,R", [(False, 4, 4), (True, 4, 4), (True, 16, 8)])
def test_verify_plan_matches_reference(tree, B, R):
    """VerifyPlan (engine/model.py:334-375): after a prefill, one pass over
    R = 4 rows per sequence (the last accepted token and three drafts, as a
    chain or as the tree 0 -> {1, 2}, 1 -> 3), and the reference's batch-16
    shape: 8 tree rows per sequence (engine.py:451), B x R = 128 rows through
    every projection, with the 8-node template its tree builder makes
    (recycle.py:75-95, prior "flat").  Row t's token must be the
    greedy token a causal restatement of the reference forward predicts after
    the prompt followed by the path root..t (positions T + depth), wherever
    that restatement's top-2 margin exceeds 0.05; a captured graph replays to
    the same tokens; every row's K/V lands in cache slot T + t."""
    from starter_amd.decode import VerifyPlan

    model = SyntheticModel(CFG, DEV, seed=9, norm_noise=0.1)
    T = 40
    plan = DecodePlan(model, B, T, 16, handoff=False)
    g = torch.Generator(device=DEV).manual_seed(21)
    ids = torch.randint(0, CFG.vocab, (B, T), device=DEV, generator=g)
    plan.ids.copy_(ids)
    plan.prefill()
    vp = VerifyPlan(plan, R, tree=tree)
    parents = {4: [-1, 0, 0, 1], 8: [-1, 0, 0, 1, 0, 2, 1, 0]}[R] if tree else [-1, 0, 1, 2]
    if tree:
        vp.set_tree(parents)
    drafts = torch.randint(0, CFG.vocab, (B, R - 1), device=DEV, generator=g)
    vp.blk.copy_(torch.cat([plan.tok[:, None], drafts], 1))
    vp.pos.copy_(plan.pos)
    k_before = plan.k_cache[:, :, :, T:T + R].clone()
    out = vp.verify()
    torch.cuda.synchronize()
    assert not torch.equal(plan.k_cache[:, :, :, T:T + R], k_before)   # slots T .. T+R-1 written
    decided = 0
    for t in range(R):
        seq = torch.cat([ids, vp.blk[:, _path(parents, t)]], 1)
        logits = _reference_logits(model, seq, plan.cos, plan.sin, first=seq.shape[1] - 1)[:, 0].float()
        top2 = logits.topk(2, dim=-1)
        clear = (top2.values[:, 0] - top2.values[:, 1]) > 0.05
        decided += int(clear.sum())
        assert torch.equal(out[clear, t], top2.indices[clear, 0]), (t, out[:, t].tolist(), top2.indices[:, 0].tolist())
    assert decided >= B * R // 2
    # the same pass captured into a graph and replayed
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        vp.verify()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g = vp.verify()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, out)


def test_verify_plan_rejects_bad_trees():
    from starter_amd.decode import VerifyPlan

    model = SyntheticModel(CFG, DEV, seed=9)
    plan = DecodePlan(model, 2, 8, 8, handoff=False)
    vp = VerifyPlan(plan, 3, tree=True)
    for bad in ([-1, 0], [0, 0, 1], [-1, 1, 0], [-1, 0, 2]):
        with pytest.raises(ValueError):
            vp.set_tree(bad)
    with pytest.raises(ValueError):
        VerifyPlan(plan, 3, tree=False).set_tree([-1, 0, 1])
    with pytest.raises(ValueError):
        VerifyPlan(plan, 64 // (CFG.heads // CFG.kv_heads) + 1)
