"""Synthetic Qwen3 greedy decode on the HIP hot path.

Mirrors the reference's decode forward (engine/model.py:182-210 ``run_layers``,
215-330 ``Plan``; engine/engine.py:198-230 graph capture and replay) with this
package's kernels in every decode-step op:

* ``mm["qkv"]`` / ``mm["gu"]`` / ``mm["lm"]``: residual add + RMSNorm fused into
  the projection (``SkinnyMatmul`` / ``SkinnyGateUp`` / ``LmArgmax`` with the
  norm prologue); ``mm["o"]`` / ``mm["d"]``: ``SkinnyMatmul``;
* q/k RMSNorm + RoPE + KV write: ``qk_norm_rope_cache``;
* attention: ``DecodeAttention`` (split-K GQA flash-decoding);
* the greedy token: argmax fused into the lm_head kernel.

The token embedding gather, the per-step position increment and the prefill
pass (bf16 GEMMs through torch, SDPA over the prompt, as the reference's own
prefill does, model.py:264-289) are torch plumbing around them.  Weights are
random (``N(0, 0.02)`` projections, unit norm gains), so the generated text is
meaningless; the work per step is that of the real model.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import kernels as K

BF16 = torch.bfloat16


@dataclass(frozen=True)
class Qwen3Config:
    """Qwen3-4B by default (RoPE theta 1e6)."""

    hidden: int = 2560
    intermediate: int = 9728
    layers: int = 36
    heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    vocab: int = 151936
    eps: float = 1e-6
    rope_theta: float = 1e6


def rope_tables(cfg: Qwen3Config, max_pos: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 cos/sin tables [max_pos, D] built like the reference (engine/model.py:85-100):
    fp32 inverse frequencies, fp32 outer product, ``cat(freqs, freqs)``, then
    cos/sin, then bf16.  Computed on the CPU (no TF32 question) and copied."""
    D = cfg.head_dim
    inv_freq = 1.0 / (cfg.rope_theta ** (torch.arange(0, D, 2, dtype=torch.int64).float() / D))
    positions = torch.arange(max_pos, dtype=torch.float32)
    freqs = (inv_freq[:, None].float() @ positions[None, :].float()).transpose(0, 1)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(BF16).contiguous().to(device), emb.sin().to(BF16).contiguous().to(device)


@dataclass
class Layer:
    in_norm: torch.Tensor
    wqkv: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    wo: torch.Tensor
    post_norm: torch.Tensor
    wgu: torch.Tensor
    wd: torch.Tensor


class SyntheticModel:
    """Random-init weights of the reference layout (engine/model.py:102-130):
    fused q|k|v and gate|up rows, tied embeddings / lm_head."""

    def __init__(self, cfg: Qwen3Config = Qwen3Config(), device="cuda:0", seed: int = 0, norm_noise: float = 0.0):
        self.cfg = cfg
        self.device = torch.device(device)
        g = torch.Generator(device=self.device).manual_seed(seed)
        H, I, D = cfg.hidden, cfg.intermediate, cfg.head_dim
        HQ, HKV = cfg.heads, cfg.kv_heads

        # Drawn in place in bf16: an fp32 draw + cast makes the caching allocator
        # release device segments, and on this platform every kernel of the
        # process runs ~7% slower after a large device free.  All projection
        # matrices are views into one allocation (256-byte aligned): a decode
        # step over them measured 0.3-0.4% faster than over one allocation per
        # matrix (5727-5729 vs 5701-5715 tok/s, alternating runs on one box).
        mats = [(cfg.vocab, H)] + [((HQ + 2 * HKV) * D, H), (H, HQ * D), (2 * I, H), (H, I)] * cfg.layers
        align = lambda n: (n + 127) // 128 * 128
        pool = torch.empty(sum(align(a * b) for a, b in mats), dtype=BF16, device=self.device)
        used = 0

        def w(*shape):
            nonlocal used
            n = shape[0] * shape[1]
            view = pool[used:used + n].view(*shape)
            used += align(n)
            return view.normal_(0.0, 0.02, generator=g)

        def gain(n):
            if norm_noise == 0.0:
                return torch.ones(n, dtype=BF16, device=self.device)
            return (1 + norm_noise * torch.randn(n, generator=g, device=self.device)).to(BF16)

        self.embed = w(cfg.vocab, H)
        self.lm_head = self.embed
        self.final_norm = gain(H)
        self.layers = [Layer(in_norm=gain(H), wqkv=w((HQ + 2 * HKV) * D, H), q_norm=gain(D), k_norm=gain(D),
                             wo=w(H, HQ * D), post_norm=gain(H), wgu=w(2 * I, H), wd=w(H, I))
                       for _ in range(cfg.layers)]
        self.scale = 1.0 / math.sqrt(D)


def decode_matmuls(m: SyntheticModel, M: int, log=None) -> dict:
    """The per-shape projection callables for M-row decode/verify steps
    (engine/model.py:137-179, the norm-fused branch): "qkv", "gu" and "lm" take
    ``(x, y, w_norm, xout, w)``, write ``xout = x + y`` and project
    ``rms_norm(xout)``; "o" and "d" take ``(a, w)``.  "lm" returns the logits
    like the reference's; "lm_argmax" is the same call with the greedy argmax
    fused in, returning ``(ids, maxv)`` without storing logits.  The configs
    come from the library's table (no warmup timing); ``log`` receives one
    line per choice."""
    cfg = m.cfg
    layer = m.layers[0]
    x = torch.empty((M, cfg.hidden), dtype=BF16, device=m.device)
    a = torch.empty((M, cfg.heads * cfg.head_dim), dtype=BF16, device=m.device)
    act = torch.empty((M, cfg.intermediate), dtype=BF16, device=m.device)
    return {
        "qkv": K.pick_normed("matmul", x, x, layer.in_norm, layer.wqkv, cfg.eps, log),
        "o": K.pick_matmul(a, layer.wo, log),
        "gu": K.pick_normed("gateup", x, x, layer.post_norm, layer.wgu, cfg.eps, log),
        "d": K.pick_matmul(act, layer.wd, log),
        "lm": K.pick_normed("matmul", x, x, m.final_norm, m.lm_head, cfg.eps, log),
        "lm_argmax": K.pick_lm_argmax(x, m.lm_head, cfg.eps, log),
    }


class DecodePlan:
    """Static buffers, KV cache and step functions for one (B, T, max_new) shape
    (engine/model.py:215-262).  ``decode()`` touches only preallocated tensors
    and library workspaces, so it can be captured into a HIP graph."""

    def __init__(self, model: SyntheticModel, B: int, T: int, max_new: int, handoff: bool = True):
        """``handoff``: run the add + RMSNorm between projections inside the
        projection kernels (the producer writes the residual and its per-row
        partial sums of squares, the consumer finishes the norm) instead of as
        the reference's normed projections (prologue per call)."""
        self.model = model
        self.handoff = handoff
        cfg = model.cfg
        self.B, self.T, self.max_new = B, T, max_new
        self.cap = ((T + max(max_new, 256) + 2 * 64 + 63) // 64) * 64     # engine/model.py:224
        dev = model.device
        H, I, D, HQ, HKV = cfg.hidden, cfg.intermediate, cfg.head_dim, cfg.heads, cfg.kv_heads
        self.cos, self.sin = rope_tables(cfg, self.cap, dev)
        self.ids = torch.zeros((B, T), dtype=torch.int64, device=dev)
        self.tok = torch.zeros((B,), dtype=torch.int64, device=dev)
        self.pos = torch.zeros((B,), dtype=torch.int32, device=dev)
        self.k_cache = torch.zeros((cfg.layers, B, HKV, self.cap, D), dtype=BF16, device=dev)
        self.v_cache = torch.zeros((cfg.layers, B, HKV, self.cap, D), dtype=BF16, device=dev)
        self.zero = torch.zeros((B, H), dtype=BF16, device=dev)
        self.xa = torch.empty((B, H), dtype=BF16, device=dev)
        self.xb = torch.empty((B, H), dtype=BF16, device=dev)
        self.q = torch.empty((B, HQ, 1, D), dtype=BF16, device=dev)
        self.attn_out = torch.empty((B, 1, HQ, D), dtype=BF16, device=dev)
        self.attention = K.DecodeAttention(B, HQ, HKV, D, self.cap, dev, maxlen=min(self.cap, T + max_new))
        # the decode-step projections (engine/model.py:137-179)
        self.mm = decode_matmuls(model, B)
        if handoff:
            # residual hand-off: partial sums of squares of the residual rows
            # (16-column groups) and one zero-filled workspace per call site
            self.sq_a = torch.zeros((B, K.sumsq_groups(B, H)), dtype=torch.float32, device=dev)
            self.sq_b = torch.zeros_like(self.sq_a)
            self.qkv = torch.empty((B, (HQ + 2 * HKV) * D), dtype=BF16, device=dev)
            self.act = torch.empty((B, I), dtype=BF16, device=dev)
            self.maxv_out = torch.empty((B,), dtype=torch.float32, device=dev)
            self.ws_o = K._workspace(K.SK_OP_RESID_GEMM, B, H, HQ * D, None, dev)
            self.ws_d = K._workspace(K.SK_OP_RESID_GEMM, B, H, I, None, dev)
            self.ws_qkv = K._workspace(K.SK_OP_PRE_GEMM, B, (HQ + 2 * HKV) * D, H, None, dev)
            self.ws_gu = K._workspace(K.SK_OP_PRE_GATEUP, B, I, H, None, dev)
            self.ws_lm = K._workspace(K.SK_OP_PRE_LM_ARGMAX, B, cfg.vocab, H, None, dev)
        self.g_decode = None
        self.steps_done = 0   # decode steps since the last prefill (host-side count)

    # -- prefill (torch GEMMs + SDPA, this package's norm/rope/swiglu/argmax) --
    @torch.inference_mode()
    def prefill(self) -> None:
        """Consume ``ids`` from position 0; leaves the first generated token in
        ``tok`` and ``pos = T`` (engine/model.py:264-289)."""
        m, cfg = self.model, self.model.cfg
        B, T = self.B, self.T
        HQ, D = cfg.heads, cfg.head_dim
        self.pos.zero_()
        x = F.embedding(self.ids.view(-1), m.embed)
        zero = torch.zeros_like(x)
        h = K.add_rms_norm(x, zero, m.layers[0].in_norm, cfg.eps, xout=torch.empty_like(x))
        q = torch.empty((B, HQ, T, D), dtype=BF16, device=x.device)
        for i, layer in enumerate(m.layers):
            k_i, v_i = self.k_cache[i], self.v_cache[i]
            qkv = h @ layer.wqkv.t()
            K.qk_norm_rope_cache(qkv, layer.q_norm, layer.k_norm, self.cos, self.sin, self.pos, q, k_i, v_i, T,
                                 cfg.eps)
            a = F.scaled_dot_product_attention(q, k_i[:, :, :T].contiguous(), v_i[:, :, :T].contiguous(),
                                               is_causal=True, scale=m.scale, enable_gqa=True)
            o = a.transpose(1, 2).reshape(B * T, HQ * D) @ layer.wo.t()
            h2 = K.add_rms_norm(x, o, layer.post_norm, cfg.eps)
            d = K.swiglu(h2 @ layer.wgu.t()) @ layer.wd.t()
            nxt = m.layers[i + 1].in_norm if i + 1 < len(m.layers) else m.final_norm
            h = K.add_rms_norm(x, d, nxt, cfg.eps)
        logits = h.view(B, T, cfg.hidden)[:, -1].contiguous() @ m.lm_head.t()
        ids, _ = K.argmax(logits)
        self.tok.copy_(ids)
        self.pos.fill_(T)
        self.steps_done = 0

    # -- one decode step: run_layers (engine/model.py:182-210) + greedy token --
    def decode(self) -> None:
        """Consume ``tok`` at ``pos``; writes the next greedy token to ``tok``
        and advances ``pos``."""
        m, cfg = self.model, self.model.cfg
        B = self.B
        # Row gather by advanced indexing: for B rows torch's index kernel takes
        # ~2 us where F.embedding's index_select kernel takes ~6.5 us.
        x = m.embed[self.tok]
        if self.handoff:
            self._decode_handoff(x)
            return
        # run_layers (engine/model.py:182-210) over the decode_matmuls callables
        mm = self.mm
        cur, y = x, self.zero
        for i, layer in enumerate(m.layers):
            qkv = mm["qkv"](cur, y, layer.in_norm, self.xa, layer.wqkv)
            K.qk_norm_rope_cache(qkv, layer.q_norm, layer.k_norm, self.cos, self.sin, self.pos, self.q,
                                 self.k_cache[i], self.v_cache[i], 1, cfg.eps)
            self.attention(self.q, self.k_cache[i], self.v_cache[i], self.pos, self.attn_out)
            o = mm["o"](self.attn_out.view(B, cfg.heads * cfg.head_dim), layer.wo)
            act = mm["gu"](self.xa, o, layer.post_norm, self.xb, layer.wgu)
            y = mm["d"](act, layer.wd)
            cur = self.xb
        ids, _ = mm["lm_argmax"](cur, y, m.final_norm, self.xa, m.lm_head)
        self.tok.copy_(ids)
        self.pos.add_(1)

    def _decode_handoff(self, x: torch.Tensor) -> None:
        """The decode step with the residual hand-off: xa/xb and their partial
        sums sq_a/sq_b pass between the projections (layer 0's input norm, on
        the embedding, keeps the normed projection), and the q/k norm, rotary
        step and cache write run inside the attention launch."""
        m, cfg = self.model, self.model.cfg
        B, I, eps = self.B, cfg.intermediate, cfg.eps
        for i, layer in enumerate(m.layers):
            if i == 0:
                qkv = self.mm["qkv"](x, self.zero, layer.in_norm, self.xa, layer.wqkv)
            else:
                qkv = K.rmsnorm_pre_gemm(self.xa, self.sq_a, layer.in_norm, eps, layer.wqkv, out=self.qkv,
                                         ws=self.ws_qkv)
            # q/k norm + rotary + cache write inside the attention launch
            self.attention.rope_attend(qkv, layer.q_norm, layer.k_norm, self.cos, self.sin, self.pos,
                                       self.k_cache[i], self.v_cache[i], self.attn_out, eps)
            # xb = xa + o (o itself is not stored), then xa = xb + down(act)
            K.gemm_residual(self.attn_out.view(B, cfg.heads * cfg.head_dim), layer.wo, self.xa, self.xb, self.sq_b,
                            ws=self.ws_o)
            act = K.rmsnorm_pre_gateup_swiglu(self.xb, self.sq_b, layer.post_norm, eps, layer.wgu[:I],
                                              layer.wgu[I:], out=self.act, ws=self.ws_gu)
            K.gemm_residual(act, layer.wd, self.xb, self.xa, self.sq_a, ws=self.ws_d)
        # the next token ids go straight into tok (read only by this step's embedding)
        K.rmsnorm_pre_lm_argmax(self.xa, self.sq_a, m.final_norm, eps, m.lm_head, ws=self.ws_lm,
                                ids=self.tok, maxv=self.maxv_out)
        self.pos.add_(1)

    def capture(self) -> None:
        """Capture one decode step into a HIP graph (engine/engine.py:198-215).
        Call after prefill; the captured step is replayed as the sequence grows
        (the attention length and cache slots come from ``pos`` on the device)."""
        tok0, pos0 = self.tok.clone(), self.pos.clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.decode()                       # warm (writes slot pos; restored below)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self.tok.copy_(tok0)
        self.pos.copy_(pos0)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.decode()
        torch.cuda.synchronize()
        self.tok.copy_(tok0)
        self.pos.copy_(pos0)
        self.g_decode = g

    def step(self) -> None:
        """One decode step (the captured graph when there is one).  Step s after
        the prefill attends over T + s keys; the attention and the cache were
        planned for T + max_new, so a step past max_new raises instead of
        silently dropping keys."""
        if self.steps_done >= self.max_new:
            raise RuntimeError(f"decode step {self.steps_done + 1} exceeds the planned max_new = {self.max_new} "
                               f"(attention planned for {self.T + self.max_new} keys)")
        if self.g_decode is None:
            self.decode()
        else:
            self.g_decode.replay()
        self.steps_done += 1

    @torch.inference_mode()
    def run(self, ids: torch.Tensor, max_new_tokens: int | None = None, depth: int = 3):
        """Yield one host list of B greedy token ids per generated position,
        keeping the GPU up to ``depth`` steps ahead of the consumer
        (engine/engine.py:388-419): step t's tokens are copied into pinned host
        slot t % depth and fenced with an event, and the following steps are
        launched before the host waits on that event, so reading step t
        overlaps the compute of steps t+1..t+depth-1.  Copies and graph replays
        share the current stream, so each copy follows its own step."""
        n = self.max_new if max_new_tokens is None else max_new_tokens
        if not 1 <= n <= self.max_new:
            raise ValueError(f"max_new_tokens must be in 1..{self.max_new}, got {n}")
        if depth < 1:
            raise ValueError("depth must be at least 1")
        if getattr(self, "_host_tok", None) is None or self._host_tok.shape[0] != depth:
            self._host_tok = torch.empty((depth, self.B), dtype=torch.int64, pin_memory=True)
            self._events = [torch.cuda.Event() for _ in range(depth)]
        host, events = self._host_tok, self._events
        self.ids.copy_(ids)
        self.prefill()
        if self.g_decode is None:
            self.capture()
        host[0].copy_(self.tok, non_blocking=True)
        events[0].record()
        launched = 1
        for step in range(n):
            while launched < n and launched - step < depth:
                slot = launched % depth
                self.step()
                host[slot].copy_(self.tok, non_blocking=True)
                events[slot].record()
                launched += 1
            slot = step % depth
            events[slot].synchronize()
            yield host[slot].tolist()

    @torch.inference_mode()
    def generate(self, ids: torch.Tensor, max_new: int | None = None) -> torch.Tensor:
        """Greedy tokens [B, max_new]: the prefill's token, then one per decode step."""
        max_new = self.max_new if max_new is None else max_new
        self.ids.copy_(ids)
        self.prefill()
        out = torch.empty((self.B, max_new), dtype=torch.int64, device=self.ids.device)
        out[:, 0] = self.tok
        for t in range(1, max_new):
            self.step()
            out[:, t] = self.tok
        return out


class VerifyPlan:
    """Speculative verification (engine/model.py:334-375): R query rows per
    sequence in one pass over the plan's model and KV cache.  Row 0 holds the
    last accepted token, rows 1..R-1 the drafts, as a chain or, with
    ``tree=True``, a draft tree given by its parent list (``set_tree``).  The
    forward writes row t of sequence b to cache slot pos[b] + t (rotated by
    position pos[b] + depth[t] in a tree) and returns the greedy token after
    every row; accepting a path is the caller's policy.  The projections run
    at M = B * R rows through ``decode_matmuls`` (the reference's run_layers
    sequence; the q/k norm, rotary step and cache write run inside the
    attention launch), so one instance can be captured into a HIP graph."""

    def __init__(self, plan: DecodePlan, R: int, tree: bool = False):
        m, cfg, B = plan.model, plan.model.cfg, plan.B
        dev = m.device
        H, HQ, HKV, D = cfg.hidden, cfg.heads, cfg.kv_heads, cfg.head_dim
        if R < 1 or R * (HQ // HKV) > 64:
            raise ValueError(f"R * (query heads per KV head) must be in 1..64, got R = {R}")
        self.plan, self.R, self.tree = plan, R, tree
        M = B * R
        self.blk = torch.zeros((B, R), dtype=torch.int64, device=dev)
        self.pos = torch.zeros((B,), dtype=torch.int32, device=dev)
        # a chain until set_tree: parent of row t is row t - 1
        self.masks = K.chain_tree(R, dev) if tree else None
        self.depth = torch.arange(R, dtype=torch.int32, device=dev) if tree else None
        self.attn_out = torch.empty((B, R, HQ, D), dtype=BF16, device=dev)
        self.zero = torch.zeros((M, H), dtype=BF16, device=dev)
        self.xa = torch.empty((M, H), dtype=BF16, device=dev)
        self.xb = torch.empty((M, H), dtype=BF16, device=dev)
        self.attention = K.DecodeAttention(B, HQ, HKV, D, plan.cap, dev, R=R, tree=tree, maxlen=plan.cap)
        self.mm = decode_matmuls(m, M)

    def set_tree(self, parents: list[int]) -> None:
        """Draft tree of the R rows: parents[t] is the row of t's parent
        (-1 for row 0 only, every parent before its child).  Sets the
        ancestor masks (kernels.ancestor_masks) and the depths."""
        if not self.tree:
            raise ValueError("this plan was built without tree=True")
        R = self.R
        if len(parents) != R or parents[0] != -1 or any(not 0 <= parents[t] < t for t in range(1, R)):
            raise ValueError("parents must list R rows: -1 for row 0, then a smaller row index for each")
        depth = [0] * R
        for t in range(1, R):
            depth[t] = depth[parents[t]] + 1
        self.masks.copy_(torch.tensor(K.ancestor_masks(parents), dtype=torch.int64))
        self.depth.copy_(torch.tensor(depth, dtype=torch.int32))

    @torch.inference_mode()
    def verify(self) -> torch.Tensor:
        """Consume ``blk`` [B, R] at ``pos``; returns the [B, R] greedy tokens
        (run_layers, engine/model.py:182-210, then the fused lm_head argmax)."""
        plan, m = self.plan, self.plan.model
        cfg = m.cfg
        B, R = plan.B, self.R
        mm = self.mm
        x = m.embed[self.blk.view(-1)]
        cur, y = x, self.zero
        for i, layer in enumerate(m.layers):
            k_i, v_i = plan.k_cache[i], plan.v_cache[i]
            qkv = mm["qkv"](cur, y, layer.in_norm, self.xa, layer.wqkv)
            # qk_norm_rope_cache (rotated by pos + depth in a tree) and the
            # attention in one launch
            self.attention.rope_attend(qkv, layer.q_norm, layer.k_norm, plan.cos, plan.sin, self.pos, k_i, v_i,
                                       self.attn_out, cfg.eps, tree=self.masks, depth=self.depth)
            o = mm["o"](self.attn_out.view(B * R, cfg.heads * cfg.head_dim), layer.wo)
            act = mm["gu"](self.xa, o, layer.post_norm, self.xb, layer.wgu)
            y = mm["d"](act, layer.wd)
            cur = self.xb
        ids, _ = mm["lm_argmax"](cur, y, m.final_norm, self.xa, m.lm_head)
        return ids.view(B, R)


def time_decode(plan: DecodePlan, steps: int) -> dict:
    """Decode throughput the way the reference defines it (B tokens per step,
    QWEN_ENGINE_CONTRACT.md:93-102): ``steps`` graph replays after a prefill,
    bracketed by HIP events on the replay stream.  Returns tok/s, ms per step
    and the prefill time.  One untimed prefill runs first, so the timed one
    finds the libraries it calls initialised (as after the reference engine's
    warmup, engine.py:149-175), whichever phase of the process ran before."""
    plan.prefill()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    plan.prefill()
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    if plan.g_decode is None:
        plan.capture()
    if steps > plan.max_new:
        raise ValueError(f"{steps} decode steps exceed the plan's max_new = {plan.max_new}")
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        plan.step()
    b.record()
    b.synchronize()
    ms = a.elapsed_time(b)
    return {"tok_s": plan.B * steps / (ms * 1e-3), "ms_per_step": ms / steps, "steps": steps,
            "prefill_s": prefill_s, "e2e_tok_s": plan.B * (steps + 1) / (prefill_s + ms * 1e-3)}


def time_delivery(plan: DecodePlan, ids: torch.Tensor, new_tokens: int, depth: int = 3) -> dict:
    """Throughput as a consumer of ``DecodePlan.run`` sees it (host clock):
    every position's tokens copied to pinned host memory and handed over as a
    Python list, the GPU kept ``depth`` steps ahead.  delivered tok/s = B x
    (new_tokens - 1) / (time from the prefill's tokens to the last step's);
    end-to-end tok/s = B x new_tokens / (time from the call to the last step's
    tokens, prefill included), the reference's definition
    (QWEN_ENGINE_CONTRACT.md:93-102).  Returns the tokens too."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    toks, times = [], []
    for row in plan.run(ids, new_tokens, depth=depth):
        times.append(time.perf_counter())
        toks.append(row)
    decode_s = times[-1] - times[0]
    return {"delivered_tok_s": plan.B * (new_tokens - 1) / decode_s if new_tokens > 1 else 0.0,
            "e2e_tok_s": plan.B * new_tokens / (times[-1] - t0), "first_token_s": times[0] - t0,
            "depth": depth, "tokens": toks}
