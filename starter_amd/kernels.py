"""Python face of the decode-GEMM hot path, mirroring the reference's kernel API.

Each class/function keeps the reference's name, argument meaning and error
behaviour (a Python exception on failure) and runs the HIP kernels of
libstarter_amd.so through the C ABI:

===========================  ==================================================
reference                    here
===========================  ==================================================
SkinnyMatmul  gemm.py:349    SkinnyMatmul (sk_gemm_bf16)
SkinnyGateUp  gemm.py:315    SkinnyGateUp (sk_gateup_swiglu_bf16)
Gemv          gemm.py:259    Gemv (sk_gemm_bf16 / sk_gateup_swiglu_bf16, GEMV path)
pick_matmul   gemm.py:516    pick_matmul (offline table instead of warmup timing)
pick_gateup   gemm.py:561    pick_gateup
pick_normed   gemm.py:602    pick_normed (sk_rmsnorm_gemm_bf16 / sk_rmsnorm_gateup_swiglu_bf16)
_norm_stats + _normed_tile   rmsnorm_gemm / rmsnorm_gateup_swiglu / rmsnorm_lm_argmax
  gemm.py:28-56, 184-208     (norm prologue fused into the projection kernel)
add_rms_norm  add_rmsnorm.py add_rms_norm (sk_add_rmsnorm_bf16)
swiglu        swiglu.py      swiglu (sk_swiglu_bf16)
fast_topk[0]  topk.py:40     argmax (sk_argmax_bf16)
fast_topk     topk.py:40     fast_topk (sk_topk_bf16, same lane-sweep algorithm)
qk_norm_rope_cache rope.py   qk_norm_rope_cache (sk_qk_norm_rope_cache_bf16)
DecodeAttention attention.py DecodeAttention (sk_decode_attention_bf16, chain masks)
logits.argmax engine.py:207  LmArgmax (sk_lm_argmax_bf16, fused into lm_head)
(none)                       gemm_residual / rmsnorm_pre_*: the add + RMSNorm
                             between two projections split across the
                             producing and consuming kernels (decode step)
===========================  ==================================================

All tensors are bf16 and live on one ROCm device; outputs are allocated per
call with ``torch.empty`` (inside a graph capture they come from the graph's
pool, as in the reference), workspaces once per instance.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from . import _lib
from ._lib import (SK_OP_ARGMAX, SK_OP_GATEUP, SK_OP_GEMM, SK_OP_LM_ARGMAX, SK_OP_PRE_GATEUP, SK_OP_PRE_GEMM,
                   SK_OP_PRE_LM_ARGMAX, SK_OP_RESID_GEMM, SK_OP_RMSNORM_GATEUP, SK_OP_RMSNORM_GEMM,
                   SK_OP_RMSNORM_LM_ARGMAX, SK_PATH_GEMV, SK_PATH_MFMA, SkConfig, check, cfg_ptr, lib)

BF16 = torch.bfloat16

__all__ = [
    "SkinnyMatmul", "SkinnyGateUp", "Gemv", "LmArgmax", "gemm", "gateup_swiglu", "lm_argmax", "argmax",
    "rmsnorm_gemm", "rmsnorm_gateup_swiglu", "rmsnorm_lm_argmax",
    "add_rms_norm", "swiglu", "pick_matmul", "pick_gateup", "pick_normed", "pick_lm_argmax", "SkConfig",
    "SK_PATH_MFMA", "SK_PATH_GEMV", "SK_OP_GEMM", "SK_OP_GATEUP", "SK_OP_LM_ARGMAX", "SK_OP_ARGMAX",
    "SK_OP_RMSNORM_GEMM", "SK_OP_RMSNORM_GATEUP", "SK_OP_RMSNORM_LM_ARGMAX",
    "qk_norm_rope_cache", "DecodeAttention", "ancestor_masks", "fast_topk",
    "gemm_residual", "rmsnorm_pre_gemm", "rmsnorm_pre_gateup_swiglu", "rmsnorm_pre_lm_argmax", "sumsq_groups",
]


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _mat(t: torch.Tensor, name: str) -> None:
    _need(t.is_cuda, f"{name} must be a ROCm device tensor")
    _need(t.dtype == BF16, f"{name} must be bfloat16, got {t.dtype}")
    _need(t.dim() == 2 and t.stride(1) == 1, f"{name} must be 2-D with unit inner stride")


def _device_guard(t: torch.Tensor) -> None:
    if torch.cuda.current_device() != t.device.index:
        torch.cuda.set_device(t.device)


def _workspace(op: int, M: int, N: int, K: int, cfg: SkConfig | None, device) -> torch.Tensor | None:
    """Zero-filled once: the library's arrival counters live at its start and
    every call leaves them at zero again."""
    n = _lib.workspace_bytes(op, M, N, K, cfg)
    return torch.zeros(n, dtype=torch.uint8, device=device) if n else None


def _ws_args(ws: torch.Tensor | None):
    return (ws.data_ptr(), ws.numel()) if ws is not None else (None, 0)


def _argmax_outputs(ids: torch.Tensor | None, maxv: torch.Tensor | None, M: int, device):
    """The (ids, maxv) outputs of an argmax call: allocated when not given, else
    checked to be what the kernel writes (int64 / float32, >= M contiguous
    elements on the call's device), so a caller-supplied buffer can never be
    written past its end."""
    if ids is None:
        ids = torch.empty((M,), dtype=torch.int64, device=device)
    if maxv is None:
        maxv = torch.empty((M,), dtype=torch.float32, device=device)
    _need(ids.dtype == torch.int64, f"ids must be int64, got {ids.dtype}")
    _need(maxv.dtype == torch.float32, f"maxv must be float32, got {maxv.dtype}")
    _need(ids.is_contiguous() and maxv.is_contiguous(), "ids and maxv must be contiguous")
    _need(ids.numel() >= M and maxv.numel() >= M, f"ids and maxv need at least M = {M} elements")
    _need(ids.device == torch.device(device) and maxv.device == torch.device(device),
          "ids and maxv must be on the device of the activations")
    return ids, maxv


def _vec(t: torch.Tensor, name: str, dtype: torch.dtype, numel: int, exact: bool = True) -> None:
    """A contiguous 1-D parameter vector (norm gains, positions) of the right dtype and length."""
    _need(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}")
    _need(t.is_contiguous(), f"{name} must be contiguous")
    _need(t.numel() == numel if exact else t.numel() >= numel,
          f"{name} must have {'' if exact else 'at least '}{numel} elements, got {t.numel()}")
    _need(t.is_cuda, f"{name} must be a ROCm device tensor")


def _config(config: SkConfig | None, kw: dict) -> SkConfig | None:
    if config is not None and kw:
        raise ValueError("pass either config= or individual config fields, not both")
    if kw:
        return SkConfig.make(**kw)
    return config


# ---------------------------------------------------------------------------
# Functional entry points
# ---------------------------------------------------------------------------

def gemm(a: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None, config: SkConfig | None = None,
         ws: torch.Tensor | None = None) -> torch.Tensor:
    """``out = a @ w.T`` (bf16, fp32 accumulation)."""
    _mat(a, "a")
    _mat(w, "w")
    M, K = a.shape
    N = w.shape[0]
    _need(w.shape[1] == K, f"K mismatch: a {tuple(a.shape)} vs w {tuple(w.shape)}")
    if out is None:
        out = torch.empty((M, N), dtype=BF16, device=a.device)
    _mat(out, "out")
    _need(tuple(out.shape) == (M, N), "out shape")
    if ws is None and _lib.workspace_bytes(SK_OP_GEMM, M, N, K, config):
        ws = _workspace(SK_OP_GEMM, M, N, K, config, a.device)
    _device_guard(a)
    wp, wn = _ws_args(ws)
    check(lib().sk_gemm_bf16(a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0), out.data_ptr(), out.stride(0),
                             M, N, K, cfg_ptr(config), wp, wn, _stream(a)), "sk_gemm_bf16")
    return out


def gateup_swiglu(a: torch.Tensor, wg: torch.Tensor, wu: torch.Tensor, out: torch.Tensor | None = None,
                  config: SkConfig | None = None, ws: torch.Tensor | None = None) -> torch.Tensor:
    """``out = swiglu(a @ wg.T, a @ wu.T)`` with the reference's bf16 casts."""
    _mat(a, "a")
    _mat(wg, "wg")
    _mat(wu, "wu")
    M, K = a.shape
    I = wg.shape[0]
    _need(wg.shape == wu.shape and wg.shape[1] == K and wg.stride(0) == wu.stride(0), "gate/up weight shapes")
    if out is None:
        out = torch.empty((M, I), dtype=BF16, device=a.device)
    _mat(out, "out")
    _need(tuple(out.shape) == (M, I), "out shape")
    if ws is None and _lib.workspace_bytes(SK_OP_GATEUP, M, I, K, config):
        ws = _workspace(SK_OP_GATEUP, M, I, K, config, a.device)
    _device_guard(a)
    wp, wn = _ws_args(ws)
    check(lib().sk_gateup_swiglu_bf16(a.data_ptr(), a.stride(0), wg.data_ptr(), wu.data_ptr(), wg.stride(0),
                                      out.data_ptr(), out.stride(0), M, I, K, cfg_ptr(config), wp, wn, _stream(a)),
          "sk_gateup_swiglu_bf16")
    return out


def lm_argmax(a: torch.Tensor, w: torch.Tensor, config: SkConfig | None = None, ws: torch.Tensor | None = None,
              ids: torch.Tensor | None = None, maxv: torch.Tensor | None = None):
    """Greedy token per row of ``bf16(a @ w.T)`` without materialising the logits.
    Returns ``(ids int64 [M], maxv float32 [M])``."""
    _mat(a, "a")
    _mat(w, "w")
    M, K = a.shape
    V = w.shape[0]
    _need(w.shape[1] == K, "K mismatch")
    ids, maxv = _argmax_outputs(ids, maxv, M, a.device)
    if ws is None:
        ws = _workspace(SK_OP_LM_ARGMAX, M, V, K, config, a.device)
    _device_guard(a)
    wp, wn = _ws_args(ws)
    check(lib().sk_lm_argmax_bf16(a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0), ids.data_ptr(),
                                  maxv.data_ptr(), M, V, K, cfg_ptr(config), wp, wn, _stream(a)),
          "sk_lm_argmax_bf16")
    return ids, maxv


def _norm_inputs(x: torch.Tensor, y: torch.Tensor, w_norm: torch.Tensor, xout: torch.Tensor) -> None:
    _mat(x, "x")
    _mat(y, "y")
    _mat(xout, "xout")
    _need(y.shape == x.shape and y.stride(0) == x.stride(0), "y must match x (shape and row stride)")
    _need(xout.shape == x.shape and xout.stride(0) == x.stride(0), "xout must match x (shape and row stride)")
    _need(w_norm.dtype == BF16 and w_norm.is_contiguous() and w_norm.numel() == x.shape[1], "w_norm must be bf16 [K]")


def rmsnorm_gemm(x: torch.Tensor, y: torch.Tensor, w_norm: torch.Tensor, eps: float, xout: torch.Tensor,
                 w: torch.Tensor, out: torch.Tensor | None = None, config: SkConfig | None = None,
                 ws: torch.Tensor | None = None) -> torch.Tensor:
    """``xout = x + y``; ``out = rms_norm(xout, w_norm) @ w.T`` in one kernel when the
    configuration allows (engine/kernels/gemm.py:602-660, prologue 28-56)."""
    _norm_inputs(x, y, w_norm, xout)
    _mat(w, "w")
    M, K = x.shape
    N = w.shape[0]
    _need(w.shape[1] == K, f"K mismatch: x {tuple(x.shape)} vs w {tuple(w.shape)}")
    if out is None:
        out = torch.empty((M, N), dtype=BF16, device=x.device)
    _mat(out, "out")
    _need(tuple(out.shape) == (M, N), "out shape")
    if ws is None and _lib.workspace_bytes(SK_OP_RMSNORM_GEMM, M, N, K, config):
        ws = _workspace(SK_OP_RMSNORM_GEMM, M, N, K, config, x.device)
    _device_guard(x)
    wp, wn = _ws_args(ws)
    check(lib().sk_rmsnorm_gemm_bf16(x.data_ptr(), y.data_ptr(), w_norm.data_ptr(), float(eps), xout.data_ptr(),
                                     x.stride(0), w.data_ptr(), w.stride(0), out.data_ptr(), out.stride(0), M, N, K,
                                     cfg_ptr(config), wp, wn, _stream(x)), "sk_rmsnorm_gemm_bf16")
    return out


def rmsnorm_gateup_swiglu(x: torch.Tensor, y: torch.Tensor, w_norm: torch.Tensor, eps: float, xout: torch.Tensor,
                          wg: torch.Tensor, wu: torch.Tensor, out: torch.Tensor | None = None,
                          config: SkConfig | None = None, ws: torch.Tensor | None = None) -> torch.Tensor:
    """``xout = x + y``; ``out = swiglu(h @ wg.T, h @ wu.T)`` with ``h = rms_norm(xout, w_norm)``."""
    _norm_inputs(x, y, w_norm, xout)
    _mat(wg, "wg")
    _mat(wu, "wu")
    M, K = x.shape
    I = wg.shape[0]
    _need(wg.shape == wu.shape and wg.shape[1] == K and wg.stride(0) == wu.stride(0), "gate/up weight shapes")
    if out is None:
        out = torch.empty((M, I), dtype=BF16, device=x.device)
    _mat(out, "out")
    _need(tuple(out.shape) == (M, I), "out shape")
    if ws is None and _lib.workspace_bytes(SK_OP_RMSNORM_GATEUP, M, I, K, config):
        ws = _workspace(SK_OP_RMSNORM_GATEUP, M, I, K, config, x.device)
    _device_guard(x)
    wp, wn = _ws_args(ws)
    check(lib().sk_rmsnorm_gateup_swiglu_bf16(x.data_ptr(), y.data_ptr(), w_norm.data_ptr(), float(eps),
                                              xout.data_ptr(), x.stride(0), wg.data_ptr(), wu.data_ptr(),
                                              wg.stride(0), out.data_ptr(), out.stride(0), M, I, K, cfg_ptr(config),
                                              wp, wn, _stream(x)), "sk_rmsnorm_gateup_swiglu_bf16")
    return out


def rmsnorm_lm_argmax(x: torch.Tensor, y: torch.Tensor, w_norm: torch.Tensor, eps: float, xout: torch.Tensor,
                      w: torch.Tensor, config: SkConfig | None = None, ws: torch.Tensor | None = None,
                      ids: torch.Tensor | None = None, maxv: torch.Tensor | None = None):
    """``xout = x + y``; greedy token per row of ``rms_norm(xout, w_norm) @ w.T``.
    Returns ``(ids int64 [M], maxv float32 [M])``."""
    _norm_inputs(x, y, w_norm, xout)
    _mat(w, "w")
    M, K = x.shape
    V = w.shape[0]
    _need(w.shape[1] == K, "K mismatch")
    ids, maxv = _argmax_outputs(ids, maxv, M, x.device)
    if ws is None:
        ws = _workspace(SK_OP_RMSNORM_LM_ARGMAX, M, V, K, config, x.device)
    _device_guard(x)
    wp, wn = _ws_args(ws)
    check(lib().sk_rmsnorm_lm_argmax_bf16(x.data_ptr(), y.data_ptr(), w_norm.data_ptr(), float(eps),
                                          xout.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0), ids.data_ptr(),
                                          maxv.data_ptr(), M, V, K, cfg_ptr(config), wp, wn, _stream(x)),
          "sk_rmsnorm_lm_argmax_bf16")
    return ids, maxv


# ---------------------------------------------------------------------------
# Residual hand-off: the add + RMSNorm between two projections of a decoder
# layer split across the producing and the consuming kernel (no norm kernel
# in between).  The producer writes the residual xout = bf16(r + bf16(a @ w.T))
# and per-row sums of squares of xout over 16-column groups; the consumer
# finishes the norm from those sums.
# ---------------------------------------------------------------------------

def _f32_vec(t: torch.Tensor, name: str, numel: int) -> None:
    _need(t.dtype == torch.float32 and t.is_contiguous() and t.numel() >= numel and t.is_cuda,
          f"{name} must be a contiguous float32 CUDA tensor with >= {numel} elements")


def sumsq_groups(M: int, N: int) -> int:
    """Columns of the partial-sums buffer of an [M, N] residual: ceil(N / 16)."""
    return (N + 15) // 16


def gemm_residual(a: torch.Tensor, w: torch.Tensor, r: torch.Tensor, r_out: torch.Tensor, sq: torch.Tensor,
                  config: SkConfig | None = None, ws: torch.Tensor | None = None) -> torch.Tensor:
    """``r_out = bf16(r + bf16(a @ w.T))`` (the projection itself is not stored) and
    ``sq[m, g] = sum(r_out[m, 16g:16g+16] ** 2)``; ``sq`` is float32 [M, ceil(N/16)].
    ``r_out`` may be ``r``.  Returns ``r_out``."""
    _mat(a, "a")
    _mat(w, "w")
    M, K = a.shape
    N = w.shape[0]
    _need(w.shape[1] == K, f"K mismatch: a {tuple(a.shape)} vs w {tuple(w.shape)}")
    _need(r.dtype == BF16 and r_out.dtype == BF16 and r.shape == (M, N) and r_out.shape == (M, N),
          "r and r_out must be bf16 [M, N]")
    _need(r.stride(1) == 1 and r_out.stride(1) == 1 and r.stride(0) == r_out.stride(0), "r / r_out row layout")
    _f32_vec(sq, "sq", M * sumsq_groups(M, N))
    if ws is None and _lib.workspace_bytes(SK_OP_RESID_GEMM, M, N, K, config):
        ws = _workspace(SK_OP_RESID_GEMM, M, N, K, config, a.device)
    _device_guard(a)
    wp, wn = _ws_args(ws)
    check(lib().sk_gemm_residual_bf16(a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0), r.data_ptr(),
                                      r_out.data_ptr(), r.stride(0), sq.data_ptr(), M, N, K, cfg_ptr(config), wp, wn,
                                      _stream(a)), "sk_gemm_residual_bf16")
    return r_out


def _pre_inputs(x: torch.Tensor, sq: torch.Tensor, w_norm: torch.Tensor) -> None:
    _mat(x, "x")
    M, K = x.shape
    _need(K % 16 == 0, "K must be a multiple of 16")
    _f32_vec(sq, "sq", M * (K // 16))
    _need(w_norm.dtype == BF16 and w_norm.is_contiguous() and w_norm.numel() == K, "w_norm must be bf16 [K]")


def rmsnorm_pre_gemm(x: torch.Tensor, sq: torch.Tensor, w_norm: torch.Tensor, eps: float, w: torch.Tensor,
                     out: torch.Tensor | None = None, config: SkConfig | None = None,
                     ws: torch.Tensor | None = None) -> torch.Tensor:
    """``out = rms_norm(x, w_norm) @ w.T`` with the row norms taken from a producer's
    partial sums ``sq`` (float32 [M, K/16], see gemm_residual)."""
    _pre_inputs(x, sq, w_norm)
    _mat(w, "w")
    M, K = x.shape
    N = w.shape[0]
    _need(w.shape[1] == K, "K mismatch")
    if out is None:
        out = torch.empty((M, N), dtype=BF16, device=x.device)
    _mat(out, "out")
    _need(tuple(out.shape) == (M, N), "out shape")
    if ws is None and _lib.workspace_bytes(SK_OP_PRE_GEMM, M, N, K, config):
        ws = _workspace(SK_OP_PRE_GEMM, M, N, K, config, x.device)
    _device_guard(x)
    wp, wn = _ws_args(ws)
    check(lib().sk_rmsnorm_pre_gemm_bf16(x.data_ptr(), x.stride(0), sq.data_ptr(), w_norm.data_ptr(), float(eps),
                                         w.data_ptr(), w.stride(0), out.data_ptr(), out.stride(0), M, N, K,
                                         cfg_ptr(config), wp, wn, _stream(x)), "sk_rmsnorm_pre_gemm_bf16")
    return out


def rmsnorm_pre_gateup_swiglu(x: torch.Tensor, sq: torch.Tensor, w_norm: torch.Tensor, eps: float,
                              wg: torch.Tensor, wu: torch.Tensor, out: torch.Tensor | None = None,
                              config: SkConfig | None = None, ws: torch.Tensor | None = None) -> torch.Tensor:
    """``out = swiglu(h @ wg.T, h @ wu.T)``, ``h = rms_norm(x, w_norm)`` from partial sums ``sq``."""
    _pre_inputs(x, sq, w_norm)
    _mat(wg, "wg")
    _mat(wu, "wu")
    M, K = x.shape
    I = wg.shape[0]
    _need(wg.shape == wu.shape and wg.shape[1] == K and wg.stride(0) == wu.stride(0), "gate/up weight shapes")
    if out is None:
        out = torch.empty((M, I), dtype=BF16, device=x.device)
    _mat(out, "out")
    _need(tuple(out.shape) == (M, I), "out shape")
    if ws is None and _lib.workspace_bytes(SK_OP_PRE_GATEUP, M, I, K, config):
        ws = _workspace(SK_OP_PRE_GATEUP, M, I, K, config, x.device)
    _device_guard(x)
    wp, wn = _ws_args(ws)
    check(lib().sk_rmsnorm_pre_gateup_swiglu_bf16(x.data_ptr(), x.stride(0), sq.data_ptr(), w_norm.data_ptr(),
                                                  float(eps), wg.data_ptr(), wu.data_ptr(), wg.stride(0),
                                                  out.data_ptr(), out.stride(0), M, I, K, cfg_ptr(config), wp, wn,
                                                  _stream(x)), "sk_rmsnorm_pre_gateup_swiglu_bf16")
    return out


def rmsnorm_pre_lm_argmax(x: torch.Tensor, sq: torch.Tensor, w_norm: torch.Tensor, eps: float, w: torch.Tensor,
                          config: SkConfig | None = None, ws: torch.Tensor | None = None,
                          ids: torch.Tensor | None = None, maxv: torch.Tensor | None = None):
    """Greedy token per row of ``rms_norm(x, w_norm) @ w.T`` with the norms from ``sq``.
    Returns ``(ids int64 [M], maxv float32 [M])``."""
    _pre_inputs(x, sq, w_norm)
    _mat(w, "w")
    M, K = x.shape
    V = w.shape[0]
    _need(w.shape[1] == K, "K mismatch")
    ids, maxv = _argmax_outputs(ids, maxv, M, x.device)
    if ws is None:
        ws = _workspace(SK_OP_PRE_LM_ARGMAX, M, V, K, config, x.device)
    _device_guard(x)
    wp, wn = _ws_args(ws)
    check(lib().sk_rmsnorm_pre_lm_argmax_bf16(x.data_ptr(), x.stride(0), sq.data_ptr(), w_norm.data_ptr(),
                                              float(eps), w.data_ptr(), w.stride(0), ids.data_ptr(), maxv.data_ptr(),
                                              M, V, K, cfg_ptr(config), wp, wn, _stream(x)),
          "sk_rmsnorm_pre_lm_argmax_bf16")
    return ids, maxv


def argmax(logits: torch.Tensor, ws: torch.Tensor | None = None):
    """``(logits.argmax(-1), logits.max(-1).float())`` over bf16 logits, lowest index on ties."""
    _mat(logits, "logits")
    M, V = logits.shape
    ids = torch.empty((M,), dtype=torch.int64, device=logits.device)
    maxv = torch.empty((M,), dtype=torch.float32, device=logits.device)
    if ws is None:
        ws = _workspace(SK_OP_ARGMAX, M, V, 0, None, logits.device)
    _device_guard(logits)
    wp, wn = _ws_args(ws)
    check(lib().sk_argmax_bf16(logits.data_ptr(), logits.stride(0), M, V, ids.data_ptr(), maxv.data_ptr(), wp, wn,
                               _stream(logits)), "sk_argmax_bf16")
    return ids, maxv


def fast_topk(logits: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """[N, V] bf16 -> (values [N, k] float32, indices [N, k] int32); indices[:, 0]
    is the exact argmax (engine/kernels/topk.py:40-46, same algorithm)."""
    _mat(logits, "logits")
    N, V = logits.shape
    vals = torch.empty((N, k), dtype=torch.float32, device=logits.device)
    idxs = torch.empty((N, k), dtype=torch.int32, device=logits.device)
    _device_guard(logits)
    check(lib().sk_topk_bf16(logits.data_ptr(), logits.stride(0), N, V, k, vals.data_ptr(), idxs.data_ptr(),
                             _stream(logits)), "sk_topk_bf16")
    return vals, idxs


def add_rms_norm(x: torch.Tensor, y: torch.Tensor, weight: torch.Tensor, eps: float,
                 xout: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """``xout = x + y`` (bf16; in place into ``x`` when ``xout`` is None), returns
    ``rms_norm(xout, weight)`` (engine/kernels/add_rmsnorm.py:65-76)."""
    _mat(x, "x")
    _mat(y, "y")
    M, K = x.shape
    _need(y.shape == x.shape and y.stride(0) == x.stride(0), "x/y shapes")
    _need(weight.dtype == BF16 and weight.is_contiguous() and weight.numel() == K, "weight")
    xout = x if xout is None else xout
    _need(xout.shape == x.shape and xout.stride(0) == x.stride(0), "xout shape")
    if out is None:
        out = torch.empty_like(x)
    _need(out.shape == x.shape and out.stride(0) == x.stride(0), "out shape")
    _device_guard(x)
    check(lib().sk_add_rmsnorm_bf16(x.data_ptr(), y.data_ptr(), weight.data_ptr(), float(eps), xout.data_ptr(),
                                    out.data_ptr(), M, K, x.stride(0), _stream(x)), "sk_add_rmsnorm_bf16")
    return out


def swiglu(gu: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(gu[:, :I]) * gu[:, I:]`` with both bf16 roundings (engine/kernels/swiglu.py:27-33)."""
    _mat(gu, "gu")
    M, two_i = gu.shape
    _need(two_i % 2 == 0, "gu must hold [gate | up]")
    I = two_i // 2
    if out is None:
        out = torch.empty((M, I), dtype=BF16, device=gu.device)
    _device_guard(gu)
    check(lib().sk_swiglu_bf16(gu.data_ptr(), gu.stride(0), out.data_ptr(), out.stride(0), M, I, _stream(gu)),
          "sk_swiglu_bf16")
    return out


# ---------------------------------------------------------------------------
# Attention side of the decode step
# ---------------------------------------------------------------------------

def _rope_params(q_norm_w: torch.Tensor, k_norm_w: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                 D: int) -> None:
    """Per-head norm gains bf16 [D]; rotary tables bf16 [rows, D], contiguous."""
    _vec(q_norm_w, "q_norm_w", BF16, D)
    _vec(k_norm_w, "k_norm_w", BF16, D)
    _need(cos.dtype == BF16 and sin.dtype == BF16, "rope tables must be bf16")
    _need(cos.dim() == 2 and cos.shape == sin.shape and cos.shape[1] == D, "rope tables must be [rows, D]")
    _need(cos.is_contiguous() and sin.is_contiguous() and cos.is_cuda and sin.is_cuda,
          "rope tables must be contiguous device tensors")


def qk_norm_rope_cache(qkv: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor, cos: torch.Tensor,
                       sin: torch.Tensor, pos: torch.Tensor, q_out: torch.Tensor, k_cache: torch.Tensor,
                       v_cache: torch.Tensor, T: int, eps: float, fused: bool = True,
                       depth: torch.Tensor | None = None) -> None:
    """Normalise, rotate and scatter one projection buffer (engine/kernels/rope.py:140-188).

    qkv [B*T, (HQ + 2*HKV)*D] rows (b, t); pos [B] int32 (row (b, t) -> slot
    pos[b] + t); q_out [B, HQ, T, D]; k_cache / v_cache [B, HKV, cap, D] (one
    layer).  ``depth`` [T] int32 (draft-tree rows): row (b, t) still goes to
    slot pos[b] + t but rotates by position pos[b] + depth[t]
    (rope.py:94-122; engine/model.py:369-370).  ``fused`` is accepted for
    signature compatibility (there is one launch either way)."""
    _mat(qkv, "qkv")
    B, HQ, T_, D = q_out.shape
    _need(T_ == T, "q_out must be [B, HQ, T, D]")
    HKV, cap = k_cache.shape[1], k_cache.shape[2]
    _need(q_out.is_contiguous() and k_cache.is_contiguous() and v_cache.is_contiguous(), "contiguous outputs")
    _need(q_out.dtype == BF16 and k_cache.dtype == BF16 and v_cache.dtype == BF16, "q_out and caches must be bf16")
    _need(k_cache.shape == v_cache.shape and k_cache.shape[0] == B and k_cache.shape[3] == D, "cache shapes")
    _need(qkv.shape[0] == B * T and qkv.shape[1] >= (HQ + 2 * HKV) * D, "qkv shape")
    _rope_params(q_norm_w, k_norm_w, cos, sin, D)
    _vec(pos, "pos", torch.int32, B, exact=False)
    if depth is not None:
        _vec(depth, "depth", torch.int32, T)
    _device_guard(qkv)
    check(lib().sk_qk_norm_rope_cache_bf16(qkv.data_ptr(), qkv.stride(0), q_norm_w.data_ptr(), k_norm_w.data_ptr(),
                                           cos.data_ptr(), sin.data_ptr(), cos.shape[0], pos.data_ptr(),
                                           depth.data_ptr() if depth is not None else None, q_out.data_ptr(),
                                           k_cache.data_ptr(), v_cache.data_ptr(), B, T, HQ, HKV, D, cap, float(eps),
                                           _stream(qkv)), "sk_qk_norm_rope_cache_bf16")


class DecodeAttention:
    """Workspace-owning wrapper; one instance per (B, HQ, cap) plan
    (engine/kernels/attention.py:152-202).  Split count and key ranges are
    fixed at construction from ``maxlen`` (default cap); the valid length of
    each sequence is read from ``pos`` on the device at every call, so one
    instance replays inside a graph while the sequences grow.  ``R`` query rows
    per sequence (speculative verify), chain-masked, or with ``tree=True``
    masked by per-row ancestor bit masks passed at call time.
    ``block_n``/``num_warps``/``num_stages`` are accepted for signature
    compatibility."""

    def __init__(self, B: int, HQ: int, HKV: int, D: int, cap: int, device, nsplit: int | None = None,
                 block_n: int = 64, num_warps: int = 4, num_stages: int = 2, R: int = 1, tree: bool = False,
                 maxlen: int | None = None):
        self.B, self.HQ, self.HKV, self.D, self.cap, self.R = B, HQ, HKV, D, cap, R
        self.tree = tree
        self.maxlen = maxlen or 0
        self.nsplit = nsplit or 0
        self.scale = 1.0 / math.sqrt(D)
        n = int(lib().sk_decode_attention_workspace_bytes(B, HQ, HKV, D, R, cap, self.maxlen, self.nsplit))
        self.ws = torch.zeros(n, dtype=torch.uint8, device=device) if n else None

    def __call__(self, q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, pos: torch.Tensor,
                 out: torch.Tensor, tree: torch.Tensor | None = None) -> None:
        """q [B, HQ, R, D] bf16; k/v_cache [B, HKV, cap, D]; pos [B] int32 (position of
        query row 0); out [B, R, HQ, D] bf16; tree [R] int64 ancestor masks when this
        instance was built with tree=True."""
        B, HQ, HKV, D, R, cap = self.B, self.HQ, self.HKV, self.D, self.R, self.cap
        _need(q.shape == (B, HQ, R, D) and q.is_contiguous() and q.dtype == BF16, "q must be [B, HQ, R, D] bf16")
        _need(k_cache.shape == (B, HKV, cap, D) and v_cache.shape == k_cache.shape, "cache shapes")
        _need(k_cache.is_contiguous() and v_cache.is_contiguous(), "contiguous caches")
        _need(out.shape == (B, R, HQ, D) and out.is_contiguous() and out.dtype == BF16, "out must be [B, R, HQ, D] bf16")
        _need(k_cache.dtype == BF16 and v_cache.dtype == BF16, "caches must be bf16")
        _vec(pos, "pos", torch.int32, B, exact=False)
        if self.tree:
            _need(tree is not None and tree.is_cuda and tree.dtype == torch.int64 and tree.numel() == R,
                  "tree=True needs tree [R] int64 on the device")
        else:
            _need(tree is None, "this instance was built without tree masks")
        _device_guard(q)
        wp, wn = _ws_args(self.ws)
        check(lib().sk_decode_attention_bf16(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), pos.data_ptr(),
                                             tree.data_ptr() if tree is not None else None, out.data_ptr(), B, HQ,
                                             HKV, D, R, cap, self.maxlen, float(self.scale), self.nsplit, wp, wn,
                                             _stream(q)), "sk_decode_attention_bf16")

    def rope_attend(self, qkv: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor, cos: torch.Tensor,
                    sin: torch.Tensor, pos: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                    out: torch.Tensor, eps: float, tree: torch.Tensor | None = None,
                    depth: torch.Tensor | None = None) -> None:
        """``qk_norm_rope_cache(qkv, q_norm_w, k_norm_w, cos, sin, pos, q, k_cache, v_cache, R, eps)``
        followed by ``self(q, k_cache, v_cache, pos, out)`` in one launch
        (sk_decode_attention_rope_bf16): same outputs and cache contents, no q
        buffer.  An instance built with ``tree=True`` takes the draft tree's
        ancestor masks ``tree`` (int64 [R]) and rotary offsets ``depth`` (int32
        [R], as ``qk_norm_rope_cache(..., depth=depth)``) and runs
        sk_decode_attention_rope_tree_bf16; a chain instance takes neither."""
        B, HQ, HKV, D, R, cap = self.B, self.HQ, self.HKV, self.D, self.R, self.cap
        if self.tree:
            _need(tree is not None and depth is not None, "a tree instance needs the masks and the depths")
            _vec(tree, "tree", torch.int64, R)
            _vec(depth, "depth", torch.int32, R)
        else:
            _need(tree is None and depth is None, "masks and depths need an instance built with tree=True")
        _mat(qkv, "qkv")
        _need(qkv.shape[0] == B * R and qkv.shape[1] >= (HQ + 2 * HKV) * D, "qkv must be [B*R, (HQ+2*HKV)*D]")
        _need(k_cache.shape == (B, HKV, cap, D) and v_cache.shape == k_cache.shape, "cache shapes")
        _need(k_cache.is_contiguous() and v_cache.is_contiguous(), "contiguous caches")
        _need(out.shape == (B, R, HQ, D) and out.is_contiguous() and out.dtype == BF16, "out must be [B, R, HQ, D] bf16")
        _need(k_cache.dtype == BF16 and v_cache.dtype == BF16, "caches must be bf16")
        _rope_params(q_norm_w, k_norm_w, cos, sin, D)
        _vec(pos, "pos", torch.int32, B, exact=False)
        _device_guard(qkv)
        wp, wn = _ws_args(self.ws)
        if self.tree:
            check(lib().sk_decode_attention_rope_tree_bf16(
                qkv.data_ptr(), qkv.stride(0), q_norm_w.data_ptr(), k_norm_w.data_ptr(), cos.data_ptr(),
                sin.data_ptr(), cos.shape[0], float(eps), k_cache.data_ptr(), v_cache.data_ptr(), pos.data_ptr(),
                tree.data_ptr(), depth.data_ptr(), out.data_ptr(), B, HQ, HKV, D, R, cap, self.maxlen,
                float(self.scale), self.nsplit, wp, wn, _stream(qkv)), "sk_decode_attention_rope_tree_bf16")
            return
        check(lib().sk_decode_attention_rope_bf16(qkv.data_ptr(), qkv.stride(0), q_norm_w.data_ptr(),
                                                  k_norm_w.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.shape[0],
                                                  float(eps), k_cache.data_ptr(), v_cache.data_ptr(), pos.data_ptr(),
                                                  out.data_ptr(), B, HQ, HKV, D, R, cap, self.maxlen,
                                                  float(self.scale), self.nsplit, wp, wn, _stream(qkv)),
              "sk_decode_attention_rope_bf16")


def ancestor_masks(parent: list[int]) -> list[int]:
    """Per-node int64 bit mask of the node and its ancestors: bit j of node
    i's mask is set when j is i or on i's path to the root, the format the
    tree attention consumes (engine/kernels/attention.py:245-254).

    A draft tree lists every parent before its children (parent[i] < i, -1
    for a root), so one pass in node order builds each mask from its parent's:
    mask[i] = mask[parent[i]] | bit i.  The masks are formed as uint64 and
    reinterpreted as int64, so node 63 gives the sign bit."""
    n = len(parent)
    if n > 64:
        raise ValueError(f"a draft tree of {n} nodes does not fit 64-bit masks")
    masks = np.zeros(n, dtype=np.uint64)
    for i, p in enumerate(parent):
        if not -1 <= p < i:
            raise ValueError(f"node {i}: parent {p} must be -1 or an earlier node")
        masks[i] = (masks[p] if p >= 0 else np.uint64(0)) | (np.uint64(1) << np.uint64(i))
    return masks.view(np.int64).tolist()


def chain_tree(R: int, device) -> torch.Tensor:
    """Ancestor masks of a plain chain, row t sees draft rows 0..t
    (engine/kernels/attention.py:257-259)."""
    return torch.tensor(ancestor_masks([t - 1 for t in range(R)]), dtype=torch.int64, device=device)


def pick_attention(B: int, HQ: int, HKV: int, D: int, cap: int, typical_len: int, device, log=None, R: int = 1,
                   tree: bool = False, maxlen: int | None = None) -> DecodeAttention:
    """engine/kernels/attention.py:262-314 signature.  The split count comes from
    the library's plan (about 256 workgroups over the key range ``maxlen``), so
    nothing is timed at warmup; ``typical_len`` only feeds the log line."""
    attn = DecodeAttention(B, HQ, HKV, D, cap, device, R=R, tree=tree, maxlen=maxlen)
    if log:
        log(f"attention B={B} R={R} len={typical_len}: HIP decode attention, tree={tree}, maxlen={maxlen or cap}")
    return attn


# ---------------------------------------------------------------------------
# Reference-shaped classes: fixed (M, N, K) and config per instance.
# ---------------------------------------------------------------------------

class _Planned:
    """Fixed (M, N, K) and config.  ``normed=True`` also plans the norm-prologue
    variant (its workspace is allocated here, outside any graph capture); a
    call with ``norm=(y, w_norm, xout, eps)`` then runs ``xout = a + y`` and
    the projection of ``rms_norm(xout, w_norm)``, fused into one kernel when
    the configuration allows (engine/kernels/gemm.py:363-366)."""

    op = SK_OP_GEMM
    norm_op = SK_OP_RMSNORM_GEMM

    def __init__(self, M: int, N: int, K: int, device, config: SkConfig | None = None, normed: bool = False,
                 **cfg_kw):
        self.M, self.N, self.K = M, N, K
        self.device = torch.device(device)
        self.config = _config(config, cfg_kw)
        if self.config is not None:
            st = _lib.check_config(self.op, M, N, K, self.config)
            if st != _lib.SK_OK:
                raise _lib.SkError(st, f"config {self.config} for op {self.op} at M={M} N={N} K={K}")
        self.ws = _workspace(self.op, M, N, K, self.config, self.device) if M > 0 else None
        self.ws_norm = None
        self._norm_planned = False
        if normed:
            self._plan_norm()

    def _plan_norm(self) -> None:
        if self.M > 0:
            self.ws_norm = _workspace(self.norm_op, self.M, self.N, self.K, self.config, self.device)
        self._norm_planned = True

    def _norm_ws(self):
        if not self._norm_planned:
            self._plan_norm()
        return self.ws_norm


class SkinnyMatmul(_Planned):
    """``C[M, N] = A[M, K] @ W[N, K]^T`` (engine/kernels/gemm.py:349-378).

    ``norm=(y, w_norm, xout, eps)`` runs ``xout = a + y; a = rms_norm(xout, w_norm)``
    in front, like the reference's fused prologue (gemm.py:363-366)."""

    op = SK_OP_GEMM
    norm_op = SK_OP_RMSNORM_GEMM

    def __call__(self, a: torch.Tensor, w: torch.Tensor, norm=None) -> torch.Tensor:
        if norm is not None:
            y, wn, xout, eps = norm
            return rmsnorm_gemm(a, y, wn, eps, xout, w, config=self.config, ws=self._norm_ws())
        return gemm(a, w, config=self.config, ws=self.ws)


class SkinnyGateUp(_Planned):
    """``swiglu(a @ wg.T, a @ wu.T)`` in one pass over both weight halves
    (engine/kernels/gemm.py:315-346)."""

    op = SK_OP_GATEUP
    norm_op = SK_OP_RMSNORM_GATEUP

    def __call__(self, a: torch.Tensor, wg: torch.Tensor, wu: torch.Tensor, norm=None) -> torch.Tensor:
        if norm is not None:
            y, wn, xout, eps = norm
            return rmsnorm_gateup_swiglu(a, y, wn, eps, xout, wg, wu, config=self.config, ws=self._norm_ws())
        return gateup_swiglu(a, wg, wu, config=self.config, ws=self.ws)


class Gemv(_Planned):
    """VALU GEMV for M <= 8 rows, optionally the SwiGLU pair (engine/kernels/gemm.py:259-292).

    Config fields are those of the GEMV path: ``rows`` weight rows per tile
    (2, 4, 8), ``ku`` 512-column units per wave, ``waves`` per workgroup."""

    def __init__(self, M: int, N: int, K: int, device, gateup: bool = False, config: SkConfig | None = None,
                 normed: bool = False, **cfg_kw):
        if M > 8:
            raise ValueError("Gemv handles at most 8 rows")
        self.op = SK_OP_GATEUP if gateup else SK_OP_GEMM
        self.norm_op = SK_OP_RMSNORM_GATEUP if gateup else SK_OP_RMSNORM_GEMM
        self.gateup = gateup
        if config is None and not cfg_kw:
            cfg_kw = dict(path=SK_PATH_GEMV, waves=1, ku=(K + 511) // 512, rows=4)
        elif cfg_kw:
            cfg_kw.setdefault("path", SK_PATH_GEMV)
        super().__init__(M, N, K, device, config, normed=normed, **cfg_kw)

    def __call__(self, a: torch.Tensor, w: torch.Tensor, w2: torch.Tensor | None = None, norm=None) -> torch.Tensor:
        if norm is not None:
            y, wn, xout, eps = norm
            if self.gateup:
                return rmsnorm_gateup_swiglu(a, y, wn, eps, xout, w, w2, config=self.config, ws=self._norm_ws())
            return rmsnorm_gemm(a, y, wn, eps, xout, w, config=self.config, ws=self._norm_ws())
        if self.gateup:
            return gateup_swiglu(a, w, w2, config=self.config, ws=self.ws)
        return gemm(a, w, config=self.config, ws=self.ws)


class LmArgmax(_Planned):
    """lm_head projection fused with the greedy argmax: ``(ids, maxv)``."""

    op = SK_OP_LM_ARGMAX
    norm_op = SK_OP_RMSNORM_LM_ARGMAX

    def __call__(self, a: torch.Tensor, w: torch.Tensor, norm=None):
        if norm is not None:
            y, wn, xout, eps = norm
            return rmsnorm_lm_argmax(a, y, wn, eps, xout, w, config=self.config, ws=self._norm_ws())
        return lm_argmax(a, w, config=self.config, ws=self.ws)


# ---------------------------------------------------------------------------
# Pickers: the reference times candidates at warmup (gemm.py:477-660); here
# the configuration comes from the library's offline-tuned table, so a picker
# only binds shapes.  The signatures are the reference's; ``log`` receives one
# line naming the chosen config, ``ws`` (the rotation list) is accepted and
# unused.
# ---------------------------------------------------------------------------

def _log_choice(log, what: str, op: int, M: int, N: int, K: int) -> None:
    if log:
        log(f"{what} M={M} N={N} K={K}: {_lib.default_config(op, M, N, K).as_dict()}")


def pick_matmul(a: torch.Tensor, w: torch.Tensor, log=None, ws: list | None = None):
    """``f(a, w) -> a @ w.T`` for this exact shape (engine/kernels/gemm.py:516-558)."""
    M, K = a.shape
    N = w.shape[0]
    mm = SkinnyMatmul(M, N, K, a.device)
    _log_choice(log, "matmul", SK_OP_GEMM, M, N, K)
    return lambda a, w: mm(a, w)


def pick_gateup(a: torch.Tensor, wgu: torch.Tensor, log=None, ws: list | None = None):
    """``f(a, wgu) -> swiglu(a @ wgu.T)`` (engine/kernels/gemm.py:561-599)."""
    M, K = a.shape
    I = wgu.shape[0] // 2
    mm = SkinnyGateUp(M, I, K, a.device)
    _log_choice(log, "gateup", SK_OP_GATEUP, M, I, K)
    return lambda a, wgu: mm(a, wgu[:I], wgu[I:])


def pick_normed(kind: str, x: torch.Tensor, y: torch.Tensor, w_norm: torch.Tensor, w: torch.Tensor, eps: float,
                log=None, ws: list | None = None):
    """``f(x, y, w_norm, xout, w) -> proj(rms_norm(x + y))`` that also writes
    ``xout = x + y`` (engine/kernels/gemm.py:602-660).  ``kind``: "matmul" or "gateup"."""
    M, K = x.shape
    if kind == "matmul":
        mm = SkinnyMatmul(M, w.shape[0], K, x.device, normed=True)
        _log_choice(log, "normed matmul", SK_OP_GEMM, M, w.shape[0], K)
        return lambda x, y, w_norm, xout, w: mm(x, w, norm=(y, w_norm, xout, eps))
    if kind == "gateup":
        I = w.shape[0] // 2
        mm = SkinnyGateUp(M, I, K, x.device, normed=True)
        _log_choice(log, "normed gateup", SK_OP_GATEUP, M, I, K)
        return lambda x, y, w_norm, xout, w: mm(x, w[:I], w[I:], norm=(y, w_norm, xout, eps))
    raise ValueError(f"unknown kind {kind!r}")


def pick_lm_argmax(x: torch.Tensor, w: torch.Tensor, eps: float, log=None):
    """``f(x, y, w_norm, xout, w) -> (ids, maxv)``: the normed lm_head with the
    greedy argmax fused in (replaces ``mm["lm"](...).argmax(-1)``)."""
    M, K = x.shape
    mm = LmArgmax(M, w.shape[0], K, x.device, normed=True)
    _log_choice(log, "normed lm_argmax", SK_OP_LM_ARGMAX, M, w.shape[0], K)
    return lambda x, y, w_norm, xout, w: mm(x, w, norm=(y, w_norm, xout, eps))
