"""Shared helpers of the test suite: seeded bf16 inputs, bit views, tolerances."""

from __future__ import annotations

import numpy as np
import torch

BF16 = torch.bfloat16

# Parity rule of the hot path: |out - ref| <= RTOL * max(|ref|, TAU * rms(ref row)).
# RTOL is the north-star bound (max relative error 1e-2 per element); the floor
# TAU * rms(row) only matters for outputs within 1e-3 of zero relative to their
# row, where two valid fp32 summation orders differ by more than 1% of the value.
RTOL = 1e-2
TAU = 1e-3


def randn_bf16(shape, scale: float, gen: torch.Generator) -> torch.Tensor:
    """fp32 randn on the CPU generator, scaled, cast to bf16 (the BASELINE recipe)."""
    return (torch.randn(*shape, generator=gen) * scale).to(BF16)


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bf16 bits of a CPU or GPU tensor as a uint16 numpy array."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def from_bits(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(BF16)


def rel_violations(out: torch.Tensor, ref: torch.Tensor, rtol: float = RTOL, tau: float = TAU) -> tuple[int, float]:
    """(number of elements outside the parity rule, worst |err| / allowed)."""
    o = out.detach().cpu().float()
    r = ref.detach().cpu().float()
    rms = r.pow(2).mean(-1, keepdim=True).sqrt()
    allowed = rtol * torch.maximum(r.abs(), tau * rms)
    err = (o - r).abs()
    ratio = err / allowed.clamp_min(1e-30)
    return int((err > allowed).sum().item()), float(ratio.max().item()) if ratio.numel() else 0.0


def assert_parity(out: torch.Tensor, ref: torch.Tensor, what: str = "") -> None:
    bad, worst = rel_violations(out, ref)
    assert bad == 0, f"{what}: {bad} elements outside 1e-2*max(|ref|, 1e-3*rms), worst ratio {worst:.3g}"


def reference_tolerance_ok(out: torch.Tensor, ref: torch.Tensor) -> bool:
    """The reference test suite's own acceptance: err <= 0.02*max|ref| + 1e-3
    (tests/test_kernels.py:123, engine/kernels/gemm.py:542-543)."""
    o, r = out.detach().cpu().float(), ref.detach().cpu().float()
    return (o - r).abs().max().item() <= 0.02 * r.abs().max().item() + 1e-3
