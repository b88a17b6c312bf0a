"""Write the seeded golden fixtures of the decode-GEMM hot path.

The reference ships no golden vectors (its tests draw random tensors at run
time and compare against torch on CUDA, tests/test_kernels.py), so these
fixtures are produced by torch's CPU library routines, the functions the
reference itself treats as ground truth:

  gemm          F.linear(x, W)                      (engine/kernels/gemm.py:527 `a @ w.t()`)
  gateup        F.silu(F.linear(x, Wg)) * F.linear(x, Wu)   (gemm.py:569 + swiglu.py)
  swiglu        F.silu(g) * u                        (tests/test_kernels.py:22-27)
  add_rmsnorm   xout = x + y; w * (h * rsqrt(mean(h^2) + eps)).to(bf16)
                                                     (tests/test_kernels.py:11-14, 90-99)
  argmax        torch.argmax / max over bf16 logits  (engine/engine.py:207)
  lm_argmax     F.linear then argmax

Inputs are drawn on a CPU torch.Generator (fp32 randn, scaled, cast to bf16).
Every array is stored as raw bf16 bits (uint16) or int64/float32, in one
.npz per case (no pickles).  Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent
BF16 = torch.bfloat16


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _randn(shape, scale, gen):
    return (torch.randn(*shape, generator=gen) * scale).to(BF16)


def ref_rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    h = x.float()
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    return w * h.to(x.dtype)


def make() -> list[Path]:
    out = []
    g = torch.Generator().manual_seed(20261201)

    # Plain GEMMs: a ragged N, a K that is only a multiple of 32, M over 16.
    for name, (M, N, K) in {"gemm_m3_n40_k96": (3, 40, 96), "gemm_m1_n48_k2560": (1, 48, 2560),
                            "gemm_m19_n33_k256": (19, 33, 256)}.items():
        x = _randn((M, K), 1.0, g)
        w = _randn((N, K), 0.02, g)
        y = F.linear(x, w)
        np.savez(HERE / f"{name}.npz", x=_bits(x), w=_bits(w), y=_bits(y))
        out.append(HERE / f"{name}.npz")

    # Gate/up with the SwiGLU epilogue.
    M, I, K = 2, 24, 256
    x = _randn((M, K), 1.0, g)
    wgu = _randn((2 * I, K), 0.05, g)
    y = F.silu(F.linear(x, wgu[:I])) * F.linear(x, wgu[I:])
    np.savez(HERE / "gateup_m2_i24_k256.npz", x=_bits(x), wgu=_bits(wgu), y=_bits(y))
    out.append(HERE / "gateup_m2_i24_k256.npz")

    # Elementwise SwiGLU, wide range (x3 like tests/test_kernels.py:24).
    gu = _randn((3, 2 * 512), 3.0, g)
    y = F.silu(gu[:, :512]) * gu[:, 512:]
    np.savez(HERE / "swiglu_m3_i512.npz", gu=_bits(gu), y=_bits(y))
    out.append(HERE / "swiglu_m3_i512.npz")

    # Residual add + RMSNorm at the hidden width.
    x = _randn((4, 2560), 1.0, g)
    yv = _randn((4, 2560), 1.0, g)
    w = (1 + 0.1 * torch.randn(2560, generator=g)).to(BF16)
    xout = x + yv
    h = ref_rmsnorm(xout, w, 1e-6)
    np.savez(HERE / "add_rmsnorm_m4_k2560.npz", x=_bits(x), y=_bits(yv), w=_bits(w), eps=np.float32(1e-6),
             xout=_bits(xout), out=_bits(h))
    out.append(HERE / "add_rmsnorm_m4_k2560.npz")

    # Argmax rows: random, unique planted max, exact tie (lowest index wins),
    # -0 vs +0 tie, NaN (first NaN wins, torch semantics), all equal.
    V = 1000
    L = (torch.randn(7, V, generator=g) * 4).to(BF16)
    L[1, 7] = L[1].max() + 1
    L[2, 100] = L[2, 200] = L[2].max() + 2
    L[3] = -1.0
    L[3, 50] = -0.0
    L[3, 20] = 0.0
    L[4, 300] = float("nan")
    L[4, 600] = float("nan")
    L[5] = 0.5
    L[6, V - 1] = L[6].max() + 1
    ids = torch.argmax(L, dim=-1)
    maxv = torch.max(L, dim=-1).values.float()
    np.savez(HERE / "argmax_m7_v1000.npz", logits=_bits(L), ids=ids.numpy().astype(np.int64),
             maxv=maxv.numpy().astype(np.float32))
    out.append(HERE / "argmax_m7_v1000.npz")

    # lm_head + argmax at a small vocabulary.
    M, V, K = 4, 777, 128
    x = _randn((M, K), 1.0, g)
    w = _randn((V, K), 0.02, g)
    logits = F.linear(x, w)
    np.savez(HERE / "lm_argmax_m4_v777_k128.npz", x=_bits(x), w=_bits(w), logits=_bits(logits),
             ids=torch.argmax(logits, -1).numpy().astype(np.int64),
             maxv=logits.max(-1).values.float().numpy().astype(np.float32))
    out.append(HERE / "lm_argmax_m4_v777_k128.npz")
    return out


if __name__ == "__main__":
    for p in make():
        print(p.name, p.stat().st_size)
