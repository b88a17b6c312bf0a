"""MI355X-native decode-GEMM hot path (Qwen3-4B shapes) behind the reference's
operator interface: split-K skinny BF16 GEMMs, gate/up with a SwiGLU epilogue,
lm_head with a fused greedy argmax, add+RMSNorm and SwiGLU, as hand-written
gfx950 HIP kernels in libstarter_amd.so (C ABI: include/starter_amd.h)."""

from ._lib import SkConfig, SkError  # noqa: F401

__version__ = "0.1.0"
