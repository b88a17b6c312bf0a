"""ctypes binding of libstarter_amd.so (the C ABI in include/starter_amd.h).

Tensors cross the boundary as raw device pointers, element strides and the
HIP stream of ``torch.cuda.current_stream()``; PyTorch is only the allocator
and stream owner.  A missing or unloadable library raises immediately: there
is no fallback path.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("STARTER_AMD_LIB", Path(__file__).resolve().parent / "lib" / "libstarter_amd.so"))

SK_OK = 0
SK_ERR_NULL = 1
SK_ERR_SHAPE = 2
SK_ERR_ALIGN = 3
SK_ERR_WORKSPACE = 4
SK_ERR_CONFIG = 5
SK_ERR_LAUNCH = 6
SK_ERR_DEVICE = 7
SK_ERR_ALIAS = 8
SK_ERR_SCRATCH = 9

SK_NOALLOC_SCRATCH_BYTES = 4 << 20

SK_OP_GEMM = 0
SK_OP_GATEUP = 1
SK_OP_LM_ARGMAX = 2
SK_OP_ARGMAX = 3
SK_OP_RMSNORM_GEMM = 4
SK_OP_RMSNORM_GATEUP = 5
SK_OP_RMSNORM_LM_ARGMAX = 6
SK_OP_RESID_GEMM = 7
SK_OP_PRE_GEMM = 8
SK_OP_PRE_GATEUP = 9
SK_OP_PRE_LM_ARGMAX = 10

SK_PATH_AUTO = 0
SK_PATH_MFMA = 1
SK_PATH_GEMV = 2
SK_PATH_MFMA_LDS = 3
SK_PATH_WIDE = 4

# Every symbol include/starter_amd.h declares (checked by the CPU tests).
EXPORTS = (
    "sk_version", "sk_strerror", "sk_default_config", "sk_check_config", "sk_workspace_bytes",
    "sk_gemm_bf16", "sk_gemm_bf16_noalloc", "sk_gateup_swiglu_bf16", "sk_lm_argmax_bf16", "sk_argmax_bf16",
    "sk_add_rmsnorm_bf16", "sk_swiglu_bf16",
    "sk_rmsnorm_gemm_bf16", "sk_rmsnorm_gateup_swiglu_bf16", "sk_rmsnorm_lm_argmax_bf16",
    "sk_gemm_residual_bf16", "sk_rmsnorm_pre_gemm_bf16", "sk_rmsnorm_pre_gateup_swiglu_bf16",
    "sk_rmsnorm_pre_lm_argmax_bf16",
    "sk_qk_norm_rope_cache_bf16", "sk_decode_attention_workspace_bytes", "sk_decode_attention_bf16",
    "sk_decode_attention_rope_bf16", "sk_decode_attention_rope_tree_bf16",
    "sk_topk_bf16",
)


class SkConfig(ctypes.Structure):
    """Mirror of ``sk_config``: path, waves, ku, rows, split, grid, groups."""

    _fields_ = [
        ("path", ctypes.c_int32),
        ("waves", ctypes.c_int32),
        ("ku", ctypes.c_int32),
        ("rows", ctypes.c_int32),
        ("split", ctypes.c_int32),
        ("grid", ctypes.c_int32),
        ("groups", ctypes.c_int32),
    ]

    def as_dict(self) -> dict:
        return {name: int(getattr(self, name)) for name, _ in self._fields_}

    @classmethod
    def make(cls, path: int = SK_PATH_MFMA, waves: int = 4, ku: int = 20, rows: int = 16, split: int = 1,
             grid: int = 0, groups: int = 0) -> "SkConfig":
        return cls(path, waves, ku, rows, split, grid, groups)

    def __repr__(self) -> str:
        return f"SkConfig({self.as_dict()})"


class SkError(RuntimeError):
    """A C-ABI call returned a non-zero sk_status."""

    def __init__(self, status: int, what: str):
        self.status = status
        super().__init__(f"{what}: {strerror(status)} (sk_status {status})")


_lib = None

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_sz = ctypes.c_size_t
_cfgp = ctypes.POINTER(SkConfig)

_SIGNATURES = {
    "sk_version": (_i32, []),
    "sk_strerror": (ctypes.c_char_p, [_i32]),
    "sk_default_config": (_i32, [_i32, _i32, _i32, _i32, _i32, _cfgp]),
    "sk_check_config": (_i32, [_i32, _i32, _i32, _i32, _cfgp]),
    "sk_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _cfgp]),
    "sk_gemm_bf16": (_i32, [_p, _i64, _p, _i64, _p, _i64, _i32, _i32, _i32, _cfgp, _p, _sz, _p]),
    "sk_gemm_bf16_noalloc": (_i32, [_p, _i64, _p, _i64, _p, _i64, _i32, _i32, _i32, _cfgp, _p]),
    "sk_gateup_swiglu_bf16": (_i32, [_p, _i64, _p, _p, _i64, _p, _i64, _i32, _i32, _i32, _cfgp, _p, _sz, _p]),
    "sk_lm_argmax_bf16": (_i32, [_p, _i64, _p, _i64, _p, _p, _i32, _i32, _i32, _cfgp, _p, _sz, _p]),
    "sk_argmax_bf16": (_i32, [_p, _i64, _i32, _i32, _p, _p, _p, _sz, _p]),
    "sk_add_rmsnorm_bf16": (_i32, [_p, _p, _p, ctypes.c_float, _p, _p, _i32, _i32, _i64, _p]),
    "sk_swiglu_bf16": (_i32, [_p, _i64, _p, _i64, _i32, _i32, _p]),
    # x, y, w_norm, eps, xout, ldx, then the projection's own arguments
    "sk_rmsnorm_gemm_bf16": (_i32, [_p, _p, _p, ctypes.c_float, _p, _i64,
                                    _p, _i64, _p, _i64, _i32, _i32, _i32, _cfgp, _p, _sz, _p]),
    "sk_rmsnorm_gateup_swiglu_bf16": (_i32, [_p, _p, _p, ctypes.c_float, _p, _i64,
                                             _p, _p, _i64, _p, _i64, _i32, _i32, _i32, _cfgp, _p, _sz, _p]),
    "sk_rmsnorm_lm_argmax_bf16": (_i32, [_p, _p, _p, ctypes.c_float, _p, _i64,
                                         _p, _i64, _p, _p, _i32, _i32, _i32, _cfgp, _p, _sz, _p]),
    "sk_gemm_residual_bf16": (_i32, [_p, _i64, _p, _i64, _p, _p, _i64, _p, _i32, _i32, _i32, _cfgp, _p, _sz, _p]),
    "sk_rmsnorm_pre_gemm_bf16": (_i32, [_p, _i64, _p, _p, ctypes.c_float, _p, _i64, _p, _i64, _i32, _i32, _i32,
                                        _cfgp, _p, _sz, _p]),
    "sk_rmsnorm_pre_gateup_swiglu_bf16": (_i32, [_p, _i64, _p, _p, ctypes.c_float, _p, _p, _i64, _p, _i64, _i32,
                                                 _i32, _i32, _cfgp, _p, _sz, _p]),
    "sk_rmsnorm_pre_lm_argmax_bf16": (_i32, [_p, _i64, _p, _p, ctypes.c_float, _p, _i64, _p, _p, _i32, _i32, _i32,
                                             _cfgp, _p, _sz, _p]),
    "sk_qk_norm_rope_cache_bf16": (_i32, [_p, _i64, _p, _p, _p, _p, _i32, _p, _p, _p, _p, _p,
                                          _i32, _i32, _i32, _i32, _i32, _i32, ctypes.c_float, _p]),
    "sk_decode_attention_workspace_bytes": (_sz, [_i32] * 8),
    "sk_topk_bf16": (_i32, [_p, _i64, _i32, _i32, _i32, _p, _p, _p]),
    "sk_decode_attention_bf16": (_i32, [_p, _p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                        ctypes.c_float, _i32, _p, _sz, _p]),
    "sk_decode_attention_rope_bf16": (_i32, [_p, _i64, _p, _p, _p, _p, _i32, ctypes.c_float, _p, _p, _p, _p,
                                             _i32, _i32, _i32, _i32, _i32, _i32, _i32, ctypes.c_float, _i32,
                                             _p, _sz, _p]),
    "sk_decode_attention_rope_tree_bf16": (_i32, [_p, _i64, _p, _p, _p, _p, _i32, ctypes.c_float, _p, _p, _p, _p,
                                                  _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, ctypes.c_float,
                                                  _i32, _p, _sz, _p]),
}


def lib() -> ctypes.CDLL:
    """Load the library once.  torch is imported first so that the HIP runtime
    already in the process (PyTorch-ROCm's) is the one the library binds to."""
    global _lib
    if _lib is None:
        import torch  # noqa: F401  (binds libamdhip64 before the library loads)

        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m starter_amd.build` "
                               "(or __graft_entry__.build()); there is no non-HIP fallback")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def strerror(status: int) -> str:
    try:
        return lib().sk_strerror(status).decode()
    except Exception:  # pragma: no cover - only when the library itself is unavailable
        return f"status {status}"


def check(status: int, what: str) -> None:
    if status != SK_OK:
        raise SkError(status, what)


def cfg_ptr(cfg: SkConfig | None):
    return ctypes.byref(cfg) if cfg is not None else None


def default_config(op: int, M: int, N: int, K: int, num_cu: int = 0) -> SkConfig:
    c = SkConfig()
    check(lib().sk_default_config(op, M, N, K, num_cu, ctypes.byref(c)), "sk_default_config")
    return c


def check_config(op: int, M: int, N: int, K: int, cfg: SkConfig) -> int:
    return lib().sk_check_config(op, M, N, K, ctypes.byref(cfg))


def workspace_bytes(op: int, M: int, N: int, K: int, cfg: SkConfig | None = None) -> int:
    return int(lib().sk_workspace_bytes(op, M, N, K, cfg_ptr(cfg)))
