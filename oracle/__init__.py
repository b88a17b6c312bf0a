"""CPU oracle of the decode-GEMM hot path (numpy in, numpy out).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the cpu_baseline leg of bench.py, always as the checker, never as a product
path.  The restatement itself is plain C (``sk_oracle.c``, one function per
reference function, each citing the reference file:line it follows), built by
``oracle/build.py`` into ``oracle/_build/libsk_oracle.so`` with gcc + OpenMP.

Pinning (tests/test_oracle.py): every function is checked against torch's CPU
library routines (``F.linear`` with fp32 accumulation, ``F.silu``,
``torch.argmax``), an fp64 closed form, exact special cases (one-hot weights,
small-integer products, constructed ties and NaNs) and the seeded fixtures
under tests/golden/.  The reference stores no golden vectors of its own
(its tests draw random tensors at runtime and compare with torch on CUDA).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "libsk_oracle.so"

_lib = None
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64
_i32 = ctypes.c_int


def threads() -> int:
    """Worker threads for the OpenMP loops (the box's CPU share is 16)."""
    return int(os.environ.get("ORACLE_THREADS", min(16, os.cpu_count() or 1)))


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            from .build import build

            build()
        h = ctypes.CDLL(str(LIB))
        h.oracle_gemm_bf16.argtypes = [_u16p, _i64, _u16p, _i64, _u16p, _i64, _i32, _i32, _i32, _i32]
        h.oracle_gemm_f32.argtypes = [_u16p, _i64, _u16p, _i64, _f32p, _i32, _i32, _i32, _i32]
        h.oracle_gateup_swiglu_bf16.argtypes = [_u16p, _i64, _u16p, _u16p, _i64, _u16p, _i64, _i32, _i32, _i32, _i32]
        h.oracle_swiglu_bf16.argtypes = [_u16p, _i64, _u16p, _i64, _i32, _i32]
        h.oracle_add_rmsnorm_bf16.argtypes = [_u16p, _u16p, _u16p, ctypes.c_float, _u16p, _u16p, _i32, _i32, _i64]
        h.oracle_argmax_bf16.argtypes = [_u16p, _i64, _i32, _i32, _i64p, _f32p]
        h.oracle_lm_argmax_bf16.argtypes = [_u16p, _i64, _u16p, _i64, _i32, _i32, _i32, _i64p, _f32p, _i32]
        h.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        h.oracle_f32_to_bf16.restype = ctypes.c_uint16
        h.oracle_swiglu_scalar.argtypes = [ctypes.c_uint16, ctypes.c_uint16]
        h.oracle_swiglu_scalar.restype = ctypes.c_uint16
        _i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
        h.oracle_qk_norm_rope_cache_bf16.argtypes = [_u16p, _i64, _u16p, _u16p, _u16p, _u16p, _i32p, _u16p, _u16p,
                                                     _u16p, _i32, _i32, _i32, _i32, _i32, _i32, ctypes.c_float,
                                                     ctypes.c_void_p]
        h.oracle_topk_bf16.argtypes = [_u16p, _i64, _i32, _i32, _i32, _f32p, _i32p]
        h.oracle_decode_attention.argtypes = [_u16p, _u16p, _u16p, _i32p, ctypes.c_void_p, _f32p, _f32p, _i32, _i32,
                                              _i32, _i32, _i32, _i32, ctypes.c_float, _i32]
        _lib = h
    return _lib


def _u16(x) -> np.ndarray:
    x = np.ascontiguousarray(x)
    if x.dtype != np.uint16:
        raise TypeError(f"expected raw bf16 bits as uint16, got {x.dtype}")
    return x


# --- bf16 <-> fp32 bit helpers (numpy) -------------------------------------

def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    """Round to nearest even (canonical quiet NaN), like torch's ``.to(bfloat16)``."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


# --- restated reference functions ------------------------------------------

def gemm(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """``bf16(a @ w.T)`` with fp32 accumulation (engine/kernels/gemm.py:59-112, 527)."""
    a, w = _u16(a), _u16(w)
    M, K = a.shape
    N = w.shape[0]
    c = np.empty((M, N), dtype=np.uint16)
    lib().oracle_gemm_bf16(a, K, w, K, c, N, M, N, K, threads())
    return c


def gemm_f32(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """The fp32 sums ``a @ w.T`` before the bf16 rounding."""
    a, w = _u16(a), _u16(w)
    M, K = a.shape
    N = w.shape[0]
    c = np.empty((M, N), dtype=np.float32)
    lib().oracle_gemm_f32(a, K, w, K, c, M, N, K, threads())
    return c


def gateup_swiglu(a: np.ndarray, wg: np.ndarray, wu: np.ndarray) -> np.ndarray:
    """``swiglu(a @ wg.T, a @ wu.T)`` (engine/kernels/gemm.py:115-181)."""
    a, wg, wu = _u16(a), _u16(wg), _u16(wu)
    M, K = a.shape
    I = wg.shape[0]
    out = np.empty((M, I), dtype=np.uint16)
    lib().oracle_gateup_swiglu_bf16(a, K, wg, wu, K, out, I, M, I, K, threads())
    return out


def swiglu(gu: np.ndarray) -> np.ndarray:
    """``silu(g) * u`` over ``gu = [g | u]`` (engine/kernels/swiglu.py:14-33)."""
    gu = _u16(gu)
    M, two_i = gu.shape
    I = two_i // 2
    out = np.empty((M, I), dtype=np.uint16)
    lib().oracle_swiglu_bf16(gu, two_i, out, I, M, I)
    return out


def add_rmsnorm(x: np.ndarray, y: np.ndarray, w: np.ndarray, eps: float):
    """``(xout, out)`` of add_rms_norm (engine/kernels/add_rmsnorm.py:15-43)."""
    x, y, w = _u16(x), _u16(y), _u16(w)
    M, K = x.shape
    xout = np.empty_like(x)
    out = np.empty_like(x)
    lib().oracle_add_rmsnorm_bf16(x, y, w, eps, xout, out, M, K, K)
    return xout, out


def argmax(logits: np.ndarray):
    """``(ids, maxv)``: first index of the row max over bf16 logits (torch.argmax rule)."""
    L = _u16(logits)
    M, V = L.shape
    ids = np.empty(M, dtype=np.int64)
    maxv = np.empty(M, dtype=np.float32)
    lib().oracle_argmax_bf16(L, V, M, V, ids, maxv)
    return ids, maxv


def lm_argmax(a: np.ndarray, w: np.ndarray):
    """``argmax(bf16(a @ w.T))`` per row without storing the logits."""
    a, w = _u16(a), _u16(w)
    M, K = a.shape
    V = w.shape[0]
    ids = np.empty(M, dtype=np.int64)
    maxv = np.empty(M, dtype=np.float32)
    lib().oracle_lm_argmax_bf16(a, K, w, K, M, V, K, ids, maxv, threads())
    return ids, maxv


def swiglu_scalar(g: int, u: int) -> int:
    return int(lib().oracle_swiglu_scalar(g, u))


def f32_to_bf16_c(f: float) -> int:
    return int(lib().oracle_f32_to_bf16(f))


def qk_norm_rope_cache(qkv: np.ndarray, qw: np.ndarray, kw: np.ndarray, cos: np.ndarray, sin: np.ndarray,
                       pos: np.ndarray, q_out: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, T: int,
                       eps: float, depth: np.ndarray | None = None) -> None:
    """In place: q_out [B, HQ, T, D], k/v_cache [B, HKV, cap, D] at slots pos[b] + t
    (engine/kernels/rope.py:140-188).  qkv [B*T, (HQ + 2*HKV)*D] bits.  The
    rotary angle of row (b, t) is that of position pos[b] + t, or with
    ``depth`` [T] int32 (a draft tree) pos[b] + depth[t] (rope.py:108-111)."""
    qkv = _u16(qkv)
    B, HQ, _, D = q_out.shape
    HKV, cap = k_cache.shape[1], k_cache.shape[2]
    for a in (q_out, k_cache, v_cache):
        if a.dtype != np.uint16 or not a.flags["C_CONTIGUOUS"]:
            raise TypeError("outputs must be contiguous uint16 arrays")
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    if pos.min() < 0 or pos.max() + T > cap:
        raise ValueError("slots outside the cache")
    dp = None
    if depth is not None:
        depth = np.ascontiguousarray(depth, dtype=np.int32)
        if depth.shape != (T,):
            raise ValueError("depth must hold one position offset per row t")
        angles = pos[:, None] + depth[None, :]
        dp = depth.ctypes.data
    else:
        angles = pos[:, None] + np.arange(T, dtype=np.int32)[None, :]
    if angles.min() < 0 or angles.max() >= cos.shape[0]:
        raise ValueError("rotary positions outside the table")
    lib().oracle_qk_norm_rope_cache_bf16(qkv, qkv.shape[1], _u16(qw), _u16(kw), _u16(cos), _u16(sin), pos, q_out,
                                         k_cache, v_cache, B, T, HQ, HKV, D, cap, eps, dp)


def decode_attention(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, pos: np.ndarray,
                     scale: float, with_abs: bool = False, tree: np.ndarray | None = None):
    """Exact attention of each query row (engine/kernels/attention.py:221-242):
    q [B, HQ, R, D] bits, caches [B, HKV, cap, D] bits, pos [B] (row t sees keys
    0 .. pos[b] + t, or with ``tree`` [R] int64 the keys < pos[b] and draft key
    pos[b] + j when bit j of tree[t] is set).  Returns fp32 [B, R, HQ, D]; with
    ``with_abs`` also the softmax-weighted mean of |v| per output element
    (error scale of bf16 probabilities)."""
    q, k_cache, v_cache = _u16(q), _u16(k_cache), _u16(v_cache)
    B, HQ, R, D = q.shape
    HKV, cap = k_cache.shape[1], k_cache.shape[2]
    out = np.empty((B, R, HQ, D), dtype=np.float32)
    wabs = np.empty_like(out)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    tr = None if tree is None else np.ascontiguousarray(tree, dtype=np.int64)
    lib().oracle_decode_attention(q, k_cache, v_cache, pos, None if tr is None else tr.ctypes.data, out, wabs, B, HQ,
                                  HKV, D, R, cap, scale, threads())
    return (out, wabs) if with_abs else out


def topk(logits: np.ndarray, k: int):
    """fast_topk's algorithm (engine/kernels/topk.py:17-37): (vals [N, k] fp32, idxs [N, k] int32)."""
    logits = _u16(logits)
    N, V = logits.shape
    vals = np.empty((N, k), dtype=np.float32)
    idxs = np.empty((N, k), dtype=np.int32)
    lib().oracle_topk_bf16(logits, logits.shape[1], N, V, k, vals, idxs)
    return vals, idxs
