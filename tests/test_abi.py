"""The C ABI on the CPU: the library loads, exports what the header declares,
and its host logic (planner, workspace sizes, argument validation) behaves.

No kernel runs here.  Calls with invalid arguments return their status code
before touching the HIP runtime; the one call that gets past validation
without a GPU must report SK_ERR_DEVICE (fail loudly, no fallback).
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from starter_amd import _lib
from starter_amd._lib import (SK_ERR_ALIAS, SK_ERR_ALIGN, SK_ERR_CONFIG, SK_ERR_DEVICE, SK_ERR_NULL, SK_ERR_SHAPE,
                              SK_ERR_WORKSPACE, SK_OK, SK_OP_ARGMAX, SK_OP_GATEUP, SK_OP_GEMM, SK_OP_LM_ARGMAX,
                              SK_OP_RMSNORM_GATEUP, SK_OP_RMSNORM_GEMM, SK_OP_RMSNORM_LM_ARGMAX, SK_PATH_GEMV,
                              SK_PATH_MFMA, SK_PATH_MFMA_LDS, SkConfig)

HEADER = Path(__file__).resolve().parents[1] / "include" / "starter_amd.h"
QWEN = {"qkv": (SK_OP_GEMM, 6144, 2560), "o": (SK_OP_GEMM, 2560, 4096), "gu": (SK_OP_GATEUP, 9728, 2560),
        "d": (SK_OP_GEMM, 2560, 9728), "lm": (SK_OP_GEMM, 151936, 2560), "lm_argmax": (SK_OP_LM_ARGMAX, 151936, 2560)}
FAKE = 0x10000   # an aligned address that is never dereferenced on the host


def _declared() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w[\w\s\*]*?\b(sk_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = _declared()
    assert set(names) == set(_lib.EXPORTS)
    for n in names:
        assert isinstance(getattr(lib, n), ctypes._CFuncPtr), n


def test_version_and_status_strings():
    lib = _lib.lib()
    assert lib.sk_version() >= 1
    msgs = {lib.sk_strerror(c).decode() for c in range(10)}
    assert len(msgs) == 10 and "ok" in msgs
    assert lib.sk_strerror(99).decode() == "unknown status"


@pytest.mark.parametrize("name", list(QWEN))
@pytest.mark.parametrize("M", [1, 2, 4, 8, 16, 32, 40, 64, 96, 128])
def test_default_config_is_valid_for_every_decode_shape(name, M):
    op, N, K = QWEN[name]
    cfg = _lib.default_config(op, M, N, K)
    assert _lib.check_config(op, M, N, K, cfg) == SK_OK, cfg
    # The waves cover K (per path: 32-column units, 512-column units, or one
    # 32*ku-column chunk per wave) and the workspace exists only where needed.
    if cfg.path == SK_PATH_MFMA:
        assert cfg.waves * cfg.ku * cfg.split >= K // 32
    elif cfg.path == SK_PATH_GEMV:
        assert cfg.waves * cfg.ku * cfg.split >= -(-K // 512)
    elif cfg.path == _lib.SK_PATH_WIDE:
        assert cfg.ku == 8 and cfg.waves in (4, 8)   # every wave walks the whole K slice
    else:
        assert cfg.path == SK_PATH_MFMA_LDS
        assert cfg.waves * cfg.split >= -(-K // (32 * cfg.ku))
    ws = _lib.workspace_bytes(op, M, N, K, cfg)
    # row groups: counters and partials per group of ceil(M / groups) rows
    # (the wide path's `groups` are wave groups, not row groups)
    g = max(cfg.groups, 1) if cfg.path != _lib.SK_PATH_WIDE else 1
    if op == SK_OP_LM_ARGMAX:
        assert ws == _tickets(g) + 8 * M
    elif cfg.split == 1:
        assert ws == 0
    else:
        # output columns per tile: 16 for MFMA gate/up (16 gate + 16 up rows), else `rows`
        out_rows = 16 if (op == SK_OP_GATEUP and cfg.path != SK_PATH_GEMV) else cfg.rows
        tiles = -(-N // out_rows)
        # partial rows: one group's rows x groups; a wide launch holds up to 128
        rows = g * -(-M // g) if g > 1 else (min(M, 128) if cfg.path == _lib.SK_PATH_WIDE else min(M, 64))
        assert ws == _tickets(g * tiles) + (2 if op == SK_OP_GATEUP else 1) * cfg.split * rows * N * 4


def test_tuned_table_drives_the_decode_shapes():
    """Measured winners: VALU GEMV for qkv at M = 1, LDS-transposed MFMA at M = 8
    (gate/up: ten 256-column waves, three tiles per workgroup)."""
    assert _lib.default_config(SK_OP_GEMM, 1, 6144, 2560).path == SK_PATH_GEMV
    assert _lib.default_config(SK_OP_GEMM, 8, 6144, 2560).path == SK_PATH_MFMA_LDS
    assert _lib.default_config(SK_OP_GATEUP, 8, 9728, 2560).as_dict() == \
        {"path": SK_PATH_MFMA_LDS, "waves": 10, "ku": 8, "rows": 16, "split": 1, "grid": 203, "groups": 0}
    assert _lib.default_config(SK_OP_LM_ARGMAX, 8, 151936, 2560).path == SK_PATH_MFMA_LDS
    # the lm_head logits GEMM shares the argmax entries; M = 5 takes the M = 8 entry
    assert _lib.default_config(SK_OP_GEMM, 5, 151936, 2560).as_dict() == \
        _lib.default_config(SK_OP_LM_ARGMAX, 8, 151936, 2560).as_dict()


def test_heuristic_for_untuned_shapes():
    assert _lib.default_config(SK_OP_GEMM, 2, 1536, 2560).path == SK_PATH_GEMV
    c = _lib.default_config(SK_OP_GEMM, 24, 1536, 2560)
    assert c.path == SK_PATH_MFMA_LDS and _lib.check_config(SK_OP_GEMM, 24, 1536, 2560, c) == SK_OK
    c = _lib.default_config(SK_OP_GEMM, 8, 777, 96)        # K not a multiple of the chunk
    assert _lib.check_config(SK_OP_GEMM, 8, 777, 96, c) == SK_OK


@pytest.mark.parametrize("name", list(QWEN) + ["rms_qkv", "rms_gu", "rms_lm"])
def test_default_config_suits_every_launch_of_the_call(name):
    """The configuration default_config returns for M rows, passed back
    explicitly, is accepted for every launch of the call at every M up to 256
    (above 128 rows the call runs as 128-row launches plus the remainder,
    which runs with as many row groups as hold a row)."""
    from starter_amd._lib import SK_OP_RMSNORM_GATEUP, SK_OP_RMSNORM_GEMM, SK_OP_RMSNORM_LM_ARGMAX

    op, N, K = {"rms_qkv": (SK_OP_RMSNORM_GEMM, 6144, 2560), "rms_gu": (SK_OP_RMSNORM_GATEUP, 9728, 2560),
                "rms_lm": (SK_OP_RMSNORM_LM_ARGMAX, 151936, 2560)}.get(name) or QWEN[name]
    for M in range(1, 257):
        cfg = _lib.default_config(op, M, N, K)
        assert _lib.check_config(op, M, N, K, cfg) == SK_OK, (name, M, cfg)
        assert _lib.workspace_bytes(op, M, N, K, cfg) == _lib.workspace_bytes(op, M, N, K, None), (name, M)


def test_default_config_prefers_no_global_split_at_decode_m():
    for name in ("qkv", "gu", "lm_argmax"):
        op, N, K = QWEN[name]
        for M in (1, 8):
            assert _lib.default_config(op, M, N, K).split == 1, (name, M)


@pytest.mark.parametrize("cfg,op,M,N,K,expect", [
    (SkConfig.make(SK_PATH_MFMA, 0, 20, 16), SK_OP_GEMM, 8, 6144, 2560, SK_ERR_CONFIG),     # no waves
    (SkConfig.make(SK_PATH_MFMA, 4, 20, 24), SK_OP_GEMM, 8, 6144, 2560, SK_ERR_CONFIG),     # rows
    (SkConfig.make(SK_PATH_MFMA, 4, 10, 16), SK_OP_GEMM, 8, 6144, 2560, SK_ERR_CONFIG),     # K not covered
    (SkConfig.make(SK_PATH_MFMA, 4, 21, 16), SK_OP_GEMM, 8, 6144, 2560, SK_ERR_CONFIG),     # no KU instance
    (SkConfig.make(SK_PATH_MFMA, 16, 20, 16), SK_OP_GEMM, 8, 6144, 2560, SK_ERR_CONFIG),    # registers
    (SkConfig.make(SK_PATH_MFMA, 2, 20, 16, 2), SK_OP_LM_ARGMAX, 8, 151936, 2560, SK_ERR_CONFIG),  # split argmax
    (SkConfig.make(SK_PATH_MFMA, 4, 20, 32), SK_OP_GATEUP, 8, 9728, 2560, SK_ERR_CONFIG),   # gate/up rows
    (SkConfig.make(SK_PATH_GEMV, 1, 5, 4), SK_OP_GEMM, 16, 6144, 2560, SK_ERR_CONFIG),      # GEMV M > 8
    (SkConfig.make(9, 4, 20, 16), SK_OP_GEMM, 8, 6144, 2560, SK_ERR_CONFIG),                # path
    (SkConfig.make(SK_PATH_MFMA, 4, 20, 16), SK_OP_GEMM, 8, 6144, 2568, SK_ERR_SHAPE),      # K % 32
    (SkConfig.make(SK_PATH_MFMA, 4, 20, 16, 1, 3), SK_OP_GEMM, 8, 6144, 2560, SK_OK),       # explicit grid
    (SkConfig.make(SK_PATH_MFMA, 4, 10, 16, 2, 3), SK_OP_GEMM, 8, 6144, 2560, SK_ERR_CONFIG),  # grid % split
    (SkConfig.make(SK_PATH_GEMV, 2, 3, 2), SK_OP_GATEUP, 4, 9728, 2560, SK_OK),
    (SkConfig.make(SK_PATH_MFMA, 16, 5, 16), SK_OP_GATEUP, 64, 9728, 2560, SK_ERR_CONFIG),  # LDS > 160 KiB
])
def test_check_config(cfg, op, M, N, K, expect):
    assert _lib.check_config(op, M, N, K, cfg) == expect


A0, W0, C0 = FAKE, FAKE + (1 << 26), FAKE + (1 << 27)   # disjoint fake operands


def _gemm(lib, A=A0, lda=2560, W=W0, ldw=2560, C=C0, ldc=6144, M=8, N=6144, K=2560, cfg=None, ws=None,
          wsb=0):
    return lib.sk_gemm_bf16(A, lda, W, ldw, C, ldc, M, N, K, _lib.cfg_ptr(cfg), ws, wsb, None)


def test_argument_validation_precedes_any_device_work():
    lib = _lib.lib()
    assert _gemm(lib, A=None) == SK_ERR_NULL
    assert _gemm(lib, C=None) == SK_ERR_NULL
    assert _gemm(lib, A=A0 + 2) == SK_ERR_ALIGN
    assert _gemm(lib, C=A0 + 4096) == SK_ERR_ALIAS   # output overlaps the activations
    assert _gemm(lib, lda=2564) == SK_ERR_ALIGN
    assert _gemm(lib, K=2568, lda=2568, ldw=2568) == SK_ERR_SHAPE
    assert _gemm(lib, ldc=100) == SK_ERR_SHAPE
    assert _gemm(lib, M=-1) == SK_ERR_SHAPE
    assert _gemm(lib, M=0) == SK_OK               # empty batch: nothing enqueued
    assert _gemm(lib, M=0, A=None, C=None) == SK_OK
    split = SkConfig.make(SK_PATH_MFMA, 4, 10, 16, 2)
    assert _gemm(lib, cfg=split) == SK_ERR_WORKSPACE
    assert _gemm(lib, cfg=split, ws=FAKE, wsb=16) == SK_ERR_WORKSPACE
    assert _gemm(lib, cfg=SkConfig.make(SK_PATH_MFMA, 4, 10, 16)) == SK_ERR_CONFIG
    assert lib.sk_lm_argmax_bf16(A0, 2560, W0, 2560, C0, C0 + 512, 8, 151936, 2560, None, None, 0, None) \
        == SK_ERR_WORKSPACE
    assert lib.sk_argmax_bf16(FAKE, 151936, 4, 151936, FAKE, FAKE, None, 0, None) == SK_ERR_WORKSPACE
    assert lib.sk_argmax_bf16(FAKE, 151935, 4, 151936, FAKE, FAKE, FAKE, 1 << 20, None) == SK_ERR_SHAPE
    X, Y, XO, OUT = FAKE, FAKE + (1 << 20), FAKE + (2 << 20), FAKE + (3 << 20)
    rms = lambda x, y, xo, out: lib.sk_add_rmsnorm_bf16(x, y, FAKE, 1e-6, xo, out, 4, 2560, 2560, None)
    assert rms(X, Y, X + 64, OUT) == 8            # SK_ERR_ALIAS: xout partially overlaps x
    assert rms(X, Y, XO, XO + 16) == 8            # out overlaps xout
    assert rms(X, Y, XO, Y) == 8                  # out overlaps y
    assert lib.sk_swiglu_bf16(FAKE, 100, FAKE, 50, 2, 60, None) == SK_ERR_SHAPE


def _tickets(n):
    return (4 * n + 255) // 256 * 256


def test_workspace_bytes():
    """[arrival counters padded to 256 B][partials | argmax candidates]."""
    assert _lib.workspace_bytes(SK_OP_ARGMAX, 4, 151936, 0) == _tickets(1) + 4 * 8
    assert _lib.workspace_bytes(SK_OP_GEMM, 0, 6144, 2560) == 0
    cfg = SkConfig.make(SK_PATH_MFMA, 4, 10, 16, 2)
    assert _lib.workspace_bytes(SK_OP_GEMM, 8, 6144, 2560, cfg) == _tickets(6144 // 16) + 2 * 8 * 6144 * 4
    assert _lib.workspace_bytes(SK_OP_GATEUP, 8, 9728, 2560, cfg) == _tickets(9728 // 16) + 2 * 2 * 8 * 9728 * 4
    lm = SkConfig.make(SK_PATH_MFMA, 4, 20, 16, 1, 500)
    assert _lib.workspace_bytes(SK_OP_LM_ARGMAX, 8, 151936, 2560, lm) == _tickets(1) + 8 * 8


def test_row_groups_planning():
    """Row groups run on the ring path only, with an explicit grid that is a
    multiple of 8 (sibling workgroups on one XCD), and every group holds a
    row; the workspace holds each group's counters and partials."""
    ring = lambda **kw: SkConfig.make(_LDS, **{"waves": 10, "ku": 8, "rows": 16, "grid": 128, **kw})
    ok = lambda cfg, op=SK_OP_GEMM, M=64, N=6144, K=2560: _lib.check_config(op, M, N, K, cfg)
    assert ok(ring(groups=2)) == SK_OK
    assert ok(ring(groups=2), SK_OP_GATEUP, N=9728) == SK_OK
    assert ok(ring(groups=2, grid=640), SK_OP_LM_ARGMAX, N=151936) == SK_OK
    assert ok(ring(groups=0)) == SK_ERR_CONFIG          # one group of 64 rows: over the ten-wave registers
    assert ok(ring(groups=2, grid=0)) == SK_ERR_CONFIG  # derived grid
    assert ok(ring(groups=2, grid=100)) == SK_ERR_CONFIG
    assert ok(ring(groups=-1)) == SK_ERR_CONFIG
    assert ok(ring(groups=2, ku=16, waves=5)) == SK_ERR_CONFIG   # whole-tile body
    assert ok(SkConfig.make(SK_PATH_MFMA, 4, 20, 16, 1, 128, 2)) == SK_ERR_CONFIG
    assert ok(ring(groups=3), M=2) == SK_ERR_CONFIG     # groups of one row: the third is empty
    assert ok(ring(groups=2), M=1) == SK_ERR_CONFIG
    assert ok(ring(groups=4), M=61) == SK_OK            # 16 + 16 + 16 + 13 rows
    # the residual hand-off producers and consumers take groups too; the fused
    # norm prologue (GEMV path) does not
    assert ok(ring(groups=2, split=4), SK_OP_RESID_GEMM, N=2560, K=9728) == SK_OK
    # consumers of 32 rows are compiled for 8 waves (the norm's registers), too
    # few for K = 2560 in 256-column chunks: 16-row groups
    assert ok(ring(groups=2), SK_OP_PRE_GEMM) == SK_ERR_CONFIG
    assert ok(ring(groups=4, grid=64), SK_OP_PRE_GEMM) == SK_OK
    assert ok(ring(groups=4, grid=64), SK_OP_PRE_GATEUP, N=9728) == SK_OK
    assert ok(ring(groups=4, grid=64), SK_OP_PRE_LM_ARGMAX, N=151936) == SK_OK
    assert ok(SkConfig.make(SK_PATH_GEMV, 1, 5, 2, 1, 8, 2), SK_OP_RMSNORM_GEMM, M=4) == SK_ERR_CONFIG
    split = ring(groups=2, waves=5, split=2)
    assert _lib.workspace_bytes(SK_OP_GEMM, 64, 6144, 2560, split) == _tickets(2 * 384) + 2 * 2 * 32 * 6144 * 4
    assert _lib.workspace_bytes(SK_OP_GATEUP, 61, 9728, 2560, ring(groups=4, waves=5, split=2)) == \
        _tickets(4 * 608) + 4 * 2 * 2 * 16 * 9728 * 4
    assert _lib.workspace_bytes(SK_OP_LM_ARGMAX, 64, 151936, 2560, ring(groups=2, grid=640)) == _tickets(2) + 64 * 8
    assert _lib.workspace_bytes(SK_OP_GEMM, 64, 6144, 2560, ring(groups=2)) == 0
    # the tuned verify-width entries use them (qkv; gate_up, down and lm_head
    # + argmax run on the two-operand wide path at 49-64 rows), and so do the
    # hand-off ops
    for name in ("qkv",):
        op, N, K = QWEN[name]
        assert _lib.default_config(op, 64, N, K).groups == 2, name
    for name in ("gu", "d", "lm_argmax", "lm"):
        op, N, K = QWEN[name]
        cfg = _lib.default_config(op, 64, N, K)
        assert cfg.path == _lib.SK_PATH_WIDE and cfg.groups == 4, name
    for op, N, K in ((SK_OP_PRE_GEMM, 6144, 2560), (SK_OP_PRE_GATEUP, 9728, 2560), (SK_OP_PRE_LM_ARGMAX, 151936, 2560),
                     (SK_OP_RESID_GEMM, 2560, 4096), (SK_OP_RESID_GEMM, 2560, 9728)):
        cfg = _lib.default_config(op, 64, N, K)
        assert cfg.groups >= 2 and _lib.check_config(op, 64, N, K, cfg) == SK_OK, (op, N, K)
    # below M = 64 a hand-off op keeps its projection's nearer entry
    assert _lib.default_config(SK_OP_RESID_GEMM, 32, 2560, 9728).as_dict() == \
        _lib.default_config(SK_OP_GEMM, 32, 2560, 9728).as_dict()


def test_wide_calls_plan_one_launch_of_row_groups():
    """Up to 128 rows run as one launch when the configuration splits them
    into row groups of at most 64 (the tuned entries do for qkv, and for
    o_proj up to 96 rows) or runs them on the wide path (every row in one
    workgroup: gate_up, down, lm_head and lm_head + argmax at 65-128 rows,
    o_proj at 97-128); more rows run as 128-row launches plus the remainder.
    An ungrouped configuration keeps 64-row launches."""
    wide = {"gu": (65, 100, 128), "d": (65, 100, 128), "lm_argmax": (65, 100, 128), "lm": (65, 100, 128),
            "o": (100, 128)}
    for name in ("qkv", "o", "gu", "d", "lm_argmax", "lm"):
        op, N, K = QWEN[name]
        for M in (65, 100, 128):
            cfg = _lib.default_config(op, M, N, K)
            if M in wide.get(name, ()):
                assert cfg.path == _lib.SK_PATH_WIDE, (name, M, cfg)
                if op == SK_OP_LM_ARGMAX:
                    assert _lib.workspace_bytes(op, M, N, K, cfg) == _tickets(1) + 8 * M   # one launch
            else:
                assert cfg.groups > 1 and -(-M // cfg.groups) <= 32, (name, M, cfg)
            assert _lib.check_config(op, M, N, K, cfg) == SK_OK, (name, M)
    # one wide launch of all 128 rows: the split-K partials of every row,
    # once; 129 rows take one more launch, which reuses that workspace
    op, N, K = QWEN["d"]
    cfg = _lib.default_config(op, 128, N, K)
    assert cfg.split > 1 and cfg.path == _lib.SK_PATH_WIDE
    one = _lib.workspace_bytes(op, 128, N, K)
    assert one == _tickets(-(-N // cfg.rows)) + cfg.split * 128 * N * 4
    assert _lib.workspace_bytes(op, 129, N, K) == one
    assert _lib.workspace_bytes(op, 256, N, K) == one
    # an explicit ungrouped configuration: 64-row launches
    plain = SkConfig.make(_LDS, 8, 8, 32, 5, 0)
    assert _lib.check_config(op, 128, N, K, plain) == SK_OK
    assert _lib.workspace_bytes(op, 128, N, K, plain) == _lib.workspace_bytes(op, 64, N, K, plain)
    # row groups hold at most 64 rows each, launches at most 128
    ring = SkConfig.make(_LDS, 10, 8, 16, 1, 64, 2)
    assert _lib.check_config(SK_OP_GEMM, 128, 6144, 2560, ring) == SK_OK   # two 64-row launches of 2 x 32
    # an explicit configuration applies to every launch: 129 rows leave a
    # one-row launch, which runs without groups (four would leave three
    # empty), 130 two groups of one row, 132 four
    four = SkConfig.make(_LDS, 10, 8, 16, 1, 64, 4)
    assert _lib.check_config(SK_OP_GEMM, 128, 6144, 2560, four) == SK_OK
    assert _lib.check_config(SK_OP_GEMM, 129, 6144, 2560, four) == SK_OK
    assert _lib.check_config(SK_OP_GEMM, 130, 6144, 2560, four) == SK_OK
    assert _lib.check_config(SK_OP_GEMM, 132, 6144, 2560, four) == SK_OK     # 128 + 4: four one-row groups
    # a single launch must still give every group a row
    assert _lib.check_config(SK_OP_GEMM, 3, 6144, 2560, four) == SK_ERR_CONFIG

    # the hand-off ops take up to 128 rows in one launch
    for op, N, K in ((SK_OP_PRE_GEMM, 6144, 2560), (SK_OP_RESID_GEMM, 2560, 9728), (SK_OP_RESID_GEMM, 2560, 4096)):
        cfg = _lib.default_config(op, 128, N, K)
        assert cfg.groups > 1 and _lib.check_config(op, 128, N, K, cfg) == SK_OK, (op, N, K)
        assert _lib.check_config(op, 129, N, K, cfg) == SK_ERR_SHAPE


def test_valid_call_without_gpu_fails_loudly():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present; the GPU tests exercise this path")
    assert _gemm(_lib.lib()) == SK_ERR_DEVICE
    assert _rms_gemm(_lib.lib(), M=1) == SK_ERR_DEVICE   # fused GEMV default: no workspace


def _gemm_noalloc(lib, A=A0, lda=2560, W=W0, ldw=2560, C=C0, ldc=6144, M=8, N=6144, K=2560, cfg=None):
    return lib.sk_gemm_bf16_noalloc(A, lda, W, ldw, C, ldc, M, N, K, _lib.cfg_ptr(cfg), None)


def test_noalloc_gemm_validates_like_the_workspace_entry_point():
    """sk_gemm_bf16_noalloc takes sk_gemm_bf16's arguments without the
    workspace: the same argument checks, and a plan whose split-K scratch
    exceeds the static array is refused with SK_ERR_SCRATCH before any device
    work (here: no GPU at all)."""
    lib = _lib.lib()
    assert _gemm_noalloc(lib, M=0) == SK_OK
    assert _gemm_noalloc(lib, A=0) == SK_ERR_NULL
    assert _gemm_noalloc(lib, K=2568) == SK_ERR_SHAPE
    assert _gemm_noalloc(lib, A=A0 + 2) == SK_ERR_ALIGN
    assert _gemm_noalloc(lib, C=A0 + 64) == SK_ERR_ALIAS
    big = SkConfig.make(SK_PATH_MFMA_LDS, waves=5, ku=8, rows=16, split=2)   # lm logits, split 2: 77.8 MB of partials
    assert _lib.workspace_bytes(SK_OP_GEMM, 64, 151936, 2560, big) > _lib.SK_NOALLOC_SCRATCH_BYTES
    assert _gemm_noalloc(lib, M=64, N=151936, ldc=151936, cfg=big) == _lib.SK_ERR_SCRATCH
    # every default plan of the Qwen3-4B projections fits the scratch
    for op, N, K in (QWEN[n] for n in ("qkv", "o", "d", "lm")):
        for M in (1, 2, 4, 8, 16, 32, 40, 64):
            assert _lib.workspace_bytes(op, M, N, K) <= _lib.SK_NOALLOC_SCRATCH_BYTES, (N, K, M)
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        assert _gemm_noalloc(lib) == SK_ERR_DEVICE   # a valid call without a GPU fails loudly


# ---------------------------------------------------------------------------
# Residual add + RMSNorm prologue ops
# ---------------------------------------------------------------------------

NORMED = {"qkv": (SK_OP_RMSNORM_GEMM, 6144, 2560), "gu": (SK_OP_RMSNORM_GATEUP, 9728, 2560),
          "lm": (SK_OP_RMSNORM_GEMM, 151936, 2560), "lm_argmax": (SK_OP_RMSNORM_LM_ARGMAX, 151936, 2560)}
BASE = {SK_OP_RMSNORM_GEMM: SK_OP_GEMM, SK_OP_RMSNORM_GATEUP: SK_OP_GATEUP, SK_OP_RMSNORM_LM_ARGMAX: SK_OP_LM_ARGMAX}
X0, Y0, XO0, NW0 = FAKE + (1 << 28), FAKE + (1 << 28) + (1 << 22), FAKE + (1 << 28) + (2 << 22), FAKE + (3 << 22)


def _rms_gemm(lib, x=X0, y=Y0, nw=NW0, xo=XO0, ldx=2560, W=W0, C=C0, M=8, N=6144, K=2560, cfg=None, ws=None, wsb=0):
    return lib.sk_rmsnorm_gemm_bf16(x, y, nw, 1e-6, xo, ldx, W, K, C, N, M, N, K, _lib.cfg_ptr(cfg), ws, wsb, None)


@pytest.mark.parametrize("name", list(NORMED))
@pytest.mark.parametrize("M", [1, 2, 4, 8, 16, 32, 40, 64])
def test_normed_default_config_valid_and_fused_at_decode_m(name, M):
    """The norm ops use their projection's tuned configuration (gate/up at
    M = 1 has its own entry: the fused GEMV beats the faster LDS-fed MFMA
    projection plus a separate norm launch); on the GEMV path with one K split
    the prologue runs inside the projection kernel, so the workspace is the
    projection's own.  Otherwise the workspace adds the normalised rows [M, K]
    bf16 after the projection's part."""
    op, N, K = NORMED[name]
    cfg = _lib.default_config(op, M, N, K)
    base = _lib.default_config(BASE[op], M, N, K)
    if not (M == 1 and name == "gu"):   # the table's one norm-specific entry
        assert cfg.as_dict() == base.as_dict()
    assert _lib.check_config(op, M, N, K, cfg) == SK_OK
    plain = _lib.workspace_bytes(BASE[op], M, N, K, cfg)
    normed = _lib.workspace_bytes(op, M, N, K, cfg)
    unfused = (plain + 255) // 256 * 256 + M * K * 2
    if cfg.path == SK_PATH_GEMV and cfg.split == 1:
        assert normed == plain            # fused: no buffer for the normalised rows
    else:
        assert normed == unfused          # MFMA paths and global splits never fuse
    if M == 1 and name in ("qkv", "gu"):
        assert cfg.path == SK_PATH_GEMV


def test_normed_workspace_layout_for_unfused_configs():
    split = SkConfig.make(SK_PATH_MFMA_LDS, 5, 8, 16, 2)
    base = _lib.workspace_bytes(SK_OP_GEMM, 8, 6144, 2560, split)
    assert base == _tickets(6144 // 16) + 2 * 8 * 6144 * 4
    assert _lib.workspace_bytes(SK_OP_RMSNORM_GEMM, 8, 6144, 2560, split) == (base + 255) // 256 * 256 + 8 * 2560 * 2
    lds = SkConfig.make(SK_PATH_MFMA_LDS, 10, 8, 16)
    assert _lib.workspace_bytes(SK_OP_RMSNORM_GEMM, 8, 6144, 2560, lds) == 8 * 2560 * 2
    gemv = SkConfig.make(SK_PATH_GEMV, 1, 5, 2)
    assert _lib.workspace_bytes(SK_OP_RMSNORM_GEMM, 4, 6144, 2560, gemv) == 0   # fused
    mfma = SkConfig.make(SK_PATH_MFMA, 8, 10, 16)
    assert _lib.workspace_bytes(SK_OP_RMSNORM_GEMM, 8, 6144, 2560, mfma) == 8 * 2560 * 2
    # rows beyond 64: the separate prologue normalises all rows at once
    mfma_split = SkConfig.make(SK_PATH_MFMA, 8, 5, 16, 2)
    base100 = _lib.workspace_bytes(SK_OP_GEMM, 100, 6144, 2560, mfma_split)
    assert base100 > 0
    assert _lib.workspace_bytes(SK_OP_RMSNORM_GEMM, 100, 6144, 2560, mfma_split) == \
        (base100 + 255) // 256 * 256 + 100 * 2560 * 2


def test_normed_argument_validation():
    lib = _lib.lib()
    assert _rms_gemm(lib, y=None) == SK_ERR_NULL
    assert _rms_gemm(lib, nw=None) == SK_ERR_NULL
    assert _rms_gemm(lib, xo=None) == SK_ERR_NULL
    assert _rms_gemm(lib, nw=NW0 + 2) == SK_ERR_ALIGN
    assert _rms_gemm(lib, y=Y0 + 8) == SK_ERR_ALIGN
    assert _rms_gemm(lib, ldx=2564) == SK_ERR_ALIGN
    assert _rms_gemm(lib, xo=X0) == SK_ERR_ALIAS          # xout is x
    assert _rms_gemm(lib, xo=Y0 + 1024) == SK_ERR_ALIAS   # xout overlaps y
    assert _rms_gemm(lib, C=Y0) == SK_ERR_ALIAS           # output overlaps y
    assert _rms_gemm(lib, C=XO0) == SK_ERR_ALIAS          # output overlaps xout
    assert _rms_gemm(lib, M=0, x=None, y=None, nw=None, xo=None, C=None) == SK_OK
    split = SkConfig.make(SK_PATH_MFMA_LDS, 5, 8, 16, 2)
    assert _rms_gemm(lib, cfg=split) == SK_ERR_WORKSPACE
    need = _lib.workspace_bytes(SK_OP_RMSNORM_GEMM, 8, 6144, 2560, split)
    assert _rms_gemm(lib, cfg=split, ws=FAKE, wsb=need - 1) == SK_ERR_WORKSPACE
    gu = lib.sk_rmsnorm_gateup_swiglu_bf16(X0, Y0, NW0, 1e-6, XO0, 2560, W0, None, 2560, C0, 9728, 8, 9728, 2560,
                                           None, None, 0, None)
    assert gu == SK_ERR_NULL                              # missing up half
    lm = lib.sk_rmsnorm_lm_argmax_bf16(X0, Y0, NW0, 1e-6, XO0, 2560, W0, 2560, C0, C0 + 512, 8, 151936, 2560,
                                       None, None, 0, None)
    assert lm == SK_ERR_WORKSPACE


# ---------------------------------------------------------------------------
# Residual hand-off ops (producer: residual + partial sums; consumers: norm
# finished from those sums)
# ---------------------------------------------------------------------------

from starter_amd._lib import (SK_OP_PRE_GATEUP, SK_OP_PRE_GEMM, SK_OP_PRE_LM_ARGMAX,  # noqa: E402
                              SK_OP_RESID_GEMM, SK_PATH_MFMA_LDS as _LDS)

HANDOFF = {  # decode-step call sites at Qwen3-4B shapes
    "o_resid": (SK_OP_RESID_GEMM, 2560, 4096, SK_OP_GEMM), "d_resid": (SK_OP_RESID_GEMM, 2560, 9728, SK_OP_GEMM),
    "qkv_pre": (SK_OP_PRE_GEMM, 6144, 2560, SK_OP_GEMM), "gu_pre": (SK_OP_PRE_GATEUP, 9728, 2560, SK_OP_GATEUP),
    "lm_pre": (SK_OP_PRE_LM_ARGMAX, 151936, 2560, SK_OP_LM_ARGMAX),
}


# hand-off ops with table entries of their own at these M (<= 16)
OWN_ENTRY = {"qkv_pre": (8, 16), "o_resid": (8, 16), "d_resid": (8,)}


@pytest.mark.parametrize("name", list(HANDOFF))
@pytest.mark.parametrize("M", [1, 2, 4, 8, 16])
def test_handoff_default_config_is_a_ring_config(name, M):
    """Hand-off ops run on the ring-streamed LDS-fed MFMA path with tiles of
    16 or 32 rows: their own tuned entry where the table has one at the
    nearest row count (the qkv consumer at M = 8 and 16, the producers at
    decode row counts), else the tuned projection configuration where the
    hand-off can take it (a ring configuration with such tiles), else a ring
    configuration; the workspace is the projection's own."""
    op, N, K, base = HANDOFF[name]
    kus = (8, 32, 40) if op == SK_OP_RESID_GEMM else (8,)
    cfg = _lib.default_config(op, M, N, K)
    assert cfg.path == _LDS and cfg.ku in kus and cfg.rows in (16, 32)
    assert _lib.check_config(op, M, N, K, cfg) == SK_OK
    b = _lib.default_config(base, M, N, K)
    if M in OWN_ENTRY.get(name, ()):
        assert cfg.rows == 16
    elif b.path == _LDS and b.ku in kus and b.rows in (16, 32):
        assert cfg.as_dict() == b.as_dict()
    assert _lib.workspace_bytes(op, M, N, K, cfg) == _lib.workspace_bytes(base, M, N, K, cfg)


def test_handoff_rejects_unsupported_configs():
    gemv = SkConfig.make(SK_PATH_GEMV, 2, 5, 2)
    tile512 = SkConfig.make(_LDS, 5, 16, 16)
    split_pre = SkConfig.make(_LDS, 5, 8, 16, 2)
    assert _lib.check_config(SK_OP_PRE_GEMM, 8, 6144, 2560, gemv) == SK_ERR_CONFIG
    assert _lib.check_config(SK_OP_PRE_GEMM, 8, 6144, 2560, tile512) == SK_ERR_CONFIG
    assert _lib.check_config(SK_OP_PRE_GEMM, 8, 6144, 2560, split_pre) == SK_ERR_CONFIG   # consumers: one K split
    assert _lib.check_config(SK_OP_RESID_GEMM, 8, 2560, 9728, SkConfig.make(_LDS, 13, 8, 16, 3)) == SK_OK
    assert _lib.check_config(SK_OP_RESID_GEMM, 8, 2560, 9728, SkConfig.make(_LDS, 4, 32, 32, 3)) == SK_OK


def test_handoff_on_the_two_operand_wide_path():
    """Above 64 rows the hand-off ops also run on the two-operand wide path
    (groups = 4): producers after split-K partials, with tiles of whole
    16-column groups (the finish writes one partial sum per group), consumers
    with one K split.  The other wide bodies take no hand-off."""
    def w2(rows, split=1, waves=8, groups=4):
        return SkConfig.make(_lib.SK_PATH_WIDE, waves, 8, rows, split, 0, groups)
    for M in (65, 100, 128):
        assert _lib.check_config(SK_OP_RESID_GEMM, M, 2560, 4096, w2(32, 3)) == SK_OK
        assert _lib.check_config(SK_OP_RESID_GEMM, M, 2560, 9728, w2(64, 2)) == SK_OK
        assert _lib.check_config(SK_OP_RESID_GEMM, M, 2560, 4096, w2(32, 1)) == SK_ERR_CONFIG   # no split-K
        assert _lib.check_config(SK_OP_RESID_GEMM, M, 2560, 4096, w2(40, 3)) == SK_ERR_CONFIG   # 40-row tiles
        assert _lib.check_config(SK_OP_RESID_GEMM, M, 2560, 4096, w2(48, 3)) == SK_ERR_CONFIG   # 48 in 4 slabs
        assert _lib.check_config(SK_OP_RESID_GEMM, M, 2560, 4096, w2(32, 3, groups=1)) == SK_ERR_CONFIG
        assert _lib.check_config(SK_OP_PRE_GEMM, M, 6144, 2560, w2(32)) == SK_OK
        assert _lib.check_config(SK_OP_PRE_GEMM, M, 6144, 2560, w2(32, 2)) == SK_ERR_CONFIG    # consumers: one split
        assert _lib.check_config(SK_OP_PRE_GATEUP, M, 9728, 2560, w2(48)) == SK_OK
        assert _lib.check_config(SK_OP_PRE_LM_ARGMAX, M, 151936, 2560, w2(128)) == SK_OK
        assert _lib.check_config(SK_OP_PRE_GEMM, M, 6144, 2560, w2(32, waves=4)) == SK_ERR_CONFIG  # not compiled
    # defaults at 65-128 rows: the producers take the projection's wide entry,
    # the gate/up and lm_head consumers their own wide entries
    for name in ("o_resid", "d_resid", "gu_pre", "lm_pre"):
        op, N, K, base = HANDOFF[name]
        cfg = _lib.default_config(op, 128, N, K)
        assert cfg.path == _lib.SK_PATH_WIDE and cfg.groups == 4, name
        assert _lib.workspace_bytes(op, 128, N, K, cfg) == _lib.workspace_bytes(base, 128, N, K, cfg)
    assert _lib.default_config(SK_OP_PRE_GEMM, 128, 6144, 2560).path == _LDS


R0, RO0, SQ0 = FAKE + (1 << 29), FAKE + (1 << 29) + (1 << 22), FAKE + (1 << 29) + (2 << 22)


def _resid(lib, A=A0, W=W0, r=R0, ro=RO0, ldr=2560, sq=SQ0, M=8, N=2560, K=4096, cfg=None, ws=None, wsb=0):
    return lib.sk_gemm_residual_bf16(A, K, W, K, r, ro, ldr, sq, M, N, K, _lib.cfg_ptr(cfg), ws, wsb, None)


def _pre(lib, x=X0, sq=SQ0, nw=NW0, W=W0, C=C0, M=8, N=6144, K=2560, cfg=None, ws=None, wsb=0):
    return lib.sk_rmsnorm_pre_gemm_bf16(x, K, sq, nw, 1e-6, W, K, C, N, M, N, K, _lib.cfg_ptr(cfg), ws, wsb, None)


def test_handoff_argument_validation_precedes_any_device_work():
    lib = _lib.lib()
    assert _resid(lib, r=None) == SK_ERR_NULL
    assert _resid(lib, sq=None) == SK_ERR_NULL
    assert _resid(lib, ro=A0 + 512) == SK_ERR_ALIAS     # residual out overlaps the projection's input
    assert _resid(lib, sq=RO0 + 64) == SK_ERR_ALIAS     # partial sums overlap the residual
    assert _resid(lib, ro=R0 + 2) == SK_ERR_ALIAS       # partially overlapping residuals
    assert _resid(lib, ldr=100) == SK_ERR_SHAPE
    assert _resid(lib, M=129) == SK_ERR_SHAPE
    assert _resid(lib, M=0, A=None, r=None, ro=None, sq=None) == SK_OK
    assert _resid(lib, K=9728, cfg=SkConfig.make(_LDS, 13, 8, 16, 3)) == SK_ERR_WORKSPACE
    assert _pre(lib, nw=None) == SK_ERR_NULL
    assert _pre(lib, nw=NW0 + 2) == SK_ERR_ALIGN
    assert _pre(lib, sq=SQ0 + 2) == SK_ERR_ALIGN
    assert _pre(lib, C=X0) == SK_ERR_ALIAS              # output overlaps the activations
    assert _pre(lib, C=SQ0) == SK_ERR_ALIAS             # output overlaps the partial sums
    lm = lib.sk_rmsnorm_pre_lm_argmax_bf16(X0, 2560, SQ0, NW0, 1e-6, W0, 2560, C0, C0 + 512, 8, 151936, 2560,
                                           None, None, 0, None)
    assert lm == SK_ERR_WORKSPACE


Q0, KC0, VC0, O0 = FAKE + (1 << 30), FAKE + (1 << 30) + (1 << 26), FAKE + (1 << 30) + (2 << 26), FAKE + (1 << 30) + (3 << 26)


def _attn_rope(lib, qkv=Q0, ld=6144, kc=KC0, vc=VC0, out=O0, B=8, R=1, cap=1408, ws=None, wsb=0):
    return lib.sk_decode_attention_rope_bf16(qkv, ld, FAKE, FAKE, FAKE, FAKE, 1408, 1e-6, kc, vc, FAKE, out,
                                             B, 32, 8, 128, R, cap, 1152, 0.088, 0, ws, wsb, None)


def test_fused_attention_argument_validation_precedes_any_device_work():
    """sk_decode_attention_rope_bf16 rejects bad arguments before it touches the
    device (fake, never dereferenced addresses); the workspace is the one
    sk_decode_attention_workspace_bytes() reports for the same plan."""
    lib = _lib.lib()
    need = lib.sk_decode_attention_workspace_bytes(8, 32, 8, 128, 1, 1408, 1152, 0)
    assert need > 0                                              # the default plan splits the keys at B = 8
    assert _attn_rope(lib) == SK_ERR_WORKSPACE
    assert _attn_rope(lib, ws=FAKE, wsb=need - 1) == SK_ERR_WORKSPACE
    assert _attn_rope(lib, qkv=None, ws=FAKE, wsb=need) == SK_ERR_NULL
    assert _attn_rope(lib, kc=None, ws=FAKE, wsb=need) == SK_ERR_NULL
    assert _attn_rope(lib, ld=6143, ws=FAKE, wsb=need) == SK_ERR_SHAPE      # row shorter than HQ + 2*HKV heads
    assert _attn_rope(lib, kc=KC0 + 2, ws=FAKE, wsb=need) == SK_ERR_ALIGN
    assert _attn_rope(lib, out=KC0 + 4096, ws=FAKE, wsb=need) == SK_ERR_ALIAS  # output inside the key cache
    assert _attn_rope(lib, out=Q0 + 64, ws=FAKE, wsb=need) == SK_ERR_ALIAS     # output inside the projection rows
    assert _attn_rope(lib, vc=KC0 + 128, ws=FAKE, wsb=need) == SK_ERR_ALIAS    # overlapping caches
    assert _attn_rope(lib, B=0, qkv=None, kc=None, vc=None, out=None) == SK_OK


def test_argmax_outputs_are_checked_before_launch():
    """Caller-supplied ids / maxv buffers of the argmax entry points must be
    what the kernel writes (int64 / float32, >= M contiguous elements on the
    activations' device), else the call raises before reaching the library."""
    import torch

    from starter_amd import kernels as K

    M = 4
    ids, maxv = K._argmax_outputs(None, None, M, "cpu")
    assert ids.dtype == torch.int64 and maxv.dtype == torch.float32 and ids.numel() == maxv.numel() == M
    good_i, good_v = torch.empty(M, dtype=torch.int64), torch.empty(M, dtype=torch.float32)
    assert K._argmax_outputs(good_i, good_v, M, "cpu")[0] is good_i
    bad = [
        (torch.empty(M, dtype=torch.int32), good_v),            # ids int32: 8-byte stores would overrun
        (good_i, torch.empty(M, dtype=torch.float16)),          # maxv not float32
        (torch.empty(M - 1, dtype=torch.int64), good_v),        # too short
        (good_i, torch.empty(M - 1, dtype=torch.float32)),
        (torch.empty(2 * M, dtype=torch.int64)[::2], good_v),   # not contiguous
    ]
    for i, v in bad:
        with pytest.raises(ValueError):
            K._argmax_outputs(i, v, M, "cpu")
    with pytest.raises(ValueError):
        K._argmax_outputs(good_i, good_v, M, "meta")             # not on the activations' device


def test_rope_and_attention_parameters_are_checked_before_launch():
    """Norm gains bf16 [D], rotary tables bf16 [rows, D], positions int32 with at
    least B entries and depths int32 [T]: anything else raises before launch
    (the kernels read w[0..D-1], pos[b] and depth[t] unconditionally)."""
    import torch

    from starter_amd import kernels as K

    D = 128
    w = torch.ones(D, dtype=torch.bfloat16)
    tab = torch.zeros(16, D, dtype=torch.bfloat16)
    for args in [(w.float(), w, tab, tab), (w, w[:64], tab, tab), (w, w, tab.float(), tab.float()),
                 (w, w, tab, tab[:, :64].contiguous()), (w, w, tab[:, :64], tab[:, :64])]:
        with pytest.raises(ValueError):
            K._rope_params(*args, D)
    for t, n, exact in [(torch.zeros(3, dtype=torch.int32), 4, False), (torch.zeros(4, dtype=torch.int64), 4, False),
                        (torch.zeros(5, dtype=torch.int32), 4, True), (torch.zeros(8, dtype=torch.int32)[::2], 4, True)]:
        with pytest.raises(ValueError):
            K._vec(t, "pos", torch.int32, n, exact=exact)
    with pytest.raises(ValueError, match="device"):
        K._vec(torch.zeros(4, dtype=torch.int32), "pos", torch.int32, 4, exact=False)   # right shape, host memory
