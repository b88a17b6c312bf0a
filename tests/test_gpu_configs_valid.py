"""Every explicit configuration the GPU tests use passes the host-side
planner (shape coverage, registers, LDS, compiled instance) on the CPU, so a
GPU run never spends time on a config the library would reject."""

from __future__ import annotations

import pytest

from starter_amd import _lib
from starter_amd._lib import SK_OK, SK_OP_GATEUP, SK_OP_GEMM, SK_OP_LM_ARGMAX

gp = pytest.importorskip("tests.test_gpu_parity")


@pytest.mark.parametrize("cfg", gp.GEMM_CONFIGS, ids=str)
@pytest.mark.parametrize("M", [1, 3, 8])
def test_gemm_test_configs_valid(cfg, M):
    assert _lib.check_config(SK_OP_GEMM, M, 1536, 2560, cfg) == SK_OK


@pytest.mark.parametrize("cfg", gp.GATEUP_CONFIGS, ids=str)
@pytest.mark.parametrize("M", [1, 4])
def test_gateup_test_configs_valid(cfg, M):
    assert _lib.check_config(SK_OP_GATEUP, M, 1024, 2560, cfg) == SK_OK


@pytest.mark.parametrize("name", list(gp.LM_CONFIGS))
@pytest.mark.parametrize("M", [1, 8, 32, 64])
def test_lm_test_configs_valid(name, M):
    cfg = gp.LM_CONFIGS[name]
    if cfg is None or (name == "gemv" and M > 8) or (name == "mfma_lds" and M > 32):
        return
    assert _lib.check_config(SK_OP_LM_ARGMAX, M, 151936, 2560, cfg) == SK_OK


@pytest.mark.parametrize("case", list(gp.MFMT_CASES))
@pytest.mark.parametrize("M", [1, 8, 16, 40, 64])
def test_mfma_lds_shape_configs_valid(case, M):
    (N, Kd), ku, rows, split = gp.MFMT_CASES[case]
    assert _lib.check_config(SK_OP_GEMM, M, N, Kd, gp.mfmt_config(Kd, ku, rows, split, M)) == SK_OK


@pytest.mark.parametrize("M", [1, 8, 40])
def test_mfma_lds_gateup_configs_valid(M):
    assert _lib.check_config(SK_OP_GATEUP, M, 9728, 2560, gp.mfmt_config(2560, 16, 16, 1, M)) == SK_OK


gn = pytest.importorskip("tests.test_gpu_norm")


@pytest.mark.parametrize("name", list(gn.NORM_CONFIGS))
@pytest.mark.parametrize("M", [1, 3, 8, 16])
def test_norm_test_configs_valid(name, M):
    """The norm-prologue test configs: fused ones (GEMV, one split) keep the
    projection's workspace, unfused ones (MFMA paths, global splits) add the
    normalised rows."""
    from starter_amd._lib import SK_OP_RMSNORM_GEMM, SK_PATH_GEMV, SK_PATH_MFMA

    cfg = gn.NORM_CONFIGS[name]
    if cfg.path == SK_PATH_GEMV and M > 8:
        return
    assert _lib.check_config(SK_OP_RMSNORM_GEMM, M, 6144, 2560, cfg) == SK_OK
    plain = _lib.workspace_bytes(SK_OP_GEMM, M, 6144, 2560, cfg)
    normed = _lib.workspace_bytes(SK_OP_RMSNORM_GEMM, M, 6144, 2560, cfg)
    if cfg.split > 1 or cfg.path != SK_PATH_GEMV:
        assert normed == (plain + 255) // 256 * 256 + M * 2560 * 2
    else:
        assert normed == plain, f"{name} should run the prologue fused"
