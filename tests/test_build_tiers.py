"""Register tiers of the kernel instances (starter_amd/build.py, csrc/sk_tiers.inc).

The build compiles every instance for the most waves per workgroup its
registers allow and refuses kernels that spill; `--retier` measures which
instances need fewer waves.  These CPU tests check the measurement loop on a
simulated compiler, the round trip of the generated table, and that the
planner in the built library enforces the committed table.
"""

from __future__ import annotations

import pytest

import starter_amd.build as B
from starter_amd import _lib
from starter_amd._lib import SK_OK, SK_OP_GEMM, SK_PATH_GEMV, SK_PATH_MFMA, SkConfig


def test_instance_names_parse():
    m = B._INSTANCE.fullmatch("_ZN2sk10mfmt_entryILi4ELi1ELi1024ELi2EEEvNS_4ArgsE")
    assert m and m.group(1) == "mfmt" and tuple(map(int, m.groups()[1:])) == (4, 1, 1024, 2)
    m = B._INSTANCE.fullmatch("_ZN2sk10gemv_entryILi8ELi8ELi10ELi7EEEvNS_4ArgsE")
    assert m and m.group(1) == "gemv" and tuple(map(int, m.groups()[1:])) == (8, 8, 10, 7)
    assert B._INSTANCE.fullmatch("_ZN2sk18decode_attn_kernelILi4ELi8ELb0ELb1EEEvNS_8AttnArgsE") is None
    m = B._INSTANCE.fullmatch("_ZN2sk18mfmt_grouped_entryILi2ELi1ELi256ELi3EEEvNS_4ArgsE")
    assert m and B._KINDS[m.group(1)] == 2 and tuple(map(int, m.groups()[1:])) == (2, 1, 256, 3)


def test_retier_moves_a_spilling_row_group_entry_with_its_plain_instance(tmp_path, monkeypatch):
    """The row-group entry shares its plain instance's tier: when only the
    grouped entry spills, the shared key moves one tier down."""
    monkeypatch.setattr(B, "TIERS_INC", tmp_path / "sk_tiers.inc")
    budget = dict(B._TIERS)

    def fake_compile(units, jobs, incremental=False, verbose=False):
        waves = B._read_tiers().get((2, 2, 1, 256, 3), 16)
        need = 150   # the grouped entry needs 150 registers: spills at 16 waves (128), fits at 12 (168)
        spills = [("_ZN2sk18mfmt_grouped_entryILi2ELi1ELi256ELi3EEEvNS_4ArgsE", need - budget[waves], budget[waves])]
        return [(None, spills if need > budget[waves] else [])]

    monkeypatch.setattr(B, "_compile", fake_compile)
    assert B.retier(jobs=1, fresh=True) == {(2, 2, 1, 256, 3): 12}


def test_tier_table_round_trip(tmp_path, monkeypatch):
    monkeypatch.setattr(B, "TIERS_INC", tmp_path / "sk_tiers.inc")
    table = {(0, 8, 8, 10, 0): 0, (1, 4, 1, 20, 2): 4, (2, 2, 1, 256, 0): 12}
    B._write_tiers(table)
    assert B._read_tiers() == table
    text = B.TIERS_INC.read_text()
    assert text.rstrip().endswith("};") and "{-1, 0, 0, 0, 0, 0}" in text


def _mangled(kind: str, a: int, b: int, c: int, e: int) -> str:
    return f"_ZN2sk10{kind}_entryILi{a}ELi{b}ELi{c}ELi{e}EEEvNS_4ArgsE"


def test_retier_moves_spilling_instances_down_one_tier(tmp_path, monkeypatch):
    """Simulated compiler: each instance has a register need; at a tier whose
    budget is smaller it reports a spill with the budget's register count.
    The loop must end with every instance at the largest tier that fits, and
    drop the one that fits nowhere."""
    monkeypatch.setattr(B, "TIERS_INC", tmp_path / "sk_tiers.inc")
    need = {("mfmt", 2, 1, 256, 0): 150,      # estimate tier 16 -> fits at 12
            ("mfma", 4, 1, 20, 2): 440,       # -> 4
            ("gemv", 8, 8, 10, 0): 900,       # spills even at 4 -> dropped
            ("gemv", 1, 2, 2, 0): 60}         # fits at 16, never listed
    kinds = {"gemv": 0, "mfma": 1, "mfmt": 2}
    budget = dict(B._TIERS)
    calls = []

    def fake_compile(units, jobs, incremental=False, verbose=False):
        table = B._read_tiers()
        spills = []
        for (k, a, b, c, e), regs in need.items():
            waves = table.get((kinds[k], a, b, c, e), 16)
            if waves and regs > budget[waves]:
                spills.append((_mangled(k, a, b, c, e), regs - budget[waves], budget[waves]))
        calls.append(len(spills))
        return [(None, spills)]

    monkeypatch.setattr(B, "_compile", fake_compile)
    out = B.retier(jobs=1, fresh=True)
    assert out == {(2, 2, 1, 256, 0): 12, (1, 4, 1, 20, 2): 4, (0, 8, 8, 10, 0): 0}
    assert calls[-1] == 0 and len(calls) <= len(B._TIERS) + 1
    assert B._read_tiers() == out


def test_committed_tiers_are_enforced_by_the_planner():
    """Every instance the committed table drops is refused, and an instance
    listed at w waves accepts w and refuses w + 1."""
    table = B._read_tiers()
    assert table, "csrc/sk_tiers.inc lists no instance"
    # GEMV, 8 activation rows, 8 weight rows per tile, K units up to 5: dropped (spills at 4 waves)
    assert table.get((0, 8, 8, 5, 0)) == 0
    assert _lib.check_config(SK_OP_GEMM, 8, 1536, 2560, SkConfig.make(SK_PATH_GEMV, 1, 5, 8)) != SK_OK
    # the register-fragment MFMA instance of 64 rows and 20 K units: 4 waves
    assert table.get((1, 4, 1, 20, 0)) in (None, 4)
    cfg4 = SkConfig.make(SK_PATH_MFMA, 4, 20, 16)
    cfg5 = SkConfig.make(SK_PATH_MFMA, 5, 20, 16)   # the same instance with one wave more than its tier
    assert _lib.check_config(SK_OP_GEMM, 64, 6144, 2560, cfg4) == SK_OK
    assert _lib.check_config(SK_OP_GEMM, 64, 6144, 2560, cfg5) != SK_OK


@pytest.mark.parametrize("waves", [4, 8])
def test_mfma_64_rows_10_units_limited_to_its_tier(waves):
    """mfma<4,1,10> spilled with 8 waves (280 registers against 256): it is
    compiled for 4, so 8 waves are refused and 4 accepted (with a K split that
    4 x 10 units cover)."""
    split = 2 if waves == 4 else 1
    st = _lib.check_config(SK_OP_GEMM, 64, 6144, 2560, SkConfig.make(SK_PATH_MFMA, waves, 10, 16, split))
    assert (st == SK_OK) == (waves == 4)


def _remarks(*kernels):
    """hipcc-style resource-usage remarks: (name, scratch bytes, VGPR spills)."""
    out = []
    for name, scratch, spill in kernels:
        tag = " [-Rpass-analysis=kernel-resource-usage]"
        out += [f"x.hip:1:1: remark: Function Name: {name}{tag}", f"x.hip:1:1: remark:     VGPRs: 128{tag}",
                f"x.hip:1:1: remark:     AGPRs: 0{tag}", f"x.hip:1:1: remark:     ScratchSize [bytes/lane]: {scratch}{tag}",
                f"x.hip:1:1: remark:     VGPRs Spill: {spill}{tag}"]
    return "\n".join(out)


def _fake_hipcc(text):
    import sys
    return [sys.executable, "-c", f"import sys; sys.stderr.write({text!r})"]


def test_remarks_report_spills_and_reject_private_arrays():
    """Spilling kernels are returned for the tier loop; a kernel that keeps a
    local array in scratch without spilling fails the compile step."""
    ok = _remarks(("_ZN2sk10mfmt_entryILi1ELi2ELi256ELi1EEEvNS_4ArgsE", 0, 0),
                  ("_ZN2sk11wide2_entryILi8ELi8ELi2EEEvNS_4ArgsE", 16, 3))
    assert B._run(_fake_hipcc(ok)) == [("_ZN2sk11wide2_entryILi8ELi8ELi2EEEvNS_4ArgsE", 3, 128)]
    stack = _remarks(("_ZN2sk11wide2_entryILi8ELi6ELi1EEEvNS_4ArgsE", 208, 0))
    with pytest.raises(RuntimeError, match="private memory"):
        B._run(_fake_hipcc(stack))
