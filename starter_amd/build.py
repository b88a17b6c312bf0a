"""Build libstarter_amd.so (gfx950) in-tree with hipcc.

The library is the C ABI declared in ``include/starter_amd.h``.  Every
translation unit is compiled to an object under ``starter_amd/_build`` in
parallel (one per epilogue for the kernel instances), then linked into
``starter_amd/lib/libstarter_amd.so``.  No CMake, no torch extension: the
library links only against the HIP runtime, which it shares with
PyTorch-ROCm when both are loaded in one process.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "lib" / "libstarter_amd.so"
TIERS_INC = CSRC / "sk_tiers.inc"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 anywhere in the device code.
COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]

N_EPI = 5       # EPI_STORE, EPI_SWIGLU, EPI_ARGMAX, EPI_PART, EPI_PART_GU
NORM_EPIS = (5, 6, 7)   # the first three with the norm prologue (GEMV path only)
HANDOFF_EPIS = (8, 9, 10, 11, 12)   # residual hand-off consumers and producers (LDS-fed ring path)
WIDE_HANDOFF_EPIS = (8, 9, 10, 12)   # the same on the two-operand wide path (no bf16-store producer)


def _units() -> list[tuple[Path, list[str], Path]]:
    units = [(CSRC / "sk_abi.hip", [], BUILD / "sk_abi.o"), (CSRC / "sk_attn.hip", [], BUILD / "sk_attn.o"),
             (CSRC / "sk_topk.hip", [], BUILD / "sk_topk.o")]
    for epi in range(N_EPI):
        units.append((CSRC / "sk_inst_mfma.hip", [f"-DSK_EPI={epi}"], BUILD / f"sk_inst_mfma_{epi}.o"))
        units.append((CSRC / "sk_inst_gemv.hip", [f"-DSK_EPI={epi}"], BUILD / f"sk_inst_gemv_{epi}.o"))
        units.append((CSRC / "sk_inst_mfmt.hip", [f"-DSK_EPI={epi}"], BUILD / f"sk_inst_mfmt_{epi}.o"))
        units.append((CSRC / "sk_inst_wide.hip", [f"-DSK_EPI={epi}"], BUILD / f"sk_inst_wide_{epi}.o"))
    for epi in NORM_EPIS:
        units.append((CSRC / "sk_inst_gemv.hip", [f"-DSK_EPI={epi}"], BUILD / f"sk_inst_gemv_{epi}.o"))
    for epi in HANDOFF_EPIS:
        units.append((CSRC / "sk_inst_mfmt.hip", [f"-DSK_EPI={epi}"], BUILD / f"sk_inst_mfmt_{epi}.o"))
    for epi in WIDE_HANDOFF_EPIS:
        units.append((CSRC / "sk_inst_wide.hip", [f"-DSK_EPI={epi}"], BUILD / f"sk_inst_wide_{epi}.o"))
    return units


def _run(cmd: list[str]) -> list[tuple[str, int, int]]:
    """Run one hipcc command; returns (kernel, VGPR spill count, VGPRs + AGPRs
    allocated) of every kernel whose resource-usage remark reports spilled
    registers.  A kernel that keeps private (scratch) memory without spilling,
    i.e. a local array the compiler did not promote to registers, fails the
    command: every kernel of this library keeps its arrays in registers."""
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    # hipcc's host pass warns about the device-only target feature and the
    # resource-usage remarks are parsed, not printed; anything else is surfaced.
    noise = ("packed-fp32-ops", "warning: feature flag", "1 warning generated", "warnings generated",
             "In file included from")
    spills, scratch, name, regs = [], [], None, 0
    for line in (r.stderr or "").splitlines():
        if "kernel-resource-usage" in line:
            field = lambda key: int(line.split(key)[1].split("[")[0])  # noqa: E731
            if "Function Name:" in line:
                name, regs = line.split("Function Name:")[1].split("[")[0].strip(), 0
            elif "ScratchSize [bytes/lane]:" in line:
                if field("ScratchSize [bytes/lane]:"):
                    scratch.append((name, field("ScratchSize [bytes/lane]:")))
            elif "VGPRs Spill:" in line:
                if field("VGPRs Spill:"):
                    spills.append((name, field("VGPRs Spill:"), regs))
            elif "VGPRs:" in line or "AGPRs:" in line:
                regs += field("VGPRs:" if "VGPRs:" in line else "AGPRs:")
            continue
        if re.match(r"\s*\d*\s*\|", line):   # source excerpt under a remark
            continue
        if line.strip() and not any(n in line for n in noise):
            print(line, file=sys.stderr)
    spilled = {n for n, _, _ in spills}
    stack = [(n, b) for n, b in scratch if n not in spilled]
    if stack:
        raise RuntimeError("kernels keep private memory (a local array not promoted to registers):\n  " +
                           "\n  ".join(f"{n} ({b} bytes per lane)" for n, b in stack))
    return spills


def _compile(units, jobs: int, incremental: bool = False, verbose: bool = False):
    """Compile units in parallel; returns [(object, spills)] in unit order."""
    headers = max(p.stat().st_mtime for p in [*CSRC.glob("*.hpp"), *CSRC.glob("*.inc"),
                                              *(ROOT / "include").glob("*.h")])
    spill_file = BUILD / "spills_by_unit.txt"
    old_spills: dict[str, list[tuple[str, int, int]]] = {}
    if incremental and spill_file.exists():
        for line in spill_file.read_text().splitlines():
            unit, name, n, regs = line.split("\t")
            old_spills.setdefault(unit, []).append((name, int(n), int(regs)))

    def compile_one(u):
        src, defs, obj = u
        if incremental and obj.exists() and obj.stat().st_mtime > max(src.stat().st_mtime, headers):
            return obj, old_spills.get(obj.name, [])
        cmd = [HIPCC, *COMMON, *defs, "-Rpass-analysis=kernel-resource-usage", "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        return obj, _run(cmd)

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        done = list(ex.map(compile_one, units))
    spill_file.write_text("".join(f"{o.name}\t{n}\t{c}\t{g}\n" for o, sp in done for n, c, g in sp))
    return done


def build(jobs: int | None = None, verbose: bool = False, incremental: bool = False) -> Path:
    """Compile every HIP translation unit and link the shared library.
    ``incremental``: recompile only the units whose object is older than their
    source or any header (a development shortcut; the default rebuilds all).
    Fails if any kernel spills VGPRs: every instance is compiled for a wave
    count at which it keeps its registers (csrc/sk_tiers.inc, see retier)."""
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found; the library needs ROCm's hipcc to build")
    BUILD.mkdir(parents=True, exist_ok=True)
    LIB.parent.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(16, os.cpu_count() or 4)
    done = _compile(_units(), jobs, incremental, verbose)
    spilled = [s for _, sp in done for s in sp]
    if spilled:
        names = "\n  ".join(f"{n} ({c} VGPRs spilled)" for n, c, _ in spilled[:20])
        raise RuntimeError(f"{len(spilled)} kernel instances spill VGPRs:\n  {names}\n"
                           "re-measure the tiers with `python -m starter_amd.build --retier`")
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, [o for o, _ in done])])
    os.replace(tmp, LIB)
    return LIB


_INSTANCE = re.compile(
    r"_ZN2sk(?:10|18)(gemv|mfma|mfmt|mfmt_grouped)_entryILi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)EEEvNS_4ArgsE")
# The row-group entry of an LDS-fed MFMA instance is compiled for the plain
# instance's tier (one table key): a spill in either moves both down.
_KINDS = {"gemv": 0, "mfma": 1, "mfmt": 2, "mfmt_grouped": 2}
# (waves per workgroup, VGPRs + AGPRs per lane the compiler may then use)
_TIERS = ((16, 128), (12, 168), (8, 256), (4, 512))


def _write_tiers(overrides: dict[tuple[int, ...], int]) -> None:
    rows = "".join(f"    {{{k[0]}, {k[1]}, {k[2]}, {k[3]}, {k[4]}, {w}}},\n" for k, w in sorted(overrides.items()))
    TIERS_INC.write_text(
        "// Generated by `python -m starter_amd.build --retier`: instances compiled for\n"
        "// fewer waves than their register estimate allows, or not compiled (waves 0).\n"
        "// Fields: {kind (0 gemv, 1 mfma, 2 mfmt), template arguments a, b, c, epilogue, waves}.\n"
        "constexpr TierOverride kTierOverrides[] = {\n" + rows +
        "    {-1, 0, 0, 0, 0, 0},   // end marker\n};\n")


def _read_tiers() -> dict[tuple[int, ...], int]:
    out = {}
    for line in TIERS_INC.read_text().splitlines() if TIERS_INC.exists() else []:
        m = re.match(r"\s*\{(\d+), (\d+), (\d+), (\d+), (\d+), (\d+)\},", line)
        if m:
            out[tuple(map(int, m.groups()[:5]))] = int(m.group(6))
    return out


def retier(jobs: int | None = None, fresh: bool = False) -> dict[tuple[int, ...], int]:
    """Measure csrc/sk_tiers.inc: compile the kernel instances at their
    estimated tiers, move every instance that spills one tier down (16, 12, 8,
    4 waves; below 4 it is dropped) and compile again until nothing spills.
    Starts from the current list unless ``fresh`` (then every instance starts
    at its estimate: use after changing a kernel body)."""
    BUILD.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(16, os.cpu_count() or 4)
    units = [u for u in _units() if u[0].name.startswith("sk_inst_")]
    overrides: dict[tuple[int, ...], int] = {} if fresh else _read_tiers()
    for rnd in range(len(_TIERS) + 1):
        _write_tiers(overrides)
        spilled = [s for _, sp in _compile(units, jobs) for s in sp]
        print(f"retier pass {rnd}: {len(spilled)} instances spill", flush=True)
        if not spilled:
            return overrides
        for name, _, regs in spilled:
            m = _INSTANCE.fullmatch(name)
            if not m:
                raise RuntimeError(f"spilling kernel {name} is not a GEMM instance")
            key = (_KINDS[m.group(1)], *map(int, m.groups()[1:]))
            cur = overrides.get(key) or next(w for w, cap in _TIERS if regs <= cap)
            lower = [w for w, _ in _TIERS if w < cur]
            overrides[key] = lower[0] if lower else 0
    raise RuntimeError("instances still spill at the 4-wave tier")


if __name__ == "__main__":
    import time

    t0 = time.time()
    if "--retier" in sys.argv:
        ov = retier(fresh="--fresh" in sys.argv)
        print(f"{len(ov)} tier overrides ({sum(w == 0 for w in ov.values())} instances dropped) in {TIERS_INC}")
    out = build(verbose="-v" in sys.argv, incremental="--incremental" in sys.argv)
    print(f"built {out} in {time.time() - t0:.1f}s")
