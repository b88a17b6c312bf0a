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
HANDOFF_EPIS = (8, 9, 10, 11, 12)   # residual hand-off consumers and producers (LDS-fed ring path only)


def _units() -> list[tuple[Path, list[str], Path]]:
    units = [(CSRC / "sk_abi.hip", [], BUILD / "sk_abi.o"), (CSRC / "sk_attn.hip", [], BUILD / "sk_attn.o"),
             (CSRC / "sk_topk.hip", [], BUILD / "sk_topk.o")]
    for epi in range(N_EPI):
        units.append((CSRC / "sk_inst_mfma.hip", [f"-DSK_EPI={epi}"], BUILD / f"sk_inst_mfma_{epi}.o"))
        units.append((CSRC / "sk_inst_gemv.hip", [f"-DSK_EPI={epi}"], BUILD / f"sk_inst_gemv_{epi}.o"))
        units.append((CSRC / "sk_inst_mfmt.hip", [f"-DSK_EPI={epi}"], BUILD / f"sk_inst_mfmt_{epi}.o"))
    for epi in NORM_EPIS:
        units.append((CSRC / "sk_inst_gemv.hip", [f"-DSK_EPI={epi}"], BUILD / f"sk_inst_gemv_{epi}.o"))
    for epi in HANDOFF_EPIS:
        units.append((CSRC / "sk_inst_mfmt.hip", [f"-DSK_EPI={epi}"], BUILD / f"sk_inst_mfmt_{epi}.o"))
    return units


def _run(cmd: list[str]) -> list[tuple[str, int]]:
    """Run one hipcc command; returns (kernel, VGPR spill count) of every
    kernel whose resource-usage remark reports spilled registers."""
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    # hipcc's host pass warns about the device-only target feature and the
    # resource-usage remarks are parsed, not printed; anything else is surfaced.
    noise = ("packed-fp32-ops", "warning: feature flag", "1 warning generated", "warnings generated")
    spills, name = [], None
    for line in (r.stderr or "").splitlines():
        if "kernel-resource-usage" in line:
            if "Function Name:" in line:
                name = line.split("Function Name:")[1].split("[")[0].strip()
            elif "VGPRs Spill:" in line:
                n = int(line.split("VGPRs Spill:")[1].split("[")[0])
                if n:
                    spills.append((name, n))
            continue
        if line.strip() and not any(n in line for n in noise):
            print(line, file=sys.stderr)
    return spills


def build(jobs: int | None = None, verbose: bool = False, incremental: bool = False) -> Path:
    """Compile every HIP translation unit and link the shared library.
    ``incremental``: recompile only the units whose object is older than their
    source or any header (a development shortcut; the default rebuilds all)."""
    if not Path(HIPCC).exists() and shutil.which("hipcc") is None:
        raise RuntimeError("hipcc not found; the library needs ROCm's hipcc to build")
    BUILD.mkdir(parents=True, exist_ok=True)
    LIB.parent.mkdir(parents=True, exist_ok=True)
    jobs = jobs or min(16, os.cpu_count() or 4)
    units = _units()
    headers = max(p.stat().st_mtime for p in [*CSRC.glob("*.hpp"), *(ROOT / "include").glob("*.h")])
    spill_file = BUILD / "spills_by_unit.txt"
    old_spills: dict[str, list[tuple[str, int]]] = {}
    if incremental and spill_file.exists():
        for line in spill_file.read_text().splitlines():
            unit, name, n = line.split("\t")
            old_spills.setdefault(unit, []).append((name, int(n)))

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
    objs = [o for o, _ in done]
    spilled = [s for _, sp in done for s in sp]
    spill_file.write_text("".join(f"{o.name}\t{n}\t{c}\n" for o, sp in done for n, c in sp))
    (BUILD / "spills.txt").write_text("".join(f"{n}\t{c}\n" for n, c in spilled))
    if spilled:
        print(f"note: {len(spilled)} kernel instances spill VGPRs (list in {BUILD / 'spills.txt'})", file=sys.stderr)
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    import time

    t0 = time.time()
    out = build(verbose="-v" in sys.argv, incremental="--incremental" in sys.argv)
    print(f"built {out} in {time.time() - t0:.1f}s")
