"""Benchmark of the MI355X decode-GEMM hot path (BASELINE.json metric).

Workload (the configuration the metric is quoted on):
one Qwen3-4B decoder layer's four decode GEMMs at M = 8 rows, bf16 —
QKV [6144, 2560], o_proj [2560, 4096], gate_up [19456, 2560] with the fused
SwiGLU epilogue, down [2560, 9728].  Weights ~N(0, 0.02) and activations
~N(0, 1), seeded, synthetic.  A *step* is those four GEMMs for one layer;
consecutive steps walk 36 distinct layers' weights (7.27 GB), so every step
streams its 201.85 MB from HBM and the 256 MB MALL cannot serve it.

``value`` = algorithmic bytes per step / device time per step (GB/s), with
inputs resident in HBM.  Algorithmic bytes per GEMM = 2NK + 2MK + out
(out = 2MN, 2*M*9728 for gate_up, 12M for lm_head+argmax); split-K
workspace traffic is not counted.

Timing: the K timed steps are captured into one HIP graph (the way the
decode step runs) and replayed once between two synchronisations; HIP
events on the launch stream give the time.  Per-kernel durations (roofline,
per-GEMM table) come from graphs of back-to-back launches of one kernel over
rotating weights, also timed with events on the launch stream; they include
the inter-kernel gap, so they slightly understate kernel-only bandwidth
(rocprofv3 --kernel-trace --stats gives kernel-only durations; see profiles/).

The ``decode`` object of the JSON line is BASELINE configuration 5: a
synthetic Qwen3-4B (36 layers, random bf16 weights) decoding greedily at
batch 16 after a 1024-token prompt, one HIP graph per decode step, reported as
decode tok/s = 16 * steps / decode time (and end-to-end tok/s including the
prefill); inside it, ``host_delivery`` is the same generation through the
pipelined host token loop and ``verify`` one speculative verify pass at the
reference's batch-16 width (16 sequences x 8 draft-tree rows = 128 rows,
engine.py:451), ``verify_r4`` the same with 4 rows per sequence.  The ``attention`` object times the decode
step's attention launch (q/k norm + rotary + KV write + GQA attention) alone at
batch 16, position 1088, with its achieved HBM bandwidth (the K and V rows read
per launch).  ``hipblaslt_us`` beside each per-GEMM point is the vendor
library's GEMM (torch.mm) on the same rotating weights.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--sweep [--wide]] [--no-cpu]
                       [--decode-steps S] [--decode-only] [--attention-only]
       python bench.py --probe --probe-op OP --M M      (launches for rocprofv3 --pmc)
       python bench.py --counters-from FOLDER           (markdown table of the counter passes)
       python bench.py --traffic-from FETCH_DIR WRITE_DIR --M M
       python bench.py --trace-from FOLDER [--trace-passes]  (markdown tables of a kernel trace)
Prints ONE JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0      # MI355X HBM3E, vendor figure
PEAK_BF16_TFLOPS = 2500.0  # dense bf16 MFMA
METRIC = "achieved HBM GB/s (% of peak) per decode GEMM at M=1/8; decode tok/s at bs=16"

SHAPES = {   # name: (N, K, kind)
    "qkv": (6144, 2560, "gemm"),
    "o_proj": (2560, 4096, "gemm"),
    "gate_up": (9728, 2560, "gateup"),     # N = I, weight [2I, K]
    "down": (2560, 9728, "gemm"),
    "lm_head": (151936, 2560, "lm_argmax"),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def alg_bytes(name: str, M: int) -> int:
    N, K, kind = SHAPES[name]
    if kind == "gateup":
        return 2 * (2 * N) * K + 2 * M * K + 2 * M * N
    if kind == "lm_argmax":
        return 2 * N * K + 2 * M * K + 12 * M
    return 2 * N * K + 2 * M * K + 2 * M * N


def alg_flops(name: str, M: int) -> int:
    N, K, kind = SHAPES[name]
    return 2 * M * (2 * N if kind == "gateup" else N) * K


class Workload:
    """36 layers of synthetic Qwen3-4B decode weights plus fixed activations."""

    def __init__(self, layers: int, M: int, device: str = "cuda:0", seed: int = 0):
        import torch

        from starter_amd import kernels as Kn

        self.torch, self.Kn = torch, Kn
        self.M, self.dev, self.L = M, device, layers
        gen = torch.Generator(device=device).manual_seed(seed)
        bf16 = torch.bfloat16

        # Drawn in place in bf16 (no fp32 temporaries): the setup then frees no
        # device memory, which on this platform leaves every later kernel of
        # the process ~7% slower.
        def w(n, k):
            return torch.empty(n, k, dtype=bf16, device=device).normal_(0.0, 0.02, generator=gen)

        self.wqkv = [w(6144, 2560) for _ in range(layers)]
        self.wo = [w(2560, 4096) for _ in range(layers)]
        self.wgu = [w(19456, 2560) for _ in range(layers)]
        self.wd = [w(2560, 9728) for _ in range(layers)]
        self.wlm = [w(151936, 2560) for _ in range(2)]
        torch.cuda.synchronize()
        self.x = torch.randn(M, 2560, generator=gen, device=device).to(bf16)
        self.attn = torch.randn(M, 4096, generator=gen, device=device).to(bf16)
        self.act = torch.randn(M, 9728, generator=gen, device=device).to(bf16)
        self.mm = {
            "qkv": Kn.SkinnyMatmul(M, 6144, 2560, device),
            "o_proj": Kn.SkinnyMatmul(M, 2560, 4096, device),
            "gate_up": Kn.SkinnyGateUp(M, 9728, 2560, device),
            "down": Kn.SkinnyMatmul(M, 2560, 9728, device),
            "lm_head": Kn.LmArgmax(M, 151936, 2560, device),
        }
        self.out = {
            "qkv": torch.empty(M, 6144, dtype=bf16, device=device),
            "o_proj": torch.empty(M, 2560, dtype=bf16, device=device),
            "gate_up": torch.empty(M, 9728, dtype=bf16, device=device),
            "down": torch.empty(M, 2560, dtype=bf16, device=device),
        }
        self.ids = torch.empty(M, dtype=torch.int64, device=device)
        self.maxv = torch.empty(M, dtype=torch.float32, device=device)

    def launch(self, name: str, layer: int) -> None:
        Kn, mm = self.Kn, self.mm[name]
        if name == "qkv":
            Kn.gemm(self.x, self.wqkv[layer], out=self.out["qkv"], config=mm.config, ws=mm.ws)
        elif name == "o_proj":
            Kn.gemm(self.attn, self.wo[layer], out=self.out["o_proj"], config=mm.config, ws=mm.ws)
        elif name == "gate_up":
            w = self.wgu[layer]
            Kn.gateup_swiglu(self.x, w[:9728], w[9728:], out=self.out["gate_up"], config=mm.config, ws=mm.ws)
        elif name == "down":
            Kn.gemm(self.act, self.wd[layer], out=self.out["down"], config=mm.config, ws=mm.ws)
        elif name == "lm_head":
            Kn.lm_argmax(self.x, self.wlm[layer % 2], config=mm.config, ws=mm.ws, ids=self.ids, maxv=self.maxv)

    def step(self, i: int) -> None:
        layer = i % self.L
        for name in ("qkv", "o_proj", "gate_up", "down"):
            self.launch(name, layer)

    def capture(self, fn, n: int):
        torch = self.torch
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for i in range(min(n, 3)):
                fn(i)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(n):
                fn(i)
        torch.cuda.synchronize()
        return g

    def time_graph(self, g, reps: int = 1) -> list[float]:
        """Milliseconds per replay, HIP events on the current (launch) stream."""
        torch = self.torch
        out = []
        for _ in range(reps):
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            g.replay()
            b.record()
            b.synchronize()
            out.append(a.elapsed_time(b))
        return out

    def kernel_us(self, name: str, launches: int, reps: int = 5) -> float:
        """Median per-launch time of back-to-back launches over rotating weights."""
        nl = 2 if name == "lm_head" else self.L
        g = self.capture(lambda i: self.launch(name, i % nl), launches)
        g.replay()
        t = self.time_graph(g, reps)
        del g
        return statistics.median(t) * 1000.0 / launches

    def launch_library(self, name: str, layer: int) -> None:
        """The vendor-library yardstick of the reference's pickers: ``a @ w.t()``
        through torch (hipBLASLt on ROCm; engine/kernels/gemm.py:527-528,
        569-570) on the same weights.  Only the GEMM is timed: gate_up's
        SwiGLU and lm_head's argmax would come on top (the library writes the
        full [M, 2I] / [M, V] output instead)."""
        mm = self.torch.mm
        if name == "qkv":
            mm(self.x, self.wqkv[layer].t(), out=self.lib_out["qkv"])
        elif name == "o_proj":
            mm(self.attn, self.wo[layer].t(), out=self.lib_out["o_proj"])
        elif name == "gate_up":
            mm(self.x, self.wgu[layer].t(), out=self.lib_out["gate_up"])
        elif name == "down":
            mm(self.act, self.wd[layer].t(), out=self.lib_out["down"])
        elif name == "lm_head":
            mm(self.x, self.wlm[layer % 2].t(), out=self.lib_out["lm_head"])

    def library_us(self, name: str, launches: int, reps: int = 5) -> float:
        """kernel_us for launch_library: graph replay of back-to-back calls."""
        nl = 2 if name == "lm_head" else self.L
        if not hasattr(self, "lib_out"):
            torch, M, bf16 = self.torch, self.M, self.torch.bfloat16
            self.lib_out = {n: torch.empty(M, (2 * N if k == "gateup" else N), dtype=bf16, device=self.dev)
                            for n, (N, K, k) in SHAPES.items()}
        g = self.capture(lambda i: self.launch_library(name, i % nl), launches)
        g.replay()
        t = self.time_graph(g, reps)
        del g
        return statistics.median(t) * 1000.0 / launches


def _cpu_model() -> str:
    cpu = platform.processor() or platform.machine()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return cpu


def _timed_steps(step, seconds: float, min_steps: int = 5) -> tuple[list[float], float]:
    """Per-step times of `step` run back to back until `seconds` of work (and
    at least `min_steps` steps) are done; returns (times, total seconds)."""
    ts = []
    t_start = time.perf_counter()
    while len(ts) < min_steps or time.perf_counter() - t_start < seconds:
        t0 = time.perf_counter()
        step()
        ts.append(time.perf_counter() - t0)
    return ts, time.perf_counter() - t_start


def cpu_baseline(M: int, seconds: float) -> dict:
    """The reference's own CPU path for one step: torch F.linear (bf16 in,
    fp32 accumulate, bf16 out; engine/kernels/gemm.py:527 `a @ w.t()`) for QKV,
    o_proj and down, F.silu(g) * u over the gate/up projection (gemm.py:569),
    on the host cores of this box.  Median step of a sample of about `seconds`
    of CPU work after 3 warmups."""
    import torch
    import torch.nn.functional as F

    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    bf = torch.bfloat16
    w = {n: (torch.randn(2 * N if k == "gateup" else N, K, generator=g) * 0.02).to(bf)
         for n, (N, K, k) in SHAPES.items() if n != "lm_head"}
    x = torch.randn(M, 2560, generator=g).to(bf)
    attn = torch.randn(M, 4096, generator=g).to(bf)
    act = torch.randn(M, 9728, generator=g).to(bf)

    def step():
        F.linear(x, w["qkv"])
        F.linear(attn, w["o_proj"])
        gu = F.linear(x, w["gate_up"])
        F.silu(gu[:, :9728]) * gu[:, 9728:]
        F.linear(act, w["down"])

    for _ in range(3):
        step()
    ts, total = _timed_steps(step, seconds)
    t = statistics.median(ts)
    step_bytes = sum(alg_bytes(n, M) for n in ("qkv", "o_proj", "gate_up", "down"))
    cpu = _cpu_model()
    return {"value": round(step_bytes / t / 1e9, 2), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "reference",
            "sample": f"{len(ts)} steps ({total:.1f} s of CPU work; median step) of the M={M} layer workload via "
                      f"torch F.linear/F.silu on CPU (the reference's a @ w.t() baseline path), "
                      f"{t * 1e3:.2f} ms/step, {cpu}"}


def cpu_config1(seconds: float) -> dict:
    """BASELINE configs[0], the reference's own CPU-runnable case: one decode
    QKV projection on the CPU path, torch F.linear (bf16 in, fp32 accumulate,
    bf16 out), x [1, 2560] ~N(0, 1) then W [6144, 2560] ~N(0, 0.02) drawn from
    one generator seeded 0.  Median call of about `seconds` of CPU work (at
    least 20 calls) after 3 warmups, on this box's host cores."""
    import torch
    import torch.nn.functional as F

    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 2560, generator=g).to(torch.bfloat16)
    w = (torch.randn(6144, 2560, generator=g) * 0.02).to(torch.bfloat16)
    for _ in range(3):
        F.linear(x, w)
    ts, total = _timed_steps(lambda: F.linear(x, w), seconds, min_steps=20)
    t = statistics.median(ts)
    return {"value": round(alg_bytes("qkv", 1) / t / 1e9, 2), "unit": "GB/s", "us": round(t * 1e6, 1),
            "cores": torch.get_num_threads(), "kind": "reference",
            "sample": f"{len(ts)} calls ({total:.1f} s of CPU work; median call) of F.linear(x [1,2560], "
                      f"W [6144,2560]) bf16, seed 0, {_cpu_model()}"}


def cpu_port(M: int, seconds: float) -> dict:
    """The CPU restatement of the hot path (oracle/, kind "port": plain C,
    fp32 accumulation, OpenMP over output rows) timed on this box's host
    cores for the same layer step: QKV, o_proj, gate_up+SwiGLU and down at
    M rows.  Median step of about `seconds` of CPU work after one warmup.  The reference's
    own path is Triton on a GPU and has no CPU build to time."""
    import numpy as np

    import oracle

    rng = np.random.default_rng(0)

    def bits(*shape, scale=1.0):
        return oracle.f32_to_bf16(rng.standard_normal(shape, dtype=np.float32) * scale)

    w = {n: bits(N, K, scale=0.02) for n, (N, K, k) in SHAPES.items() if k == "gemm"}
    wg, wu = bits(9728, 2560, scale=0.02), bits(9728, 2560, scale=0.02)
    x, attn, act = bits(M, 2560), bits(M, 4096), bits(M, 9728)

    def step():
        oracle.gemm(x, w["qkv"])
        oracle.gemm(attn, w["o_proj"])
        oracle.gateup_swiglu(x, wg, wu)
        oracle.gemm(act, w["down"])

    step()
    ts, total = _timed_steps(step, seconds, min_steps=3)
    t = statistics.median(ts)
    step_bytes = sum(alg_bytes(n, M) for n in ("qkv", "o_proj", "gate_up", "down"))
    cpu = _cpu_model()
    return {"value": round(step_bytes / t / 1e9, 2), "unit": "GB/s", "cores": oracle.threads(),
            "kind": "port",
            "sample": f"{len(ts)} steps ({total:.1f} s of CPU work; median step) of the M={M} layer workload "
                      f"(qkv, o_proj, gate_up+swiglu, down) through the C oracle, {t * 1e3:.2f} ms/step, "
                      f"{oracle.threads()} OpenMP threads, {cpu}"}


PROBE_LAUNCHES = 24
PROBE_COPY_BYTES = 512 << 20


def probe(M: int, name: str = "gate_up", config: str | None = None) -> int:
    """Untimed launches for the hardware-counter passes: PROBE_LAUNCHES
    launches of one projection (default gate_up+SwiGLU) at M rows over rotating
    weights (12 layers, or the two lm_head copies: no launch finds its weights
    in the MALL), then three copies of PROBE_COPY_BYTES with torch's copy
    kernel as the calibration of known size.  ``config`` ("path,waves,ku,rows,
    split,grid,groups") replaces the projection's default configuration."""
    import torch

    if name == "attention":   # the decode step's fused rope + attention launch (B = 16, position 1088)
        log(f"probe: {PROBE_LAUNCHES} attention launches (B = 16, position {ATTN_POS})")
        attention_benchmark(launches=PROBE_LAUNCHES, timed=False)
    else:
        wl = Workload(12, M)
        if config:
            from starter_amd import kernels as Kn
            from starter_amd._lib import SkConfig

            mm = wl.mm[name]
            mm.config = SkConfig.make(*[int(v) for v in config.split(",")])
            mm.ws = Kn._workspace(mm.op, M, mm.N, mm.K, mm.config, wl.dev)
            log(f"probe: {name} at M={M} with {mm.config}")
        nl = 2 if name == "lm_head" else wl.L
        wl.launch(name, 0)
        torch.cuda.synchronize()
        log(f"probe: {PROBE_LAUNCHES} {name} launches at M={M}")
        for i in range(PROBE_LAUNCHES):
            wl.launch(name, i % nl)
        torch.cuda.synchronize()
    src = torch.empty(PROBE_COPY_BYTES // 2, dtype=torch.bfloat16, device="cuda:0").fill_(1.0)
    dst = torch.empty_like(src)
    log(f"probe: 3 copies of {PROBE_COPY_BYTES} bytes")
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log("probe: done")
    return 0


def _counter_rows(folder: str, counter: str) -> list[tuple[str, float]]:
    """(kernel name, counter value) per dispatch, in dispatch order, from
    rocprofv3's counter_collection.csv under folder."""
    import csv

    files = sorted(Path(folder).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no counter_collection.csv under {folder}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                if r.get("Counter_Name") == counter:
                    rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    return [(n, v) for _, n, v in sorted(rows)]


def traffic_summary(fetch_dir: str, write_dir: str, M: int, name: str = "gate_up") -> int:
    """HBM bytes per launch of the probed projection from FETCH_SIZE /
    WRITE_SIZE (KiB per dispatch), each scaled by copy_bytes / (what the
    counter reads for the PROBE_COPY_BYTES copy), written next to the
    profiles it came from."""
    out = {"op": name, "M": M, "copy_bytes": PROBE_COPY_BYTES}
    total = 0.0
    for key, folder, counter in (("fetch", fetch_dir, "FETCH_SIZE"), ("write", write_dir, "WRITE_SIZE")):
        rows = _counter_rows(folder, counter)
        gu = [v for n, v in rows if "sk::" in n]   # the probe launches no other library kernel
        cp = [v for n, v in rows if "copy" in n.lower()][-3:]   # the probe ends with its three copies
        if not gu or not cp:
            raise SystemExit(f"{counter}: {name} dispatches {len(gu)}, copy dispatches {len(cp)} in {folder}")
        gu = gu[1:] if len(gu) > 1 else gu     # first launch warms code and workspace
        kib = statistics.median(gu)
        copy_kib = statistics.median(cp)
        factor = (PROBE_COPY_BYTES / 1024.0) / copy_kib
        out[key] = {"counter": counter, "kib_per_launch": kib, "copy_kib": copy_kib, "factor": round(factor, 4),
                    "bytes_per_launch": round(kib * 1024.0 * factor)}
        total += kib * 1024.0 * factor
    out["hbm_bytes_per_launch"] = round(total)
    out["algorithmic_bytes_per_launch"] = alg_bytes(name, M)
    out["ratio"] = round(total / alg_bytes(name, M), 4)
    path = ROOT / "profiles" / f"traffic_{name}_m{M}.json"
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(json.dumps(out))
    return 0


COUNTER_PASSES = {   # rocprofv3 --pmc sets, each within one run's per-block limits
    "A": "SQ_WAVES SQ_BUSY_CU_CYCLES SQ_WAVE_CYCLES SQ_WAIT_INST_ANY SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS "
         "SQ_LDS_BANK_CONFLICT",
    "B": "SQ_VALU_MFMA_BUSY_CYCLES SQ_ACTIVE_INST_VMEM SQ_ACTIVE_INST_LDS SQ_INSTS_VMEM_RD SQ_LDS_IDX_ACTIVE "
         "SQ_WAIT_INST_LDS GRBM_GUI_ACTIVE TA_BUSY_avr TA_BUSY_max",
    "C": "FETCH_SIZE",
    "D": "WRITE_SIZE TCC_HIT_sum TCC_MISS_sum",
}
MI355X_SIMDS = 1024
SHADER_GHZ = 2.4   # MI355X peak engine clock: busy fractions are of the kernel's duration at this clock


def _dispatches(folder: Path, csv_name: str) -> list[dict]:
    """Rows of rocprofv3's csv_name files under folder grouped per dispatch, in dispatch order."""
    import csv

    per = {}
    for f in sorted(folder.rglob(f"*{csv_name}")):
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                d = per.setdefault(int(r.get("Dispatch_Id") or r.get("Correlation_Id")), {"_name": r["Kernel_Name"]})
                if "Counter_Name" in r:
                    d[r["Counter_Name"]] = float(r["Counter_Value"])
                    d["_grid"] = int(r["Grid_Size"]) // int(r["Workgroup_Size"])
                    d["_wg"] = int(r["Workgroup_Size"])
                else:
                    d["_us"] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
    return [per[k] for k in sorted(per)]


def trace_summary(folder: str, regex: str = "sk::", per: int = 0) -> int:
    """One markdown row per kernel launch shape in the rocprofv3 kernel trace(s)
    under ``folder``: kernels whose name matches ``regex``, grouped by (name,
    workgroups, workgroup size) in order of first appearance, with launch
    count, kernel-only average / median / min / max duration and, when ``per``
    is given, the launches and microseconds per unit (e.g. per decode step)."""
    import csv
    import re

    pat = re.compile(regex)
    groups: dict = {}
    for f in sorted(Path(folder).rglob("*kernel_trace.csv")):
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                name = r["Kernel_Name"]
                if not pat.search(name):
                    continue
                wg = int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"])
                grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"]) // max(wg, 1)
                key = (name.replace("void ", "").split("(")[0], grid, wg, r.get("VGPR_Count", ""))
                groups.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
    head = "| kernel | workgroups | threads | VGPR | launches | avg us | median us | min us | max us |"
    print(head + (" launches per unit | us per unit |" if per else ""))
    print("|---|---:|---:|---:|---:|---:|---:|---:|---:|" + ("---:|---:|" if per else ""))
    total = 0.0
    for (name, grid, wg, vgpr), us in groups.items():
        line = (f"| `{name}` | {grid} | {wg} | {vgpr} | {len(us)} | {statistics.mean(us):.2f} | "
                f"{statistics.median(us):.2f} | {min(us):.2f} | {max(us):.2f} |")
        if per:
            line += f" {len(us) / per:.1f} | {sum(us) / per:.1f} |"
            total += sum(us) / per
        print(line)
    if per:
        print(f"\nSum of the listed kernels per unit: {total:.1f} us ({per} units).")
    return 0


def trace_passes(folder: str, marker: str = "decode_attn_kernel<16") -> int:
    """The verify passes of a ``--decode-only`` kernel trace, one markdown row
    per (pass, kernel instance, launch shape, occurrence within the layer).
    Launches are taken in start order from the first ``marker`` launch (the
    tree attention, one per layer) on; each marker launch starts a layer, its
    grid names the pass (workgroups of the attention), and a kernel's k-th
    launch since the last marker is occurrence k (o_proj and down share one
    wide instance: occurrences 1 and 2).  The kernel before the first marker
    of a replay (the layer-0 qkv) and the lm_head launch after the last layer
    count as occurrences of the preceding layer."""
    import csv
    import re

    rows = []
    for f in sorted(Path(folder).rglob("*kernel_trace.csv")):
        with open(f, newline="") as fh:
            rows += [r for r in csv.DictReader(fh) if "sk::" in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    start = next((i for i, r in enumerate(rows) if marker in r["Kernel_Name"]), None)
    if start is None:
        print(f"no launch of {marker} in {folder}")
        return 1
    groups: dict = {}
    pass_grid, seen = None, {}
    for r in rows[start:]:
        name = re.sub(r"^void ", "", r["Kernel_Name"]).split("(")[0]
        wg = int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"])
        grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"]) // max(wg, 1)
        if marker in name:
            pass_grid, seen = grid, {}
        k = seen[(name, grid)] = seen.get((name, grid), 0) + 1
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
        groups.setdefault((pass_grid, name, grid, k), []).append(us)
    print("| pass (attention workgroups) | kernel | workgroups | occurrence | launches | avg us | median us |")
    print("|---:|---|---:|---:|---:|---:|---:|")
    for (pg, name, grid, k), us in groups.items():
        print(f"| {pg} | `{name}` | {grid} | {k} | {len(us)} | {statistics.mean(us):.2f} | {statistics.median(us):.2f} |")
    return 0


def counters_summary(folder: str) -> int:
    """One markdown row per probe from the counter passes of ``--probe`` runs
    laid out as <folder>/<op>_m<M>_{kt,A,B,C,D} (kernel trace, then the four
    COUNTER_PASSES).  Library launches (kernel names in namespace sk) are kept
    and the first one dropped (it warms code and workspace); FETCH_SIZE and
    WRITE_SIZE are scaled by copy bytes / what the counter reads for the
    probe's PROBE_COPY_BYTES copies.  Busy fractions divide by the kernel
    trace's average duration in cycles at SHADER_GHZ (times the SIMD count
    for MFMA busy cycles, which the counter sums over SIMDs); TA_BUSY_avr and
    _max are per texture-address unit."""
    root = Path(folder)
    probes = sorted({p.name[:-3] for p in root.glob("*_kt")})
    print("| op | M | instance | WGs x threads | avg us | % of 8 TB/s | TFLOP/s (% of 2.5 P) | MFMA busy % "
          "| MFMA insts/wave | VALU insts/wave | LDS bank confl % | wait % of wave cycles | TA busy avg/max % "
          "| HBM read MB (alg MB) | HBM write MB | L2 hit % |")
    print("|---|---:|---|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|")

    def med(rs, k):
        v = [r[k] for r in rs if k in r]
        return statistics.median(v) if v else float("nan")

    for pr in probes:
        op, m = pr.rsplit("_m", 1)
        m, _, tag = m.partition("-")   # <op>_m<M>[-<tag>]: a probe of an explicit configuration
        M = int(m)
        sets = {x: _dispatches(root / f"{pr}_{x}", "counter_collection.csv") for x in "ABCD"}
        lib = {x: [r for r in rs if "sk::" in r["_name"]][1:] for x, rs in sets.items()}
        cal = {}
        for x, ctr in (("C", "FETCH_SIZE"), ("D", "WRITE_SIZE")):
            cp = [r[ctr] for r in sets[x] if "copy" in r["_name"].lower() and ctr in r][-3:]
            cal[ctr] = (PROBE_COPY_BYTES / 1024.0) / statistics.median(cp) if cp else float("nan")
        kt = [r["_us"] for r in _dispatches(root / f"{pr}_kt", "kernel_trace.csv") if "sk::" in r["_name"]][1:]
        A, B, C, D = lib["A"], lib["B"], lib["C"], lib["D"]
        if op == "attention":
            alg, flops = 16 * 8 * (ATTN_POS + 1) * 128 * 2 * 2, 16 * 32 * (ATTN_POS + 1) * 128 * 2 * 2
        else:
            alg, flops = alg_bytes(op, M), alg_flops(op, M)
        us = statistics.mean(kt)
        cycles = us * SHADER_GHZ * 1e3          # kernel duration in shader cycles
        waves = med(A, "SQ_WAVES")
        name = A[0]["_name"].replace("void ", "").split("(")[0]
        hits, miss = med(D, "TCC_HIT_sum"), med(D, "TCC_MISS_sum")
        print(f"| {op}{f' ({tag})' if tag else ''} | {M if op != 'attention' else 16} | `{name}` | {A[0]['_grid']} x {A[0]['_wg']} | {us:.2f} "
              f"| {100 * alg / us / 1e3 / PEAK_HBM_GBS:.1f} "
              f"| {flops / us / 1e6:.1f} ({100 * flops / us / 1e6 / PEAK_BF16_TFLOPS:.2f}) "
              f"| {100 * med(B, 'SQ_VALU_MFMA_BUSY_CYCLES') / (cycles * MI355X_SIMDS):.2f} "
              f"| {med(A, 'SQ_INSTS_MFMA') / waves:.0f} | {med(A, 'SQ_INSTS_VALU') / waves:.0f} "
              f"| {100 * med(A, 'SQ_LDS_BANK_CONFLICT') / max(med(B, 'SQ_LDS_IDX_ACTIVE'), 1):.1f} "
              f"| {100 * med(A, 'SQ_WAIT_INST_ANY') / med(A, 'SQ_WAVE_CYCLES'):.1f} "
              f"| {100 * med(B, 'TA_BUSY_avr') / cycles:.0f} / {100 * med(B, 'TA_BUSY_max') / cycles:.0f} "
              f"| {med(C, 'FETCH_SIZE') * 1024 * cal['FETCH_SIZE'] / 1e6:.1f} ({alg / 1e6:.1f}) "
              f"| {med(D, 'WRITE_SIZE') * 1024 * cal['WRITE_SIZE'] / 1e6:.2f} "
              f"| {100 * hits / max(hits + miss, 1):.1f} |")
    return 0


def decode_benchmark(steps: int, B: int = 16, T: int = 1024, max_new: int | None = None) -> dict:
    """synthetic Qwen3-4B (36 layers, random bf16
    weights ~N(0, 0.02)), B prompts of T uniform-random token ids, prefill, then
    ``steps`` greedy decode steps replayed from one captured HIP graph.
    decode tok/s = B * steps / decode time (HIP events on the replay stream);
    end-to-end tok/s = B * (steps + 1) / (prefill + decode)."""
    import torch

    from starter_amd.decode import DecodePlan, Qwen3Config, SyntheticModel, time_decode, time_delivery

    log(f"decode: building the synthetic Qwen3-4B (B={B}, prompt {T}, {steps} steps)")
    model = SyntheticModel(Qwen3Config(), "cuda:0", seed=7)
    # the plan (attention length, cache) covers every timed step: 128 new
    # tokens (the prefill's and 127 steps) unless more steps are asked for
    max_new = max(128, steps + 1) if max_new is None else max_new
    plan = DecodePlan(model, B, T, max_new)
    g = torch.Generator(device="cuda:0").manual_seed(11)
    plan.ids.copy_(torch.randint(0, model.cfg.vocab, (B, T), device="cuda:0", generator=g))
    ids = plan.ids.clone()
    r = time_decode(plan, steps)
    log(f"decode: {r['tok_s']:.0f} tok/s ({r['ms_per_step']:.3f} ms/step), prefill {r['prefill_s']:.3f} s, "
        f"end-to-end {r['e2e_tok_s']:.0f} tok/s")
    # the same generation through the pipelined host delivery loop (every
    # step's tokens copied to pinned host memory, GPU kept 3 steps ahead)
    d = time_delivery(plan, ids, steps + 1)
    log(f"decode with host delivery: {d['delivered_tok_s']:.0f} tok/s delivered, end-to-end {d['e2e_tok_s']:.0f} tok/s")
    v = verify_benchmark(plan)
    v4 = verify_benchmark(plan, 4, (-1, 0, 0, 1))
    out = {"tok_s": round(r["tok_s"], 1), "ms_per_step": round(r["ms_per_step"], 4), "steps": steps, "B": B,
           "prompt": T, "prefill_s": round(r["prefill_s"], 4), "e2e_tok_s": round(r["e2e_tok_s"], 1),
           "host_delivery": {"delivered_tok_s": round(d["delivered_tok_s"], 1), "e2e_tok_s": round(d["e2e_tok_s"], 1),
                             "first_token_s": round(d["first_token_s"], 4), "depth": d["depth"]},
           "workload": "synthetic qwen3-4b greedy decode, 36 layers, GQA 32/8, cap %d, HIP graph per step" % plan.cap,
           "verify": v, "verify_r4": v4}
    return out


# The reference's 8-node draft tree (its greedy template builder, recycle.py:75-95,
# under the default "flat" rank prior): node t's parent.
TREE8 = (-1, 0, 0, 1, 0, 2, 1, 0)


def verify_benchmark(plan, R: int = 8, parents=TREE8, replays: int = 20) -> dict:
    """One speculative verify pass (engine/model.py:334-375) over the decode
    model's cache: B sequences x R rows (a draft tree), M = B*R rows through
    every projection, tree-masked attention, greedy token per row; captured
    into a HIP graph and replayed at the position the decode left (the same
    cache slots are rewritten each replay).  Reports the pass time and rows
    verified per second."""
    import statistics

    import torch

    from starter_amd.decode import VerifyPlan

    vp = VerifyPlan(plan, R, tree=True)
    vp.set_tree(list(parents))
    g = torch.Generator(device="cuda:0").manual_seed(5)
    vp.blk.copy_(torch.randint(0, plan.model.cfg.vocab, vp.blk.shape, device="cuda:0", generator=g))
    vp.pos.copy_(plan.pos)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        vp.verify()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        vp.verify()
    graph.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(replays):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        graph.replay()
        b.record()
        b.synchronize()
        ts.append(a.elapsed_time(b))
    ms = statistics.median(ts)
    B = plan.B
    pos = int(plan.pos[0])
    _KEEP.append((vp, graph))
    log(f"verify: B={B} x R={R} rows (tree {list(parents)}) at position {pos}: {ms:.3f} ms per pass, "
        f"{B * R / ms * 1e3:.0f} rows/s")
    return {"B": B, "R": R, "tree_parents": list(parents), "position": pos, "ms_per_pass": round(ms, 4),
            "rows_per_s": round(B * R / ms * 1e3, 1), "replays": replays}


_KEEP: list = []   # attention workloads stay allocated until the process ends (no device frees)


def verify_recycle_benchmark(B: int = 16, R: int = 8, k: int = 8, chains: int = 8, reps: int = 7) -> dict:
    """The reference's production verify chain at batch 16 (recycle mode,
    engine/model.py:370-373, engine/recycle.py:164-184): the lm_head call
    ``mm["lm"](x, y, w_norm, xout, w)`` producing the full logits of the
    M = B x R verify rows ([128, 151936] bf16: add + RMSNorm, then the logits
    GEMM, sk_gemm_bf16), then ``fast_topk(logits, k)`` (sk_topk_bf16).  A graph of
    ``chains`` chains over two rotating lm_head weight copies (1.56 GB, beyond
    the 256 MB Infinity Cache); HIP events on the replay stream, median of
    ``reps`` replays.  The logits GEMM and the top-k are also timed alone, and
    the library's logits GEMM (torch.mm on hipBLASLt) beside them."""
    import statistics

    import torch

    from starter_amd import kernels as K
    from starter_amd._lib import SK_OP_RMSNORM_GEMM

    dev = "cuda:0"
    M, H, V = B * R, 2560, 151936
    g = torch.Generator(device=dev).manual_seed(21)
    ws_ = [torch.empty(V, H, dtype=torch.bfloat16, device=dev).normal_(0.0, 0.02, generator=g) for _ in range(2)]
    x = torch.empty(M, H, dtype=torch.bfloat16, device=dev).normal_(generator=g)
    y = torch.empty(M, H, dtype=torch.bfloat16, device=dev).normal_(generator=g)
    wn = torch.ones(H, dtype=torch.bfloat16, device=dev)
    xout = torch.empty_like(x)
    logits = torch.empty(M, V, dtype=torch.bfloat16, device=dev)
    lib_logits = torch.empty(M, V, dtype=torch.bfloat16, device=dev)
    n = K._lib.workspace_bytes(SK_OP_RMSNORM_GEMM, M, V, H)
    ws = torch.zeros(max(n, 1), dtype=torch.uint8, device=dev)
    _KEEP.extend([ws_, x, y, wn, xout, logits, lib_logits, ws])
    res: dict = {}

    def chain(i):
        K.rmsnorm_gemm(x, y, wn, 1e-6, xout, ws_[i % 2], out=logits, ws=ws)
        res["topk"] = K.fast_topk(logits, k)

    def logits_only(i):
        K.rmsnorm_gemm(x, y, wn, 1e-6, xout, ws_[i % 2], out=logits, ws=ws)

    def topk_only(i):
        K.fast_topk(logits, k)

    def library(i):
        torch.mm(x, ws_[i % 2].t(), out=lib_logits)

    def time_us(fn, n_calls):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn(0)
            fn(1)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(n_calls):
                fn(i)
        graph.replay()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            graph.replay()
            b.record()
            b.synchronize()
            ts.append(a.elapsed_time(b) * 1e3 / n_calls)
        _KEEP.append(graph)
        return statistics.median(ts)

    chain_us = time_us(chain, chains)
    logits_us = time_us(logits_only, chains)
    topk_us = time_us(topk_only, 4 * chains)
    lib_us = time_us(library, chains)
    log(f"verify recycle chain (M={M}): {chain_us:.1f} us per chain; logits {logits_us:.1f} us "
        f"(hipBLASLt GEMM alone {lib_us:.1f} us), top-{k} {topk_us:.1f} us")
    return {"M": M, "B": B, "R": R, "k": k, "us_per_chain": round(chain_us, 2), "logits_us": round(logits_us, 2),
            "topk_us": round(topk_us, 2), "hipblaslt_logits_us": round(lib_us, 2),
            "logits_GB/s": round((V * H * 2 + M * H * 2 + M * V * 2) / (logits_us * 1e-6) / 1e9, 1),
            "workload": f"mm['lm'] (add + RMSNorm + logits GEMM [{M}, {H}] x [{V}, {H}]) then fast_topk k={k}, "
                        f"two rotating weight copies"}


ATTN_POS = 1088


def attention_benchmark(launches: int = 64, B: int = 16, pos: int = ATTN_POS, cap: int = 1408, ncache: int = 8,
                        timed: bool = True) -> dict:
    """Decode attention with the rotary step (sk_decode_attention_rope_bf16, the
    launch the decode step makes per layer) at the Qwen3-4B decode shape: B
    sequences at position ``pos``, 32/8 heads of 128, plan length 1152 (one key
    split per (sequence, KV head) at B = 16).  ``ncache`` K/V cache pairs of
    92 MB rotate so that a launch does not find its rows in the 256 MB Infinity
    Cache.  One graph of ``launches`` launches, HIP events on its stream; HBM
    bytes per launch = the K and V rows read, B x 8 x (pos + 1) x 128 x 2 x 2."""
    import statistics

    import torch

    from starter_amd import kernels as K
    from starter_amd.decode import Qwen3Config, rope_tables

    dev = "cuda:0"
    cfg = Qwen3Config()
    HQ, HKV, D = cfg.heads, cfg.kv_heads, cfg.head_dim
    g = torch.Generator(device=dev).manual_seed(13)

    def rnd(*shape):
        return torch.empty(*shape, dtype=torch.bfloat16, device=dev).normal_(generator=g)

    ks = [rnd(B, HKV, cap, D) for _ in range(ncache)]
    vs = [rnd(B, HKV, cap, D) for _ in range(ncache)]
    qkv = rnd(B, (HQ + 2 * HKV) * D)
    qw = torch.ones(D, dtype=torch.bfloat16, device=dev)
    cos, sin = rope_tables(cfg, cap, dev)
    posv = torch.full((B,), pos, dtype=torch.int32, device=dev)
    out = torch.empty(B, 1, HQ, D, dtype=torch.bfloat16, device=dev)
    attn = K.DecodeAttention(B, HQ, HKV, D, cap, dev, maxlen=1152)
    _KEEP.extend([ks, vs, qkv, qw, cos, sin, posv, out, attn])

    def call(i):
        attn.rope_attend(qkv, qw, qw, cos, sin, posv, ks[i % ncache], vs[i % ncache], out, cfg.eps)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(2):
            call(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    if not timed:   # counter probe: untimed eager launches only
        for i in range(launches):
            call(i)
        torch.cuda.synchronize()
        return {}
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(launches):
            call(i)
    graph.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(5):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        graph.replay()
        b.record()
        b.synchronize()
        ts.append(a.elapsed_time(b) * 1e3 / launches)
    us = statistics.median(ts)
    byts = B * HKV * (pos + 1) * D * 2 * 2
    log(f"attention: {us:.2f} us per launch, {byts / us / 1e3:.0f} GB/s")
    return {"us": round(us, 3), "GB/s": round(byts / us / 1e3, 1), "frac_peak": round(byts / us / 1e3 / PEAK_HBM_GBS, 4),
            "bytes": byts, "launches": launches,
            "workload": f"q/k norm + rotary + KV write + GQA decode attention, B={B}, 32/8 heads x 128, "
                        f"position {pos}, {ncache} rotating caches of cap {cap}"}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=72)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--M", type=int, default=8)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--sweep", action="store_true", help="also time all five shapes at M in 1..64 (BASELINE config 4)")
    ap.add_argument("--wide", action="store_true",
                    help="with --sweep, also M = 96 and 128 (the reference's batch-16 verify width)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="CPU work in the reference baseline's sample (the oracle port gets half)")
    ap.add_argument("--decode-steps", type=int, default=127,
                    help="C5: greedy decode steps timed after a B=16, T=1024 prefill (0 skips it)")
    ap.add_argument("--attention-only", action="store_true",
                    help="run only the decode-attention measurement and print its JSON object")
    ap.add_argument("--recycle-only", action="store_true",
                    help="run only the verify recycle-chain measurement (logits at M = 128 + top-k)")
    ap.add_argument("--decode-only", action="store_true",
                    help="run only the C5 decode measurement and print its JSON object")
    ap.add_argument("--probe", action="store_true",
                    help="launch --probe-op at --M (untimed) and a 512 MiB copy, for rocprofv3 --pmc passes")
    ap.add_argument("--probe-op", default="gate_up", choices=list(SHAPES) + ["attention"],
                    help="the projection --probe launches (default gate_up)")
    ap.add_argument("--probe-config", metavar="P,W,KU,ROWS,SPLIT,GRID,GROUPS",
                    help="with --probe: launch this configuration instead of the default one")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="turn two rocprofv3 --pmc output folders of --probe (FETCH_SIZE, WRITE_SIZE) into "
                         "profiles/traffic_<probe-op>_m<M>.json and exit")
    ap.add_argument("--trace-from", metavar="FOLDER",
                    help="print a markdown table of the library's kernels in the rocprofv3 kernel trace under "
                         "FOLDER and exit (--trace-regex, --trace-per)")
    ap.add_argument("--trace-regex", default="sk::", help="kernel-name pattern for --trace-from")
    ap.add_argument("--trace-per", type=int, default=0, help="with --trace-from: units to divide totals by")
    ap.add_argument("--trace-passes", action="store_true",
                    help="with --trace-from on a --decode-only trace: the verify passes by pass and layer position")
    ap.add_argument("--counters-from", metavar="FOLDER",
                    help="print a markdown row per probe from the rocprofv3 passes under FOLDER "
                         "(<op>_m<M>_kt, _A, _B, _C, _D) and exit")
    args = ap.parse_args()
    if args.counters_from:
        return counters_summary(args.counters_from)
    if args.trace_from:
        if args.trace_passes:
            return trace_passes(args.trace_from)
        return trace_summary(args.trace_from, args.trace_regex, args.trace_per)
    if args.traffic_from:
        return traffic_summary(args.traffic_from[0], args.traffic_from[1], args.M, args.probe_op)

    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: this build measures the single-GPU hot path "
              f"(--gpus {args.gpus} requested; multi-GPU sharding is a design note, not a measured path)",
              file=sys.stderr)
        return 2

    import torch

    from starter_amd import _lib

    if not _lib.LIB_PATH.exists():
        from starter_amd.build import build

        log("library missing; building")
        build()
    if not torch.cuda.is_available():
        log("no ROCm GPU visible")
        return 1
    torch.cuda.set_device(0)
    if args.probe:
        return probe(args.M, args.probe_op, args.probe_config)
    if args.attention_only:
        print(json.dumps({"attention": attention_benchmark()}), flush=True)
        return 0
    if args.decode_only:
        print(json.dumps({"decode": decode_benchmark(max(1, args.decode_steps))}), flush=True)
        return 0
    if args.recycle_only:
        print(json.dumps({"verify_recycle": verify_recycle_benchmark()}), flush=True)
        return 0
    log(f"device {torch.cuda.get_device_name(0)}; building workload (36 layers of weights)")
    wl = Workload(args.layers, args.M)

    layer_names = ("qkv", "o_proj", "gate_up", "down")
    step_bytes = sum(alg_bytes(n, args.M) for n in layer_names)
    step_flops = sum(alg_flops(n, args.M) for n in layer_names)

    if args.warmup > 0:
        gw = wl.capture(wl.step, args.warmup)
        gw.replay()
        torch.cuda.synchronize()
        del gw
    g = wl.capture(wl.step, args.steps)
    g.replay()   # untimed replay of the captured graph (first-touch of its pool)
    torch.cuda.synchronize()
    log(f"timing {args.steps} steps")
    times = wl.time_graph(g, 5)   # five replays of the K-step graph: the median is the value
    ms = statistics.median(times)
    ms_per_step = ms / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    value_best = step_bytes / (min(times) / args.steps * 1e-3) / 1e9
    del g

    # Per-kernel timing: the dominant kernel of the step (gate_up) and the
    # per-GEMM table at M = 1 and M = 8.  Every workload stays referenced until
    # the process ends: on this platform a large device free (torch releasing a
    # segment) leaves every later kernel of the process several percent slower,
    # so nothing is freed between the timed phases.
    per_gemm = {}
    keep = [wl]
    for M in sorted({1, args.M}):
        wlM = wl if M == args.M else Workload(args.layers, M, seed=1)
        keep.append(wlM)
        for name in SHAPES:
            n = 8 if name == "lm_head" else 72
            us = wlM.kernel_us(name, n)
            lib_us = wlM.library_us(name, n)
            gbs = alg_bytes(name, M) / (us * 1e-6) / 1e9
            per_gemm.setdefault(name, {})[f"M{M}"] = {
                "us": round(us, 3), "GB/s": round(gbs, 1), "frac_peak": round(gbs / PEAK_HBM_GBS, 4),
                "TFLOP/s": round(alg_flops(name, M) / (us * 1e-6) / 1e12, 3),
                "hipblaslt_us": round(lib_us, 3), "vs_hipblaslt": round(lib_us / us, 3)}
            log(f"{name:8s} M={M:2d}: {us:8.2f} us  {gbs:7.1f} GB/s  ({100 * gbs / PEAK_HBM_GBS:.1f}% of 8 TB/s); "
                f"hipBLASLt GEMM alone {lib_us:8.2f} us")

    sweep = None
    if args.sweep:
        sweep = {}
        for M in (1, 2, 4, 8, 16, 32, 40, 64) + ((96, 128) if args.wide else ()):
            wlM = Workload(min(args.layers, 12), M, seed=2)
            for name in SHAPES:
                n = 8 if name == "lm_head" else 36
                us = wlM.kernel_us(name, n)
                lib_us = wlM.library_us(name, n)
                gbs = alg_bytes(name, M) / (us * 1e-6) / 1e9
                sweep.setdefault(name, {})[f"M{M}"] = {"us": round(us, 3), "GB/s": round(gbs, 1),
                                                       "TFLOP/s": round(alg_flops(name, M) / (us * 1e-6) / 1e12, 3),
                                                       "hipblaslt_us": round(lib_us, 3),
                                                       "vs_hipblaslt": round(lib_us / us, 3)}
                log(f"sweep {name:8s} M={M:2d}: {us:8.2f} us {gbs:7.1f} GB/s; hipBLASLt {lib_us:8.2f} us")
            keep.append(wlM)

    dom = per_gemm["gate_up"][f"M{args.M}"]
    traffic = None
    tfile = ROOT / "profiles" / f"traffic_gate_up_m{args.M}.json"
    if tfile.exists():
        try:
            traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    roofline = {"bound": "hbm", "achieved": dom["GB/s"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(dom["GB/s"] / PEAK_HBM_GBS, 4), "traffic": traffic,
                "kernel": f"gate_up+swiglu M={args.M} ({alg_bytes('gate_up', args.M)} algorithmic bytes/launch, "
                          f"{dom['us']} us/launch)"}

    # attention before the decode measurement, whose model and caches (~11 GB)
    # leave the process in a state where the isolated launch reads ~1 us slower
    attention = attention_benchmark()
    recycle = verify_recycle_benchmark()
    decode = None
    if args.decode_steps > 0:
        decode = decode_benchmark(args.decode_steps)

    cpu = port = cpu1 = None
    if not args.no_cpu:
        log("timing the CPU baseline")
        cpu = cpu_baseline(args.M, args.cpu_seconds)
        log("timing the C oracle on the CPU")
        port = cpu_port(args.M, args.cpu_seconds / 2)
        log("timing BASELINE config 1 (QKV, M = 1) on the CPU reference path")
        cpu1 = cpu_config1(args.cpu_seconds / 4)

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) activations)",
        "value_best_of_5": round(value_best, 1),
        "config": {"workload": "qwen3-4b decoder-layer decode GEMMs: qkv 6144x2560, o_proj 2560x4096, "
                               "gate_up 19456x2560+swiglu, down 2560x9728",
                   "M": args.M, "layers_rotated": args.layers, "step_bytes": step_bytes,
                   "step_tflops": round(step_flops / (ms_per_step * 1e-3) / 1e12, 3),
                   "frac_peak_hbm": round(value / PEAK_HBM_GBS, 4)},
        "roofline": roofline,
        "decode": decode,
        "attention": attention,
        "verify_recycle": recycle,
        "cpu_baseline": cpu,
        "cpu_port": port,
        "cpu_config1": cpu1,
        "per_gemm": per_gemm,
    }
    if sweep is not None:
        line["sweep"] = sweep
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
