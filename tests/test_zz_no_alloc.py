"""sk_gemm_bf16_noalloc on the GPU, through the C ABI (needs an MI355X).

The allocation-free entry point runs the same plan and kernels as
sk_gemm_bf16, with the split-K counters and partials in the library's static
device scratch instead of a caller workspace, so its outputs must equal
sk_gemm_bf16's bit for bit.  Two calls in a row share the scratch; the second
is smaller than the first, so stale partials and counters of the first call
would show up in its output.  Also checked against the CPU oracle (the
parity bar of every GEMM).
"""

from __future__ import annotations

import pytest
import torch

import oracle
from starter_amd import _lib
from starter_amd._lib import SK_OK, SK_PATH_MFMA_LDS, SkConfig
from tests._util import BF16, assert_parity, bits, from_bits, randn_bf16

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _pair(M: int, N: int, K: int, seed: int):
    g = torch.Generator().manual_seed(seed)
    return randn_bf16((M, K), 1.0, g), randn_bf16((N, K), 0.02, g)


def _with_workspace(a: torch.Tensor, w: torch.Tensor, cfg: SkConfig | None) -> torch.Tensor:
    """sk_gemm_bf16 through the C ABI with its own zero-filled workspace."""
    M, K = a.shape
    N = w.shape[0]
    out = torch.empty(M, N, dtype=BF16, device=DEV)
    n = _lib.workspace_bytes(_lib.SK_OP_GEMM, M, N, K, cfg)
    ws = torch.zeros(max(n, 1), dtype=torch.uint8, device=DEV)
    st = _lib.lib().sk_gemm_bf16(a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0), out.data_ptr(), out.stride(0),
                                 M, N, K, _lib.cfg_ptr(cfg), ws.data_ptr() if n else None, n,
                                 torch.cuda.current_stream().cuda_stream)
    assert st == SK_OK, _lib.strerror(st)
    return out


def _noalloc(a: torch.Tensor, w: torch.Tensor, cfg: SkConfig | None) -> torch.Tensor:
    M, K = a.shape
    N = w.shape[0]
    out = torch.full((M, N), float("nan"), dtype=BF16, device=DEV)
    st = _lib.lib().sk_gemm_bf16_noalloc(a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0), out.data_ptr(),
                                         out.stride(0), M, N, K, _lib.cfg_ptr(cfg),
                                         torch.cuda.current_stream().cuda_stream)
    assert st == SK_OK, _lib.strerror(st)
    return out


SPLIT3 = SkConfig.make(SK_PATH_MFMA_LDS, waves=13, ku=8, rows=32, split=3)   # the down producer's plan at M = 16
SPLIT4 = SkConfig.make(SK_PATH_MFMA_LDS, waves=10, ku=8, rows=16, split=4)
# two row groups, each with its own counters and partials in the scratch
GROUPS_A = SkConfig.make(SK_PATH_MFMA_LDS, waves=10, ku=8, rows=16, split=4, grid=128, groups=2)
GROUPS_B = SkConfig.make(SK_PATH_MFMA_LDS, waves=10, ku=8, rows=16, split=4, grid=64, groups=2)


@pytest.mark.parametrize("first,second", [
    ((16, SPLIT3), (3, SPLIT3)),      # down projection, three K splits, then a smaller batch
    ((64, None), (48, None)),         # the M = 64 default (wide path, three K splits), then 48 rows on it
    ((8, SPLIT4), (5, SPLIT3)),       # explicit split counts: the second call uses fewer tiles
    ((64, GROUPS_A), (40, GROUPS_B)),  # row groups with split K, then fewer rows and workgroups
])
def test_noalloc_equals_workspace_entry_point_on_two_calls(first, second):
    N, K = 2560, 9728                 # down: every plan above splits K, so the scratch is used
    outs = []
    for i, (M, cfg) in enumerate((first, second)):
        assert _lib.workspace_bytes(_lib.SK_OP_GEMM, M, N, K, cfg) > 0, "the case must use the scratch"
        a, w = _pair(M, N, K, seed=100 * i + M)
        ad, wd = a.to(DEV), w.to(DEV)
        got = _noalloc(ad, wd, cfg)
        ref = _with_workspace(ad, wd, cfg)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"call {i}: M={M} cfg={cfg}"
        outs.append((got.cpu(), a, w))
    for got, a, w in outs:
        assert_parity(got, from_bits(oracle.gemm(bits(a), bits(w))), "noalloc gemm vs oracle")


def test_noalloc_unsplit_plan_and_graph_replay():
    """A one-split plan touches no scratch; a split plan captured into a HIP
    graph (the counter clear is a kernel node) replays to the eager result."""
    M, N, K = 4, 6144, 2560           # qkv M = 4: one K split
    a, w = _pair(M, N, K, seed=7)
    ad, wd = a.to(DEV), w.to(DEV)
    assert _lib.workspace_bytes(_lib.SK_OP_GEMM, M, N, K) == 0
    assert torch.equal(_noalloc(ad, wd, None), _with_workspace(ad, wd, None))

    M, N, K = 8, 2560, 9728
    a, w = _pair(M, N, K, seed=8)
    ad, wd = a.to(DEV), w.to(DEV)
    out = torch.empty(M, N, dtype=BF16, device=DEV)
    stream = torch.cuda.Stream()
    assert _lib.workspace_bytes(_lib.SK_OP_GEMM, M, N, K, SPLIT3) > 0

    def call():
        st = _lib.lib().sk_gemm_bf16_noalloc(ad.data_ptr(), ad.stride(0), wd.data_ptr(), wd.stride(0),
                                             out.data_ptr(), out.stride(0), M, N, K, _lib.cfg_ptr(SPLIT3),
                                             torch.cuda.current_stream().cuda_stream)
        assert st == SK_OK

    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        call()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for _ in range(3):
        out.zero_()
        # eager work between replays, also through the shared scratch (a smaller split call)
        small = _noalloc(ad[:3], wd, SPLIT3)
        torch.cuda.synchronize()
        assert torch.equal(small, _with_workspace(ad[:3], wd, SPLIT3))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    assert torch.equal(eager, _with_workspace(ad, wd, SPLIT3))


_FIRST_CALL_IN_CAPTURE = r'''
import sys, torch
sys.path.insert(0, sys.argv[1])
from starter_amd import _lib
from starter_amd._lib import SK_OK, SK_PATH_MFMA_LDS, SkConfig
dev = "cuda:0"
torch.cuda.set_device(0)
M, N, K = 8, 2560, 9728
cfg = SkConfig.make(SK_PATH_MFMA_LDS, waves=13, ku=8, rows=32, split=3)   # uses the scratch
g = torch.Generator().manual_seed(5)
a = (torch.randn(M, K, generator=g)).to(torch.bfloat16).to(dev)
w = (0.02 * torch.randn(N, K, generator=g)).to(torch.bfloat16).to(dev)
out = torch.zeros(M, N, dtype=torch.bfloat16, device=dev)
L = _lib.lib()
def noalloc():
    return L.sk_gemm_bf16_noalloc(a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0), out.data_ptr(),
                                  out.stride(0), M, N, K, _lib.cfg_ptr(cfg), torch.cuda.current_stream().cuda_stream)
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    st = noalloc()      # the process's first call of the entry point
assert st == SK_OK, _lib.strerror(st)
ref = torch.empty_like(out)
n = _lib.workspace_bytes(_lib.SK_OP_GEMM, M, N, K, cfg)
ws = torch.zeros(n, dtype=torch.uint8, device=dev)
assert L.sk_gemm_bf16(a.data_ptr(), a.stride(0), w.data_ptr(), w.stride(0), ref.data_ptr(), ref.stride(0), M, N, K,
                      _lib.cfg_ptr(cfg), ws.data_ptr(), n, torch.cuda.current_stream().cuda_stream) == SK_OK
for i in range(3):
    out.zero_()
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {i}"
print("first-call-in-capture ok", flush=True)
'''


def test_noalloc_first_call_inside_graph_capture():
    """A fresh process whose first sk_gemm_bf16_noalloc call is made under
    HIP graph capture: the scratch address is looked up there, and every
    replay equals sk_gemm_bf16 with a workspace."""
    import subprocess
    import sys
    from pathlib import Path

    root = str(Path(__file__).resolve().parents[1])
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_IN_CAPTURE, root], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "first-call-in-capture ok" in r.stdout
