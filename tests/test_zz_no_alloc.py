"""The allocation-free GEMM entry point (wq8_gemm_noalloc; no counterpart in the reference, for callers that cannot
allocate): through the C-ABI its outputs equal wq8_gemm's bit for bit, for the modes whose kernels use a workspace
(block: transposed activation scales; block+g and exact+g: transposed weight scales too) and two that use none (row,
exact), on two calls in a row, the second with a smaller input, and with the residual in place. A call needing more than the
library's array is rejected with -5 before any launch."""
import ctypes

import pytest
import torch

from conftest import DT

pytestmark = pytest.mark.gpu
LIMIT = 32 << 20


def operands(m, n, k, mode, seed):
    g = torch.Generator().manual_seed(seed)
    kb = (k + 127) // 128
    base = mode.removesuffix("+g")
    a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).cuda()
    a_lo = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8).cuda() if base == "exact" else None
    sa = (((torch.rand(m, kb, generator=g) if base == "block" else torch.rand(m, generator=g)) + 0.5) / 127).cuda()
    b = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).cuda()
    sb = (((torch.rand(n, kb, generator=g) if mode.endswith("+g") else torch.rand(n, generator=g)) + 0.5) / 127).cuda()
    bias = (0.02 * torch.randn(n, generator=g)).bfloat16().cuda()
    res = torch.randn(m, n, generator=g).bfloat16().cuda()
    rs = torch.full((n,), 0.5).bfloat16().cuda()
    return a, a_lo, sa, b, sb, bias, res, rs


def p(t):
    return None if t is None else t.data_ptr()


@pytest.mark.parametrize("mode,variant", [("block", 10), ("block", 11), ("block", 15), ("block+g", 12), ("exact+g", 14), ("row", 0), ("exact", 1)])
def test_noalloc_equals_gemm(wq, mode, variant):
    lib = wq.library()
    stream = torch.cuda.current_stream().cuda_stream
    for call, (m, n, k) in enumerate(((4100, 1536, 5120), (700, 1024, 2304))):  # second call smaller
        print(f"noalloc mode={mode} variant={variant} call={call} m={m} n={n} k={k}", flush=True)
        a, a_lo, sa, b, sb, bias, res, rs = operands(m, n, k, mode, seed=variant * 10 + call)
        sizes = (ctypes.c_int64 * 2)()
        lib.wq8_gemm_workspace(m, n, k, variant, 256, 0, sizes)
        ws = torch.empty(max(1, sizes[0]), dtype=torch.uint8, device="cuda")
        want = res.clone()
        assert lib.wq8_gemm(p(a), p(a_lo), p(sa), p(b), p(sb), p(bias), p(want), p(rs), p(want), m, n, k, DT[torch.bfloat16], variant, 256, 0,
                            p(ws), None, stream) == 0
        got = res.clone()
        assert lib.wq8_gemm_noalloc(p(a), p(a_lo), p(sa), p(b), p(sb), p(bias), p(got), p(rs), p(got), m, n, k, DT[torch.bfloat16], variant,
                                    256, 0, stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(got, want)
        assert not torch.equal(got, res)


@pytest.mark.parametrize("mode,variant,shape", [("block", 15, (70, 900, 4096)), ("block", 10, (200, 300, 2048)), ("row", 6, (90, 700, 3072)),
                                                ("exact", 7, (60, 500, 2048)), ("block", 10, (300, 500, 3072))], ids=str)
def test_noalloc_split_equals_gemm(wq, mode, variant, shape):
    """With split 1 (the deep split of launches of few tiles: partial planes in the array and a second launch; with 4 CUs
    counted, the split-K tail with its counters in the array, cleared by a kernel): the same bits as wq8_gemm with a
    workspace, on two calls in a row."""
    lib = wq.library()
    stream = torch.cuda.current_stream().cuda_stream
    m, n, k = shape
    cus = 4 if shape == (300, 500, 3072) else 256
    sizes = (ctypes.c_int64 * 2)()
    lib.wq8_gemm_workspace(m, n, k, variant, cus, 1, sizes)
    assert 0 < sizes[0] + sizes[1] <= LIMIT
    ws = torch.empty(sizes[0], dtype=torch.uint8, device="cuda")
    counters = torch.zeros(max(1, sizes[1] // 4), dtype=torch.int32, device="cuda")
    for call in range(2):
        print(f"noalloc split mode={mode} variant={variant} shape={shape} call={call}", flush=True)
        a, a_lo, sa, b, sb, bias, res, rs = operands(m, n, k, mode, seed=variant * 10 + call + 5)
        want = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
        assert lib.wq8_gemm(p(a), p(a_lo), p(sa), p(b), p(sb), p(bias), None, None, p(want), m, n, k, DT[torch.bfloat16], variant, cus, 1,
                            p(ws), p(counters), stream) == 0
        got = torch.empty_like(want)
        assert lib.wq8_gemm_noalloc(p(a), p(a_lo), p(sa), p(b), p(sb), p(bias), None, None, p(got), m, n, k, DT[torch.bfloat16], variant,
                                    cus, 1, stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(got, want)


def test_noalloc_rejects_beyond_its_array(wq):
    lib = wq.library()
    m, k = 65536, 16384  # block scales m * k / 128 * 4 bytes = 32 MiB + 256: one row too many
    m = LIMIT // ((k // 128) * 4) + 1
    sizes = (ctypes.c_int64 * 2)()
    lib.wq8_gemm_workspace(m, 256, k, 10, 256, 0, sizes)
    assert sizes[0] > LIMIT  # else the call below would launch on null operands: checked on the host first
    rc = lib.wq8_gemm_noalloc(None, None, None, None, None, None, None, None, None, m, 256, k, DT[torch.bfloat16], 10, 256, 0,
                              torch.cuda.current_stream().cuda_stream)
    assert rc == -5


def test_noalloc_under_graph_capture(wq):
    """Captured once in a HIP graph (the callers it is for), replayed with new activations and eager wq8_gemm calls in
    between: every replay equals the eager entry point's result bit for bit."""
    lib = wq.library()
    m, n, k, variant = 1024, 768, 2048, 10
    a, _, sa, b, sb, bias, _, _ = operands(m, n, k, "block", seed=99)
    out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    capture = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.stream(capture):
        with torch.cuda.graph(graph, stream=capture):
            assert lib.wq8_gemm_noalloc(p(a), None, p(sa), p(b), p(sb), p(bias), None, None, p(out), m, n, k, DT[torch.bfloat16], variant, 256, 0,
                                        capture.cuda_stream) == 0
    sizes = (ctypes.c_int64 * 2)()
    lib.wq8_gemm_workspace(m, n, k, variant, 256, 0, sizes)
    ws = torch.empty(sizes[0], dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    for replay in range(4):
        print(f"noalloc graph replay {replay}", flush=True)
        a.copy_(torch.randint(-127, 128, (m, k), dtype=torch.int8, device="cuda"))
        sa.copy_(torch.rand(m, (k + 127) // 128, device="cuda") / 127)
        graph.replay()
        want = torch.empty_like(out)
        assert lib.wq8_gemm(p(a), None, p(sa), p(b), p(sb), p(bias), None, None, p(want), m, n, k, DT[torch.bfloat16], variant, 256, 0,
                            p(ws), None, stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(out, want)


FRESH = r"""
import ctypes, sys, torch
sys.path.insert(0, {root!r})
from wgpkernels_amd.int8 import _native
lib = _native.Library({path!r})  # no Python-layer set-up: nothing resolved the array yet
m, n, k = 512, 384, 1024
a = torch.randint(-127, 128, (m, k), dtype=torch.int8, device="cuda")
b = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda")
sa = torch.rand(m, k // 128, device="cuda") / 127
sb = torch.rand(n, device="cuda") / 127
out = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
p = lambda t: t.data_ptr()
capture = torch.cuda.Stream()
graph = torch.cuda.CUDAGraph()
torch.cuda.synchronize()
with torch.cuda.stream(capture):
    with torch.cuda.graph(graph, stream=capture):
        rc = lib.wq8_gemm_noalloc(p(a), None, p(sa), p(b), p(sb), None, None, None, p(out), m, n, k, 1, 10, 256, 0, capture.cuda_stream)
print("first call under capture:", rc, flush=True)
assert rc == -6, rc
sizes = (ctypes.c_int64 * 2)()
lib.wq8_gemm_workspace(m, n, k, 10, 256, 0, sizes)  # resolves the array outside capture
graph = torch.cuda.CUDAGraph()
with torch.cuda.stream(capture):
    with torch.cuda.graph(graph, stream=capture):
        rc = lib.wq8_gemm_noalloc(p(a), None, p(sa), p(b), p(sb), None, None, None, p(out), m, n, k, 1, 10, 256, 0, capture.cuda_stream)
assert rc == 0, rc
ws = torch.empty(sizes[0], dtype=torch.uint8, device="cuda")
want = torch.empty_like(out)
for _ in range(3):
    graph.replay()
    assert lib.wq8_gemm(p(a), None, p(sa), p(b), p(sb), None, None, None, p(want), m, n, k, 1, 10, 256, 0, p(ws), None,
                        torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, want)
print("fresh process ok", flush=True)
"""


def test_noalloc_first_call_under_capture_in_fresh_process(wq):
    """In a fresh process whose first allocation-free call on the GPU is made under graph capture (nothing resolved the
    array before), the call returns -6 and launches nothing; after a workspace query outside capture, the captured call
    works and every replay equals wq8_gemm."""
    import subprocess
    import sys
    from pathlib import Path
    root = str(Path(__file__).resolve().parents[1])
    code = FRESH.format(root=root, path=str(wq.library().path))
    done = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    print(done.stdout[-2000:], done.stderr[-2000:], flush=True)
    assert done.returncode == 0 and "fresh process ok" in done.stdout
