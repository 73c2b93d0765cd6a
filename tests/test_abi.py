"""The C-ABI boundary without a GPU: libwgp_int8.so loads, exports every entry point include/wq8.h declares (the symbols
the reference's ctypes layer binds, I:66-89), reports ABI 11, and rejects bad arguments with the reference's negative
codes before any launch (K8:1404-1976). No call here reaches a kernel."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "wq8.h"


@pytest.fixture(scope="module")
def lib():
    from wgpkernels_amd import build
    path = build.library_file("int8")
    if not path.exists():
        build.build("int8")
    return ctypes.CDLL(str(path))


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|void)\s+(wq8_\w+)\s*\(", text, re.M)))


def test_header_declares_the_reference_interface():
    names = set(declared())
    # bound by the reference's load_library (I:69-89) and its optional entry points (K8:1396, K8:1637, K8:1926)
    required = {"wq8_abi", "wq8_features", "wq8_quantize", "wq8_quantize_blocks", "wq8_transform_rows", "wq8_rotate_groups",
                "wq8_gemm", "wq8_gemm_workspace", "wq8_gemm_select", "wq8_small", "wq8_small_workspace", "wq8_gemv_lines",
                "wq8_l2_flush", "wq8_l2_flush_release", "wq8_gemm_segments", "wq8_quantize_at", "wq8_quantize_blocks_at",
                "wq8_gemm_at"}
    assert required <= names, required - names


def test_every_declared_symbol_is_exported(lib):
    missing = [name for name in declared() if not hasattr(lib, name)]
    assert not missing
    exported = subprocess.run(["nm", "-D", "--defined-only", str(Path(lib._name))], capture_output=True, text=True, check=True).stdout
    public = set(re.findall(r"\bT (wq8_\w+)", exported))
    assert public == set(declared()), public ^ set(declared())  # nothing exported that the header does not declare


def test_abi_version_and_features(lib):
    assert lib.wq8_abi() == 11
    assert lib.wq8_features() & 1  # per-(n, k-block) weight scales


def test_workspace_queries(lib):
    sizes = (ctypes.c_int64 * 2)(-1, -1)
    lib.wq8_gemm_workspace(32760, 13824, 5120, 0, 256, 0, sizes)
    assert list(sizes) == [0, 0]  # whole tiles: no split-K slots or counters
    lib.wq8_gemm_workspace(32760, 13824, 5120, 10, 256, 0, sizes)
    assert list(sizes) == [32760 * 40 * 4, 0]  # block mode: the activation scales transposed per k-block
    lib.wq8_gemm_workspace(100, 13824, 5120, 12, 256, 0, sizes)
    assert list(sizes) == [(100 * 40 * 4 + 255) // 256 * 256 + 13824 * 40 * 4, 0]  # plus the weight-group scales
    lib.wq8_small_workspace(32, 5120, 13824, 256, sizes)
    assert list(sizes) == [3 * 32 * 5120 * 4, 0]  # row-balanced over 3 K splits: their FP32 partials
    lib.wq8_small_workspace(32, 13824, 5120, 256, sizes)
    assert list(sizes) == [0, 0]  # row-balanced over the whole of K: none
    lib.wq8_small_workspace(32, 1536, 5120, 256, sizes)
    assert list(sizes) == [10 * 32 * 1536 * 4, 0]  # split form: one slot per 512-element K split
    # empty shapes (the Python layer queries before it skips the call): no division by zero, no workspace
    for m, n, k in ((3, 0, 512), (0, 256, 512), (0, 0, 0)):
        lib.wq8_small_workspace(m, n, k, 256, sizes)
        assert list(sizes) == [0, 0]
        for variant in (0, 1, 10, 12, 14):
            lib.wq8_gemm_workspace(m, n, k, variant, 256, 0, sizes)


def test_gemm_select_returns_a_known_variant(lib):
    for hilo in (0, 1):
        for m in (40, 4096, 32760):
            assert lib.wq8_gemm_select(m, 5120, 5120, hilo, 256) in ((1, 7) if hilo else (0, 6))


def test_argument_rejection_before_launch(lib):
    p, i, i64, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
    lib.wq8_quantize_blocks.argtypes = [p, p, p, i, i, i64, i, i, i, p, f, p, p]
    lib.wq8_quantize.argtypes = [p, p, p, p, i, i, i64, i, i, i, p, f, p]
    lib.wq8_gemm.argtypes = [p, p, p, p, p, p, p, p, p, i, i, i, i, i, i, i, p, p, p]
    lib.wq8_small.argtypes = [p, i64, p, p, p, p, p, p, i, i, i, i, i, p, p, p]
    lib.wq8_gemv_lines.argtypes = [p, i64, p, p, p, p, p, p, i, i, i, i, p]
    lib.wq8_rotate_groups.argtypes = [p, p, i, i, i64, i, i, p]
    # quantizers: bad dtype / group / act, FP32 input with an activation, K not a multiple of 8, rms above 16384 without inv_rms
    assert lib.wq8_quantize_blocks(None, None, None, 4, 128, 128, 3, 0, 0, None, 0.0, None, None) == -1
    assert lib.wq8_quantize_blocks(None, None, None, 4, 128, 128, 1, 32, 0, None, 0.0, None, None) == -1
    assert lib.wq8_quantize_blocks(None, None, None, 4, 128, 128, 1, 0, 4, None, 0.0, None, None) == -1
    assert lib.wq8_quantize_blocks(None, None, None, 4, 128, 128, 2, 0, 3, None, 0.0, None, None) == -1
    assert lib.wq8_quantize_blocks(None, None, None, 4, 100, 100, 1, 0, 0, None, 0.0, None, None) == -2
    assert lib.wq8_quantize_blocks(None, None, None, 4, 16392, 16392, 1, 0, 1, None, 0.0, None, None) == -2
    assert lib.wq8_quantize(None, None, None, None, 4, 96, 96, 1, 64, 0, None, 0.0, None) == -2
    assert lib.wq8_rotate_groups(None, None, 4, 128, 128, 1, 8, None) == -1
    # GEMM: unknown variant, hi/lo operand against the variant, K not a multiple of 16
    assert lib.wq8_gemm(None, None, None, None, None, None, None, None, None, 64, 64, 128, 1, 99, 256, 0, None, None, None) == -3
    assert lib.wq8_gemm(None, None, None, None, None, None, None, None, None, 64, 64, 128, 1, 1, 256, 0, None, None, None) == -2
    assert lib.wq8_gemm(None, None, None, None, None, None, None, None, None, 64, 64, 120, 1, 0, 256, 0, None, None, None) == -2
    # block variants need their workspace (the transposed scales)
    assert lib.wq8_gemm(None, None, None, None, None, None, None, None, None, 64, 64, 128, 1, 10, 256, 0, None, None, None) == -2
    # ... 16-byte aligned (a misaligned one is refused before anything runs)
    assert lib.wq8_gemm(None, None, None, None, None, None, None, None, None, 64, 64, 128, 1, 10, 256, 0, 0x1008, None, None) == -2
    # few-token paths: more rows than the path takes, K off its multiple
    assert lib.wq8_small(None, 128, None, None, None, None, None, None, 33, 64, 128, 1, 256, None, None, None) == -2
    assert lib.wq8_small(None, 96, None, None, None, None, None, None, 8, 64, 96, 1, 256, None, None, None) == -2
    assert lib.wq8_gemv_lines(None, 128, None, None, None, None, None, None, 5, 64, 128, 1, None) == -2
    assert lib.wq8_gemv_lines(None, 130, None, None, None, None, None, None, 2, 64, 130, 1, None) == -2
