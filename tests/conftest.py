"""Shared test helpers. Marker `gpu`: needs an MI355X (run with -m gpu); everything else runs on the CPU."""
import os
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X GPU (gfx950) and the built HIP library")


def bits(t):
    """numpy view of a CPU tensor: uint16 bit patterns for BF16 / FP16, the values otherwise."""
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


DT = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def from_bits(a, dtype):
    """torch tensor (CPU) of dtype from uint16 bit patterns."""
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dtype)


def rel_err(y, ref):
    y, ref = y.double(), ref.double()
    return ((y - ref).norm() / ref.norm()).item()


@pytest.fixture(scope="session")
def oracle():
    import oracle as o
    o.build()
    return o


@pytest.fixture(scope="session")
def wq():
    """The product package with its HIP library loaded (GPU tests only)."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from wgpkernels_amd import int8 as wq
    wq.load_library()
    return wq


@pytest.fixture
def whole_tiles(wq, monkeypatch, tmp_path):
    """The tile choice timed from an empty store over whole tiles only (split 0): every tile it can pick for a mode folds
    in the same order (block: 10 and 15 both biased; row and exact: INT32), so that outputs of different shapes, chunks
    or entry points compare bit for bit whatever tile wins. (With split 1 the split-K order depends on the tiles.)"""
    monkeypatch.setattr(wq._tuning, "store", wq._tuning.Store(str(tmp_path / "tiles.json")))
    monkeypatch.setattr(wq, "_plans", {})
    monkeypatch.setattr(wq, "tile_candidates", lambda mode: [(v, 0) for v in wq.TILES[mode] if v is not None])
    return wq


def gemm_exact64(a, a_lo, sa, b, sb, bias_bits, dtype, mode, residual_bits=None, rscale_bits=None):
    """The INT8 GEMM epilogue's value in float64, before the output rounding: exact INT64 block sums, scales and epilogue
    in float64 (numpy inputs as the oracle takes them; bias / residual / rscale as uint16 bits of `dtype`). mode 'row',
    'exact' or 'block'; weight groups when sb is 2-D."""
    a64, b64 = a.astype(np.int64), b.astype(np.int64)
    k = a.shape[1]
    kb = (k + 127) // 128
    groups = sb.ndim == 2
    f = np.zeros((a.shape[0], b.shape[0]))
    for blk in range(kb):
        cols = slice(blk * 128, min(k, blk * 128 + 128))
        s = (a64[:, cols] @ b64[:, cols].T).astype(np.float64)
        if a_lo is not None:
            s = s + (a_lo[:, cols].astype(np.int64) @ b64[:, cols].T).astype(np.float64) / 254.0
        if mode == "block":
            s = s * sa[:, blk].astype(np.float64)[:, None]
        if groups:
            s = s * sb[:, blk].astype(np.float64)[None, :]
        f += s
    if mode != "block":
        f *= sa.astype(np.float64)[:, None]
    if not groups:
        f *= sb.astype(np.float64)[None, :]
    as_float = lambda v: from_bits(v, dtype).double().numpy()
    if bias_bits is not None:
        f += as_float(bias_bits)[None, :]
    if residual_bits is not None:
        rs = as_float(rscale_bits)[None, :] if rscale_bits is not None else 1.0
        f = f * rs + as_float(residual_bits)
    return f
