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
