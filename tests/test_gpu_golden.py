"""The GPU path against the committed golden fixture of the reference's plumbing configuration (K = N = 1536, seed 0;
tests/golden/make_golden.py): M = 4 through 'lines' within 1e-3 of the FP64 reference, M = 512 through 'block' bit for
bit (INT8 activations, block scales and BF16 outputs) when the reference-order tile runs."""
import hashlib
import importlib.util
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import bits, rel_err

HERE = Path(__file__).resolve().parent / "golden"


def _generator():
    spec = importlib.util.spec_from_file_location("make_golden", HERE / "make_golden.py")
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    return gen


@pytest.mark.gpu
def test_config1_lines(wq):
    gen, golden = _generator(), np.load(HERE / "config1.npz")
    x, w, s, bias = (t.cuda() for t in gen.inputs(4))
    y = wq.linear(x, w, s, bias, mode="lines")
    ref = torch.from_numpy(golden["lines_y"]).bfloat16().float()
    assert rel_err(y.float().cpu(), ref) <= 1e-3


@pytest.mark.gpu
@pytest.mark.parametrize("variant", [11, 10, 15])
def test_config1_block(wq, variant):
    gen, golden = _generator(), np.load(HERE / "config1.npz")
    x, w, s, bias = (t.cuda() for t in gen.inputs(512))
    q, sa = wq.quantize_blocks(x)
    digest = lambda t: hashlib.sha256(np.ascontiguousarray(bits(t)).tobytes()).digest()
    assert digest(q) == bytes(golden["block_q_sha256"])
    assert digest(sa) == bytes(golden["block_sa_sha256"])
    y = wq.gemm(q, None, sa, w, s, bias, torch.bfloat16, 0, variant)
    if variant == 11:  # the reference's fold order: bit-exact
        assert digest(y) == bytes(golden["block_y_sha256"])
        np.testing.assert_array_equal(bits(y[:4]), golden["block_y_head"])
    # either fold: the error against the FP32 definition stays within 1.05x of the reference block math's
    from oracle import torch_reference as tr
    ref = tr.reference_linear(*(t.cpu() for t in (x, w, s, bias)))
    assert rel_err(y.float().cpu(), ref) <= 1.05 * float(golden["block_rel_err"])
