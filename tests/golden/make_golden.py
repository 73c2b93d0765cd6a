"""Writes tests/golden/config1.npz: the CPU oracle's outputs at the reference's plumbing configuration (K = N = 1536,
weights U[-127, 127], per-channel scales U(0.5, 1.5) / 127, FP32 bias 0.02 N(0, 1) cast to BF16, BF16 N(0, 1) activations
with 8 outlier channels x 50; M = 4 through the lines math and M = 512 through the block math; seed 0).

Inputs are regenerated from the seeded CPU generator (inputs()), so the fixture holds only outputs: the lines outputs in
full, the block path's INT8 activations, block scales and BF16 outputs as SHA-256 digests plus the first rows in full, and
the reference's FP32 dequantize-and-matmul error of each path. Run from the repository root:

    python tests/golden/make_golden.py
"""
import hashlib
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

K = N = 1536
ROWS_KEPT = 4


def inputs(m, seed=0):
    """(x bf16 (m, K), w int8 (N, K), s f32 (N,), bias bf16 (N,)) of the plumbing configuration."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s = (torch.rand(N, generator=g) + 0.5) / 127
    bias = (0.02 * torch.randn(N, generator=g)).to(torch.bfloat16)
    x = torch.randn(m, K, generator=g)
    outliers = torch.randperm(K, generator=g)[:8]
    x[:, outliers] *= 50
    return x.to(torch.bfloat16), w, s, bias


def u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def digest(a):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), np.uint8)


def outputs(oracle):
    from oracle import torch_reference as tr
    out = {}
    x, w, s, bias = inputs(4)
    lines = oracle.linear_f64(u16(x), 1, w.numpy(), s.numpy(), u16(bias))
    out["lines_y"] = lines
    ref = tr.reference_linear(x, w, s, bias)
    out["lines_rel_err"] = np.float64(((torch.from_numpy(lines).double() - ref.double()).norm() / ref.double().norm()).item())
    x, w, s, bias = inputs(512)
    q, sa = oracle.quantize_blocks(u16(x), 1)
    y = oracle.gemm(q, None, sa, w.numpy(), s.numpy(), u16(bias), 1, "block")
    out["block_q_sha256"], out["block_sa_sha256"], out["block_y_sha256"] = digest(q), digest(sa), digest(y)
    out["block_q_head"], out["block_sa_head"], out["block_y_head"] = q[:ROWS_KEPT], sa[:ROWS_KEPT], y[:ROWS_KEPT]
    yf = torch.from_numpy(y.view(np.int16)).view(torch.bfloat16).double()
    ref = tr.reference_linear(x, w, s, bias).double()
    out["block_rel_err"] = np.float64(((yf - ref).norm() / ref.norm()).item())
    return out


if __name__ == "__main__":
    import oracle
    oracle.build()
    np.savez_compressed(Path(__file__).with_name("config1.npz"), **outputs(oracle))
    print("wrote", Path(__file__).with_name("config1.npz"))
