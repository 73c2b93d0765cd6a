"""A seeded sweep of ragged shapes through every GEMM variant and both few-token paths, against the CPU oracle: GEMM
outputs bit-exact (the variant's own fold order), few-token outputs within the 1e-3 bound of the FP32 reference
rounded to the output dtype. The shapes are drawn once from a fixed seed (M, N, K not multiples of the tiles; K a
multiple of 16 for the GEMM, 64 for small, 4 for lines), with and without bias and residual, in BF16 and FP16."""
import numpy as np
import pytest
import torch

from conftest import DT, bits, from_bits, rel_err
from test_gpu_gemm import BIASED, check_gemm, operands

pytestmark = pytest.mark.gpu

GEMM_VARIANTS = [("row", 0), ("row", 6), ("exact", 1), ("exact", 7), ("block", 10), ("block", 11), ("block", 15), ("block+g", 12),
                 ("block+g", 13), ("exact+g", 14)]


def shapes(seed, count, k_multiple, m_max):
    rng = np.random.default_rng(seed)
    for _ in range(count):
        m = int(rng.integers(1, m_max + 1))
        n = int(rng.integers(1, 700))
        k = int(rng.integers(1, 40)) * k_multiple
        yield m, n, k, bool(rng.integers(0, 2)), bool(rng.integers(0, 2)), (torch.bfloat16, torch.float16)[int(rng.integers(0, 2))]


@pytest.mark.parametrize("mode,variant", GEMM_VARIANTS)
def test_gemm_sweep(wq, oracle, mode, variant):
    groups = mode.endswith("+g")
    base = mode.removesuffix("+g")
    oracle_mode = "block_biased" if base == "block" and not groups and variant in BIASED else base
    if groups and base == "exact":
        oracle_mode = "exact_combined"
    for i, (m, n, k, with_bias, with_res, dtype) in enumerate(shapes(variant * 101, 6, 16, 600)):
        print(f"sweep {mode} v{variant} #{i}: m={m} n={n} k={k} bias={with_bias} residual={with_res} {dtype}", flush=True)
        a, a_lo, sa, b, sb, bias, res, rs = operands(m, n, k, variant * 1000 + i, groups, base == "exact", base == "block", dtype, with_res)
        bias = bias if with_bias else None
        cu = lambda t: None if t is None else t.cuda()
        y = wq.gemm(cu(a), cu(a_lo), cu(sa), cu(b), cu(sb), cu(bias), dtype, 0, variant, residual=cu(res), residual_scale=cu(rs))
        torch.cuda.synchronize()
        ref = oracle.gemm(a.numpy(), None if a_lo is None else a_lo.numpy(), sa.numpy(), b.numpy(), sb.numpy(),
                          None if bias is None else bits(bias), DT[dtype], oracle_mode, None if res is None else bits(res),
                          None if rs is None else bits(rs))
        check_gemm(y, ref)


@pytest.mark.parametrize("path,k_multiple,m_max", [("gemv_lines", 4, 4), ("small", 64, 32)])
def test_fewtoken_sweep(wq, oracle, path, k_multiple, m_max):
    for i, (m, n, k, with_bias, with_res, dtype) in enumerate(shapes(k_multiple * 7 + m_max, 8, k_multiple * 16, m_max)):
        print(f"sweep {path} #{i}: m={m} n={n} k={k} bias={with_bias} residual={with_res} {dtype}", flush=True)
        g = torch.Generator().manual_seed(i)
        x = torch.randn(m, k, generator=g).to(dtype)
        w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
        s = (torch.rand(n, generator=g) + 0.5) / 127
        bias = (0.02 * torch.randn(n, generator=g)).to(dtype) if with_bias else None
        res = torch.randn(m, n, generator=g).to(dtype) if with_res else None
        rs = torch.rand(n, generator=g).to(dtype) if with_res else None
        cu = lambda t: None if t is None else t.cuda()
        y = getattr(wq, path)(x.cuda(), w.cuda(), s.cuda(), cu(bias), cu(res), cu(rs))
        torch.cuda.synchronize()
        ref = oracle.linear_f64(bits(x), DT[dtype], w.numpy(), s.numpy(), None if bias is None else bits(bias),
                                None if res is None else bits(res), None if rs is None else bits(rs))
        assert rel_err(y.cpu().float(), torch.from_numpy(ref).to(dtype).float()) <= 1e-3
