"""GPU parity of the few-token paths (lines: 1-4 tokens; small: up to 32) against the FP32 reference of the T-rounded
prepared input (FP64-accumulated CPU oracle), norm-relative error <= 1e-3 (the north star's bound); the reference's own
selftest bound is 5e-3. Also: residual in place, odd N, K tails (K % 16 != 0 for lines), FP16.
"""
import numpy as np
import pytest
import torch

from conftest import DT, bits, from_bits, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-3


def case(m, n, k, seed, dtype=torch.bfloat16, residual=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).to(dtype)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    s = (torch.rand(n, generator=g) + 0.5) / 127
    bias = (0.02 * torch.randn(n, generator=g)).to(dtype)
    res = torch.randn(m, n, generator=g).to(dtype) if residual else None
    rs = torch.rand(n, generator=g).to(dtype) if residual else None
    return x, w, s, bias, res, rs


def check(wq, oracle, fn, m, n, k, seed, dtype=torch.bfloat16, residual=False, in_place=False):
    x, w, s, bias, res, rs = case(m, n, k, seed, dtype, residual)
    print(f"{fn} m={m} n={n} k={k} dtype={dtype} residual={residual} in_place={in_place}", flush=True)
    cu = lambda t: None if t is None else t.cuda()
    out = cu(res).clone() if in_place else None
    y = getattr(wq, fn)(x.cuda(), w.cuda(), s.cuda(), bias.cuda(), out if in_place else cu(res), cu(rs), out)
    torch.cuda.synchronize()
    ref = oracle.linear_f64(bits(x), DT[dtype], w.numpy(), s.numpy(), bits(bias), None if res is None else bits(res),
                            None if rs is None else bits(rs))
    ref_t = torch.from_numpy(ref).to(dtype).float()  # the FP32 reference rounded to the output dtype
    err = rel_err(y.cpu().float(), ref_t)
    err_unrounded = rel_err(y.cpu().float(), torch.from_numpy(ref))
    print(f"  rel err vs T-rounded ref {err:.3e}, vs unrounded {err_unrounded:.3e}")
    assert err <= TOL


@pytest.mark.parametrize("m", (1, 2, 3, 4))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_lines(wq, oracle, m, dtype):
    check(wq, oracle, "gemv_lines", m, 520, 5120, seed=m, dtype=dtype)
    check(wq, oracle, "gemv_lines", m, 37, 13824, seed=m + 10, dtype=dtype, residual=True, in_place=True)
    check(wq, oracle, "gemv_lines", m, 64, 1028, seed=m + 20, dtype=dtype, residual=True)  # K % 16 == 4


@pytest.mark.parametrize("m", (1, 3, 4, 5, 8, 16, 17, 32))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_small(wq, oracle, m, dtype):
    """M <= 4 runs the kernel that stages 4 token rows (fragment rows past 4 wrap; rows past M read zeros), M <= 16 one
    16-token tile, M > 16 two."""
    check(wq, oracle, "small", m, 520, 5120, seed=m, dtype=dtype)
    check(wq, oracle, "small", m, 200, 13824, seed=m + 30, dtype=dtype, residual=True, in_place=True)
    check(wq, oracle, "small", m, 1000, 64, seed=m + 40, dtype=dtype)  # a single 64-element step


@pytest.mark.parametrize("m", (1, 5, 16, 17, 32))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_small_row_balanced(wq, oracle, monkeypatch, m, dtype):
    """Above 32 weight rows per CU small runs the row-balanced kernel: one workgroup per CU, an equal share of the
    channels over the whole of K. The CU count is forced low so that modest shapes take it: shares of 33-38 rows, more
    than 64 rows per CU (at M > 16: two rounds of 8 workgroups of at most 64 rows; at M <= 16 the split form), K of one
    64-element step and K % 256 != 0, odd N, the residual epilogue in place. (Config 2's N = 13824 takes it at the real
    CU count.)"""
    from wgpkernels_amd.int8 import _native
    monkeypatch.setattr(_native.gpu(torch.device("cuda")), "cus", 8)
    check(wq, oracle, "small", m, 300, 64 * 67, seed=m + 60, dtype=dtype)
    check(wq, oracle, "small", m, 1001, 320, seed=m + 70, dtype=dtype, residual=True, in_place=True)
    check(wq, oracle, "small", m, 264, 64, seed=m + 80, dtype=dtype, residual=True)


@pytest.mark.parametrize("m", (5, 17, 32))
def test_small_row_balanced_k_split(wq, oracle, m):
    """Weights of 48 MiB or more with fewer than 33 rows per CU (N = 5120, K = 13824 on 256 CUs) run the row-balanced
    kernel over K splits (3 here, shares of 60 rows) whose FP32 partials are added in order by the reduction kernel; the
    residual epilogue in place. K = 13888 ends the last split in a partial chunk of 256 (64 of its elements)."""
    check(wq, oracle, "small", m, 5120, 13824, seed=m + 90, residual=True, in_place=True)
    check(wq, oracle, "small", m, 5120, 13888, seed=m + 95)


def test_fewtoken_dispatch_edges(wq, oracle):
    """Shapes at the edges of the few-token dispatch: one token with two rows per wave and an odd last row (N >= 8192),
    one token past the staged kernel's 16 KiB rows (looped kernel), 3-4 tokens through the LDS-staged kernel with two
    rows per wave, and small with a prime number of 64-element steps
    (67: splits of one step), N not a multiple of 4 (partial stores of the split partials) and a single split."""
    check(wq, oracle, "gemv_lines", 1, 8193, 1040, seed=51)
    check(wq, oracle, "gemv_lines", 1, 300, 17408, seed=52, residual=True)
    check(wq, oracle, "gemv_lines", 2, 8193, 1040, seed=53)
    check(wq, oracle, "gemv_lines", 3, 8193, 5120, seed=57, residual=True)  # staged activations, two rows per wave
    check(wq, oracle, "gemv_lines", 4, 9000, 8192, seed=58)  # 4 tokens at the staged kernel's longest rows
    check(wq, oracle, "small", 16, 300, 64 * 67, seed=54)
    check(wq, oracle, "small", 32, 37, 5120, seed=55, residual=True, in_place=True)
    check(wq, oracle, "small", 9, 8200, 128, seed=56)


@pytest.mark.parametrize("m", (3, 4))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_quads(wq, oracle, m, dtype):
    """3-4 tokens with K % 16 == 0 run the persistent matrix-core kernel: 2 quads x 4 k ranges per workgroup up to 32
    chunks of 256 k, 1 x 8 beyond (NL chunks per range from 1 to 8). Covers a last chunk holding 16 of its 256 k, a
    last quad with 1-3 rows (N < 4 included), more quad groups than workgroups (the loop's both buffers, an odd and an even count),
    and one chunk."""
    check(wq, oracle, "gemv_lines", m, 8200, 1040, seed=60 + m, dtype=dtype)          # 2 x 4, NL 2, 1025 groups
    check(wq, oracle, "gemv_lines", m, 4097, 8192, seed=62 + m, dtype=dtype, residual=True)  # 2 x 4, NL 8
    check(wq, oracle, "gemv_lines", m, 1026, 8208, seed=64 + m, dtype=dtype)          # 1 x 8, NL 5, partial chunk
    check(wq, oracle, "gemv_lines", m, 2050, 16384, seed=66 + m, dtype=dtype, residual=True, in_place=True)  # 1 x 8, NL 8
    check(wq, oracle, "gemv_lines", m, 99, 16, seed=68 + m, dtype=dtype)              # one chunk
    check(wq, oracle, "gemv_lines", m, 3, 512, seed=72 + m, dtype=dtype, residual=True)  # one partial quad


def test_quads_strided_rows(wq, oracle):
    """Token rows with a stride past K (a column slice of a wider tensor) and zero rows past M read as zeros."""
    m, n, k = 3, 700, 2560
    x, w, s, bias, _, _ = case(m, n, k, seed=70)
    wide = torch.randn(m, k + 512).to(torch.bfloat16)
    wide[:, :k] = x
    y = wq.gemv_lines(wide.cuda()[:, :k], w.cuda(), s.cuda(), bias.cuda())
    torch.cuda.synchronize()
    ref = oracle.linear_f64(bits(x), DT[torch.bfloat16], w.numpy(), s.numpy(), bits(bias), None, None)
    assert rel_err(y.cpu().float(), torch.from_numpy(ref).to(torch.bfloat16).float()) <= TOL


def test_small_repeated_counters_left_zero(wq, oracle):
    """Many calls in a row stay correct (the split partials are rewritten by every call; the counters stay zero)."""
    for i in range(5):
        check(wq, oracle, "small", 16, 4096, 5120, seed=100 + i)
    from wgpkernels_amd.int8 import _native
    assert _native.gpu(torch.device("cuda", 0)).counters.abs().sum().item() == 0


def test_selftest(wq):
    assert wq.selftest() is None
