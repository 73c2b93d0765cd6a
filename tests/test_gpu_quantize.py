"""GPU parity of activation preparation: the gfx950 quantizers against the CPU oracle, bit for bit.

quantize_blocks (block path: INT8 codes and per-128-block FP32 scales), quantize (row / exact paths: hi, lo, row
scales), transform_rows and rotate_groups (few-token prologue, rounded once) -- every input operation, ConvRot group
and dtype, the reference's edge cases (zero rows, outlier channels, K not a multiple of 128, swiglu width 2K, long
rows read twice), at sizes the oracle finishes in seconds.
"""
import numpy as np
import pytest
import torch

from conftest import DT, bits

pytestmark = pytest.mark.gpu

GROUPS = (0, 16, 64, 256)
ACTS = (None, "rms_norm", "swiglu", "gelu")


def make_x(m, k, dtype, act, seed, outliers=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    width = 2 * k if act == "swiglu" else k
    x = torch.randn(m, width, generator=g) * scale
    if outliers:
        cols = torch.randperm(width, generator=g)[:outliers]
        x[:, cols] *= 50
    if m > 2:
        x[1] = 0  # an all-zero row: scale 0, codes 0
    return x.to(dtype)


def make_w(k, dtype, seed):
    g = torch.Generator().manual_seed(seed + 1)
    return (1 + 0.1 * torch.randn(k, generator=g)).to(dtype)


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("group", GROUPS)
def test_quantize_blocks_bit_exact(wq, oracle, dtype, act, group):
    m, k = 37, 1280 if group != 256 else 1536
    x = make_x(m, k, dtype, act, seed=group + 7, outliers=8)
    aw = make_w(k, dtype, 3) if act == "rms_norm" else None
    print(f"quantize_blocks dtype={dtype} act={act} group={group} m={m} k={k}", flush=True)
    q, s = wq.quantize_blocks(x.cuda(), group, act, None if aw is None else aw.cuda(), 1e-6)
    torch.cuda.synchronize()
    q_ref, s_ref = oracle.quantize_blocks(bits(x), DT[dtype], group, act, None if aw is None else bits(aw), 1e-6)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("k", (8, 136, 2056, 5120, 13824, 16392))
def test_quantize_blocks_widths(wq, oracle, k):
    """K not a multiple of 128 (partial last block), register caches of 1 to 8 chunks, and rows read twice (K > 16384)."""
    m = 9
    x = make_x(m, k, torch.bfloat16, "rms_norm", seed=k, outliers=min(8, k // 8))
    aw = make_w(k, torch.bfloat16, k)
    print(f"quantize_blocks widths k={k}", flush=True)
    q, s = wq.quantize_blocks(x.cuda(), 0, "rms_norm", aw.cuda(), 1e-6)
    torch.cuda.synchronize()
    q_ref, s_ref = oracle.quantize_blocks(bits(x), 1, 0, "rms_norm", bits(aw), 1e-6)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


def test_quantize_blocks_fp32_input(wq, oracle):
    x = make_x(5, 1024, torch.float32, None, seed=11)
    q, s = wq.quantize_blocks(x.cuda(), 64)
    torch.cuda.synchronize()
    q_ref, s_ref = oracle.quantize_blocks(x.numpy(), 2, 64)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("group", (0, 64))
@pytest.mark.parametrize("hilo", (False, True))
def test_quantize_rows_bit_exact(wq, oracle, dtype, act, group, hilo):
    m, k = 21, 2048 + 512
    x = make_x(m, k, dtype, act, seed=31 + group, outliers=20)
    aw = make_w(k, dtype, 5) if act == "rms_norm" else None
    print(f"quantize rows dtype={dtype} act={act} group={group} hilo={hilo}", flush=True)
    hi, lo, s = wq.quantize(x.cuda(), group, hilo, act, None if aw is None else aw.cuda(), 1e-5)
    torch.cuda.synchronize()
    hi_ref, lo_ref, s_ref = oracle.quantize(bits(x), DT[dtype], group, hilo, act, None if aw is None else bits(aw), 1e-5)
    np.testing.assert_array_equal(hi.cpu().numpy(), hi_ref)
    if hilo:
        np.testing.assert_array_equal(lo.cpu().numpy(), lo_ref)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("k", (16392, 24576))
def test_quantize_rows_long(wq, oracle, k):
    x = make_x(3, k, torch.bfloat16, "rms_norm", seed=k)
    aw = make_w(k, torch.bfloat16, 9)
    hi, lo, s = wq.quantize(x.cuda(), 0, True, "rms_norm", aw.cuda(), 1e-6)
    torch.cuda.synchronize()
    hi_ref, lo_ref, s_ref = oracle.quantize(bits(x), 1, 0, True, "rms_norm", bits(aw), 1e-6)
    np.testing.assert_array_equal(hi.cpu().numpy(), hi_ref)
    np.testing.assert_array_equal(lo.cpu().numpy(), lo_ref)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("group", GROUPS)
def test_transform_rows_bit_exact(wq, oracle, dtype, act, group):
    m, k = 5, 5120 if group != 256 else 4096
    x = make_x(m, k, dtype, act, seed=41 + group)
    aw = make_w(k, dtype, 6) if act == "rms_norm" else None
    print(f"transform_rows dtype={dtype} act={act} group={group}", flush=True)
    if act is None and group == 0:
        pytest.skip("identity: prepare() passes x through")
    y = wq.transform_rows(x.cuda(), group, act, None if aw is None else aw.cuda(), 1e-6) if act else wq.rotate_groups(x.cuda(), group)
    torch.cuda.synchronize()
    ref = oracle.transform_rows(bits(x), DT[dtype], group, act, None if aw is None else bits(aw), 1e-6)
    np.testing.assert_array_equal(bits(y), ref)


def test_quantize_blocks_row_stride(wq, oracle):
    """Rows ldx elements apart (a column slice of a wider tensor), as the reference's callers pass."""
    big = make_x(7, 4096, torch.bfloat16, None, seed=3)
    x = big[:, :2048]
    q, s = wq.quantize_blocks(big.cuda()[:, :2048], 0, "gelu")
    torch.cuda.synchronize()
    q_ref, s_ref = oracle.quantize_blocks(bits(x.contiguous()), 1, 0, "gelu")
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)


def test_quantize_blocks_extremes(wq, oracle):
    """Huge and tiny magnitudes (subnormal scales), single-element blocks standing out, negative zeros."""
    k = 1024
    x = torch.zeros(6, k)
    x[0] = torch.linspace(-3e4, 3e4, k)
    x[1, 5] = 1e-30
    x[2] = -0.0
    x[3] = torch.randn(k) * 1e-20
    x[4, ::128] = 65000.0
    x[5] = torch.randn(k)
    for dtype in (torch.bfloat16, torch.float16):
        xd = x.to(dtype)
        q, s = wq.quantize_blocks(xd.cuda())
        torch.cuda.synchronize()
        q_ref, s_ref = oracle.quantize_blocks(bits(xd), DT[dtype])
        np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
        np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16))
@pytest.mark.parametrize("act", ("gelu", "swiglu"))
def test_activation_full_range(wq, oracle, act, dtype):
    """gelu and swiglu on inputs spread densely over [-100, 100], through both ends of the exp clamp and the zero branch
    of the logistic: the results (rounded once to the input dtype) equal the oracle's bit for bit."""
    m, k = 64, 16384
    width = 2 * k if act == "swiglu" else k
    x = torch.linspace(-100, 100, m * width, dtype=torch.float64).reshape(m, width)
    if act == "swiglu":
        x[:, k:] = torch.randn(m, k, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    x = x.to(dtype)
    print(f"activation range act={act} dtype={dtype}", flush=True)
    y = wq.transform_rows(x.cuda(), 0, act, None, 1e-6)
    torch.cuda.synchronize()
    ref = oracle.transform_rows(bits(x), DT[dtype], 0, act, None, 1e-6)
    np.testing.assert_array_equal(bits(y), ref)


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
def test_quantize_blocks_nan_inf(wq, oracle, dtype):
    """NaN and infinite inputs: the block maximum ignores NaNs, a NaN's code is 0, and a block holding an infinity gets
    scale inf and codes 0, as in the oracle (FP32 input NaNs with a nonzero payload included)."""
    m, k = 6, 1024
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(8)).to(dtype)
    x[0, 5] = float("nan")
    x[1, 130] = float("inf")
    x[2, 300] = -float("inf")
    x[3, :128] = float("nan")  # a block of NaNs only: amax 0, scale 0
    if dtype == torch.float32:
        x.view(torch.int32)[4, 17] = 0x7FC000AB  # quiet NaN, payload low byte 0xAB
    print(f"quantize_blocks NaN/inf dtype={dtype}", flush=True)
    q, s = wq.quantize_blocks(x.cuda(), 0, None)
    torch.cuda.synchronize()
    q_ref, s_ref = oracle.quantize_blocks(bits(x), DT[dtype], 0, None)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert q[0, 5] == 0 and torch.isinf(s[1, 1]).item() and (dtype != torch.float32 or q[4, 17] == 0)


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float32))
def test_quantize_rows_nan_inf(wq, oracle, dtype):
    """The row quantizer (hi / lo) on NaN and infinite inputs: NaNs are ignored by the row maximum and get codes 0, a row
    holding an infinity gets scale inf and codes 0, as in the oracle."""
    m, k = 4, 1536
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(9)).to(dtype)
    x[0, 7] = float("nan")
    x[1, 900] = float("inf")
    x[2] = float("nan")
    print(f"quantize rows NaN/inf dtype={dtype}", flush=True)
    hi, lo, s = wq.quantize(x.cuda(), 0, True, None, None, 0.0)
    torch.cuda.synchronize()
    hi_ref, lo_ref, s_ref = oracle.quantize(bits(x), DT[dtype], 0, True, None, None, 0.0)
    np.testing.assert_array_equal(hi.cpu().numpy(), hi_ref)
    np.testing.assert_array_equal(lo.cpu().numpy(), lo_ref)
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert hi[0, 7] == 0 and lo[0, 7] == 0 and torch.isinf(s[1]).item() and int(hi[1].abs().max()) == 0
