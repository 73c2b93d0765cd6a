"""Pins the CPU oracle (oracle/wq8_oracle.c) before it is trusted as the GPU kernels' checker.

Each oracle function is checked against something it does not share code with: libm / numpy in float64, torch's own
dtype conversions, closed forms (the Kronecker rotation of I:579-584), integer brute force, invariants of the quantizers
(K8:269-450), the FP64 dequantize-and-matmul of the reference's definition (I:523-539), and the committed golden
fixture of the plumbing configuration (tests/golden/config1.npz). The reference ships no golden vectors of its own.
"""
import math

import numpy as np
import pytest
import torch

from conftest import bits, from_bits, gemm_exact64

DT_CODE = {torch.float16: 0, torch.bfloat16: 1}


def ulp32(x):
    """Spacing of float32 at |x| (float64 array)."""
    x = np.abs(np.asarray(x, np.float64)).astype(np.float32)
    return np.spacing(x).astype(np.float64)


# ---- element conversions --------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_conversions_match_torch(oracle, dtype):
    g = torch.Generator().manual_seed(1)
    v = torch.cat([torch.randn(20000, generator=g) * 10.0 ** torch.randint(-8, 6, (20000,), generator=g),
                   torch.tensor([0.0, -0.0, 65504.0, 65520.0, 1e6, -1e6, 6e-8, 3e-8, 1e-40, float("inf"), -float("inf")])])
    ours = oracle.to_dtype(v.numpy(), DT_CODE[dtype])
    np.testing.assert_array_equal(ours, bits(v.to(dtype)))
    back = oracle.from_dtype(ours, DT_CODE[dtype])
    np.testing.assert_array_equal(back, v.to(dtype).float().numpy())


# ---- exp / reciprocal / logistic / gelu / swiglu: this build's own functions, pinned by libm in float64 ------------
def test_exp_error_bound(oracle):
    x = np.concatenate([np.linspace(-87.0, 80.0, 400001, dtype=np.float32), np.float32([0.0, -0.0, 1.0, -1.0, 1e-30])])
    got = oracle.exp(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    assert np.all(np.abs(got - ref) <= 2 * ulp32(ref)), "exp beyond 2 ulp"
    assert oracle.exp(np.float32([0.0]))[0] == 1.0


def test_recip_error_bound(oracle):
    rng = np.random.default_rng(5)
    d = np.concatenate([np.linspace(1, 2, 1_000_001, dtype=np.float32), (2.0 ** rng.uniform(0, 116, 1_000_000)).astype(np.float32),
                        np.float32([1.0, 2.0, 3.0, 1.5, 2.0 ** 116])])
    got = oracle.recip(d).astype(np.float64)
    ref = 1.0 / d.astype(np.float64)
    assert np.all(np.abs(got - ref) <= 0.51 * ulp32(ref)), "reciprocal beyond 0.51 ulp"
    assert oracle.recip(np.float32([1.0]))[0] == 1.0


def test_logistic_error_bound(oracle):
    s = np.concatenate([np.linspace(-100, 100, 400001, dtype=np.float32), np.float32([0.0, -80.0, -79.99, 87.0, 200.0, -200.0])])
    got = oracle.logistic(s).astype(np.float64)
    ref = 1.0 / (1.0 + np.exp(-s.astype(np.float64)))
    live = s > -80
    assert np.all(np.abs(got - ref)[live] <= 4 * ulp32(ref[live])), "logistic beyond 4 ulp"
    # from s <= -80 the clamped exponent holds the result at 1 / (1 + e^80): within 2^-115 of the true value
    assert np.all(np.abs(got - ref)[~live] <= 2.0 ** -115) and np.all(got[~live] < 2.0 ** -115)
    assert oracle.logistic(np.float32([0.0]))[0] == 0.5 and oracle.logistic(np.float32([200.0]))[0] == 1.0


def test_div127_three_ops_is_the_ieee_quotient(oracle):
    """The quantizers' scale amax * norm / 127 as q = x RN(1/127), q + fma(-q, 127, x) RN(1/127) (+inf kept): equal to
    the IEEE quotient (checked over every non-negative float up to +inf once; here every pattern of the binades around 1,
    of the denormals' top and of the largest binade with +inf, and every 997th pattern of the rest)."""
    for lo, hi in ((0x3F000000, 0x40000000), (0x00700000, 0x00900000), (0x7F000000, 0x7F800001)):
        assert oracle.check_div127(lo, hi) == 0
    assert oracle.check_div127(0, 0x7F800000, 997) == 0


def test_swiglu_matches_float64_formula(oracle):
    rng = np.random.default_rng(6)
    g = np.concatenate([np.linspace(-90, 90, 200001, dtype=np.float32), rng.standard_normal(200001).astype(np.float32)])
    u = rng.standard_normal(g.size).astype(np.float32)
    got = oracle.swiglu(g, u).astype(np.float64)
    gd, ud = g.astype(np.float64), u.astype(np.float64)
    ref = gd / (1 + np.exp(-gd)) * ud
    # below -80 the logistic stays at 1 / (1 + e^80) < 2^-115 (the true value is smaller still): g * logistic(g) * u then
    # differs by at most |g u| 2^-115
    assert np.all(np.abs(got - ref) <= 8 * ulp32(ref) + np.abs(gd * ud) * 2.0 ** -115)


def test_gelu_matches_float64_formula(oracle):
    x = np.linspace(-20, 20, 400001, dtype=np.float32)
    got = oracle.gelu(x).astype(np.float64)
    xd = x.astype(np.float64)
    ref = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd ** 3)))
    # float32 evaluation of the formula: a few ulp of the result, plus cancellation near 1 + tanh = 0 (x << 0)
    assert np.all(np.abs(got - ref) <= 8 * ulp32(ref) + 4 * np.abs(xd) * 2.0 ** -24)
    # torch's own tanh-GELU evaluates the same formula in FP32: the two agree within the same bound, twice over
    tg = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").double().numpy()
    assert np.all(np.abs(got - tg) <= 16 * ulp32(ref) + 8 * np.abs(xd) * 2.0 ** -24)


# ---- fixed reduction tree and rotation ----------------------------------------------------------------------------
@pytest.mark.parametrize("k", [8, 128, 1536, 5120, 16392])
def test_ss_tree_sum_of_squares(oracle, k):
    v = np.random.default_rng(k).standard_normal(k).astype(np.float32)
    got = oracle.ss_tree(v)
    ref = float(np.sum(v.astype(np.float64) ** 2))
    assert abs(got - ref) <= ref * 2e-6


def test_ss_tree_order_brute_force(oracle):
    """Slot s sums the 8-element chunks s, s + 256, ... (one rounding per element), lanes of a 64-slot wave are combined
    by xor butterflies, the four waves left to right: the order the gfx950 kernels reduce in."""
    k = 4096
    v = (np.random.default_rng(7).standard_normal(k) * 10.0 ** np.random.default_rng(8).integers(-3, 3, k)).astype(np.float32)
    chunks = v.reshape(-1, 8)
    slots = []
    for s in range(256):
        acc = np.float32(0)
        for c in range(s, chunks.shape[0], 256):
            for e in chunks[c]:
                acc = np.float32(np.float64(e) * np.float64(e) + np.float64(acc))  # fmaf: exact product, one rounding
        slots.append(acc)
    slots = np.array(slots, np.float32)
    waves = []
    for w in range(4):
        lane = slots[64 * w:64 * w + 64].copy()
        for d in (32, 16, 8, 4, 2, 1):
            lane = (lane + lane[np.arange(64) ^ d]).astype(np.float32)
        assert np.all(lane == lane[0])
        waves.append(lane[0])
    assert oracle.ss_tree(v) == np.float32(np.float32(np.float32(waves[0] + waves[1]) + waves[2]) + waves[3])


@pytest.mark.parametrize("group", [16, 64, 256])
def test_rotation_closed_form(oracle, group):
    k = 1024
    v = np.random.default_rng(group).standard_normal(k).astype(np.float32)
    h = np.ones((4, 4)) - 2 * np.eye(4)[::-1]
    r = h
    while r.shape[0] < group:
        r = np.kron(r, h)
    ref = (v.astype(np.float64).reshape(-1, group) @ r).reshape(-1)  # unnormalised: sqrt(group) * I:579-584
    got = oracle.rotate_row(v, group).astype(np.float64)
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))
    # H4 @ H4 = 4 I: rotating twice multiplies by the group size
    twice = oracle.rotate_row(oracle.rotate_row(v, group), group).astype(np.float64)
    np.testing.assert_allclose(twice, group * v.astype(np.float64), rtol=0, atol=1e-4 * group * np.max(np.abs(v)))


# ---- quantizers ---------------------------------------------------------------------------------------------------
def _acts_input(m, k, act, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, 2 * k if act == "swiglu" else k, generator=g)
    x[:, :3] *= 40
    x[0, :] = 0 if m > 2 else x[0, :]  # an all-zero row
    x = x.to(dtype)
    aw = (1 + 0.1 * torch.randn(k, generator=g)).to(dtype) if act == "rms_norm" else None
    return x, aw


def _op_f64(x, act, aw, eps):
    v = x.double()
    if act == "swiglu":
        gt, u = v.chunk(2, dim=-1)
        v = gt / (1 + torch.exp(-gt)) * u
    elif act == "gelu":
        v = 0.5 * v * (1 + torch.tanh(math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3)))
    elif act == "rms_norm":
        v = v / torch.sqrt((v * v).mean(-1, keepdim=True) + eps) * aw.double()
    return v


@pytest.mark.parametrize("act", [None, "rms_norm", "swiglu", "gelu"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_transform_rows_matches_float64_op(oracle, act, dtype):
    """op(x) rounded once to the dtype: equal to the float64 op rounded to the dtype, except at a rounding boundary."""
    x, aw = _acts_input(6, 512, act, dtype, 3)
    got = from_bits(oracle.transform_rows(bits(x), DT_CODE[dtype], 0, act, None if aw is None else bits(aw), 1e-6), dtype).double()
    ref = _op_f64(x, act, aw, 1e-6)
    near = ref.to(dtype).double()
    off = got != near
    assert off.float().mean() < 0.01
    # where they differ, the FP32 evaluation sits within a few FP32 ulp of the float64 value: one dtype ulp at most
    step = (near.abs() * (2 ** -7 if dtype == torch.bfloat16 else 2 ** -10)).clamp_min(1e-30)
    assert torch.all((got - ref).abs()[off] <= step[off])


@pytest.mark.parametrize("group", [0, 16, 256])
@pytest.mark.parametrize("act", [None, "rms_norm", "swiglu", "gelu"])
def test_quantize_blocks_invariants(oracle, group, act):
    m, k = 5, 1536 + 16 * (group == 0)  # a ragged last block where the rotation allows it
    x, aw = _acts_input(m, k, act, torch.bfloat16, 11)
    q, sa = oracle.quantize_blocks(bits(x), 1, group, act, None if aw is None else bits(aw), 1e-6)
    assert q.shape == (m, k) and sa.shape == (m, (k + 127) // 128)
    assert np.abs(q.astype(np.int32)).max() <= 127
    kb = sa.shape[1]
    v = _op_f64(x, act, aw, 1e-6).numpy()
    if group:
        h = np.ones((4, 4)) - 2 * np.eye(4)[::-1]
        r = h
        while r.shape[0] < group:
            r = np.kron(r, h)
        v = (v.reshape(m, -1, group) @ (r / math.sqrt(group))).reshape(m, k)
    for r_ in range(m):
        for b in range(kb):
            blk = slice(128 * b, min(128 * b + 128, k))
            qb = q[r_, blk].astype(np.float64)
            if sa[r_, b] == 0:
                assert np.all(qb == 0)
                continue
            assert np.abs(qb).max() == 127
            # dequantized values reconstruct op(x) within half a step (plus the FP32 error of evaluating op)
            step = float(sa[r_, b])
            err = np.abs(qb * step - v[r_, blk])
            assert np.all(err <= 0.5 * step * (1 + 1e-4) + 1e-5 * np.abs(v[r_, blk]).max()), (r_, b, err.max() / step)
    if m > 2:
        assert np.all(sa[0] == 0) and np.all(q[0] == 0)


def test_quantize_blocks_numpy_restatement(oracle):
    """act None, group 0: amax per block, inv = 127 / amax, q = round-half-even(v * inv), scale = amax / 127, all float32."""
    x = (torch.randn(7, 1040, generator=torch.Generator().manual_seed(2)) * 3).to(torch.bfloat16)
    q, sa = oracle.quantize_blocks(bits(x), 1)
    v = x.float().numpy()
    for b in range(sa.shape[1]):
        vb = v[:, 128 * b:128 * b + 128]
        amax = np.abs(vb).max(axis=1).astype(np.float32)
        inv = np.where(amax > 0, np.float32(127) / amax, np.float32(0)).astype(np.float32)
        np.testing.assert_array_equal(sa[:, b], (amax / np.float32(127)).astype(np.float32))
        np.testing.assert_array_equal(q[:, 128 * b:128 * b + 128], np.rint((vb * inv[:, None]).astype(np.float32)).astype(np.int8))


@pytest.mark.parametrize("act", [None, "rms_norm", "gelu"])
def test_quantize_hilo_invariants(oracle, act):
    m, k = 4, 2048
    x, aw = _acts_input(m, k, act, torch.bfloat16, 5)
    hi, lo, sa = oracle.quantize(bits(x), 1, 0, True, act, None if aw is None else bits(aw), 1e-6)
    assert np.abs(hi.astype(int)).max() <= 127 and np.abs(lo.astype(int)).max() <= 127
    v = _op_f64(x, act, aw, 1e-6).numpy()
    for r in range(m):
        if sa[r] == 0:
            assert not hi[r].any() and not lo[r].any()
            continue
        assert np.abs(hi[r].astype(int)).max() == 127
        t = v[r] / float(sa[r])  # v * 127 / amax
        recon = hi[r] + lo[r] / 254.0
        assert np.all(np.abs(recon - t) <= 1 / 508 + 1e-5 * np.abs(t).max())
    hi2, lo2, sa2 = oracle.quantize(bits(x), 1, 0, False, act, None if aw is None else bits(aw), 1e-6)
    assert lo2 is None
    np.testing.assert_array_equal(hi2, hi)
    np.testing.assert_array_equal(sa2, sa)


def test_quantize_rejects_bad_arguments(oracle):
    x = np.zeros((2, 100), np.uint16)
    with pytest.raises(RuntimeError):
        oracle.quantize_blocks(x, 1)  # K not a multiple of 8
    with pytest.raises(RuntimeError):
        oracle.quantize_blocks(np.zeros((2, 96), np.uint16), 1, group=64)  # K not a multiple of the group


# ---- block sums and GEMM epilogue ----------------------------------------------------------------------------------
@pytest.mark.parametrize("m,n,k", [(3, 5, 128), (7, 9, 700 - 700 % 16), (4, 6, 1040)])
def test_block_sums_brute_force(oracle, m, n, k):
    rng = np.random.default_rng(m * n)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (n, k), dtype=np.int8)
    got = oracle.block_sums(a, b)
    for blk in range((k + 127) // 128):
        sl = slice(128 * blk, min(128 * blk + 128, k))
        np.testing.assert_array_equal(got[:, :, blk], a[:, sl].astype(np.int64) @ b[:, sl].astype(np.int64).T)
    # extremes: the largest block sum is exact
    a = np.full((1, 128), -127, np.int8)
    b = np.full((1, 128), -127, np.int8)
    assert oracle.block_sums(a, b)[0, 0, 0] == 128 * 127 * 127


def _gemm_operands(m, n, k, seed, groups=False):
    rng = np.random.default_rng(seed)
    kb = (k + 127) // 128
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    lo = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (n, k), dtype=np.int8)
    sa_row = (rng.random(m) / 127).astype(np.float32)
    sa_blk = (rng.random((m, kb)) / 127).astype(np.float32)
    sb = ((rng.random((n, kb)) if groups else rng.random(n)) / 127 + 1e-4).astype(np.float32)
    bias = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(torch.bfloat16)
    res = torch.from_numpy(rng.standard_normal((m, n)).astype(np.float32)).to(torch.bfloat16)
    rs = torch.from_numpy(rng.random(n).astype(np.float32)).to(torch.bfloat16)
    return a, lo, b, sa_row, sa_blk, sb, bias, res, rs


def _bf16(y):
    return from_bits(y, torch.bfloat16).double()


@pytest.mark.parametrize("mode", ["row", "exact", "block", "block_biased"])
@pytest.mark.parametrize("residual", [False, True])
def test_gemm_modes_vs_float64(oracle, mode, residual):
    m, n, k = 9, 33, 1040
    a, lo, b, sa_row, sa_blk, sb, bias, res, rs = _gemm_operands(m, n, k, 4)
    kb = (k + 127) // 128
    sa = sa_blk if mode.startswith("block") else sa_row
    y = oracle.gemm(a, lo if mode == "exact" else None, sa, b, sb, bits(bias), 1, mode,
                    bits(res) if residual else None, bits(rs) if residual else None)
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    if mode == "exact":
        a64 = a64 + lo / 254.0
    if mode.startswith("block"):
        ref = sum((a64[:, 128 * i:128 * i + 128] * sa_blk[:, i:i + 1]) @ b64[:, 128 * i:128 * i + 128].T for i in range(kb))
    else:
        ref = (a64 * sa_row[:, None]) @ b64.T
    ref = ref * sb[None, :] + bias.double().numpy()[None, :]
    if residual:
        ref = res.double().numpy() + rs.double().numpy()[None, :] * ref
    got = _bf16(y).numpy()
    # one BF16 rounding of the output (2^-9 relative) plus FP32 accumulation error
    bound = 2 ** -8 * np.abs(ref) + 1e-5 * np.abs(ref).max()
    if mode == "block_biased":
        # the biased fold accumulates 1.5 * 2^23 * sa next to the sums: each of its kb FMAs rounds at the scale of that
        # running bias, removed exactly at the end (corr), so the absolute error is kb roundings of it
        corr = 12582912.0 * sa_blk.astype(np.float64).sum(axis=1)
        extra = 2 * kb * ulp32(corr)[:, None] * sb[None, :]
        bound = bound + (extra * rs.double().numpy()[None, :] if residual else extra)
    assert np.all(np.abs(got - ref) <= bound)


def test_gemm_biased_fold_close_to_reference_order(oracle):
    m, n, k = 6, 40, 5120
    a, _, b, _, sa_blk, sb, bias, _, _ = _gemm_operands(m, n, k, 9)
    y0 = _bf16(oracle.gemm(a, None, sa_blk, b, sb, bits(bias), 1, "block"))
    y3 = _bf16(oracle.gemm(a, None, sa_blk, b, sb, bits(bias), 1, "block_biased"))
    assert ((y0 - y3).norm() / y0.norm()).item() < 2e-3


@pytest.mark.parametrize("mode", ["block", "exact", "exact_combined"])
def test_gemm_group_scales_vs_float64(oracle, mode):
    m, n, k = 5, 24, 1024
    a, lo, b, _, sa_blk, sbg, bias, _, _ = _gemm_operands(m, n, k, 6, groups=True)
    sa_row = (np.random.default_rng(1).random(m) / 127).astype(np.float32)
    sa = sa_blk if mode == "block" else sa_row
    hilo = mode.startswith("exact")
    y = _bf16(oracle.gemm(a, lo if hilo else None, sa, b, sbg, bits(bias), 1, mode)).numpy()
    a64 = a.astype(np.float64) + (lo / 254.0 if hilo else 0)
    ref = np.zeros((m, n))
    for i in range(k // 128):
        sl = slice(128 * i, 128 * i + 128)
        rows = sa_blk[:, i:i + 1] if mode == "block" else sa_row[:, None]
        ref += (a64[:, sl] * rows) @ (b[:, sl].astype(np.float64) * sbg[:, i:i + 1]).T
    ref += bias.double().numpy()[None, :]
    assert np.all(np.abs(y - ref) <= 2 ** -8 * np.abs(ref) + 1e-5 * np.abs(ref).max())


def test_exact_combined_fold_close_to_reference_order(oracle):
    """The integer-combined exact+g fold (254 H + L, scaled by sb / 254) differs from the reference's
    fmaf(L, 1/254, H) order only by FP32 rounding; with extreme block sums the combination stays exact in INT32."""
    m, n, k = 4, 48, 3072
    a, lo, b, _, _, sbg, bias, _, _ = _gemm_operands(m, n, k, 10, groups=True)
    sa_row = (np.random.default_rng(2).random(m) / 127).astype(np.float32)
    y0 = oracle.gemm(a, lo, sa_row, b, sbg, bits(bias), 1, "exact")
    y4 = oracle.gemm(a, lo, sa_row, b, sbg, bits(bias), 1, "exact_combined")
    d = np.abs(_bf16(y0).numpy() - _bf16(y4).numpy())
    assert np.all(d <= 2 ** -7 * np.abs(_bf16(y0).numpy()) + 1e-6)  # at most one BF16 rounding step apart
    # extremes: every product +/-127 * 127 in hi and lo; 254 * 128 * 127 * 127 + 128 * 127 * 127 < 2^31
    hi = np.full((1, 128), -127, np.int8)
    w = np.full((2, 128), 127, np.int8)
    y = oracle.gemm(hi, hi, np.ones(1, np.float32), w, np.ones((2, 1), np.float32), None, 1, "exact_combined")
    expect = -(128 * 127 * 127) * (1 + 1 / 254)
    assert np.allclose(_bf16(y).numpy(), expect, rtol=2 ** -8)


@pytest.mark.parametrize("mode,groups", [("block", False), ("block_biased", False), ("block", True)])
@pytest.mark.parametrize("pieces", [2, 3, 4])
def test_gemm_pieces_exact_when_fp32_is_exact(oracle, mode, groups, pieces):
    """With power-of-two scales and few enough blocks every FP32 fold step is exact, so the split-K order must give the
    unsplit result bit for bit: a block dropped, counted twice or folded into the wrong piece changes it."""
    m, n, k = 7, 19, 1280 + 48  # 11 k-blocks, the last one partial
    kb = (k + 127) // 128
    a, _, b, *_ = _gemm_operands(m, n, k, 20 + pieces)
    # operands that are multiples of 4: |S| < 2^19 and S a multiple of 16, so that every folded value (with the biased
    # fold's 1.5 * 2^23 * 2^-8 per block) is a multiple of 2^-4 below 2^20: exact in FP32
    a, b = (a // 4 * 4).astype(np.int8), (b // 4 * 4).astype(np.int8)
    sa = np.full((m, kb), 2.0 ** -8, np.float32)
    sb = np.full((n, kb) if groups else n, 2.0 ** -6, np.float32)
    args = (a, None, sa, b, sb, None, 1, mode)
    np.testing.assert_array_equal(oracle.gemm(*args, pieces=pieces), oracle.gemm(*args))


@pytest.mark.parametrize("mode,groups", [("block", False), ("block_biased", False), ("block", True), ("exact_combined", True)])
def test_gemm_pieces_vs_float64(oracle, mode, groups):
    """The split-K order against float64, within one BF16 rounding plus the fold's FP32 error (random scales)."""
    m, n, k = 6, 30, 2048
    a, lo, b, sa_row, sa_blk, sb, bias, _, _ = _gemm_operands(m, n, k, 31, groups=groups)
    hilo = mode.startswith("exact")
    sa = sa_row if hilo else sa_blk
    ref = gemm_exact64(a, lo if hilo else None, sa, b, sb, bits(bias), torch.bfloat16, "exact" if hilo else "block")
    for pieces in (2, 4):
        got = _bf16(oracle.gemm(a, lo if hilo else None, sa, b, sb, bits(bias), 1, mode, pieces=pieces)).numpy()
        assert np.all(np.abs(got - ref) <= 2 ** -8 * np.abs(ref) + 2e-5 * np.abs(ref).max())


def test_gemm_pieces_leave_integer_modes_unchanged(oracle):
    m, n, k = 5, 17, 1024
    a, lo, b, sa_row, _, sb, bias, _, _ = _gemm_operands(m, n, k, 40)
    for mode, a_lo in (("row", None), ("exact", lo)):
        np.testing.assert_array_equal(oracle.gemm(a, a_lo, sa_row, b, sb, bits(bias), 1, mode, pieces=4),
                                      oracle.gemm(a, a_lo, sa_row, b, sb, bits(bias), 1, mode))


def test_linear_f64_vs_torch(oracle):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(3, 640, generator=g).to(torch.bfloat16)
    w = torch.randint(-127, 128, (50, 640), generator=g, dtype=torch.int8)
    s = torch.rand(50, generator=g) / 127
    bias = torch.randn(50, generator=g).to(torch.bfloat16)
    res = torch.randn(3, 50, generator=g).to(torch.bfloat16)
    rs = torch.rand(50, generator=g).to(torch.bfloat16)
    got = oracle.linear_f64(bits(x), 1, w.numpy(), s.numpy(), bits(bias), bits(res), bits(rs))
    ref = res.double() + rs.double() * (x.double() @ (w.double() * s.double()[:, None]).T + bias.double())
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-6, atol=1e-6)


# ---- golden fixture of the plumbing configuration ----------------------------------------------------------------
def test_golden_config1(oracle):
    import importlib.util
    from pathlib import Path
    here = Path(__file__).resolve().parent / "golden"
    spec = importlib.util.spec_from_file_location("make_golden", here / "make_golden.py")
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    golden = np.load(here / "config1.npz")
    fresh = gen.outputs(oracle)
    np.testing.assert_array_equal(fresh["lines_y"], golden["lines_y"])
    for key in ("block_q", "block_sa", "block_y"):
        assert bytes(fresh[key + "_sha256"]) == bytes(golden[key + "_sha256"]), key
        np.testing.assert_array_equal(fresh[key + "_head"], golden[key + "_head"])
    # lines math is exact up to FP32 output rounding; the block math's error is the INT8 activation error (8 outliers
    # x 50 flatten their blocks), well inside the reference's selftest tolerance of 3e-2 (I:572-573)
    assert float(golden["lines_rel_err"]) < 1e-6
    assert 5e-3 < float(golden["block_rel_err"]) < 3e-2
