"""GPU parity of the INT8 GEMM (row, exact, block, +g modes; residual epilogue, in place; tails; segments; row offsets)
against the CPU oracle: bit-exact outputs (every mode folds in block order on both sides) and bit-exact INT32 block sums.
"""
import numpy as np
import pytest
import torch

from conftest import DT, bits, from_bits, rel_err

pytestmark = pytest.mark.gpu

VARIANTS = {"row": (0, 6), "exact": (1, 7), "block": (10, 11, 15), "block+g": (12, 13), "exact+g": (14,)}


def operands(m, n, k, seed, groups=False, hilo=False, block=False, dtype=torch.bfloat16, residual=False):
    g = torch.Generator().manual_seed(seed)
    kb = (k + 127) // 128
    a = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8)
    a_lo = torch.randint(-127, 128, (m, k), generator=g, dtype=torch.int8) if hilo else None
    sa = (torch.rand(m, kb, generator=g) + 0.5) / 127 if block else (torch.rand(m, generator=g) + 0.5) / 127
    b = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    sb = (torch.rand(n, kb, generator=g) + 0.5) / 127 if groups else (torch.rand(n, generator=g) + 0.5) / 127
    bias = (0.02 * torch.randn(n, generator=g)).to(dtype)
    res = torch.randn(m, n, generator=g).to(dtype) if residual else None
    rs = torch.full((n,), 0.5).to(dtype) if residual else None
    return a, a_lo, sa, b, sb, bias, res, rs


# variants whose block fold is the wide kernel's single-FMA form (oracle mode 'block_biased'); the others fold in the
# reference's order
BIASED = {10, 15}


def check_gemm(got, ref_bits):
    """Bit-exact against the oracle's order for the variant."""
    got = bits(got)
    if not np.array_equal(got, ref_bits):
        diff = np.nonzero(got != ref_bits)
        raise AssertionError(f"{len(diff[0])} of {got.size} outputs differ; first at {diff[0][0]},{diff[1][0]}: "
                             f"got {got[diff[0][0], diff[1][0]]:#06x} ref {ref_bits[diff[0][0], diff[1][0]]:#06x}")


def run_case(wq, oracle, mode, variant, m, n, k, seed, dtype=torch.bfloat16, residual=False, in_place=False, bias=True):
    groups = mode.endswith("+g")
    base = mode.removesuffix("+g")
    oracle_mode = "block_biased" if base == "block" and not groups and variant in BIASED else base
    if groups and base == "exact":
        oracle_mode = "exact_combined"  # the exact+g kernel combines the hi / lo block sums in INT32
    a, a_lo, sa, b, sb, bs, res, rs = operands(m, n, k, seed, groups, base == "exact", base == "block", dtype, residual)
    if not bias:
        bs = None
    print(f"gemm mode={mode} variant={variant} m={m} n={n} k={k} dtype={dtype} residual={residual} in_place={in_place}", flush=True)
    cu = lambda t: None if t is None else t.cuda()
    out = cu(res).clone() if in_place else None
    y = wq.gemm(cu(a), cu(a_lo), cu(sa), cu(b), cu(sb), cu(bs), dtype, 0, variant, out=out, residual=out if in_place else cu(res),
                residual_scale=cu(rs))
    torch.cuda.synchronize()
    ref = oracle.gemm(a.numpy(), None if a_lo is None else a_lo.numpy(), sa.numpy(), b.numpy(), sb.numpy(), None if bs is None else bits(bs),
                      DT[dtype], oracle_mode, None if res is None else bits(res), None if rs is None else bits(rs))
    check_gemm(y, ref)


@pytest.mark.parametrize("mode", list(VARIANTS))
def test_modes_bit_exact(wq, oracle, mode):
    for variant in VARIANTS[mode]:
        run_case(wq, oracle, mode, variant, 200, 264, 640, seed=variant)


@pytest.mark.parametrize("mode", list(VARIANTS))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_residual_in_place(wq, oracle, mode, dtype):
    run_case(wq, oracle, mode, VARIANTS[mode][0], 96, 160, 384, seed=5, dtype=dtype, residual=True, in_place=True)
    run_case(wq, oracle, mode, VARIANTS[mode][-1], 33, 96, 256, seed=6, dtype=dtype, residual=True, in_place=False, bias=False)


@pytest.mark.parametrize("shape", ((1, 8, 16), (31, 33, 48), (129, 130, 144), (257, 12, 1040), (5, 1000, 5120)))
def test_tails(wq, oracle, shape):
    """M, N not multiples of the tile, K not a multiple of 128 (a partial scale block), N odd."""
    m, n, k = shape
    for mode in ("row", "block", "exact", "exact+g"):
        for variant in VARIANTS[mode]:
            run_case(wq, oracle, mode, variant, m, n, k, seed=m + n + k)


@pytest.mark.parametrize("cus", (256, 1))
def test_exact_long_tiles(wq, oracle, monkeypatch, cus):
    """The long exact tile is 128 x 192 or 128 x 256, whichever leaves its last wave of workgroups fuller: at N = 512
    with one CU counted, 128 x 256 (2 tiles a row of tiles against 3); with 256 CUs, 128 x 192. Both bit-exact, with the
    residual epilogue in place."""
    from wgpkernels_amd.int8 import _native
    monkeypatch.setattr(_native.gpu(torch.device("cuda")), "cus", cus)
    run_case(wq, oracle, "exact", 1, 200, 512, 640, seed=cus)
    run_case(wq, oracle, "exact", 1, 130, 512, 1040, seed=cus + 1, residual=True, in_place=True)


@pytest.mark.parametrize("kernel", [0, 1], ids=["ring", "pingpong_block"])
@pytest.mark.parametrize("shape", [(70, 100, 704), (300, 400, 1536 + 48)])
def test_block_sums_bit_exact(wq, oracle, kernel, shape):
    """The exact INT32 sums of each 128-element K block, as a GEMM mainloop computes them: the ring kernel's, and the
    ping-pong kernel that runs the long block tiles (the headline GEMM: biased chains, sums read off their start)."""
    from wgpkernels_amd.int8 import _native
    m, n, k = shape
    a, _, _, b, *_ = operands(m, n, k, seed=17 + kernel)
    a[:, :128] = -127  # the extreme block sums, +-128 * 127^2
    b[: n // 2, :128] = -127
    b[n // 2:, :128] = 127
    sums = torch.empty(m, n, (k + 127) // 128, dtype=torch.int32, device="cuda")
    test_lib = _native.load_test_library()
    ac, bc = a.cuda(), b.cuda()
    print(f"block sums kernel={kernel} m={m} n={n} k={k}", flush=True)
    assert test_lib.wq8_debug_block_sums(ac.data_ptr(), bc.data_ptr(), sums.data_ptr(), m, n, k, kernel,
                                         torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(sums.cpu().numpy(), oracle.block_sums(a.numpy(), b.numpy()))


def test_segments(wq, oracle, whole_tiles):
    """linear_prepared_segments: 3 weights (fused QKV) in one launch equal 3 separate GEMMs (whole tiles in both, as
    the segments entry point runs them)."""
    torch.manual_seed(0)
    x = torch.randn(80, 512, dtype=torch.bfloat16, device="cuda")
    ws = [torch.randint(-127, 128, (96, 512), dtype=torch.int8, device="cuda") for _ in range(3)]
    ss = [torch.rand(96, device="cuda") / 127 for _ in range(3)]
    bs = [torch.randn(96, dtype=torch.bfloat16, device="cuda"), None, torch.randn(96, dtype=torch.bfloat16, device="cuda")]
    for path in ("exact", "block", "row"):
        p = wq.prepare(x, path=path)
        outs = [torch.empty(80, 96, dtype=torch.bfloat16, device="cuda") for _ in range(3)]
        wq.linear_prepared_segments(p, ws, ss, bs, outs)
        for w, s, bvec, o in zip(ws, ss, bs, outs):
            ref = wq.linear_prepared(p, w, s, bvec)
            torch.testing.assert_close(o, ref, rtol=0, atol=0)


def test_block_path_error_vs_reference_definition(wq, oracle):
    """The block path's error against the FP32 dequantize-and-matmul of the unquantized input equals the error of the
    reference's block math (CPU oracle) -- ratio 1.0 here since the outputs are bit-identical; bound 1.05."""
    g = torch.Generator().manual_seed(0)
    m, n, k = 256, 512, 1536
    x = torch.randn(m, k, generator=g)
    x[:, torch.randperm(k, generator=g)[:8]] *= 50
    x = x.bfloat16()
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    s = (torch.rand(n, generator=g) + 0.5) / 127
    bias = (0.02 * torch.randn(n, generator=g)).bfloat16()
    y = wq.linear(x.cuda(), w.cuda(), s.cuda(), bias.cuda(), mode="block").cpu()
    q, sa = oracle.quantize_blocks(bits(x), 1)
    y_cpu = from_bits(oracle.gemm(q, None, sa, w.numpy(), s.numpy(), bits(bias), 1, "block"), torch.bfloat16)
    ref = x.float() @ (w.float() * s[:, None]).T + bias.float()
    e_gpu, e_cpu = rel_err(y.float(), ref), rel_err(y_cpu.float(), ref)
    print(f"block error gpu {e_gpu:.3e} cpu-reference-math {e_cpu:.3e}")
    assert e_gpu <= 1.05 * e_cpu
    # every block variant: the biased fold of the long and short tiles and the reference-order fold of the short tile
    for variant in (10, 11, 15):
        qg, sag = wq.quantize_blocks(x.cuda())
        yv = wq.gemm(qg, None, sag, w.cuda(), s.cuda(), bias.cuda(), torch.bfloat16, 0, variant).cpu()
        assert rel_err(yv.float(), ref) <= 1.05 * e_cpu


def test_block_channel_split(wq, oracle, monkeypatch):
    """When the last wave of 256 x 192 block workgroups would be at most half full, the long biased block tiles run in
    two launches: 256 x 192 tiles over the first channels (a whole number of waves) and 256 x 128 tiles over the rest.
    With 4 CUs counted, M = 512 and N = 5120 split at channel 4608 (12 + 2 waves instead of 13.5 in 14); K tails and the
    residual epilogue in place included. With 16 CUs counted, M = 256 and N = 1280 run as 256 x 128 tiles only (10 tiles
    in one wave instead of 7 wider ones). Bit-exact against the oracle, as without the split."""
    from wgpkernels_amd.int8 import _native
    monkeypatch.setattr(_native.gpu(torch.device("cuda")), "cus", 4)
    run_case(wq, oracle, "block", 10, 512, 5120, 640, seed=71, residual=True, in_place=True)
    run_case(wq, oracle, "block", 10, 300, 5120, 1040, seed=72, dtype=torch.float16)
    monkeypatch.setattr(_native.gpu(torch.device("cuda")), "cus", 16)
    run_case(wq, oracle, "block", 10, 256, 1280, 640, seed=73, residual=True)
    run_case(wq, oracle, "block", 10, 200, 1280, 1040, seed=74, dtype=torch.float16)


def test_block_channel_split_segments(wq, monkeypatch):
    """The channel split also serves the segments entry point (fused weights): two 2560-row weights (N = 5120) on the long
    biased tile (variant 10) with 4 CUs counted split at channel 4608, inside the second weight; each output equals the
    same variant's GEMM of its weight alone (with all CUs counted: one launch)."""
    from wgpkernels_amd.int8 import _native
    torch.manual_seed(3)
    x = torch.randn(512, 640, dtype=torch.bfloat16, device="cuda")
    ws = [torch.randint(-127, 128, (2560, 640), dtype=torch.int8, device="cuda") for _ in range(2)]
    ss = [torch.rand(2560, device="cuda") / 127 for _ in range(2)]
    bs = [torch.randn(2560, dtype=torch.bfloat16, device="cuda"), None]
    p = wq.prepare(x, path="block")
    refs = [wq.gemm(p.x, None, p.scale, w, s, b, torch.bfloat16, 0, 10) for w, s, b in zip(ws, ss, bs)]  # no split
    monkeypatch.setattr(_native.gpu(torch.device("cuda")), "cus", 4)
    import ctypes
    sizes = (ctypes.c_int64 * 2)()
    wq.library().wq8_gemm_workspace(512, 5120, 640, 10, 4, 0, sizes)
    monkeypatch.setattr(wq, "_plans", {("block", 512, 5120, 640, 0): (10, 0, sizes[0], sizes[1])})  # the long biased tile
    outs = [torch.empty(512, 2560, dtype=torch.bfloat16, device="cuda") for _ in range(2)]
    wq.linear_prepared_segments(p, ws, ss, bs, outs)
    torch.cuda.synchronize()
    for o, r in zip(outs, refs):
        torch.testing.assert_close(o, r, rtol=0, atol=0)
