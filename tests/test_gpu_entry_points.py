"""GPU parity of the graph-loop entry points (wq8_quantize_at, wq8_quantize_blocks_at, wq8_gemm_at; the reference's
int8_gemm.cu:1396, :1926, :1637) and of inputs whose row pitch is not their width, against the CPU oracle.

The *_at entry points read their row offset from an int64 on the GPU (`counter`), so that a captured graph can be
replayed over consecutive chunks of a long input: input rows in_first + counter * in_step, output / residual rows
first + counter * step, residual scales of row t from row (shift + t) / span * scale_step of a (spans, N) table.
"""
import numpy as np
import pytest
import torch

from conftest import DT, bits, rel_err
from test_gpu_gemm import BIASED

pytestmark = pytest.mark.gpu
BF16 = DT[torch.bfloat16]


def stream():
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("act", (None, "rms_norm", "gelu", "swiglu"))
def test_quantize_at_entry_points(wq, oracle, act):
    """Both quantizers read rows first + counter * step; their outputs equal the oracle on those rows, bit for bit."""
    m, k, total = 24, 640, 200
    width = 2 * k if act == "swiglu" else k
    g = torch.Generator().manual_seed(11)
    x = torch.randn(total, width, generator=g).bfloat16()
    x[:, torch.randperm(width, generator=g)[:4]] *= 50
    aw = (1 + 0.1 * torch.randn(k, generator=g)).bfloat16() if act == "rms_norm" else None
    counter = torch.tensor([3], dtype=torch.int64, device="cuda")
    first, step = 17, 40
    start = first + 3 * step
    lib = wq.library()
    xc, awc = x.cuda(), None if aw is None else aw.cuda()
    ACT = wq.ACTS[act]
    print(f"quantize_at act={act} rows {start}..{start + m}", flush=True)

    q = torch.empty(m, k, dtype=torch.int8, device="cuda")
    sa = torch.empty(m, (k + 127) // 128, dtype=torch.float32, device="cuda")
    assert lib.wq8_quantize_blocks_at(xc.data_ptr(), q.data_ptr(), sa.data_ptr(), m, k, width, BF16, 0, ACT, None if awc is None else awc.data_ptr(),
                                      1e-6, None, counter.data_ptr(), first, step, stream()) == 0
    hi = torch.empty(m, k, dtype=torch.int8, device="cuda")
    lo = torch.empty_like(hi)
    sr = torch.empty(m, dtype=torch.float32, device="cuda")
    assert lib.wq8_quantize_at(xc.data_ptr(), hi.data_ptr(), lo.data_ptr(), sr.data_ptr(), m, k, width, BF16, 0, ACT,
                               None if awc is None else awc.data_ptr(), 1e-6, counter.data_ptr(), first, step, stream()) == 0
    torch.cuda.synchronize()
    rows = bits(x[start:start + m])
    aw_bits = None if aw is None else bits(aw)
    q_ref, sa_ref = oracle.quantize_blocks(rows, BF16, 0, act, aw_bits, 1e-6)
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(sa.cpu().numpy().view(np.uint32), sa_ref.view(np.uint32))
    hi_ref, lo_ref, sr_ref = oracle.quantize(rows, BF16, 0, True, act, aw_bits, 1e-6)
    np.testing.assert_array_equal(hi.cpu().numpy(), hi_ref)
    np.testing.assert_array_equal(lo.cpu().numpy(), lo_ref)
    np.testing.assert_array_equal(sr.cpu().numpy().view(np.uint32), sr_ref.view(np.uint32))


@pytest.mark.parametrize("mode,variant", [("row", 0), ("row", 6), ("block", 10), ("block", 11), ("block", 15), ("exact", 1), ("exact", 7)])
def test_gemm_at_offsets_vs_oracle(wq, oracle, mode, variant):
    """wq8_gemm_at with shifted input rows (in_first + counter * in_step), shifted output / residual rows and per-span
    residual scales; only the addressed output rows are written, and they equal the oracle bit for bit."""
    m, n, k, spans = 72, 136, 384, 4
    total = 5 * m
    g = torch.Generator().manual_seed(variant + 40)
    kb = (k + 127) // 128
    a = torch.randint(-127, 128, (total, k), generator=g, dtype=torch.int8)
    a_lo = torch.randint(-127, 128, (total, k), generator=g, dtype=torch.int8) if mode == "exact" else None
    sa = ((torch.rand(total, kb, generator=g) if mode == "block" else torch.rand(total, generator=g)) + 0.5) / 127
    b = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    sb = (torch.rand(n, generator=g) + 0.5) / 127
    bias = (0.02 * torch.randn(n, generator=g)).bfloat16()
    residual = torch.randn(spans * m, n, generator=g).bfloat16()
    rscale = torch.rand(spans, n, generator=g).bfloat16()
    c = 2
    in_first, in_step, first, step = 5, m + 3, 0, m
    in_rows = slice(in_first + c * in_step, in_first + c * in_step + m)
    out_rows = slice(first + c * step, first + c * step + m)
    cu = lambda t: None if t is None else t.cuda()
    a_d, lo_d, sa_d, b_d, sb_d, bias_d, rscale_d = map(cu, (a, a_lo, sa, b, sb, bias, rscale))
    out = torch.zeros(spans * m, n, dtype=torch.bfloat16, device="cuda")
    res_d = residual.cuda()
    counter = torch.tensor([c], dtype=torch.int64, device="cuda")
    lib = wq.library()
    sizes = (__import__("ctypes").c_int64 * 2)()
    lib.wq8_gemm_workspace(m, n, k, variant, 256, 0, sizes)
    ws = torch.empty(max(1, sizes[0]), dtype=torch.uint8, device="cuda")
    print(f"gemm_at mode={mode} variant={variant} input rows {in_rows} output rows {out_rows}", flush=True)
    rc = lib.wq8_gemm_at(a_d.data_ptr(), None if lo_d is None else lo_d.data_ptr(), sa_d.data_ptr(), b_d.data_ptr(), sb_d.data_ptr(),
                         bias_d.data_ptr(), res_d.data_ptr(), rscale_d.data_ptr(), out.data_ptr(), m, n, k, BF16, variant, 256, 0,
                         ws.data_ptr(), None, counter.data_ptr(), first, step, m, n, in_first, in_step, stream())
    assert rc == 0
    torch.cuda.synchronize()
    oracle_mode = "block_biased" if variant in BIASED else mode
    ref = oracle.gemm(a[in_rows].numpy(), None if a_lo is None else a_lo[in_rows].numpy(), sa[in_rows].numpy(), b.numpy(), sb.numpy(),
                      bits(bias), BF16, oracle_mode, bits(residual[out_rows]), bits(rscale[c]))
    got = out.cpu()
    np.testing.assert_array_equal(bits(got[out_rows]), ref)
    assert got[:out_rows.start].abs().sum().item() == 0 and got[out_rows.stop:].abs().sum().item() == 0


@pytest.mark.parametrize("path", ("lines", "small"))
def test_one_row_transposed_column(wq, oracle, path):
    """A (K, 1) column transposed to (1, K) has stride (1, 1): it is one row, read at its own width, and gives the
    contiguous row's result bit for bit."""
    k, n = 2048, 320
    g = torch.Generator().manual_seed(3)
    col = torch.randn(k, 1, generator=g).bfloat16().cuda()
    x = col.t()
    assert x.stride() == (1, 1)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8).cuda()
    s = ((torch.rand(n, generator=g) + 0.5) / 127).cuda()
    bias = (0.02 * torch.randn(n, generator=g)).bfloat16().cuda()
    print(f"one-row transposed input path={path}", flush=True)
    y = wq.linear(x, w, s, bias, mode=path)
    y_ref = wq.linear(x.contiguous(), w, s, bias, mode=path)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
    ref = torch.from_numpy(oracle.linear_f64(bits(x.cpu()), BF16, w.cpu().numpy(), s.cpu().numpy(), bits(bias.cpu()))).bfloat16().float()
    assert rel_err(y.cpu().float(), ref) <= 1e-3
    assert y.abs().sum() > bias.float().abs().sum()  # not the bias alone


@pytest.mark.parametrize("mode", ("block", "exact"))
def test_chunked_linear_equals_one_chunk(wq, oracle, mode, monkeypatch, whole_tiles):
    """linear() over several row chunks (SCRATCH_BYTES forced small) equals one chunk bit for bit, with the residual
    written in place, and sampled rows equal the oracle (whole tiles: every chunk folds in the same order)."""
    m, k, n = 3000, 1280, 768
    g = torch.Generator().manual_seed(21)
    x = torch.randn(m, k, generator=g).bfloat16()
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    s = (torch.rand(n, generator=g) + 0.5) / 127
    bias = (0.02 * torch.randn(n, generator=g)).bfloat16()
    r = torch.randn(m, n, generator=g).bfloat16()
    rs = torch.full((n,), 0.5).bfloat16()
    xc, wc, sc, bc, rsc = x.cuda(), w.cuda(), s.cuda(), bias.cuda(), rs.cuda()
    one = r.cuda()
    wq.linear(xc, wc, sc, bc, mode=mode, act="gelu", residual=one, residual_scale=rsc, out=one)
    row_bytes = {"block": k + 4 * ((k + 127) // 128), "exact": 2 * k + 4}[mode]
    monkeypatch.setattr(wq, "SCRATCH_BYTES", 1024 * row_bytes)
    step = wq.chunk_rows(mode, k)
    assert -(-m // step) >= 3, step
    print(f"chunked {mode}: {-(-m // step)} chunks of {step} rows", flush=True)
    many = r.cuda()
    wq.linear(xc, wc, sc, bc, mode=mode, act="gelu", residual=many, residual_scale=rsc, out=many)
    torch.cuda.synchronize()
    assert torch.equal(one, many)
    rows = torch.tensor([0, step - 1, step, 2 * step + 7, m - 1])
    xr = bits(x[rows])
    if mode == "block":
        q, sa = oracle.quantize_blocks(xr, BF16, 0, "gelu")
        refs = [oracle.gemm(q, None, sa, w.numpy(), s.numpy(), bits(bias), BF16, fold, bits(r[rows]), bits(rs)) for fold in ("block", "block_biased")]
    else:
        hi, lo, sa = oracle.quantize(xr, BF16, 0, True, "gelu")
        refs = [oracle.gemm(hi, lo, sa, w.numpy(), s.numpy(), bits(bias), BF16, "exact", bits(r[rows]), bits(rs))]
    got = bits(many[rows.cuda()].cpu())
    assert any(np.array_equal(got, ref) for ref in refs)


@pytest.mark.parametrize("mode", (None, "lines", "small", "exact", "block", "row"))
def test_empty_inputs(wq, mode):
    """No tokens, or no output channels: every path returns the empty result without launching a kernel."""
    w = torch.randint(-127, 128, (256, 512), dtype=torch.int8, device="cuda")
    s = torch.rand(256, device="cuda") / 127
    y = wq.linear(torch.randn(0, 512, dtype=torch.bfloat16, device="cuda"), w, s, mode=mode)
    assert tuple(y.shape) == (0, 256)
    y = wq.linear(torch.randn(3, 512, dtype=torch.bfloat16, device="cuda"), w[:0], s[:0], mode=mode or "small")
    torch.cuda.synchronize()
    assert tuple(y.shape) == (3, 0)
