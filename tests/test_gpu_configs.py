"""GPU parity at the full sizes of the reference's benchmark configurations (configs 2-5 of the hot path), through the
public API (linear / prepare / linear_prepared / linear_prepared_segments) with the autotuned tiles. Every check
compares sampled rows (or sampled output channels) with the CPU oracle on the same inputs:
- INT8 activations, hi/lo parts and scales bit for bit;
- GEMM outputs bit for bit in the fold order of the tile that ran (the reference's order or the single-FMA biased one),
  on 64 rows per linear: every tile-boundary class of the long tiles, the last partial tile, and seeded random rows
  (each row whole: at config 3's second linear the channel split at channel 4608, or the split-K tiles of the last wave,
  whichever the tuner keeps, run through every checked row);
- lines / small / exact within 1e-3 of the FP32 reference rounded to the output dtype, block within 1.05x of the
  reference block math's own error (I:523-539 definition).
Inputs follow the configurations: seeded CPU generators for the sampled parts, BF16 N(0, 1) activations, INT8 weights
U[-127, 127], scales U(0.5, 1.5) / 127, bias 0.02 N(0, 1).
"""
import numpy as np
import pytest
import torch

from conftest import bits, from_bits, rel_err

pytestmark = pytest.mark.gpu
BF16 = 1


def weights(n, k, seed, groups=False):
    g = torch.Generator().manual_seed(seed)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    s = (torch.rand(n, (k + 127) // 128, generator=g) if groups else torch.rand(n, generator=g)) / 127 + 0.5 / 127
    bias = (0.02 * torch.randn(n, generator=g)).to(torch.bfloat16)
    return w, s, bias


def activations(m, k, seed, outliers=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g)
    if outliers:
        x[:, torch.randperm(k, generator=g)[:outliers]] *= scale
    return x.to(torch.bfloat16)


def sample_rows(m, count=64, seed=0):
    """count rows to check bit for bit: every class of tile boundary of the long tiles (256 tokens: 255 / 256, 511 / 512;
    128 tokens: 127 / 128), the rows of the last, partial tile and of the tile before it, the first and last rows, and
    seeded random rows for the rest."""
    last_tile = (m - 1) // 256 * 256
    fixed = [0, 1, 127, 128, 129, 255, 256, 257, 383, 384, 511, 512, 513, 1023, 1024, 2047, 2048, 4095, 4096,
             last_tile - 256, last_tile - 129, last_tile - 128, last_tile - 1, last_tile, last_tile + 1,
             (last_tile + m) // 2, m - 2, m - 1]
    fixed = [r for r in fixed if 0 <= r < m]
    g = torch.Generator().manual_seed(seed)
    rows = torch.unique(torch.tensor(fixed))
    while rows.numel() < min(count, m):
        rows = torch.unique(torch.cat([rows, torch.randint(0, m, (count - rows.numel(),), generator=g)]))
    return rows


def as_bf16(a):
    return from_bits(a, torch.bfloat16)


def planned_folds(wq, fold, mode, m, n, k, rows, names):
    """name -> oracle outputs (bits) of `rows` in the fold order of the tile plan the library decided for (mode, m, n,
    k) on GPU 0: whole tiles unsplit, the tiles of a split last wave in the split-K order. fold(name, pieces) gives the
    oracle's outputs of the sampled rows for one order."""
    from test_gpu_split import split_tiles
    variant, split = wq._plans[(mode, m, n, k, 0)][:2]
    folds = {name: fold(name, 1) for name in names}
    if split:
        cus = wq._native.gpu(torch.device("cuda", 0)).cus
        bm, bn, tiles, pieces = split_tiles(variant, m, n, k, cus)
        if pieces > 1:
            for name in names:
                pieced = fold(name, pieces)
                for tm, tn in tiles:
                    sel = (rows // bm == tm).numpy()
                    folds[name][sel, tn * bn:(tn + 1) * bn] = pieced[sel, tn * bn:(tn + 1) * bn]
    return folds


def oracle_rows_exact(oracle, y_rows, ref_modes):
    """The fold order (among ref_modes: name -> oracle outputs) that y_rows matches bit for bit, or None."""
    for name, ref in ref_modes.items():
        if np.array_equal(bits(y_rows), ref):
            return name
    return None


# ---- config 2: few-token paths at Wan-14B widths ----------------------------------------------------------------
@pytest.mark.parametrize("k,n", [(5120, 5120), (5120, 13824), (13824, 5120)])
@pytest.mark.parametrize("m", [1, 2, 4, 16, 32])
def test_config2_few_token(wq, oracle, k, n, m):
    path = "lines" if m <= 4 else "small"
    print(f"config2 path={path} m={m} k={k} n={n}", flush=True)
    w, s, bias = weights(n, k, 20 + m)
    x = activations(m, k, 30 + m)
    y = wq.linear(x.cuda(), w.cuda(), s.cuda(), bias.cuda(), mode=path).cpu()
    # every output channel, against the FP64-accumulated reference rounded to BF16
    ref = torch.from_numpy(oracle.linear_f64(bits(x), BF16, w.numpy(), s.numpy(), bits(bias))).bfloat16().float()
    assert rel_err(y.float(), ref) <= 1e-3
    # and per token: no row may hide behind the others' norm
    for t in range(m):
        assert rel_err(y[t].float(), ref[t]) <= 1e-3


# ---- config 3: long-sequence block path ---------------------------------------------------------------------------
def test_config3_block_gelu_then_residual(wq, oracle):
    from oracle import torch_reference as tr
    m, k1, n1 = 32760, 5120, 13824
    print("config3 first linear: block, gelu, M=32760 K=5120 N=13824", flush=True)
    x = activations(m, k1, 3)
    w, s, bias = weights(n1, k1, 4)
    rows = sample_rows(m)
    p = wq.prepare(x.cuda(), 0, "block", "gelu")
    q_ref, sa_ref = oracle.quantize_blocks(bits(x[rows]), BF16, 0, "gelu")
    np.testing.assert_array_equal(p.x[rows.cuda()].cpu().numpy(), q_ref)
    np.testing.assert_array_equal(p.scale[rows.cuda()].cpu().numpy(), sa_ref)
    y = wq.linear_prepared(p, w.cuda(), s.cuda(), bias.cuda())
    y_rows = y[rows.cuda()].cpu()
    folds = planned_folds(wq, lambda mode, pieces: oracle.gemm(q_ref, None, sa_ref, w.numpy(), s.numpy(), bits(bias), BF16, mode,
                                                               pieces=pieces), "block", m, n1, k1, rows, ("block", "block_biased"))
    assert oracle_rows_exact(oracle, y_rows, folds) is not None
    ref = tr.reference_linear(x[rows], w, s, bias, act="gelu")
    assert rel_err(y_rows.float(), ref) <= 1.05 * rel_err(as_bf16(folds["block"]).float(), ref)
    del p, y

    print("config3 second linear: block, residual in place, M=32760 K=13824 N=5120", flush=True)
    k2, n2 = 13824, 5120
    gen = torch.Generator(device="cuda").manual_seed(5)
    x2 = torch.randn(m, k2, device="cuda", generator=gen).to(torch.bfloat16)
    r = torch.randn(m, n2, device="cuda", generator=gen).to(torch.bfloat16)
    r_rows = r[rows.cuda()].cpu()
    w2, s2, bias2 = weights(n2, k2, 6)
    rs = torch.full((n2,), 0.5).to(torch.bfloat16)
    out = wq.linear(x2, w2.cuda(), s2.cuda(), bias2.cuda(), mode="block", residual=r, residual_scale=rs.cuda(), out=r)
    assert out.data_ptr() == r.data_ptr()
    x2_rows = x2[rows.cuda()].cpu()
    q2, sa2 = oracle.quantize_blocks(bits(x2_rows), BF16)
    folds = planned_folds(wq, lambda mode, pieces: oracle.gemm(q2, None, sa2, w2.numpy(), s2.numpy(), bits(bias2), BF16, mode, bits(r_rows),
                                                               bits(rs), pieces=pieces), "block", m, n2, k2, rows, ("block", "block_biased"))
    assert oracle_rows_exact(oracle, r[rows.cuda()].cpu(), folds) is not None


# ---- config 4: exact path, massive activations, fused QKV ---------------------------------------------------------
def test_config4_exact_rms_qkv(wq, oracle):
    from oracle import torch_reference as tr
    m, k, n = 4096, 5120, 3 * 5120
    print("config4 exact rms_norm M=4096 K=5120 N=3x5120", flush=True)
    x = activations(m, k, 7, outliers=k // 100, scale=100.0)
    g = torch.Generator().manual_seed(8)
    aw = (1 + 0.1 * torch.randn(k, generator=g)).to(torch.bfloat16)
    w, s, bias = weights(n, k, 9)
    rows = sample_rows(m)
    p = wq.prepare(x.cuda(), 0, "exact", "rms_norm", aw.cuda(), 1e-6)
    hi, lo, sa = oracle.quantize(bits(x[rows]), BF16, 0, True, "rms_norm", bits(aw), 1e-6)
    np.testing.assert_array_equal(p.x[rows.cuda()].cpu().numpy(), hi)
    np.testing.assert_array_equal(p.lo[rows.cuda()].cpu().numpy(), lo)
    np.testing.assert_array_equal(p.scale[rows.cuda()].cpu().numpy(), sa)
    wc, sc, bc = w.cuda(), s.cuda(), bias.cuda()
    ys = [wq.linear_prepared(p, wc[i * 5120:(i + 1) * 5120], sc[i * 5120:(i + 1) * 5120], bc[i * 5120:(i + 1) * 5120]) for i in range(3)]
    ref = tr.reference_linear(x[rows], w, s, bias, act="rms_norm", act_weight=aw, eps=1e-6)
    for i in range(3):
        sl = slice(i * 5120, (i + 1) * 5120)
        y_rows = ys[i][rows.cuda()].cpu()
        exact = oracle.gemm(hi, lo, sa, w[sl].numpy(), s[sl].numpy(), bits(bias[sl]), BF16, "exact")
        np.testing.assert_array_equal(bits(y_rows), exact)
        assert rel_err(y_rows.float(), ref[:, sl].bfloat16().float()) <= 1e-3
    if wq.segments_supported():
        outs = [torch.empty(m, 5120, dtype=torch.bfloat16, device="cuda") for _ in range(3)]
        wq.linear_prepared_segments(p, [wc[i * 5120:(i + 1) * 5120] for i in range(3)], [sc[i * 5120:(i + 1) * 5120] for i in range(3)],
                                    [bc[i * 5120:(i + 1) * 5120] for i in range(3)], outs)
        for i in range(3):
            assert torch.equal(outs[i], ys[i])


# ---- config 5: group-128 weight scales, swiglu, residual ---------------------------------------------------------
@pytest.mark.parametrize("path", ["exact", "block"])
def test_config5_group128_swiglu_residual(wq, oracle, path):
    from oracle import torch_reference as tr
    m, k, n = 8192, 3072, 12288
    print(f"config5 {path} group-128 swiglu residual M=8192 K=3072 N=12288", flush=True)
    x = activations(m, 2 * k, 10)
    w, sg, bias = weights(n, k, 11, groups=True)
    g = torch.Generator().manual_seed(12)
    r = torch.randn(m, n, generator=g).to(torch.bfloat16)
    rs = (torch.rand(n, generator=g) + 0.5).to(torch.bfloat16)
    rows = sample_rows(m)
    out = r.cuda()
    y = wq.linear(x.cuda(), w.cuda(), sg.cuda(), bias.cuda(), mode=path, act="swiglu", residual=out, residual_scale=rs.cuda(), out=out)
    y_rows = y[rows.cuda()].cpu()
    if path == "exact":
        hi, lo, sa = oracle.quantize(bits(x[rows]), BF16, 0, True, "swiglu")
        ref_bits = planned_folds(wq, lambda mode, pieces: oracle.gemm(hi, lo, sa, w.numpy(), sg.numpy(), bits(bias), BF16, mode, bits(r[rows]),
                                                                      bits(rs), pieces=pieces), "exact+g", m, n, k, rows, ("exact_combined",))["exact_combined"]
    else:
        q, sa = oracle.quantize_blocks(bits(x[rows]), BF16, 0, "swiglu")
        ref_bits = planned_folds(wq, lambda mode, pieces: oracle.gemm(q, None, sa, w.numpy(), sg.numpy(), bits(bias), BF16, mode, bits(r[rows]),
                                                                      bits(rs), pieces=pieces), "block+g", m, n, k, rows, ("block",))["block"]
    np.testing.assert_array_equal(bits(y_rows), ref_bits)
    ref = tr.reference_linear(x[rows], w, sg, bias, act="swiglu", residual=r[rows], residual_scale=rs)
    if path == "exact":
        assert rel_err(y_rows.float(), ref.bfloat16().float()) <= 1e-3
    else:
        assert rel_err(y_rows.float(), ref) <= 1.05 * rel_err(as_bf16(ref_bits).float(), ref) + 1e-7
