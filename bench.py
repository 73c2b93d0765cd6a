#!/usr/bin/env python3
"""Benchmark of the INT8 weight linear on one MI355X (gfx950): prints ONE JSON line on stdout.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu]

Headline workload (first linear): the block path at M = 32760 tokens, K = 5120, N = 13824 with the
act='gelu' prologue, BF16 N(0,1) activations, INT8 weights U[-127, 127], per-channel FP32 scales, BF16 bias; synthetic
data from a CPU generator seeded 0. One step = one whole linear: quantize_blocks(gelu(x)) + the block GEMM, inputs already
resident in HBM.
- value: whole-linear INT8 TOPS (2 M N K / step time), the reference README's definition (quantization included);
- roofline: the dominant kernel (the block GEMM), achieved TOPS from its launch durations measured with HIP events on its
  own stream during the timed steps, against MI355X's dense INT8 peak (5.0 POPS) and, as frac_probe, against the INT8
  matrix-core rate this GPU sustains in the same run on random operands with no memory traffic, for the 16x16x64
  instruction the GEMM runs (the power-limited
  ceiling); traffic: HBM bytes per launch from the committed rocprofv3 summary named in traffic_source;
- lines: the M = 1 GEMV at K = 5120, N = 13824 (config 2), algorithmic bytes N K + 6 N + 2 K M + 2 N M per call, weights
  cycled over 8 copies (> L2 + 256 MiB MALL) so that every call streams from HBM; against 8 TB/s;
- few_token: config 2 per call: M = 2 (lines), M = 4 (the faster of lines and small), M = 16 and 32 (small) at K = 5120,
  N = 13824; M = 1 (lines), 4 (the faster), 16 and 32 (small) at K = 13824, N = 5120; M = 1, 2 (lines), 4 (the faster),
  16 and 32 (small) at K = N = 5120;
- configs: the other GEMM configurations (config 3 second linear, config 4 exact fused QKV, config 5 block+g / exact+g),
  quantize and GEMM timed apart;
- error: norm-relative error against the FP32 reference on sampled rows, next to the reference's own block math (CPU
  oracle) on the same rows;
- cpu_baseline: the reference's numerical definition (PyTorch-CPU FP32 block quantize + dequantize-and-matmul) on a bounded
  sample of rows of the same workload, on this host's cores.
"""
import argparse
import contextlib
import json
import os
import sys
import time

import torch

METRIC = "INT8 linear TOPS at M=32760 (block); HBM GB/s at M≤4; max rel err vs FP32"
INT8_PEAK_TOPS = 5000.0      # MI355X dense INT8 MFMA
HBM_PEAK_GBPS = 8000.0       # MI355X HBM3E


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def synthetic(m, k, n, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    s = (torch.rand(n, generator=g) + 0.5) / 127
    bias = (0.02 * torch.randn(n, generator=g)).to(torch.bfloat16)
    return x, w, s, bias


def rel(y, ref):
    y, ref = y.double(), ref.double()
    return ((y - ref).norm() / ref.norm()).item()


def bench_block(wq, steps, warmup):
    m, k, n = 32760, 5120, 13824
    log(f"[bench] generating block workload M={m} K={k} N={n}")
    x_cpu, w_cpu, s_cpu, b_cpu = synthetic(m, k, n)
    x, w, s, bias = x_cpu.cuda(), w_cpu.cuda(), s_cpu.cuda(), b_cpu.cuda()
    y = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.current_stream()
    events = []

    def step(timed):
        p = wq.prepare(x, 0, "block", "gelu")
        if timed:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
        wq.linear_prepared(p, w, s, bias, out=y)
        if timed:
            e1.record(stream)
            events.append((e0, e1))

    log("[bench] warmup (first call tunes the tile)")
    for _ in range(warmup):
        step(False)
    torch.cuda.synchronize()
    log(f"[bench] timing {steps} steps")
    t0 = time.perf_counter()
    for _ in range(steps):
        step(True)
    torch.cuda.synchronize()
    step_ms = (time.perf_counter() - t0) * 1e3 / steps
    gemm_ms = sum(e0.elapsed_time(e1) for e0, e1 in events) / len(events)
    ops = 2.0 * m * n * k
    rows = torch.tensor([0, 1, 777, 4096, 12345, 20000, 32000, m - 1])
    y_rows = y[rows.cuda()].cpu()
    return {
        "m": m, "k": k, "n": n, "step_ms": step_ms, "gemm_ms": gemm_ms, "ops": ops,
        "whole_tops": ops / (step_ms * 1e-3) / 1e12, "gemm_tops": ops / (gemm_ms * 1e-3) / 1e12,
        "rows": rows, "y_rows": y_rows, "inputs": (x_cpu, w_cpu, s_cpu, b_cpu),
    }


def bench_lines(wq, m=1, path="lines", calls=200, copies=None, k=5120, n=13824):
    fn = wq.gemv_lines if path == "lines" else wq.small
    # weight copies larger than every L2 plus the 256 MiB MALL, so that every call streams its weights from HBM
    copies = copies or max(8, (2 * (32 << 20) + (256 << 20)) // (n * k) + 2)
    log(f"[bench] {path} M={m} K={k} N={n}, {copies} weight copies")
    x_cpu, w_cpu, s_cpu, b_cpu = synthetic(m, k, n, seed=1)
    x, s, bias = x_cpu.cuda(), s_cpu.cuda(), b_cpu.cuda()
    ws = [w_cpu.cuda()] + [torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda") for _ in range(copies - 1)]
    y = torch.empty(m, n, dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.current_stream()
    for i in range(copies):
        fn(x, ws[i], s, bias, out=y)
    torch.cuda.synchronize()
    # the launches go through a HIP graph (one launch per weight copy, replayed), so host submission is out of the
    # timed region; HIP events on the replay stream bracket `calls` launches, including the GPU's gap between dependent
    # launches (a few us, more than the difference between a 13 us kernel and the eager-call rate)
    graph = torch.cuda.CUDAGraph()
    capture = torch.cuda.Stream()
    capture.wait_stream(stream)
    with torch.cuda.stream(capture):
        with torch.cuda.graph(graph, stream=capture):
            for i in range(copies):
                fn(x, ws[i], s, bias, out=y)
    stream.wait_stream(capture)
    replays = max(1, calls // copies)
    calls = replays * copies
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(replays):
        graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / calls * 1e3
    nbytes = n * k + 6 * n + 2 * k * m + 2 * n * m
    fn(x, ws[0], s, bias, out=y)
    y_out = y.cpu()
    del graph, ws
    return {"m": m, "k": k, "n": n, "path": path, "us": us, "bytes": nbytes,
            "gbps": nbytes / (us * 1e-6) / 1e9, "y": y_out, "inputs": (x_cpu, w_cpu, s_cpu, b_cpu)}


def timed_calls(fn, reps, warm=20):
    """Median ms of `reps` calls of fn, each between HIP events on the current stream (the stream the kernels run on),
    after `warm` untimed calls (the clock settles under load within a few ms)."""
    stream = torch.cuda.current_stream()
    for _ in range(warm):
        fn()
    torch.cuda.synchronize()
    marks = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        fn()
        e1.record(stream)
        marks.append((e0, e1))
    torch.cuda.synchronize()
    times = sorted(e0.elapsed_time(e1) for e0, e1 in marks)
    return times[len(times) // 2]


def bench_configs(wq, reps=20):
    """The other GEMM configurations of the metric's configs, quantize and GEMM timed apart.
    Synthetic inputs from a GPU generator (parity at these shapes is covered by tests/test_gpu_configs.py)."""
    g = torch.Generator(device="cuda").manual_seed(0)
    randn = lambda *shape: torch.randn(*shape, device="cuda", generator=g).to(torch.bfloat16)
    w8 = lambda n, k: torch.randint(-127, 128, (n, k), device="cuda", generator=g, dtype=torch.int8)
    scale = lambda *shape: (torch.rand(*shape, device="cuda", generator=g) + 0.5) / 127
    out = []

    def record(name, m, n, k, path, prep_ms, gemm_ms):
        ops = 2.0 * m * n * k
        out.append({"config": name, "m": m, "n": n, "k": k, "path": path, "quantize_us": round(prep_ms * 1e3, 1),
                    "gemm_us": round(gemm_ms * 1e3, 1), "gemm_tops": round(ops / gemm_ms / 1e9, 1),
                    "gemm_frac": round(ops / gemm_ms / 1e9 / INT8_PEAK_TOPS, 4),
                    "whole_tops": round(ops / (prep_ms + gemm_ms) / 1e9, 1)})
        log(f"[bench] {name}: quantize {prep_ms * 1e3:.1f} us, GEMM {gemm_ms * 1e3:.1f} us = {ops / gemm_ms / 1e9:.0f} TOPS")

    # config 3, second linear: K = 13824, N = 5120, residual (scale 0.5) written in place
    m, k, n = 32760, 13824, 5120
    x, w, s, bias, r = randn(m, k), w8(n, k), scale(n), randn(n), randn(m, n)
    rs = torch.full((n,), 0.5, device="cuda").to(torch.bfloat16)
    p = wq.prepare(x, 0, "block")
    prep = timed_calls(lambda: wq.prepare(x, 0, "block"), reps)
    gemm = timed_calls(lambda: wq.linear_prepared(p, w, s, bias, r, rs, r), reps)
    record("3b block residual in place", m, n, k, "block", prep, gemm)
    del x, w, r, p
    # config 4: exact, rms_norm, fused QKV over three 5120-row ranges in one launch
    m, k, n = 4096, 5120, 3 * 5120
    x, w, s, bias = randn(m, k), w8(n, k), scale(n), randn(n)
    aw = (1 + 0.1 * torch.randn(k, device="cuda", generator=g)).to(torch.bfloat16)
    p = wq.prepare(x, 0, "exact", "rms_norm", aw, 1e-6)
    prep = timed_calls(lambda: wq.prepare(x, 0, "exact", "rms_norm", aw, 1e-6), reps)
    parts = [slice(i * 5120, (i + 1) * 5120) for i in range(3)]
    outs = [torch.empty(m, 5120, dtype=torch.bfloat16, device="cuda") for _ in parts]
    gemm = timed_calls(lambda: wq.linear_prepared_segments(p, [w[sl] for sl in parts], [s[sl] for sl in parts], [bias[sl] for sl in parts], outs), reps)
    record("4 exact rms_norm fused QKV", m, n, k, "exact", prep, gemm)
    del x, w, p, outs
    # config 5: group-128 weight scales, swiglu over [gate | value] rows, residual
    m, k, n = 8192, 3072, 12288
    x, w, sg, bias, r = randn(m, 2 * k), w8(n, k), scale(n, k // 128), randn(n), randn(m, n)
    rs = (torch.rand(n, device="cuda", generator=g) + 0.5).to(torch.bfloat16)
    for path in ("block", "exact"):
        p = wq.prepare(x, 0, path, "swiglu")
        prep = timed_calls(lambda: wq.prepare(x, 0, path, "swiglu"), reps)
        y = r.clone()
        gemm = timed_calls(lambda: wq.linear_prepared(p, w, sg, bias, y, rs, y), reps)
        record(f"5 {path}+g swiglu residual", m, n, k, path + "+g", prep, gemm)
        del p, y
    return out


def cpu_baseline_leg(block, lines, budget_s=12.0, time_it=True):
    """CPU leg: the reference's numerical definition in PyTorch-CPU FP32 (block quantize + dequantize-and-matmul) timed on
    a bounded sample of rows of the headline workload, and the checks of the GPU outputs against the CPU oracle (the
    reference's own block math on the sampled rows; the FP64 few-token reference for lines)."""
    import numpy as np
    import oracle
    from oracle import torch_reference as tr
    u16 = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16)
    x, w, s, bias = block["inputs"]
    rows = block["rows"]
    ref = tr.reference_linear(x[rows], w, s, bias, act="gelu")
    q, sa = oracle.quantize_blocks(u16(x[rows]), 1, 0, "gelu")
    def oracle_rows(mode):
        y = oracle.gemm(q, None, sa, w.numpy(), s.numpy(), u16(bias), 1, mode)
        return torch.from_numpy(y.view(np.int16)).view(torch.bfloat16)
    y_or = oracle_rows("block")
    err_gpu, err_ref_math = rel(block["y_rows"].float(), ref), rel(y_or.float(), ref)
    # the long block tiles fold with the biased single-FMA order, the short ones with the reference's order: the
    # sampled rows must match one of the two bit for bit
    exact = [mode for mode in ("block", "block_biased")
             if torch.equal(block["y_rows"].view(torch.int16), oracle_rows(mode).view(torch.int16))]
    error = {"block_rel_err_vs_fp32": err_gpu, "reference_block_math_rel_err": err_ref_math, "ratio": err_gpu / err_ref_math,
             "bit_exact_sampled_rows": bool(exact), "oracle_fold": exact[0] if exact else None}
    lx, lw, ls, lb = lines["inputs"]
    lref = torch.from_numpy(oracle.linear_f64(u16(lx), 1, lw.numpy(), ls.numpy(), u16(lb))).bfloat16().float()
    error["lines_rel_err_vs_rounded_fp32"] = rel(lines["y"].float(), lref)
    if not time_it:
        return None, error
    threads = os.cpu_count()
    torch.set_num_threads(threads)
    # grow the row sample until one call costs about a quarter of the budget (or covers every row), then repeat calls
    # until the budget is spent
    n_rows = 256
    while True:
        t0 = time.perf_counter()
        tr.block_linear(x[:n_rows], w, s, bias, act="gelu")
        dt = time.perf_counter() - t0
        if dt * 4 > budget_s or n_rows >= x.shape[0]:
            break
        n_rows = min(n_rows * 4, x.shape[0])
    calls, total = 0, 0.0
    while total < budget_s:
        t0 = time.perf_counter()
        tr.block_linear(x[:n_rows], w, s, bias, act="gelu")
        total += time.perf_counter() - t0
        calls += 1
    ops = 2.0 * n_rows * w.shape[0] * w.shape[1] * calls
    baseline = {"value": round(ops / total / 1e12, 4), "unit": "TOPS", "cores": threads, "kind": "port",
                "sample": f"{calls} calls on {n_rows} of 32760 rows (K=5120, N=13824, gelu): PyTorch-CPU FP32 block quantize + "
                          f"dequantize-and-matmul, {total:.2f} s"}
    return baseline, error


TRAFFIC_PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic_bench_workloads.md")


def measured_traffic():
    """(HBM bytes per launch of the block GEMM at the headline shape, where they come from): the committed rocprofv3
    --pmc summary's line 'traffic_bytes_per_launch: <int>' and the commit its counters were read at
    ('measured_at_commit: <hash>'), or (None, None) when no summary is present."""
    traffic, commit = None, None
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    traffic = int(line.split(":", 1)[1])
                elif line.startswith("measured_at_commit:"):
                    commit = line.split(":", 1)[1].strip()
    except OSError:
        return None, None
    source = os.path.relpath(TRAFFIC_PROFILE, os.path.dirname(os.path.abspath(__file__)))
    return traffic, f"{source} (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE" + (f", measured at commit {commit})" if commit else ")")


def copy_probe(nbytes=1 << 30, reps=3):
    """A plain device copy of known size: src read once, dst written once per launch (FETCH_SIZE / WRITE_SIZE scale)."""
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] copy probe: {reps} copies of {nbytes} bytes")


def mfma_probe(wq, blocks=512, iters=2000, reps=3, operands=("zero", "random"), shapes=(1, 0)):
    """INT8 matrix-core rate with no memory traffic in the loop (test library entry point wq8_debug_mfma_probe), on zero
    operands and on uniformly random int8 operands (the gap is what the power limit takes for real data), for
    v_mfma_i32_16x16x64_i8 (shape 1, the instruction the GEMMs run; keys "zero", "random") and v_mfma_i32_32x32x32_i8
    (shape 0; keys suffixed "_32x32x32")."""
    from wgpkernels_amd.int8 import _native
    lib = _native.load_test_library()
    out = torch.empty(blocks * 256, dtype=torch.int32, device="cuda")
    ops = blocks * 4 * iters * 16 * 65536.0
    rates = {}
    for name in operands:
        frags = torch.zeros(blocks * 2048 * 16, dtype=torch.uint8, device="cuda")
        if name == "random":
            frags = torch.randint(-127, 128, (blocks * 2048 * 16,), dtype=torch.int8, device="cuda").view(torch.uint8)
        stream = torch.cuda.current_stream()
        for shape in shapes:
            key = name if shape == 1 else f"{name}_32x32x32"
            times = []
            for _ in range(reps + 1):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                lib.call("wq8_debug_mfma_probe", frags.data_ptr(), out.data_ptr(), blocks, iters, shape, stream.cuda_stream)
                e1.record(stream)
                e1.synchronize()
                times.append(e0.elapsed_time(e1))
            ms = sorted(times[1:])[len(times[1:]) // 2]
            rates[key] = round(ops / ms / 1e9, 1)
            log(f"[bench] MFMA probe {key}: {ms:.3f} ms = {ops / ms / 1e9:.0f} TOPS")
    return rates


def main():
    parser = argparse.ArgumentParser(description="INT8 linear benchmark (one MI355X)")
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--mfma-probe", action="store_true",
                        help="run the INT8 matrix-core rate probe on zero operands too, and longer (the default run measures it on random "
                             "operands only)")
    parser.add_argument("--copy-probe", action="store_true",
                        help="also run a plain 1 GiB device copy (calibrates HBM byte counters under rocprofv3 --pmc)")
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build's path runs on a single MI355X (no multi-GPU configuration).",
              file=sys.stderr)
        sys.exit(2)
    # stdout carries the JSON line only: the library's own messages (autotuning, as the reference prints them) go to stderr
    with contextlib.redirect_stdout(sys.stderr):
        result = run(args)
    print(json.dumps(result), flush=True)


def run(args):
    torch.cuda.set_device(0)
    from wgpkernels_amd import int8 as wq
    wq.load_library()
    block = bench_block(wq, args.steps, args.warmup)
    lines = bench_lines(wq)
    # the other few-token counts of the metric (HBM GB/s at M <= 4), each on its faster path
    few = []
    for (k, n), m, paths in (((5120, 13824), 2, ("lines",)), ((5120, 13824), 4, ("lines", "small")), ((5120, 13824), 16, ("small",)),
                             ((5120, 13824), 32, ("small",)), ((13824, 5120), 1, ("lines",)), ((13824, 5120), 4, ("lines", "small")),
                             ((13824, 5120), 16, ("small",)), ((13824, 5120), 32, ("small",)), ((5120, 5120), 1, ("lines",)),
                             ((5120, 5120), 2, ("lines",)), ((5120, 5120), 4, ("lines", "small")), ((5120, 5120), 16, ("small",)),
                             ((5120, 5120), 32, ("small",))):
        runs = [bench_lines(wq, m, path, calls=96, k=k, n=n) for path in paths]
        best = min(runs, key=lambda r: r["us"])
        few.append({"m": m, "k": k, "n": n, "path": best["path"], "gbps": round(best["gbps"], 1), "us": round(best["us"], 2),
                    "frac": round(best["gbps"] / HBM_PEAK_GBPS, 4)})
    configs = bench_configs(wq)
    log("[bench] CPU leg: oracle checks" + ("" if args.no_cpu else " and CPU baseline"))
    cpu, error = cpu_baseline_leg(block, lines, time_it=not args.no_cpu)
    if args.copy_probe:
        copy_probe()
    probe = mfma_probe(wq) if args.mfma_probe else mfma_probe(wq, iters=1000, operands=("random",))
    traffic, traffic_source = measured_traffic()
    result = {
        "metric": METRIC,
        "value": round(block["whole_tops"], 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(block["step_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "block linear M=32760 K=5120 N=13824 act=gelu, bf16 in/out (BASELINE config 3)",
                   "m": block["m"], "k": block["k"], "n": block["n"], "act": "gelu", "path": "block"},
        "roofline": {"bound": "mfma", "achieved": round(block["gemm_tops"], 2), "peak": INT8_PEAK_TOPS, "unit": "TOPS",
                     "frac": round(block["gemm_tops"] / INT8_PEAK_TOPS, 4), "traffic": traffic, "traffic_source": traffic_source,
                     "probe_tops": probe["random"], "frac_probe": round(block["gemm_tops"] / probe["random"], 4),
                     "kernel": "gemm_i8 block (quantize excluded)", "gemm_ms": round(block["gemm_ms"], 4)},
        "cpu_baseline": cpu,
        "lines": {"config": "M=1 K=5120 N=13824", "gbps": round(lines["gbps"], 1), "us": round(lines["us"], 2), "frac": round(lines["gbps"] / HBM_PEAK_GBPS, 4)},
        "few_token": {"config": "per call, weights streamed from HBM (BASELINE config 2)", "runs": few},
        "configs": configs,
        "error": error,
    }
    result["mfma_probe"] = {"unit": "TOPS", **probe}
    return result


if __name__ == "__main__":
    main()
