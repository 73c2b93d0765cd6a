"""GPU tests of the timed path choice (choose_path(), used by linear() without mode=; the reference's
wgpkernels/int8/__init__.py:474-509) at the BASELINE config-2 shapes.

For every shape the chosen path is checked against an independent cold measurement: each candidate path timed over a
rotation of weight copies larger than every cache (L2 + 256 MiB MALL), so each call streams its weights from HBM as a
model layer does. The choice must be the path the decision rule picks from those timings, or cost at most 10% more.
linear() without mode= must then give that path's result (checked against the CPU oracle).
"""
import pytest
import torch

from conftest import DT, bits, rel_err

pytestmark = pytest.mark.gpu
BF16 = DT[torch.bfloat16]
CACHE_BYTES = 2 * (8 * 4 * 1024 * 1024 + 256 * 1024 * 1024)


@pytest.fixture
def fresh_store(wq, tmp_path, monkeypatch):
    from wgpkernels_amd.int8 import _tuning
    monkeypatch.setattr(_tuning, "store", _tuning.Store(tmp_path / "tuning.json"))
    monkeypatch.setattr(wq, "_decided_paths", {})
    monkeypatch.setattr(wq, "_plans", {})
    return _tuning.store


def cold_path_ms(wq, path, x, copies, s, bias, reps=3):
    """Median per-call ms of `path` cycling over the weight copies (nothing cached), after one untimed pass."""
    for w in copies:
        wq.linear(x, w, s, bias, mode=path)
    times = []
    for _ in range(reps):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for w in copies:
            wq.linear(x, w, s, bias, mode=path)
        end.record()
        end.synchronize()
        times.append(start.elapsed_time(end) / len(copies))
    return sorted(times)[len(times) // 2]


@pytest.mark.parametrize("k,n", [(5120, 13824), (13824, 5120), (5120, 5120)])
def test_choice_matches_cold_measurement(wq, oracle, fresh_store, k, n):
    from wgpkernels_amd.int8 import _policy
    g = torch.Generator().manual_seed(k + n)
    w0 = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    s = ((torch.rand(n, generator=g) + 0.5) / 127).cuda()
    bias = (0.02 * torch.randn(n, generator=g)).bfloat16()
    count = CACHE_BYTES // (n * k) + 2
    copies = [w0.cuda()] + [torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda") for _ in range(count - 1)]
    report = []
    for m in (1, 2, 4, 16, 32):
        x = torch.randn(m, k, generator=g).bfloat16()
        xc = x.cuda()
        shape = _policy.LinearShape(m, n, k)
        print(f"path choice m={m} k={k} n={n}", flush=True)
        chosen = wq.choose_path(xc, copies[0], s, bias.cuda())
        timings = {p: cold_path_ms(wq, p, xc, copies, s, bias.cuda()) for p in shape.candidates()}
        expected = _policy.decide(timings, False)
        report.append(f"m={m}: chose {chosen}, cold {', '.join(f'{p} {t * 1e3:.1f} us' for p, t in timings.items())}")
        assert chosen in timings
        assert chosen == expected or timings[chosen] <= 1.10 * timings[expected], report[-1]
        # linear() without mode= runs the chosen path
        y = wq.linear(xc, copies[0], s, bias.cuda())
        torch.cuda.synchronize()
        ref = torch.from_numpy(oracle.linear_f64(bits(x), BF16, w0.numpy(), s.cpu().numpy(), bits(bias))).float()
        if chosen == "block":
            assert rel_err(y.cpu().float(), ref) <= 3e-2
        else:
            assert rel_err(y.cpu().float(), ref.bfloat16().float()) <= 1e-3
    print("\n".join(report))
    assert sum(key.startswith("path|") for key in fresh_store.entries()) == 5  # one decision per token bucket


def test_long_inputs_take_block_untimed(wq, fresh_store):
    x = torch.zeros(4097, 256, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(64, 256, dtype=torch.int8, device="cuda")
    assert wq.choose_path(x, w, torch.ones(64, device="cuda")) == "block"
    assert wq.choose_path(x, w, torch.ones(64, device="cuda"), precise=True) == "exact"
    assert not any(key.startswith("path|") for key in fresh_store.entries())


def test_choice_is_cached_per_bucket(wq, fresh_store, capsys):
    k, n = 1024, 512
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, device="cuda")
    s = torch.rand(n, device="cuda") / 127
    first = wq.choose_path(torch.randn(20, k, device="cuda").bfloat16(), w, s)
    assert "Autotuning INT8 path" in capsys.readouterr().out
    # 19 tokens fall in the same bucket (multiples of 8 above 16): no new timing, same path
    wq._decided_paths.clear()
    assert wq.choose_path(torch.randn(19, k, device="cuda").bfloat16(), w, s) == first
    assert "Autotuning" not in capsys.readouterr().out
