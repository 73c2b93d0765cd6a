"""Host-side logic of wgpkernels_amd.int8 on the CPU: buckets and cache keys of the per-GPU autotune (I:195-216,
I:453-468), the path policy used under capture (I:453-465), the tuning cache's tolerance of damaged files (I:204-216),
Prepared.rows (I:367-377), operand validation, and the loud failure when the HIP library is missing (no CPU fallback)."""
import json

import pytest
import torch

from wgpkernels_amd import int8 as wq


def test_rows_bucket():
    assert [wq._rows_bucket(m) for m in (1, 64, 65, 4096)] == [64, 64, 128, 4096]
    assert [wq._rows_bucket(m) for m in (4097, 8192, 8193, 32760, 100000)] == [8192, 8192, 16384, 16384, 16384]


def test_path_bucket():
    assert [wq._path_bucket(m) for m in (1, 16, 17, 24, 128, 129, 5000)] == [1, 16, 24, 24, 128, 192, 8192]


def test_static_path_policy():
    assert wq._static_path(4, 5120, False) == "lines"
    assert wq._static_path(4, 5122, False) == "exact"  # K fits neither few-token kernel
    assert wq._static_path(32, 5120, False) == "small"
    assert wq._static_path(33, 5120, False) == "exact"
    assert wq._static_path(65, 5120, False) == "block"
    assert wq._static_path(65, 5120, True) == "exact"
    assert wq._static_path(2, 5120, False, groups=True) == "exact"  # group scales: no few-token paths


def test_precise_candidates():
    assert wq._precise_paths(4, 5120) == ["lines", "small", "exact"]
    assert wq._precise_paths(16, 5120) == ["small", "exact"]
    assert wq._precise_paths(16, 5124) == ["exact"]
    assert wq._precise_paths(2, 5120, groups=True) == ["exact"]


def test_candidates_cover_every_mode():
    for mode, candidates in wq._CANDIDATES.items():
        for variant, split in candidates:
            assert wq._MODES[variant] == mode and split == 0


def test_width_and_rows_checks():
    x = torch.zeros(3, 64, dtype=torch.bfloat16)
    assert wq._width(x, None) == 64 and wq._width(x, "swiglu") == 32
    wq._check_rows(x)
    with pytest.raises(ValueError):
        wq._check_rows(x.t())
    with pytest.raises(ValueError):
        wq._check_rows(torch.zeros(3, 63, dtype=torch.bfloat16)[:, :60])  # 126-byte row stride


def test_gemm_operand_checks():
    m, n, k = 8, 16, 256
    a, b = torch.zeros(m, k, dtype=torch.int8), torch.zeros(n, k, dtype=torch.int8)
    y = torch.zeros(m, n, dtype=torch.bfloat16)
    wq._check_gemm_operands(a, None, torch.zeros(m), b, torch.zeros(n), y, "row")
    wq._check_gemm_operands(a, None, torch.zeros(m, 2), b, torch.zeros(n), y, "block")
    wq._check_gemm_operands(a, None, torch.zeros(m, 2), b, torch.zeros(n, 2), y, "block+g")
    with pytest.raises(ValueError):
        wq._check_gemm_operands(a, None, torch.zeros(m), b, torch.zeros(n), y, "block")  # row scales on the block path
    with pytest.raises(ValueError):
        wq._check_gemm_operands(a, None, torch.zeros(m, 2), b, torch.zeros(n), y, "row")
    with pytest.raises(ValueError):
        wq._check_gemm_operands(a, None, torch.zeros(m), torch.zeros(n, k + 16, dtype=torch.int8), torch.zeros(n), y, "row")
    with pytest.raises(ValueError):
        wq._check_gemm_operands(a, torch.zeros(m, k - 16, dtype=torch.int8), torch.zeros(m), b, torch.zeros(n), y, "exact")
    with pytest.raises(ValueError):
        wq._check_gemm_operands(a, None, torch.zeros(m), b, torch.zeros(n), torch.zeros(n, m, dtype=torch.bfloat16).t(), "row")


def test_prepared_rows():
    q = torch.arange(40, dtype=torch.int8).reshape(10, 4)
    p = wq.Prepared("block", q, None, torch.arange(20.0).reshape(10, 2), torch.bfloat16)
    part = p.rows(2, 5)
    assert part.path == "block" and part.lo is None and part.dtype == torch.bfloat16
    assert torch.equal(part.x, q[2:5]) and torch.equal(part.scale, p.scale[2:5])
    assert part.x.data_ptr() == q[2:5].data_ptr()  # a view, not a copy


def test_linear_prepared_rejects_group_scales_on_few_token_paths():
    p = wq.Prepared("lines", torch.zeros(1, 256, dtype=torch.bfloat16), None, None, torch.bfloat16)
    with pytest.raises(ValueError):
        wq.linear_prepared(p, torch.zeros(8, 256, dtype=torch.int8), torch.zeros(8, 2))


def test_prepare_rejects_unknown_path():
    with pytest.raises(ValueError):
        wq.prepare(torch.zeros(2, 64, dtype=torch.bfloat16), path="fast")


def test_tuning_cache_survives_damaged_files(tmp_path, monkeypatch):
    path = tmp_path / "cache.json"
    monkeypatch.setattr(wq, "_TUNING_PATH", path)
    for payload in ("not json", json.dumps([1, 2]), json.dumps({"version": 0, "configs": {"k": [1, 0]}}),
                    json.dumps({"version": wq._TUNING_VERSION, "configs": [1]})):
        path.write_text(payload)
        monkeypatch.setattr(wq, "_tuned", None)
        assert wq._cache() == {}
    monkeypatch.setattr(wq, "_tuned", None)
    path.write_text(json.dumps({"version": wq._TUNING_VERSION, "configs": {"block|16384x13824x5120|gfx950x256": [10, 0]}}))
    assert wq._cache()["block|16384x13824x5120|gfx950x256"] == [10, 0]
    wq._cache()["row|64x64x64|gfx950x256"] = [6, 0]
    wq._save_cache()
    assert json.loads(path.read_text())["configs"]["row|64x64x64|gfx950x256"] == [6, 0]
    monkeypatch.setattr(wq, "_tuned", None)


def test_check_raises_on_error_codes():
    wq._check(0)
    with pytest.raises(RuntimeError, match="rejected"):
        wq._check(-2)
    with pytest.raises(RuntimeError, match="HIP error"):
        wq._check(700)


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="not found"):
        wq.load_library(tmp_path / "libwgp_int8.so")


def test_reference_rotation_is_orthonormal():
    for group in (16, 64, 256):
        eye = torch.eye(group)
        r = wq._reference_rotation(eye, group)
        assert torch.allclose(r @ r.T, eye, atol=1e-5)
