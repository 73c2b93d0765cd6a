"""Host-side logic of wgpkernels_amd.int8 on the CPU: the token-count buckets and cache keys of the per-GPU autotune
(reference formats, wgpkernels/int8/__init__.py:195-197, :467-468, :485-486), the path rule used where nothing is timed,
the decision rule of the timed choice (:503-505), the tuning store's tolerance of damaged files, row chunking, Prepared
views, operand validation, the ctypes signature table against include/wq8.h, the `wgpkernels.int8` import name, and the
loud failure when the HIP library is missing (there is no CPU fallback)."""
import json
import re
from pathlib import Path

import pytest
import torch

from wgpkernels_amd import int8 as wq
from wgpkernels_amd.int8 import _native, _policy, _tuning

ROOT = Path(__file__).resolve().parents[1]


def test_reference_import_name():
    from wgpkernels import int8 as alias
    import wgpkernels.int8 as dotted
    assert alias is wq and dotted is wq
    for name in ("linear", "prepare", "linear_prepared", "linear_prepared_segments", "choose_path", "selftest", "quantize_blocks",
                 "quantize", "transform_rows", "rotate_groups", "gemm", "small", "gemv_lines", "load_library", "prepare_stream",
                 "weight_groups_supported", "segments_supported", "Prepared", "SCRATCH_BYTES", "EXACT_TOLERANCE"):
        assert hasattr(alias, name), name


def test_rows_buckets():
    assert [_tuning.gemm_rows_bucket(m) for m in (1, 64, 65, 4096)] == [64, 64, 128, 4096]
    assert [_tuning.gemm_rows_bucket(m) for m in (4097, 8192, 8193, 16384, 32760, 100000)] == [8192, 8192, 16384, 16384, 16384, 16384]
    assert [_tuning.path_rows_bucket(m) for m in (1, 16, 17, 24, 128, 129, 5000)] == [1, 16, 24, 24, 128, 192, 8192]


def test_path_key_format():
    shape = _policy.LinearShape(32, 13824, 5120, 16, "gelu", True, True)
    assert shape.key(32, "gfx950x256") == "path+precise|32x13824x5120|g16|gelu|wgroups|gfx950x256"
    assert _policy.LinearShape(5, 64, 128).key(5, "d") == "path|5x64x128|g0|d"


def test_untimed_rule():
    S = _policy.LinearShape
    assert S(4, 1, 5120).untimed() == "lines"
    assert S(4, 1, 5122).untimed() == "exact"  # K fits neither few-token kernel
    assert S(32, 1, 5120).untimed() == "small"
    assert S(5, 1, 5124).untimed() == "exact"
    assert S(33, 1, 5120).untimed() == "exact"
    assert S(65, 1, 5120).untimed() == "block"
    assert S(65, 1, 5120, precise=True).untimed() == "exact"
    assert S(2, 1, 5120, weight_groups=True).untimed() == "exact"


def test_candidates():
    S = _policy.LinearShape
    assert S(4, 1, 5120).candidates() == ["lines", "small", "exact", "block"]
    assert S(16, 1, 5120, precise=True).candidates() == ["small", "exact"]
    assert S(16, 1, 5124).candidates() == ["exact", "block"]
    assert S(2, 1, 5120, weight_groups=True).candidates() == ["exact", "block"]


def test_decision_rule():
    assert _policy.decide({"small": 1.0, "exact": 2.0, "block": 0.95}, False) == "small"
    assert _policy.decide({"small": 1.2, "exact": 2.0, "block": 1.0}, False) == "block"   # 20% over block
    assert _policy.decide({"small": 1.1, "exact": 2.0, "block": 1.0}, False) == "small"   # exactly at the tolerance
    assert _policy.decide({"small": 1.2, "exact": 2.0, "block": 1.0}, True) == "small"    # precise: never block
    assert _policy.decide({"exact": 3.0}, True) == "exact"


def test_tile_candidates_keep_modes():
    for mode in wq.TILES:
        candidates = wq.tile_candidates(mode)
        assert candidates[0] == (wq.TILES[mode][0], 1)  # the untimed default: the long tile with the split-K tail
        for variant, split in candidates:
            assert wq.VARIANT_MODES[variant] == mode and split in (0, 1)
        assert {split for _, split in candidates} == {0, 1}


def test_chunk_rows(monkeypatch):
    assert wq.chunk_rows("block", 5120) >= 32760  # one chunk at the headline shape
    monkeypatch.setattr(wq, "SCRATCH_BYTES", 4 * 1024 * 1024)
    rows = wq.chunk_rows("block", 5120)
    assert rows % wq.CHUNK_ROW_MULTIPLE == 0 and rows * (5120 + 4 * 40) <= 4 * 1024 * 1024
    assert wq.chunk_rows("exact", 5120) * (2 * 5120 + 4) <= 4 * 1024 * 1024
    monkeypatch.setattr(wq, "SCRATCH_BYTES", 1)
    assert wq.chunk_rows("row", 5120) == wq.CHUNK_ROW_MULTIPLE  # never less than one tile of rows


def test_activation_checks():
    x = torch.zeros(3, 64, dtype=torch.bfloat16)
    assert wq._op_width(x, None) == 64 and wq._op_width(x, "swiglu") == 32
    wq._check_activation(x)
    with pytest.raises(ValueError):
        wq._check_activation(x.t())
    with pytest.raises(ValueError):
        wq._check_activation(torch.zeros(3, 63, dtype=torch.bfloat16)[:, :60])  # 126-byte row pitch
    with pytest.raises(ValueError):
        wq._check_activation(torch.zeros(3, 64, dtype=torch.float64))


def test_one_row_pitch():
    """A one-row input is read with its own width as pitch, whatever stride PyTorch reports for it."""
    col = torch.zeros(256, 1, dtype=torch.bfloat16).t()
    assert col.stride() == (1, 1)
    wq._check_activation(col)
    assert wq._row_pitch(col) == 256
    x = torch.zeros(4, 512, dtype=torch.bfloat16)[:, :256]
    assert wq._row_pitch(x) == 512


def test_gemm_operand_checks():
    m, n, k = 8, 16, 256
    a, b = torch.zeros(m, k, dtype=torch.int8), torch.zeros(n, k, dtype=torch.int8)
    y = torch.zeros(m, n, dtype=torch.bfloat16)
    wq._check_gemm(a, None, torch.zeros(m), b, torch.zeros(n), y, "row")
    wq._check_gemm(a, None, torch.zeros(m, 2), b, torch.zeros(n), y, "block")
    wq._check_gemm(a, None, torch.zeros(m, 2), b, torch.zeros(n, 2), y, "block+g")
    bad = [
        (a, None, torch.zeros(m), b, torch.zeros(n), y, "block"),      # row scales on the block path
        (a, None, torch.zeros(m, 2), b, torch.zeros(n), y, "row"),
        (a, None, torch.zeros(m), torch.zeros(n, k + 16, dtype=torch.int8), torch.zeros(n), y, "row"),
        (a, torch.zeros(m, k - 16, dtype=torch.int8), torch.zeros(m), b, torch.zeros(n), y, "exact"),
        (a, None, torch.zeros(m), b, torch.zeros(n), torch.zeros(n, m, dtype=torch.bfloat16).t(), "row"),
    ]
    for args in bad:
        with pytest.raises(ValueError):
            wq._check_gemm(*args)


def test_gemm_rejects_unknown_variant():
    a, b = torch.zeros(8, 256, dtype=torch.int8), torch.zeros(16, 256, dtype=torch.int8)
    with pytest.raises(ValueError, match="variant"):
        wq.gemm(a, None, torch.zeros(8), b, torch.zeros(16), None, torch.bfloat16, 0, 99)


def test_prepared_rows_are_views():
    q = torch.arange(40, dtype=torch.int8).reshape(10, 4)
    p = wq.Prepared("block", q, None, torch.arange(20.0).reshape(10, 2), torch.bfloat16)
    part = p.rows(2, 5)
    assert part.path == "block" and part.lo is None and part.dtype == torch.bfloat16
    assert torch.equal(part.x, q[2:5]) and torch.equal(part.scale, p.scale[2:5])
    assert part.x.data_ptr() == q[2:5].data_ptr()


def test_linear_prepared_rejects_group_scales_on_few_token_paths():
    p = wq.Prepared("lines", torch.zeros(1, 256, dtype=torch.bfloat16), None, None, torch.bfloat16)
    with pytest.raises(ValueError):
        wq.linear_prepared(p, torch.zeros(8, 256, dtype=torch.int8), torch.zeros(8, 2))


def test_prepare_rejects_unknown_path():
    with pytest.raises(ValueError):
        wq.prepare(torch.zeros(2, 64, dtype=torch.bfloat16), path="fast")


def test_store_survives_damaged_files(tmp_path):
    path = tmp_path / "cache.json"
    for payload in ("not json", json.dumps([1, 2]), json.dumps({"version": 0, "configs": {"k": [1, 0]}}),
                    json.dumps({"version": _tuning.TUNING_VERSION, "configs": [1]})):
        path.write_text(payload)
        assert _tuning.Store(path).entries() == {}
    path.write_text(json.dumps({"version": _tuning.TUNING_VERSION, "configs": {"block|16384x13824x5120|gfx950x256": [10, 0]}}))
    store = _tuning.Store(path)
    assert store.get("block|16384x13824x5120|gfx950x256") == [10, 0]
    store.put("row|64x64x64|gfx950x256", [6, 0])
    assert json.loads(path.read_text())["configs"] == {"block|16384x13824x5120|gfx950x256": [10, 0], "row|64x64x64|gfx950x256": [6, 0]}
    assert not list(tmp_path.glob(".wgp-int8-*"))  # the temporary file was renamed into place


def test_store_in_unwritable_place_only_warns(tmp_path, capsys):
    blocker = tmp_path / "file"
    blocker.write_text("")
    store = _tuning.Store(blocker / "sub" / "cache.json")
    store.put("k", "block")
    assert store.get("k") == "block" and "Could not save" in capsys.readouterr().out


def test_error_codes_raise():
    with pytest.raises(RuntimeError, match="rejected"):
        _native.raise_code(-2, "wq8_gemm")
    with pytest.raises(RuntimeError, match="HIP error 700"):
        _native.raise_code(700, "wq8_gemm")


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="not found"):
        wq.load_library(tmp_path / "libwgp_int8.so")


_C_LETTER = {"const void*": "p", "void*": "p", "int8_t*": "p", "const int8_t*": "p", "float*": "p", "const float*": "p", "int*": "p",
             "int32_t*": "p", "int64_t*": "p", "const long long*": "p", "const int8_t* const*": "p", "const float* const*": "p",
             "const void* const*": "p", "void* const*": "p", "wq8_stream_t": "p", "int": "i", "int64_t": "l", "long long": "q",
             "float": "f"}


@pytest.mark.parametrize("header,table", [("wq8.h", "SIGNATURES"), ("wq8_test.h", "TEST_SIGNATURES")])
def test_signature_table_matches_header(header, table):
    """Every ctypes signature equals the C declaration in include/ (the product library's wq8.h, the test library's
    wq8_test.h), argument by argument, and each table holds exactly its header's entry points."""
    signatures = getattr(_native, table)
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / header).read_text(), flags=re.S)
    decls = dict(re.findall(r"^(?:int|void)\s+(wq8_\w+)\s*\(([^)]*)\)\s*;", text, re.M))
    results = dict(re.findall(r"^(int|void)\s+(wq8_\w+)\s*\(", text, re.M)[i][::-1] for i in range(len(decls)))
    assert set(decls) == set(signatures)
    for name, params in decls.items():
        assert name in signatures, name
        letters = ""
        for param in filter(None, (p.strip() for p in params.replace("\n", " ").split(","))):
            if param == "void":
                continue
            ctype = re.sub(r"\s+", " ", param.rsplit(" ", 1)[0].replace(" *", "*")).strip()
            if param.split()[-1].startswith("*"):
                ctype += "*"
            letters += _C_LETTER[ctype]
        result, args = signatures[name]
        assert args == letters, (name, args, letters)
        assert result == ("-" if results[name] == "void" else "i"), name


def test_reference_rotation_is_orthonormal():
    for group in (16, 64, 256):
        eye = torch.eye(group)
        r = wq._reference_rotation(eye, group)
        assert torch.allclose(r @ r.T, eye, atol=1e-5)
