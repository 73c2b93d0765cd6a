"""Checkpoint adapters (Quanto INT8, ConvRot, group-128) on the CPU: layouts recognised, scales reshaped to what linear()
takes, bad layouts rejected, a .safetensors round trip, and the writers' quantization against its closed form."""
import pytest
import torch

from wgpkernels_amd.int8 import checkpoint as ck


def test_quanto_layout():
    w = torch.randn(48, 256)
    t = ck.quanto_tensors("blocks.0.attn.q", w, bias=torch.randn(48))
    assert t["blocks.0.attn.q.weight._scale"].shape == (48, 1) and t["blocks.0.attn.q.weight._scale"].dtype == torch.bfloat16
    got = ck.load(t, "blocks.0.attn.q")
    assert got.weight.dtype == torch.int8 and got.weight.data_ptr() == t["blocks.0.attn.q.weight._data"].data_ptr()  # not copied
    assert got.scale.shape == (48,) and got.scale.dtype == torch.float32 and got.group == 0 and got.bias is not None
    # dequantized weight within half a step of the float weight (scales kept in FP32 here; BF16 rounds them)
    exact = ck.load(ck.quanto_tensors("l", w, dtype=torch.float32), "l")
    err = (exact.weight.float() * exact.scale[:, None] - w).abs()
    assert (err <= exact.scale[:, None] * 0.5 * 1.0001 + 1e-6).all()


def test_group128_layout():
    w = torch.randn(32, 384)
    w[:, 128:256] *= 20  # one block much larger: its own scale
    t = ck.group128_tensors("l", w)
    got = ck.load(t, "l")
    assert got.block_scales and got.scale.shape == (32, 3)
    assert torch.allclose(got.scale[:, 1] / got.scale[:, 0], w[:, 128:256].abs().amax(1) / w[:, :128].abs().amax(1))
    deq = got.weight.float() * got.scale.repeat_interleave(128, dim=1)
    assert ((deq - w).abs() <= got.scale.repeat_interleave(128, dim=1) * 0.5 * 1.01 + 1e-4).all()


@pytest.mark.parametrize("group", ck.ROTATION_GROUPS)
def test_convrot_layout_and_rotation(group):
    w = torch.randn(16, 512)
    t = ck.convrot_tensors("l", w, group)
    got = ck.load(t, "l", group=group)
    assert got.group == group and got.scale.shape == (16,)
    r = ck.rotation(group)
    assert torch.allclose(r @ r.T, torch.eye(group), atol=1e-5)
    # undoing the rotation of the dequantized weight gives back the float weight
    deq = got.weight.float() * got.scale[:, None]
    back = (deq.reshape(16, -1, group) @ r.T).reshape(16, 512)
    assert (back - w).norm() / w.norm() < 1e-2


def test_rejects_bad_layouts():
    good = ck.quanto_tensors("l", torch.randn(8, 64))
    with pytest.raises(KeyError):
        ck.from_quanto(good, "m")
    bad = dict(good)
    bad["l.weight._scale"] = torch.ones(9, 1)
    with pytest.raises(ValueError):
        ck.from_quanto(bad, "l")
    bad = dict(good)
    bad["l.weight._data"] = torch.zeros(8, 64, dtype=torch.int16)
    with pytest.raises(ValueError):
        ck.from_quanto(bad, "l")
    with pytest.raises(ValueError):
        ck.from_convrot(good, "l", 32)  # not a rotation group
    with pytest.raises(ValueError):
        ck.from_convrot(ck.quanto_tensors("l", torch.randn(8, 80)), "l", 64)  # K not a multiple of the group
    g = ck.group128_tensors("l", torch.randn(8, 256))
    g["l.weight_scale"] = g["l.weight_scale"][:, :1].expand(8, 1).contiguous()
    with pytest.raises(ValueError):
        ck.from_group128(g, "l")


def test_safetensors_round_trip(tmp_path):
    from safetensors.torch import save_file
    tensors = {**ck.quanto_tensors("a", torch.randn(16, 128), torch.randn(16)), **ck.group128_tensors("b", torch.randn(24, 256))}
    path = tmp_path / "model.safetensors"
    save_file(tensors, str(path))
    loaded = ck.load_safetensors(path, ["a", "b"], device="cpu", dtype=torch.float16)
    assert torch.equal(loaded["a"].weight, tensors["a.weight._data"]) and loaded["a"].bias.dtype == torch.float16
    assert loaded["b"].block_scales and torch.equal(loaded["b"].scale, tensors["b.weight_scale"])
