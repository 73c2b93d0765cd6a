"""Checkpoint formats that feed the INT8 linear: the adapters that turn a checkpoint's tensors into linear() arguments.

The reference takes (weight, scale) tensors and leaves loading to its caller; it names the checkpoints it serves
(README.md:5, :27-30, :103): Quanto INT8, ConvRot and group-128 INT8 (Hunyuan's DiT). Their tensor layouts:

- Quanto INT8 (optimum-quanto `qint8` weights, per output channel): `<layer>.weight._data` int8 (N, K) and
  `<layer>.weight._scale` (N, 1) in the model's float dtype, W = _data * _scale; `<layer>.bias` optional.
- ConvRot: the same INT8 (N, K) weight and per-channel scales, but quantized after a rotation of K in groups of 16, 64
  or 256: the stored matrix is quantize(W @ R), R the block-diagonal group rotation. The activation must get the same
  rotation, which is linear()'s `group` argument: rot(x) @ (W R)^T = x R R^T W^T = x W^T.
- Group-128 INT8: `<layer>.weight` int8 (N, K) with `<layer>.weight_scale` (N, ceil(K / 128)), one scale per output
  channel and 128-element block of K; linear() takes such scales directly (the 'exact' and 'block' paths).

Every adapter returns an `Int8Weight`: the INT8 matrix as stored (never copied or dequantized), its FP32 scales in the
layout linear() takes, the bias in the activation dtype, and the rotation group.
"""
from dataclasses import dataclass
from typing import Mapping, Optional

import torch

ROTATION_GROUPS = (16, 64, 256)
WEIGHT_BLOCK = 128


@dataclass
class Int8Weight:
    """One INT8 linear's parameters in the form linear() takes."""
    weight: torch.Tensor                  # int8 (N, K), as stored
    scale: torch.Tensor                   # float32 (N,) or (N, ceil(K / 128))
    bias: Optional[torch.Tensor] = None   # (N,) in the activation dtype, or None
    group: int = 0                        # ConvRot rotation group of the activation (0: none)

    @property
    def out_features(self):
        return self.weight.shape[0]

    @property
    def in_features(self):
        return self.weight.shape[1]

    @property
    def block_scales(self):
        return self.scale.dim() == 2

    def to(self, device=None, dtype=None):
        """Moves the tensors to `device`; `dtype` is the activation dtype the bias is cast to (the INT8 weight and the
        FP32 scales keep theirs)."""
        bias = self.bias
        if bias is not None:
            bias = bias.to(device=device, dtype=dtype or bias.dtype)
        return Int8Weight(self.weight.to(device), self.scale.to(device), bias, self.group)

    def linear(self, x, **kwargs):
        """linear(x, ...) with this weight: the rotation group and the bias come from the checkpoint."""
        from . import linear
        bias = self.bias if self.bias is None or self.bias.dtype == x.dtype else self.bias.to(x.dtype)
        return linear(x, self.weight, self.scale, bias, group=self.group, **kwargs)


def _check_weight(weight, name):
    if weight.dtype != torch.int8 or weight.dim() != 2:
        raise ValueError(f"{name}: expected an int8 (N, K) matrix, got {weight.dtype} {tuple(weight.shape)}")
    if weight.shape[1] % 16:
        raise ValueError(f"{name}: K = {weight.shape[1]} is not a multiple of 16")
    return weight.contiguous()


def channel_scales(scale, n, name="scale"):
    """Per-channel scales in any float dtype, shaped (N,), (N, 1) or (1, N) (Quanto keeps (N, 1)), as FP32 (N,)."""
    if not scale.is_floating_point() or scale.numel() != n:
        raise ValueError(f"{name}: expected {n} per-channel float scales, got {scale.dtype} {tuple(scale.shape)}")
    return scale.reshape(n).to(torch.float32).contiguous()


def block_scales(scale, n, k, name="scale"):
    """Per-(channel, 128-element K block) scales as FP32 (N, ceil(K / 128))."""
    blocks = (k + WEIGHT_BLOCK - 1) // WEIGHT_BLOCK
    if not scale.is_floating_point() or tuple(scale.shape) != (n, blocks):
        raise ValueError(f"{name}: expected float scales of shape {(n, blocks)} (one per channel and {WEIGHT_BLOCK}-element block of "
                         f"K = {k}), got {scale.dtype} {tuple(scale.shape)}")
    return scale.to(torch.float32).contiguous()


def _get(tensors, key, required=True):
    value = tensors.get(key)
    if value is None and required:
        raise KeyError(f"checkpoint has no tensor {key!r}")
    return value


def from_quanto(tensors: Mapping[str, torch.Tensor], prefix: str) -> Int8Weight:
    """A Quanto qint8 linear: `prefix.weight._data` int8 (N, K), `prefix.weight._scale` (N, 1), optional `prefix.bias`."""
    weight = _check_weight(_get(tensors, f"{prefix}.weight._data"), f"{prefix}.weight._data")
    scale = channel_scales(_get(tensors, f"{prefix}.weight._scale"), weight.shape[0], f"{prefix}.weight._scale")
    return Int8Weight(weight, scale, _get(tensors, f"{prefix}.bias", False))


def from_convrot(tensors: Mapping[str, torch.Tensor], prefix: str, group: int) -> Int8Weight:
    """A ConvRot linear: an INT8 weight quantized after the group rotation of K, per-channel scales, and the rotation
    group (16, 64 or 256) the activations need. Takes Quanto's keys (`weight._data` / `weight._scale`) or plain ones
    (`weight` / `weight_scale`)."""
    if group not in ROTATION_GROUPS:
        raise ValueError(f"ConvRot group must be one of {ROTATION_GROUPS}, not {group}")
    if f"{prefix}.weight._data" in tensors:
        loaded = from_quanto(tensors, prefix)
    else:
        weight = _check_weight(_get(tensors, f"{prefix}.weight"), f"{prefix}.weight")
        loaded = Int8Weight(weight, channel_scales(_get(tensors, f"{prefix}.weight_scale"), weight.shape[0], f"{prefix}.weight_scale"),
                            _get(tensors, f"{prefix}.bias", False))
    if loaded.in_features % group:
        raise ValueError(f"{prefix}: K = {loaded.in_features} is not a multiple of the rotation group {group}")
    loaded.group = group
    return loaded


def from_group128(tensors: Mapping[str, torch.Tensor], prefix: str) -> Int8Weight:
    """A group-128 INT8 linear (Hunyuan's DiT checkpoints): `prefix.weight` int8 (N, K) and `prefix.weight_scale`
    (N, ceil(K / 128)), optional `prefix.bias`."""
    weight = _check_weight(_get(tensors, f"{prefix}.weight"), f"{prefix}.weight")
    n, k = weight.shape
    scale = block_scales(_get(tensors, f"{prefix}.weight_scale"), n, k, f"{prefix}.weight_scale")
    return Int8Weight(weight, scale, _get(tensors, f"{prefix}.bias", False))


def load(tensors: Mapping[str, torch.Tensor], prefix: str, group: int = 0) -> Int8Weight:
    """Recognizes the layout of `prefix`'s tensors: Quanto keys, or a plain INT8 weight with per-channel or group-128
    scales. `group` > 0 marks a ConvRot checkpoint."""
    if group:
        return from_convrot(tensors, prefix, group)
    if f"{prefix}.weight._data" in tensors:
        return from_quanto(tensors, prefix)
    scale = _get(tensors, f"{prefix}.weight_scale")
    if scale.dim() == 2 and scale.shape[1] > 1:
        return from_group128(tensors, prefix)
    weight = _check_weight(_get(tensors, f"{prefix}.weight"), f"{prefix}.weight")
    return Int8Weight(weight, channel_scales(scale, weight.shape[0], f"{prefix}.weight_scale"), _get(tensors, f"{prefix}.bias", False))


def load_safetensors(path, prefixes, device="cuda", dtype=torch.bfloat16, group=0):
    """Int8Weight per prefix from a .safetensors file (read without executing anything from it), on `device`, biases in
    `dtype`."""
    from safetensors.torch import load_file
    tensors = load_file(str(path))
    return {prefix: load(tensors, prefix, group).to(device, dtype) for prefix in prefixes}


class Int8Linear(torch.nn.Module):
    """A torch module over one Int8Weight: forward(x) = linear(x, ...) on x's leading dimensions flattened to rows."""

    def __init__(self, weight: Int8Weight, **linear_kwargs):
        super().__init__()
        self.register_buffer("weight", weight.weight)
        self.register_buffer("scale", weight.scale)
        self.register_buffer("bias", weight.bias)
        self.group = weight.group
        self.linear_kwargs = linear_kwargs

    def forward(self, x, **kwargs):
        from . import linear
        rows = x.reshape(-1, x.shape[-1])
        if not rows.is_contiguous():
            rows = rows.contiguous()
        bias = self.bias if self.bias is None or self.bias.dtype == x.dtype else self.bias.to(x.dtype)
        y = linear(rows, self.weight, self.scale, bias, group=self.group, **{**self.linear_kwargs, **kwargs})
        return y.reshape(*x.shape[:-1], self.weight.shape[0])


# ---- writers: the same layouts from a float weight (used to make checkpoints and by the tests) ----------------------
def rotation(group, device=None):
    """The ConvRot group rotation: Kronecker power of H4 (ones with a negated anti-diagonal) over `group` values, scaled
    by group^-1/2 (orthonormal)."""
    h4 = torch.ones(4, 4, device=device)
    h4[torch.arange(4), 3 - torch.arange(4)] = -1.0
    r = h4
    while r.shape[0] < group:
        r = torch.kron(r, h4)
    return r / group ** 0.5


def quantize_channels(w):
    """Symmetric per-channel INT8 of a float (N, K) weight: (int8 (N, K), FP32 scales (N,) = amax / 127)."""
    w = w.float()
    scale = w.abs().amax(dim=1) / 127
    safe = torch.where(scale > 0, scale, torch.ones_like(scale))
    return torch.round(w / safe[:, None]).clamp(-127, 127).to(torch.int8), scale


def quantize_blocks_of_k(w):
    """Symmetric INT8 of a float (N, K) weight with one scale per channel and 128-element block of K."""
    w = w.float()
    n, k = w.shape
    blocks = (k + WEIGHT_BLOCK - 1) // WEIGHT_BLOCK
    padded = torch.nn.functional.pad(w, (0, blocks * WEIGHT_BLOCK - k)).reshape(n, blocks, WEIGHT_BLOCK)
    scale = padded.abs().amax(dim=2) / 127
    safe = torch.where(scale > 0, scale, torch.ones_like(scale))
    q = torch.round(padded / safe[..., None]).clamp(-127, 127).reshape(n, blocks * WEIGHT_BLOCK)[:, :k]
    return q.to(torch.int8).contiguous(), scale


def quanto_tensors(prefix, w, bias=None, dtype=torch.bfloat16):
    """The Quanto qint8 tensors of a float weight (scale (N, 1) in `dtype`, as Quanto stores it)."""
    q, scale = quantize_channels(w)
    out = {f"{prefix}.weight._data": q, f"{prefix}.weight._scale": scale.to(dtype)[:, None]}
    if bias is not None:
        out[f"{prefix}.bias"] = bias.to(dtype)
    return out


def convrot_tensors(prefix, w, group, bias=None, dtype=torch.bfloat16):
    """ConvRot tensors of a float weight: W rotated over K in groups (W @ R per group), then per-channel INT8."""
    n, k = w.shape
    rotated = (w.float().reshape(n, k // group, group) @ rotation(group, w.device)).reshape(n, k)
    q, scale = quantize_channels(rotated)
    out = {f"{prefix}.weight": q, f"{prefix}.weight_scale": scale}
    if bias is not None:
        out[f"{prefix}.bias"] = bias.to(dtype)
    return out


def group128_tensors(prefix, w, bias=None, dtype=torch.bfloat16):
    """Group-128 INT8 tensors of a float weight."""
    q, scale = quantize_blocks_of_k(w)
    out = {f"{prefix}.weight": q, f"{prefix}.weight_scale": scale}
    if bias is not None:
        out[f"{prefix}.bias"] = bias.to(dtype)
    return out
