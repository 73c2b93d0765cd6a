"""PyTorch-CPU FP32 restatement of the reference's numerical definition -- TEST INFRASTRUCTURE ONLY.

Used by tests/ (tolerance checks), __graft_entry__.smoke() and bench.py's cpu_baseline leg; never by the product path.

- ``reference_linear``: the reference's FP32 reference of linear() (wgpkernels/int8/__init__.py:523-539, I:579-584 for
  ConvRot): op(x) -> rotation -> optional rounding to x's dtype -> x @ (w * scale).T + bias -> residual.
- ``block_linear``: the same with the block path's activation quantization (one scale per row and 128-element block,
  K8:392-409 of wgpkernels/int8/int8_gemm.cu) applied before the FP32 dequantize-and-matmul: the definition the CPU
  baseline times. It uses torch's own tanh-GELU, so its codes can differ from the GPU's (which follow the C oracle) in
  rare rounding ties; it is a timing and tolerance baseline, not a bit-exact one.
"""
import torch


def op(x, act=None, act_weight=None, eps=0.0):
    v = x.float()
    if act == "swiglu":
        gate, value = v.chunk(2, dim=-1)
        v = torch.nn.functional.silu(gate) * value
    elif act == "rms_norm":
        v = v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + eps) * (1 if act_weight is None else act_weight.float())
    elif act == "gelu":
        v = torch.nn.functional.gelu(v, approximate="tanh")
    return v


def rotation(group, device="cpu"):
    h = torch.ones(4, 4, device=device) - 2 * torch.eye(4, device=device).flip(0)
    r = h
    while r.shape[0] < group:
        r = torch.kron(r, h)
    return r * group ** -0.5


def weight_scale(s, k):
    return s.repeat_interleave(128, dim=1)[:, :k] if s.dim() == 2 else s[:, None]


def reference_linear(x, w, s, bias=None, group=0, act=None, act_weight=None, eps=0.0, residual=None, residual_scale=None,
                     round_input=False):
    v = op(x, act, act_weight, eps)
    if group:
        v = (v.reshape(v.shape[0], -1, group) @ rotation(group, v.device)).reshape(v.shape)
    if round_input:
        v = v.to(x.dtype).float()
    out = v @ (w.float() * weight_scale(s, w.shape[1])).T
    if bias is not None:
        out = out + bias.float()
    if residual is not None:
        out = residual.float() + (1 if residual_scale is None else residual_scale.float()) * out
    return out


def quantize_blocks(v):
    """Per-row, per-128-block symmetric INT8 of an FP32 matrix: (q as float, scale (M, ceil(K/128)))."""
    m, k = v.shape
    kb = (k + 127) // 128
    padded = torch.nn.functional.pad(v, (0, kb * 128 - k)).reshape(m, kb, 128)
    amax = padded.abs().amax(-1)
    inv = torch.where(amax > 0, 127.0 / amax, torch.zeros_like(amax))
    q = torch.round(padded * inv[..., None])
    return q.reshape(m, kb * 128)[:, :k], amax / 127.0


def block_linear(x, w, s, bias=None, act=None, act_weight=None, eps=0.0, residual=None, residual_scale=None):
    """FP32 dequantize-and-matmul of the block-quantized op(x) (the reference's block math, in torch)."""
    v = op(x, act, act_weight, eps)
    q, sa = quantize_blocks(v)
    deq = q * sa.repeat_interleave(128, dim=1)[:, :v.shape[1]]
    out = deq @ (w.float() * weight_scale(s, w.shape[1])).T
    if bias is not None:
        out = out + bias.float()
    if residual is not None:
        out = residual.float() + (1 if residual_scale is None else residual_scale.float()) * out
    return out
