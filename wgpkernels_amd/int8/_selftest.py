"""selftest(): the API-level gate a caller runs before trusting the kernels on a GPU (the reference's wgpkernels/int8/
__init__.py:542-576 has the same contract: None when every kernel agrees with PyTorch, else the reason).

Each path runs on small random inputs through its fixed tiles (both tile sizes of every GEMM mode, no tuning), over a
rotation of input operations, ConvRot groups and residual epilogues, in BF16 and FP16. Outputs are compared with an
FP32 PyTorch reference by norm-relative error: 5e-3 for the full-precision paths, 3e-2 for the one-pass 'block' and
'row' paths (the reference's bounds, wgpkernels/int8/__init__.py:572-573).
"""
import torch

ACTS = (None, "rms_norm", "swiglu", "gelu")
GROUPS = (0, 16, 64, 256)
# path -> token count, fixed tiles (variant ids) of the GEMM modes
PATHS = {"lines": (3, ()), "small": (5, ()), "exact": (40, (1, 7)), "block": (40, (10, 11)), "row": (40, (0, 6)),
         "exact+g": (40, (14,)), "block+g": (40, (12, 13))}
K, N = 256, 96
TOLERANCE = {"lines": 5e-3, "small": 5e-3, "exact": 5e-3, "exact+g": 5e-3, "block": 3e-2, "block+g": 3e-2, "row": 3e-2}


def reference_rotation(v, group):
    """ConvRot over groups of `group` values: the Kronecker power of the 4x4 Hadamard-like matrix H4 (ones with a
    negated anti-diagonal), scaled by group^-1/2 (an orthonormal rotation)."""
    h4 = torch.ones(4, 4, device=v.device)
    h4[torch.arange(4), 3 - torch.arange(4)] = -1.0
    rotation = h4
    while rotation.shape[0] < group:
        rotation = torch.kron(rotation, h4)
    return (v.reshape(v.shape[0], -1, group) @ rotation).reshape(v.shape) / group ** 0.5


def apply_op(v, act, act_weight, eps):
    """op(x) in FP32: RMSNorm (times an optional weight), SwiGLU over rows [gate | value], or tanh-GELU."""
    if act == "rms_norm":
        v = v / torch.sqrt(v.square().mean(dim=-1, keepdim=True) + eps)
        return v if act_weight is None else v * act_weight.float()
    if act == "swiglu":
        gate, value = v[:, :v.shape[1] // 2], v[:, v.shape[1] // 2:]
        return gate * torch.sigmoid(gate) * value
    if act == "gelu":
        return torch.nn.functional.gelu(v, approximate="tanh")
    return v


def reference_linear(x, w, s, bias, group, act, act_weight, eps, residual, residual_scale, round_input):
    """FP32 linear(): op, rotation, optional rounding of the op's result to x's dtype (the few-token paths keep it in
    16 bits), dequantized weights (per channel or per channel and 128-element block), bias, residual epilogue."""
    v = apply_op(x.float(), act, act_weight, eps)
    if group:
        v = reference_rotation(v, group)
    if round_input:
        v = v.to(x.dtype).float()
    wf = w.float()
    if s.dim() == 2:
        wf = wf * torch.repeat_interleave(s, 128, dim=1)[:, :w.shape[1]]
    else:
        wf = wf * s[:, None]
    y = v @ wf.T
    if bias is not None:
        y = y + bias.float()
    if residual is not None:
        y = residual.float() + (y if residual_scale is None else residual_scale.float() * y)
    return y


def _cases():
    """(path, variant, tokens, act, group, residual) rotating acts, groups and residuals over every path and tile."""
    index = 0
    for path, (tokens, variants) in PATHS.items():
        for variant in variants or (None,):
            for repeat in range(2):
                act = ACTS[(index + repeat) % len(ACTS)]
                group = GROUPS[(3 * index + repeat) % len(GROUPS)]
                yield path, variant, tokens, act, group, (index + repeat) % 2 == 1
            index += 1


def selftest(device=None):
    """Runs every kernel once on small inputs: None when all match PyTorch, else a description of the first mismatch."""
    from . import gemm, library, linear_prepared, prepare, weight_groups_supported
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    library()
    rng = torch.Generator(device=device).manual_seed(0)
    for dtype in (torch.bfloat16, torch.float16):
        w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=device, generator=rng)
        channel_scale = (torch.rand(N, device=device, generator=rng) + 0.5) / 127
        block_scale = (torch.rand(N, (K + 127) // 128, device=device, generator=rng) + 0.5) / 127
        bias = torch.randn(N, device=device, generator=rng).to(dtype)
        norm_weight = (torch.rand(K, device=device, generator=rng) + 0.5).to(dtype)
        for path, variant, tokens, act, group, with_residual in _cases():
            groups = path.endswith("+g")
            if groups and not weight_groups_supported():
                continue
            x = torch.randn(tokens, 2 * K if act == "swiglu" else K, device=device, generator=rng).to(dtype)
            act_weight = norm_weight if act == "rms_norm" else None
            residual = (4 * torch.randn(tokens, N, device=device, generator=rng)).to(dtype) if with_residual else None
            rscale = torch.rand(N, device=device, generator=rng).to(dtype) if with_residual else None
            scale = block_scale if groups else channel_scale
            ref = reference_linear(x, w, scale, bias, group, act, act_weight, 1e-6, residual, rscale, path in ("lines", "small"))
            prepared = prepare(x, group, path.removesuffix("+g"), act, act_weight, 1e-6)
            out = residual  # written in place of the residual when there is one
            if variant is None:
                y = linear_prepared(prepared, w, scale, bias, residual, rscale, out)
            else:
                y = gemm(prepared.x, prepared.lo, prepared.scale, w, scale, bias, dtype, 0, variant, out=out, residual=residual,
                         residual_scale=rscale)
            error = ((y.float() - ref).norm() / ref.norm()).item()
            if not error < TOLERANCE[path]:
                return (f"{path} kernel mismatch ({dtype}, {tokens} rows{f', tiles {variant}' if variant is not None else ''}, group {group}, "
                        f"{act or 'no input op'}{', residual' if with_residual else ''}): relative error {error:.3g}")
    torch.cuda.synchronize(device)
    return None
