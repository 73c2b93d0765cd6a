"""GPU runs of the checkpoint formats (Quanto INT8, ConvRot, group-128) through their adapters, on synthetic tensors of
each layout made from a float weight:
- the adapter passes linear() exactly the arguments the raw tensors mean (bit-identical outputs);
- the result approximates x @ W.T of the float weight within the weight quantization's error (for ConvRot: only with
  the checkpoint's rotation group; without it the output is unrelated), on each path the format supports;
- the module wrapper flattens leading dimensions."""
import pytest
import torch

from conftest import rel_err

pytestmark = pytest.mark.gpu


def float_weight(n, k, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(n, k, generator=g) / k ** 0.5, 0.02 * torch.randn(n, generator=g)


def inputs(m, k, seed):
    g = torch.Generator().manual_seed(seed + 1)
    return torch.randn(m, k, generator=g).bfloat16()


@pytest.mark.parametrize("fmt", ["quanto", "convrot16", "convrot64", "convrot256", "group128"])
def test_format_through_linear(wq, fmt):
    from wgpkernels_amd.int8 import checkpoint as ck
    n, k = 768, 1536
    w, bias = float_weight(n, k, seed=len(fmt))
    group = int(fmt[7:]) if fmt.startswith("convrot") else 0
    tensors = {"quanto": lambda: ck.quanto_tensors("l", w, bias), "group128": lambda: ck.group128_tensors("l", w, bias)}.get(
        fmt, lambda: ck.convrot_tensors("l", w, group, bias))()
    loaded = ck.load(tensors, "l", group).to("cuda", torch.bfloat16)
    paths = ("exact", "block") if fmt == "group128" else ("lines", "small", "exact", "block")
    for m, path in [(m, p) for p in paths for m in ((2,) if p == "lines" else (16,) if p == "small" else (300,))]:
        print(f"checkpoint {fmt} path={path} m={m}", flush=True)
        x = inputs(m, k, seed=m)
        xc = x.cuda()
        y = loaded.linear(xc, mode=path)
        raw = wq.linear(xc, loaded.weight, loaded.scale, loaded.bias, group=group, mode=path)
        torch.cuda.synchronize()
        assert torch.equal(y, raw)
        ref = x.float() @ w.T + bias.bfloat16().float()
        err = rel_err(y.cpu().float(), ref)
        assert err < (3e-2 if path == "block" else 1.5e-2), err
        if group:
            unrotated = wq.linear(xc, loaded.weight, loaded.scale, loaded.bias, mode=path)
            assert rel_err(unrotated.cpu().float(), ref) > 0.5


def test_module_wrapper(wq):
    from wgpkernels_amd.int8 import checkpoint as ck
    w, bias = float_weight(256, 512, seed=9)
    module = ck.Int8Linear(ck.load(ck.quanto_tensors("l", w, bias), "l").to("cuda", torch.bfloat16))
    x = torch.randn(2, 3, 512).bfloat16().cuda()
    y = module(x, mode="exact")
    assert y.shape == (2, 3, 256)
    flat = wq.linear(x.reshape(6, 512), module.weight, module.scale, module.bias, mode="exact")
    assert torch.equal(y.reshape(6, 256), flat)
