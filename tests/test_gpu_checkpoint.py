"""GPU parity of FP8 layers that come from a checkpoint rather than from quantizing a Linear:
the on-disk format (tfp8.save_fp8 / load_fp8) loaded onto the device, and
FP8Linear.from_fp8_checkpoint (tfp8/linear.py:82-98) with a per-tensor (scalar) scale and with
float8_e4m3fn / float8_e5m2-typed codes (tests/test_tfp8.py:309-319 covers the CPU side in the
reference).  Loaded codes and scales must be bit-identical to what was saved, and the GEMV (M=1)
and GEMM (M=40) outputs on the device within the reference tolerance of the float64 oracle."""
import os

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import fp8_oracle as O
from tfp8 import load_fp8, save_fp8
from tfp8.linear import FP8Linear

pytestmark = pytest.mark.gpu
DTN = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}


def _check(layer, x, label):
    y = layer(x)
    torch.cuda.synchronize()
    ref = O.linear_ref64(x.float().cpu().numpy().astype(np.float64), layer.qweight.cpu().numpy(),
                         layer.weight_scale.cpu().numpy(), layer.group_size, layer.fmt,
                         None if layer.bias_f32 is None else layer.bias_f32.cpu().numpy())
    d = np.abs(y.double().cpu().numpy() - ref)
    tol = O.tolerance(ref, DTN[layer.out_dtype])
    assert (d <= tol).all(), f"{label}: max excess {float((d - tol).max()):.3g}"


class _Net(nn.Module):
    def __init__(self):
        super().__init__()
        self.chan = nn.Linear(512, 384)              # per-channel f32 scales, E4M3FN
        self.grp = nn.Linear(512, 256, bias=False)   # 32-groups, UE8M0 scales, E5M2
        self.tensor = nn.Linear(256, 128)            # per-tensor scale from an FP8 checkpoint
        self.norm = nn.LayerNorm(128)


def _converted(seed):
    torch.manual_seed(seed)
    net = _Net()
    with torch.no_grad():
        for lin in (net.chan, net.grp, net.tensor):
            lin.weight.mul_(0.5)
    net.chan = FP8Linear.from_linear(net.chan, "e4m3fn")
    net.grp = FP8Linear.from_linear(net.grp, "e5m2", group_size=32, scale_format="ue8m0")
    codes = torch.randint(0, 0x7E, (128, 256), dtype=torch.uint8)          # finite E4M3FN codes
    codes[torch.rand(128, 256) < 0.5] |= 0x80
    net.tensor = FP8Linear.from_fp8_checkpoint(codes.view(torch.float8_e4m3fn), torch.tensor(0.0078125),
                                               net.tensor.bias.detach(), fmt="e4m3fn")
    return net


def test_checkpoint_round_trip_onto_gpu(tmp_path):
    print("[checkpoint] save_fp8 -> load_fp8 onto cuda", flush=True)
    src = _converted(31)
    path = os.path.join(tmp_path, "net.safetensors")
    save_fp8(src, path)
    dst = load_fp8(_Net(), path, device="cuda")
    dst.norm.cuda()
    layouts = {"chan": ("e4m3fn", 512, torch.float32), "grp": ("e5m2", 32, torch.uint8),
               "tensor": ("e4m3fn", 256, torch.float32)}
    for name, (fmt, G, sdt) in layouts.items():
        a, b = getattr(src, name), getattr(dst, name)
        assert isinstance(b, FP8Linear) and b.qweight.is_cuda
        assert (b.fmt, b.group_size, b.weight_scale.dtype) == (fmt, G, sdt), name
        assert torch.equal(b.qweight.cpu(), a.qweight) and torch.equal(b.weight_scale.cpu(), a.weight_scale)
        assert (b.bias_f32 is None) == (a.bias_f32 is None)
        if a.bias_f32 is not None:
            assert torch.equal(b.bias_f32.cpu(), a.bias_f32)
    assert bool((dst.tensor.weight_scale == 0.0078125).all()) and dst.tensor.weight_scale.shape == (128, 1)
    assert torch.equal(dst.norm.weight.cpu(), src.norm.weight)
    g = torch.Generator().manual_seed(32)
    for M in (1, 40):
        for name in layouts:
            layer = getattr(dst, name)
            layer.out_dtype = torch.float32
            x = torch.randn(M, layer.in_features, generator=g).bfloat16().cuda()
            _check(layer, x, f"{name} M={M}")
    assert dst.chan.stats["gemv"] == 1 and dst.chan.stats["gemm"] == 1


@pytest.mark.parametrize("fmt", ["e4m3fn", "e5m2"])
def test_from_fp8_checkpoint_per_tensor_and_float8_codes(fmt):
    """A scalar f32 scale (per tensor, expanded to one scale per row as tfp8/linear.py:91 does) and
    codes given as torch float8 tensors of the declared format, run on the device."""
    print(f"[from_fp8_checkpoint] per-tensor {fmt}", flush=True)
    torch.manual_seed(33)
    tdt = torch.float8_e4m3fn if fmt == "e4m3fn" else torch.float8_e5m2
    w = (torch.randn(320, 1024) * 0.05).to(tdt)            # float8-typed weight codes
    scale = torch.tensor(0.75)                              # not a power of two
    bias = torch.randn(320) * 0.1
    layer = FP8Linear.from_fp8_checkpoint(w.cuda(), scale.cuda(), bias.cuda(), fmt=fmt, out_dtype=torch.float32)
    assert torch.equal(layer.qweight.cpu(), w.view(torch.uint8))
    assert layer.weight_scale.shape == (320, 1) and bool((layer.weight_scale == 0.75).all())
    g = torch.Generator().manual_seed(34)
    # (fp32 activations only at M <= 8: the GEMV multiplies them as given, the GEMM path would
    # first round them to fp16 with a row scale)
    for M, xdt in ((1, torch.bfloat16), (40, torch.float16), (3, torch.float32)):
        _check(layer, torch.randn(M, 1024, generator=g).to(xdt).cuda(), f"per-tensor {fmt} M={M} {xdt}")
    # per-channel [N] f32 scales with float8 codes, and a mismatched float8 dtype is refused
    sc = torch.rand(320) + 0.25
    lc = FP8Linear.from_fp8_checkpoint(w.cuda(), sc.cuda(), None, fmt=fmt, out_dtype=torch.float32)
    assert torch.equal(lc.weight_scale[:, 0].cpu(), sc)
    _check(lc, torch.randn(40, 1024, generator=g).bfloat16().cuda(), f"per-channel {fmt}")
    other = "e5m2" if fmt == "e4m3fn" else "e4m3fn"
    with pytest.raises(ValueError):
        FP8Linear.from_fp8_checkpoint(w.cuda(), scale, fmt=other)
