"""The reference's CPU FP8Linear forward, restated in torch (CPU) -- TEST INFRASTRUCTURE ONLY.

y = F.linear(x.float(), lut[q.long()].float() * scale[n, k//G], bias_f32).to(out_dtype)
following tfp8/linear.py:179-181 with tfp8/quantize.py:39-44 (dequantize_weight: fp16 table
gather, f32 widen, f32 scale multiply) and tfp8/formats.py:63-69 (the 256-entry fp16 table).
UE8M0 scales are widened with the fp8_gemm_kernel.cu:22-30 rule.  This is the CPU baseline that
bench.py times beside the GPU kernels, and a second (fp32, host BLAS) parity reference.
"""
import numpy as np
import torch
import torch.nn.functional as F

from . import fp8_oracle as O


def lut16(fmt):
    """fp16 table built from the oracle decode (tfp8/formats.py:63-69)."""
    return torch.from_numpy(O.lut_f16_bits(fmt).view(np.float16).copy())


def cpu_forward(x, q, s, group_size, fmt, bias, out_dtype, table=None):
    """One full reference CPU forward; the fp32 weight is re-materialised per call, as in the
    reference (tfp8/linear.py:104-105, 179-181)."""
    table = lut16(fmt) if table is None else table
    N, K = q.shape
    sv = torch.from_numpy(O.ue8m0_decode(s.numpy())) if s.dtype == torch.uint8 else s.float()
    W = (table[q.long()].float().reshape(N, K // group_size, group_size) * sv[..., None]).reshape(N, K)
    return F.linear(x.float(), W, bias).to(out_dtype)


def dequant_weight_f32(q, s, group_size, fmt):
    """lut[q].float() * scale[n, k//G] on q's own device (tfp8/quantize.py:39-44), so the reference
    forward can run as an fp32 GPU matmul for model-sized checks.  UE8M0 bytes widen as the
    oracle does (255 -> NaN, b -> 2^(b-127), exact through ldexp)."""
    table = lut16(fmt).to(q.device)
    if s.dtype == torch.uint8:
        e = s.to(torch.int32)
        sv = torch.ldexp(torch.ones(e.shape, dtype=torch.float32, device=e.device), e - 127)
        sv = torch.where(e == 255, torch.full_like(sv, float("nan")), sv)
    else:
        sv = s.float()
    N, K = q.shape
    return (table[q.long()].float().reshape(N, K // group_size, group_size) * sv[..., None]).reshape(N, K)


def ref_linear(x, W, bias, out_dtype):
    """The reference CPU forward's arithmetic (tfp8/linear.py:179-181) on a pre-dequantized weight."""
    return F.linear(x.float(), W, bias).to(out_dtype)
