"""Symmetric FP8 weight quantization and the activation row scale (API of tfp8/quantize.py:1-62).

    scale = max|w| / FP8_MAX   (rounded up to a power of two by default)
    q     = RNE(clamp(w / scale, -FP8_MAX, FP8_MAX))

Scales are float32, or UE8M0 bytes (scale = 2^(byte-127), always a power of two) when
`scale_format="ue8m0"`.  CUDA tensors run the gfx950 quantize / dequant / prep kernels; CPU
tensors run the torch code here, which computes the same numbers.
"""
import torch

from . import _ext
from .formats import _table, encode, get_format

SCALE_FORMATS = ("f32", "ue8m0")


def pow2_ceil(s: torch.Tensor) -> torch.Tensor:
    """2^ceil(log2 s) through torch's fp32 log2, the formula of tfp8/quantize.py:11-12.

    A value a few ULP above a power of two 2^k can have an fp32 log2 that rounds to exactly k, and
    then the result is 2^k (below s), not 2^(k+1); the gfx950 kernels reproduce that rounding
    (ceil_log2_ref in tfp8_common.h), so CPU and GPU give the same scales as the reference."""
    return torch.exp2(torch.ceil(torch.log2(s)))


def ue8m0_encode(s: torch.Tensor) -> torch.Tensor:
    """Power-of-two scale -> UE8M0 byte ceil(log2 s) + 127, clamped to [0, 254]; NaN -> 255
    (fp8_cuda.py:85-88 encode rule, fp8_gemm_kernel.cu:22-30 decode rule)."""
    _, e = torch.frexp(pow2_ceil(s.float()))
    b = (e - 1).clamp(-127, 127) + 127
    return torch.where(torch.isnan(s), torch.full_like(b, 255), b).to(torch.uint8)


def ue8m0_decode(b: torch.Tensor) -> torch.Tensor:
    e = b.to(torch.int32) - 127
    v = torch.ldexp(torch.ones(b.shape, dtype=torch.float32, device=b.device), e)
    return torch.where(b == 255, torch.full_like(v, float("nan")), v)


def scale_values(s: torch.Tensor) -> torch.Tensor:
    """float32 view of a weight_scale tensor of either storage (f32 or UE8M0 bytes)."""
    return ue8m0_decode(s) if s.dtype == torch.uint8 else s.float()


def quantize_weight(w: torch.Tensor, fmt="e4m3fn", group_size=None, pow2_scale=True, scale_format="f32"):
    """w [N,K] -> (qweight uint8 [N,K], scale [N, K/G], G).

    group_size None -> one scale per output channel (G = K). scale is float32, or uint8 UE8M0
    bytes for scale_format="ue8m0" (which implies power-of-two scales).
    Runs on whatever device w lives on; call it layer by layer so the full-precision model
    never has to sit in VRAM next to the quantized one.
    """
    f = get_format(fmt)
    if scale_format not in SCALE_FORMATS:
        raise ValueError(f"scale_format must be one of {SCALE_FORMATS}, got {scale_format!r}")
    N, K = w.shape
    G = K if group_size is None else group_size
    if G <= 0 or K % G:
        raise ValueError(f"K={K} not divisible by group_size={G}")
    ue8m0 = scale_format == "ue8m0"
    if w.is_cuda:
        q, s = _ext.quantize_weight(w, f.name, G, pow2_scale, ue8m0)
        return q, s, G
    wg = w.float().reshape(N, K // G, G)
    amax = wg.abs().amax(-1)
    s = (amax / f.max_finite).clamp_min(torch.finfo(torch.float32).tiny)
    if pow2_scale or ue8m0:
        s = pow2_ceil(s)
    s = torch.where(amax == 0, torch.ones_like(s), s)
    q = encode(wg / s[..., None], f).reshape(N, K)   # the encoder saturates = clamp then RNE
    s = s.contiguous()
    return q.contiguous(), (ue8m0_encode(s) if ue8m0 else s), G


def dequantize_weight(q: torch.Tensor, s: torch.Tensor, fmt, group_size) -> torch.Tensor:
    """Dequantization to float32 [N,K]. Never used on the forward hot path."""
    f = get_format(fmt)
    N, K = q.shape
    if q.is_cuda:
        out = torch.empty(N, K, dtype=torch.float32, device=q.device)
        return _ext.dequant_into(out, q.contiguous(), None, s.contiguous(), group_size, f.name)
    v = _table(f)[q.long()].reshape(N, K // group_size, group_size)
    return (v * scale_values(s)[..., None]).reshape(N, K)


ACT_TARGET_EXP = 8  # row amax is mapped into [2^7, 2^8): far from fp16 overflow, ~30 binades of headroom


def activation_to_fp16(x: torch.Tensor):
    """BF16/FP32 activation rows -> (fp16 [M,K], power-of-two row scale f32 [M]).

    Dividing by an exact power of two is lossless, so BF16 -> FP16 only loses values that
    would land in fp16's subnormal range. FP16 input passes through.
    """
    if x.dtype == torch.float16:
        return x.contiguous(), torch.ones(x.shape[0], dtype=torch.float32, device=x.device)
    if x.is_cuda:
        return _ext.prepare_activations(x)
    amax = x.abs().amax(-1).float()
    e = torch.ceil(torch.log2(amax.clamp_min(2.0 ** -100))) - ACT_TARGET_EXP   # quantize.py:58-60
    e = torch.where(amax > 0, e, torch.zeros_like(e))
    xs = torch.exp2(e)
    return (x.float() / xs[:, None]).half().contiguous(), xs.contiguous()
