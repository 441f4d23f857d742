"""Weight quantization to FP8 codes with per-row / per-K-group scales, its inverse, and the
power-of-two row rescale of activations (functions of the reference's tfp8/quantize.py:1-62).

For every weight row n and group g of G consecutive inputs the scale is the group's largest
magnitude divided by the format's largest finite value (raised to a power of two unless
pow2_scale=False; 1 for an all-zero group), and each code is the round-to-nearest-even FP8 value
of w / scale, saturated at the largest finite code.  Scales are stored as float32, or with
scale_format="ue8m0" as one byte e per scale meaning 2^(e-127).  On a CUDA tensor the gfx950
kernels (quantize, dequant, prep) do the work; on a CPU tensor the torch code below does, with
identical results.
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
    """Quantize a [N, K] weight: returns (codes uint8 [N, K], scales [N, K // G], G).

    G = K (one scale per output row) when group_size is None.  Scales come back as float32, or as
    UE8M0 bytes for scale_format="ue8m0", which always uses power-of-two scales.  The work happens
    on w's device, so a model can be converted one layer at a time without holding a second
    full-precision copy.
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


ACT_TARGET_EXP = 8  # a row's largest magnitude lands in (2^7, 2^8]: fp16 keeps ~7 binades above it, ~30 below


def activation_to_fp16(x: torch.Tensor):
    """Rescale each activation row by a power of two so it fits fp16: returns (x16 fp16 [M, K],
    xs f32 [M]) with x = x16 * xs.

    The division by 2^e is exact, so only entries far below the row maximum (in fp16's subnormal
    range after the shift) lose bits.  fp16 rows are returned unchanged with xs = 1.
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
