"""FP8 x FP8 linear (W8A8) with 32-wide K-block scales on MI355X: the API of the reference's
fp8_cuda.py (FORMATS, BLOCK, lut, quantize_k, Fp8Weight, fp8_linear, dequant_ref).

The reference compiles fp8_gemm_kernel.cu with NVRTC and launches it through the CUDA driver; here
the quantizer and the GEMM are the gfx950 kernels of libtfp8_hip.so (tfp8_w8a8_quantize,
tfp8_w8a8_gemm), called on torch's current stream without host synchronisation.

One layout difference: Fp8Weight keeps its codes and scales N-major ([N, K] and [N, K/32], k
contiguous, as the quantizer produces them for w.T) so that both matrix-core operands load as
contiguous k runs; `.q` and `.s` are the reference's [K, N] / [K/32, N] as transposed views.
"""
import torch

from tfp8 import _ext
from tfp8.formats import lut as _tfp8_lut

FORMATS = {  # name -> (torch dtype, max finite)            (fp8_cuda.py:28-31)
    "e4m3": (torch.float8_e4m3fn, 448.0),
    "e5m2": (torch.float8_e5m2, 57344.0),
}
BLOCK = 32
_FMT_ID = {"e4m3": _ext.FMT_ID["e4m3fn"], "e5m2": _ext.FMT_ID["e5m2"]}
_TFP8_NAME = {"e4m3": "e4m3fn", "e5m2": "e5m2"}


def lut(fmt, device="cuda"):
    """uint8 -> fp16 decode table of `fmt` (fp8_cuda.py:68-71)."""
    if fmt not in FORMATS:
        raise ValueError(f"unknown FP8 format {fmt!r}")
    return _tfp8_lut(_TFP8_NAME[fmt], device)


def quantize_k(x, fmt, ue8m0=False):
    """Quantize x (R, K) in blocks of 32 along K. Returns uint8 codes (R, K) and scales (R, K/32):
    FP32, or UE8M0 bytes (value 2^(e-127)) when ue8m0 (fp8_cuda.py:74-92)."""
    if fmt not in FORMATS:
        raise ValueError(f"unknown FP8 format {fmt!r}")
    if not x.is_cuda:
        raise ValueError("quantize_k: x must be a CUDA tensor")
    R, K = x.shape
    if K % BLOCK:
        raise ValueError(f"quantize_k: K={K} must be a multiple of {BLOCK}")
    lib = _ext.require()
    if x.dtype not in _ext.DTYPE_ID:
        x = x.float()
    x = x.contiguous()
    q = torch.empty(R, K, dtype=torch.uint8, device=x.device)
    s = torch.empty(R, K // BLOCK, dtype=torch.uint8 if ue8m0 else torch.float32, device=x.device)
    dev = x.get_device()
    _ext._check(lib.tfp8_w8a8_quantize(x.data_ptr(), _ext.DTYPE_ID[x.dtype], R, K, _FMT_ID[fmt], int(bool(ue8m0)),
                                       q.data_ptr(), s.data_ptr(), _ext._stream(dev)), "tfp8_w8a8_quantize")
    return q, s


class Fp8Weight:
    """B (K, N) quantized along K per output column; scales laid out (K/32, N) (fp8_cuda.py:95-106)."""

    def __init__(self, w, fmt="e4m3", ue8m0=False):
        if not w.is_cuda:
            raise ValueError("Fp8Weight: w must be a CUDA tensor")
        if w.shape[0] % BLOCK:
            raise ValueError(f"Fp8Weight: K={w.shape[0]} must be a multiple of {BLOCK}")
        self.qt, self.st = quantize_k(w.t().contiguous(), fmt, ue8m0)   # [N, K], [N, K/32]
        self.fmt, self.ue8m0 = fmt, ue8m0
        self.K, self.N = w.shape

    @property
    def q(self):
        return self.qt.t()

    @property
    def s(self):
        return self.st.t()


def fp8_linear(x, w, bias, act_fmt=None, *, native_fp8=False):
    """x (M, K) float -> fused FP8 GEMM -> (M, N) fp32 (+bias). Activations are quantized
    dynamically per row and 32-wide K block, in the same format family as the weights
    (fp8_cuda.py:109-138).

    native_fp8=False multiplies on f16 matrix cores after an exact FP8 -> f16 decode (the
    reference's fp16-WMMA numerics, ~1e-7 of max|out| from a float64 sum); True uses the FP8 / MX
    matrix cores, whose dot products keep ~13 fraction bits below their largest term (~1e-5..1e-4
    of max|out|)."""
    act_fmt = act_fmt or w.fmt
    M, K = x.shape
    if not (x.is_cuda and w.qt.is_cuda and w.st.is_cuda and bias.is_cuda):
        raise ValueError("fp8_linear: x, weights and bias must all be CUDA tensors")
    if not (x.device == w.qt.device == w.st.device == bias.device):
        raise ValueError(f"fp8_linear: tensors on different devices ({x.device}, {w.qt.device}, "
                         f"{w.st.device}, {bias.device})")
    if M % 32 or K % 32 or w.N % 32 or K != w.K:
        raise ValueError(f"fp8_linear: need M, K, N multiples of 32 and K == w.K; "
                         f"got M={M} K={K} N={w.N} w.K={w.K}")
    lib = _ext.require()
    aq, sa = quantize_k(x, act_fmt, w.ue8m0)
    out = torch.empty(M, w.N, dtype=torch.float32, device=x.device)
    b = bias.float().contiguous()
    _ext._check(lib.tfp8_w8a8_gemm(aq.data_ptr(), _FMT_ID[act_fmt], sa.data_ptr(), w.qt.data_ptr(), _FMT_ID[w.fmt],
                                   w.st.data_ptr(), int(bool(w.ue8m0)), 0, int(bool(native_fp8)), b.data_ptr(),
                                   out.data_ptr(), M, w.N, K,
                                   _ext._stream(x.get_device())), "tfp8_w8a8_gemm")
    return out


def dequant_ref(q, s, fmt, ue8m0, k_axis_last):
    """float64 dequantization used as the reference; q, s as produced above (A layout if
    k_axis_last) (fp8_cuda.py:141-147)."""
    v = lut(fmt, q.device)[q.long()].double()
    sc = torch.exp2(s.double() - 127) if ue8m0 else s.double()
    if k_axis_last:
        return v * sc.repeat_interleave(BLOCK, dim=1)
    return v * sc.repeat_interleave(BLOCK, dim=0)
