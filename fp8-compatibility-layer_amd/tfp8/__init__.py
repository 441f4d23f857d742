"""tfp8 on MI355X: FP8 weights (uint8 codes + f32/UE8M0 scales) decoded inside gfx950 kernels --
a streaming GEMV and matrix-core decode kernel for small M, MFMA GEMMs above -- with fp32
accumulation.

Drop-in for the reference package's API (tfp8/__init__.py:9-16): FP8Config, FP8Linear,
prepare_model, plan, report, weight_bytes, quantize_weight, dequantize_weight, decode, encode,
lut, E4M3FN, E5M2; plus save_fp8 / load_fp8, an on-disk FP8 checkpoint format the reference lacks.
"""
__version__ = "0.1.0"

from .checkpoint import load_fp8, save_fp8
from .config import FP8Config
from .formats import E4M3FN, E5M2, decode, encode, lut
from .linear import FP8Linear
from .planner import plan, prepare_model, report, weight_bytes
from .quantize import dequantize_weight, quantize_weight

__all__ = ["FP8Config", "FP8Linear", "prepare_model", "plan", "report", "weight_bytes",
           "quantize_weight", "dequantize_weight", "decode", "encode", "lut", "E4M3FN", "E5M2",
           "save_fp8", "load_fp8"]
