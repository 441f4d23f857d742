"""FP8 formats: descriptors, decode, the 256-entry fp16 table, RNE + saturating encode.

API of the reference tfp8/formats.py:11-96. CUDA tensors are decoded/encoded by the gfx950
kernels (tfp8_decode / tfp8_encode); CPU tensors by the torch code below, which follows the same
bit-level rules so both devices give identical codes and values.
"""
import math
from dataclasses import dataclass

import torch

from . import _ext


@dataclass(frozen=True)
class Fp8Format:
    name: str
    ebits: int
    mbits: int
    bias: int
    has_inf: bool          # E5M2 is IEEE-like; E4M3FN has no inf
    max_finite: float
    torch_dtype: torch.dtype

    def is_nan(self, c: torch.Tensor) -> torch.Tensor:
        e = (c >> self.mbits) & ((1 << self.ebits) - 1)
        m = c & ((1 << self.mbits) - 1)
        emax = (1 << self.ebits) - 1
        if self.has_inf:
            return (e == emax) & (m != 0)
        return (e == emax) & (m == (1 << self.mbits) - 1)

    @property
    def nan_code(self) -> int:
        """Canonical NaN code produced by encode (tfp8/formats.py:94)."""
        return 0x7E if self.has_inf else 0x7F

    @property
    def max_code(self) -> int:
        """Largest finite positive code (saturation target)."""
        return (((1 << self.ebits) - 2) << self.mbits) | ((1 << self.mbits) - 1) if self.has_inf \
            else (((1 << self.ebits) - 1) << self.mbits) | ((1 << self.mbits) - 2)


E4M3FN = Fp8Format("e4m3fn", 4, 3, 7, False, 448.0, torch.float8_e4m3fn)
E5M2 = Fp8Format("e5m2", 5, 2, 15, True, 57344.0, torch.float8_e5m2)
FORMATS = {f.name: f for f in (E4M3FN, E5M2)}


def get_format(fmt) -> Fp8Format:
    if isinstance(fmt, Fp8Format):
        return fmt
    if fmt not in FORMATS:
        raise ValueError(f"unsupported FP8 format {fmt!r}; expected one of {sorted(FORMATS)}")
    return FORMATS[fmt]


def _code_value(c: int, f: Fp8Format) -> float:
    """Value of one code from its bit fields."""
    s = -1.0 if c & 0x80 else 1.0
    e = (c >> f.mbits) & ((1 << f.ebits) - 1)
    m = c & ((1 << f.mbits) - 1)
    emax = (1 << f.ebits) - 1
    if f.has_inf and e == emax:
        return s * math.inf if m == 0 else math.nan
    if not f.has_inf and e == emax and m == (1 << f.mbits) - 1:
        return math.nan
    if e == 0:
        return s * math.ldexp(m, 1 - f.bias - f.mbits)
    return s * math.ldexp(m + (1 << f.mbits), e - f.bias - f.mbits)


_TABLES = {}


def _table(f: Fp8Format) -> torch.Tensor:
    t = _TABLES.get(f.name)
    if t is None:
        t = _TABLES[f.name] = torch.tensor([_code_value(c, f) for c in range(256)], dtype=torch.float32)
    return t


def decode(codes: torch.Tensor, fmt) -> torch.Tensor:
    """uint8 codes -> float32 (exact; NaN codes give NaN, E5M2 0x7C/0xFC give +-inf)."""
    f = get_format(fmt)
    if codes.is_cuda:
        return _ext.decode(codes.to(torch.uint8), f.name, torch.float32)
    return _table(f)[codes.to(torch.uint8).long()]


_LUT_CACHE = {}


def lut(fmt, device="cpu") -> torch.Tensor:
    """256-entry fp16 table. Every FP8 value (incl. subnormals, +-0, NaN, inf) is exact in fp16."""
    f = get_format(fmt)
    key = (f.name, str(device))
    if key not in _LUT_CACHE:
        codes = torch.arange(256, dtype=torch.uint8, device=device)
        if codes.is_cuda:
            _LUT_CACHE[key] = _ext.decode(codes, f.name, torch.float16)
        else:
            _LUT_CACHE[key] = _table(f).half()
    return _LUT_CACHE[key]


def _encode_cpu(x: torch.Tensor, f: Fp8Format) -> torch.Tensor:
    """Arithmetic RNE on the float64 bit pattern (every f16/bf16/f32/f64 input is exact there)."""
    xd = x.double().contiguous()
    b = xd.view(torch.int64)
    sign = ((b >> 56) & 0x80).to(torch.int64)
    a = b & 0x7FFFFFFFFFFFFFFF
    af = a.view(torch.float64)
    # normal range: round the 52-bit mantissa to mbits, ties to even, then rebias 1023 -> bias
    sh = 52 - f.mbits
    r = (a + ((1 << (sh - 1)) - 1) + ((a >> sh) & 1)) >> sh
    r = r - ((1023 - f.bias) << f.mbits)
    # subnormal range: mantissa = rne(|x| * 2^(bias - 1 + mbits))
    sub = torch.round(af * float(2 ** (f.bias - 1 + f.mbits))).to(torch.int64)   # torch.round: half to even
    min_normal = math.ldexp(1.0, 1 - f.bias)
    q = torch.where(af < min_normal, sub, r)
    q = torch.where(af >= f.max_finite, torch.full_like(q, f.max_code), q)     # saturate (inf too)
    q = q | sign
    q = torch.where(torch.isnan(xd), torch.full_like(q, f.nan_code), q)
    return q.to(torch.uint8)


def encode(x: torch.Tensor, fmt) -> torch.Tensor:
    """float -> uint8 codes. Round-to-nearest-even, saturating to +-max_finite (never produces
    inf), NaN -> canonical NaN code. Matches torch's `.to(float8)` for in-range values."""
    f = get_format(fmt)
    if x.is_cuda:
        return _ext.encode(x, f.name)
    return _encode_cpu(x, f)
