"""CPU oracle for the tfp8 FP8Linear path -- TEST INFRASTRUCTURE, not product code.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and
only as the checker (or the timed CPU baseline), never as the thing measured or shipped.

A numpy restatement of the reference algorithm, one function per reference function, each citing
the file:line it follows (paths relative to the reference repository). Byte/integer work is
exact integer arithmetic; the linear product is float64 (the reference test oracle,
tests/test_tfp8.py:75-90). How each function is pinned (golden vectors, closed forms, brute
force, torch's own float8 casts) is listed in tests/test_oracle.py; every function here has at
least one independent check there.
"""
import math

import numpy as np

# name -> (ebits, mbits, bias, has_inf, max_finite)          tfp8/formats.py:30-31, fp8.h:18-19
FORMATS = {
    "e4m3fn": (4, 3, 7, False, 448.0),
    "e5m2": (5, 2, 15, True, 57344.0),
}


def _fields(fmt):
    eb, mb, bias, has_inf, mx = FORMATS[fmt]
    return eb, mb, bias, has_inf, mx


def is_nan(c, fmt):
    """tfp8/formats.py:21-27, fp8.h:21-26."""
    eb, mb, _, has_inf, _ = _fields(fmt)
    c = np.asarray(c, dtype=np.int64)
    e = (c >> mb) & ((1 << eb) - 1)
    m = c & ((1 << mb) - 1)
    emax = (1 << eb) - 1
    if has_inf:
        return (e == emax) & (m != 0)
    return (e == emax) & (m == (1 << mb) - 1)


def decode(codes, fmt):
    """uint8 codes -> float64 values from the bit fields (tfp8/formats.py:43-57, fp8.h:35-44).
    Subnormal m*2^(1-bias-mbits); normal (m+2^mbits)*2^(e-bias-mbits); E5M2 inf; NaN; sign."""
    eb, mb, bias, has_inf, _ = _fields(fmt)
    c = np.asarray(codes, dtype=np.int64)
    s = (c >> 7) & 1
    e = (c >> mb) & ((1 << eb) - 1)
    m = (c & ((1 << mb) - 1)).astype(np.float64)
    sub = np.ldexp(m, 1 - bias - mb)
    nrm = np.ldexp(m + (1 << mb), (e - bias - mb).astype(np.int32))
    v = np.where(e == 0, sub, nrm)
    if has_inf:
        v = np.where((e == (1 << eb) - 1) & ((c & ((1 << mb) - 1)) == 0), np.inf, v)
    v = np.where(is_nan(c, fmt), np.nan, v)
    return np.where(s == 1, -v, v)


def lut_f16_bits(fmt):
    """256 x uint16 fp16 bit patterns, NaN codes -> 0x7E00 | sign<<15 (fp8.h:47-52). This is the
    layout of the reference's lut_e4m3fn.bin / lut_e5m2.bin data files."""
    codes = np.arange(256)
    v = decode(codes, fmt).astype(np.float16).view(np.uint16).copy()
    nan = is_nan(codes, fmt)
    v[nan] = (0x7E00 | ((codes[nan] >> 7) << 15)).astype(np.uint16)
    return v


def _finite_table(fmt):
    """Non-negative codes 0..127 with their values; non-finite ones dropped (tfp8/formats.py:72-74, 84-86)."""
    codes = np.arange(128)
    vals = decode(codes, fmt)
    keep = np.isfinite(vals)
    return codes[keep], vals[keep]


def encode(x, fmt):
    """float -> uint8 code: nearest finite code to min(|x|, max_finite), ties to the even code,
    sign from signbit, NaN -> 0x7F (E4M3FN) / 0x7E (E5M2) (tfp8/formats.py:77-96)."""
    _, _, _, has_inf, mx = _fields(fmt)
    xd = np.asarray(x, dtype=np.float64)
    flat = xd.reshape(-1)
    ax = np.minimum(np.abs(flat), mx)
    codes, vals = _finite_table(fmt)
    hi = np.clip(np.searchsorted(vals, ax), 0, len(vals) - 1)
    lo = np.clip(hi - 1, 0, None)
    dlo = ax - vals[lo]
    dhi = vals[hi] - ax
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (codes[hi] % 2 == 0))
    q = np.where(pick_hi, codes[hi], codes[lo])
    q = q | (np.signbit(flat).astype(np.int64) << 7)
    q = np.where(np.isnan(flat), 0x7E if has_inf else 0x7F, q)
    return q.astype(np.uint8).reshape(xd.shape)


def ceil_log2_f32(s):
    """ceil(log2 s) of the reference's fp32 formula (tfp8/quantize.py:11-12 and :58-59): the
    log2 of an fp32 value rounded once to fp32, then the ceiling.  Computed as float64 log2
    rounded to float32, i.e. the correctly rounded fp32 log2 (float64 carries 29 bits more than
    that rounding needs).  A value a few ULP above 2^k has an fp32 log2 of exactly k, so its
    ceiling is k, not k + 1."""
    s = np.asarray(s, dtype=np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        return np.ceil(np.log2(s.astype(np.float64)).astype(np.float32))


def pow2_ceil_exact(s):
    """2^ceil(log2 s) from the exponent bits (no rounded log2): the power of two at or above s."""
    s = np.asarray(s, dtype=np.float32)
    m, e = np.frexp(s)
    p = np.where(m == 0.5, s, np.ldexp(np.float32(1.0), e).astype(np.float32))
    return np.where(np.isfinite(s), p, s).astype(np.float32)


def pow2_ceil(s):
    """torch.exp2(torch.ceil(torch.log2(s))) (tfp8/quantize.py:11-12) for s > 0; inf and NaN pass
    through.  Equals pow2_ceil_exact except a few ULP above a power of two (ceil_log2_f32)."""
    s = np.asarray(s, dtype=np.float32)
    c = ceil_log2_f32(s)
    fin = np.isfinite(c)
    p = np.ldexp(np.float32(1.0), np.where(fin, c, 0).astype(np.int32)).astype(np.float32)
    return np.where(fin, p, s).astype(np.float32)


def ue8m0_encode(s):
    """pow2 scale -> byte ceil(log2 s)+127 clamped to [-127,127]+127 (fp8_cuda.py:85-88); NaN -> 255."""
    s = np.asarray(s, dtype=np.float32)
    _, e = np.frexp(pow2_ceil(s))
    b = np.clip(e.astype(np.int64) - 1, -127, 127) + 127
    return np.where(np.isnan(s), 255, b).astype(np.uint8)


def ue8m0_decode(b):
    """byte -> 2^(b-127), 255 -> NaN (fp8_gemm_kernel.cu:22-30, fp8_gemm_host.cpp:75-84)."""
    b = np.asarray(b, dtype=np.int64)
    v = np.ldexp(np.float32(1.0), (b - 127).astype(np.int32)).astype(np.float32)
    return np.where(b == 255, np.float32(np.nan), v).astype(np.float32)


def scale_values(s):
    s = np.asarray(s)
    return ue8m0_decode(s) if s.dtype == np.uint8 else s.astype(np.float32)


def quantize_weight(w, fmt="e4m3fn", group_size=None, pow2_scale=True, scale_format="f32"):
    """w [N,K] -> (q uint8 [N,K], s [N,K/G] f32 or UE8M0 uint8, G)  (tfp8/quantize.py:15-36).
    amax per group; s = max(amax/max_finite, FLT_MIN); pow2 ceiling; s = 1 where amax == 0;
    q = RNE(clamp(w/s, +-max)) with f32 division."""
    _, _, _, _, mx = _fields(fmt)
    w = np.asarray(w, dtype=np.float32)
    N, K = w.shape
    G = K if group_size is None else group_size
    if K % G:
        raise ValueError(f"K={K} not divisible by group_size={G}")
    wg = w.reshape(N, K // G, G)
    amax = np.abs(wg).max(-1)
    with np.errstate(invalid="ignore"):
        s = np.maximum((amax / np.float32(mx)).astype(np.float32), np.float32(np.finfo(np.float32).tiny))
    s = np.where(np.isnan(amax), np.float32(np.nan), s).astype(np.float32)
    ue8m0 = scale_format == "ue8m0"
    if pow2_scale or ue8m0:
        s = pow2_ceil(s)
    s = np.where(amax == 0, np.float32(1.0), s).astype(np.float32)
    with np.errstate(invalid="ignore", divide="ignore"):
        r = (wg / s[..., None]).astype(np.float32)
    q = encode(np.clip(r, -mx, mx), fmt).reshape(N, K)   # np.clip keeps NaN, like torch.clamp
    return q, (ue8m0_encode(s) if ue8m0 else s), G


def dequantize_weight(q, s, fmt, group_size):
    """fp32 W[n,k] = fp32(decode(q)) * fp32 scale[n, k//G], one f32 multiply (tfp8/quantize.py:39-44)."""
    q = np.asarray(q)
    N, K = q.shape
    v = decode(q, fmt).astype(np.float32).reshape(N, K // group_size, group_size)
    return (v * scale_values(s)[..., None]).astype(np.float32).reshape(N, K)


ACT_TARGET_EXP = 8


def activation_to_fp16(x):
    """(x16 fp16, xs f32 pow2) per row: e = ceil(log2 max(amax, 2^-100)) - 8 with the fp32 log2
    rounding of ceil_log2_f32, 0 for amax == 0 (tfp8/quantize.py:47-62; the kernel variant
    tfp8_kernels.cu:513-532 rescales fp16 input too)."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.abs(x).max(-1)
    cl = ceil_log2_f32(np.maximum(amax, np.float32(2.0 ** -100)))
    ex = np.where(amax > 0, np.nan_to_num(cl) - ACT_TARGET_EXP, 0).astype(np.int32)
    xs = np.ldexp(np.float32(1.0), ex).astype(np.float32)
    return (x / xs[:, None]).astype(np.float16), xs


def linear_ref64(x, q, s, group_size, fmt, bias=None):
    """float64 y = x @ W_deq^T + bias -- the reference kernel-test oracle (tests/test_tfp8.py:82-85)
    with x taken at face value (the gfx950 GEMV/GEMM consume f16/bf16 x exactly)."""
    W = dequantize_weight(q, s, fmt, group_size).astype(np.float64)
    y = np.asarray(x, dtype=np.float64) @ W.T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)
    return y


def tolerance(ref, out_dtype_name):
    """|y - ref| bound of tests/test_tfp8.py:86-89: eps*|ref| + 1e-4*max|ref| + 1e-6 with
    eps = 2^-11 for fp16 outputs and 2^-8 for bf16/fp32 outputs."""
    eps = 2.0 ** -11 if out_dtype_name == "float16" else 2.0 ** -8
    ref = np.asarray(ref, dtype=np.float64)
    return eps * np.abs(ref) + 1e-4 * np.abs(ref).max(initial=0.0) + 1e-6


def bruteforce_linear(x, W, bias=None):
    """Triple-loop y = x W^T + b in Python floats, for tiny shapes only (pins linear_ref64)."""
    M, K = len(x), len(x[0])
    N = len(W)
    out = [[0.0] * N for _ in range(M)]
    for m in range(M):
        for n in range(N):
            acc = 0.0
            for k in range(K):
                acc += float(x[m][k]) * float(W[n][k])
            out[m][n] = acc + (float(bias[n]) if bias is not None else 0.0)
    return out


def bruteforce_encode(v, fmt):
    """Nearest finite code by exhaustive scan over the 128 non-negative codes, ties to the even
    code, saturating (fp8.h:55-76 rule); Python floats, for small samples only."""
    _, _, _, has_inf, mx = _fields(fmt)
    if math.isnan(v):
        return 0x7E if has_inf else 0x7F
    sign = 0x80 if math.copysign(1.0, v) < 0 else 0
    a = min(abs(v), mx)
    best, best_d = 0, math.inf
    for c in range(128):
        cv = float(decode(np.array([c]), fmt)[0])
        if not math.isfinite(cv):
            continue
        d = abs(a - cv)
        if d < best_d or (d == best_d and c % 2 == 0):
            best, best_d = c, d
    return sign | best
