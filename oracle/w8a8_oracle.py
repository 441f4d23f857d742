"""CPU oracle for the W8A8 block-32 path -- TEST INFRASTRUCTURE, not product code.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, as
the checker (or the timed CPU baseline).  numpy restatement of the reference's fp8_cuda.py
quantizer and of the double-precision reference of its host test (tests/fp8_gemm_host.cpp);
paths are relative to the reference repository.  How each function is pinned is listed in
tests/test_w8a8_oracle.py (closed forms, brute force, torch's float8 casts, planted mistakes).

Two documented choices where the reference's own pieces disagree or leave behaviour open:
  * ceil(log2 s) for UE8M0 is exact (from frexp), as in fp8_gemm_host.cpp:75-84 (log2 in
    double).  fp8_cuda.py:85 takes log2 in fp32, which rounds log2 of an s one or two ulps
    above a power of two to the integer, so its ceil lands one exponent low there.
  * a block holding a NaN gets a NaN scale (UE8M0 byte 255, the kernel's NaN code,
    fp8_gemm_kernel.cu:8) and NaN codes 0x7F (torch's positive NaN code in both formats);
    torch's float -> uint8 cast of the NaN exponent is undefined.
"""
import numpy as np

from .fp8_oracle import FORMATS, decode, encode, ue8m0_decode

BLOCK = 32                                   # fp8_cuda.py:32
_API_FMT = {"e4m3": "e4m3fn", "e5m2": "e5m2", "e4m3fn": "e4m3fn"}


def _fmt(fmt):
    return _API_FMT[fmt]


def ceil_log2_exact(s):
    """ceil(log2 s) for finite s > 0, exactly (fp8_gemm_host.cpp:78)."""
    m, e = np.frexp(np.asarray(s, dtype=np.float32))
    return np.where(m == 0.5, e - 1, e).astype(np.int64)


def quantize_k(x, fmt, ue8m0=False):
    """x (R, K) float -> (codes uint8 (R, K), scales (R, K/32) float32 or UE8M0 uint8).
    s = max(amax/max_finite, 1e-12) per 32-block; UE8M0 e = clamp(ceil log2 s, -127, 127),
    s = 2^e, byte e + 127; q = encode(clamp(x/s, +-max_finite)) in fp32 (fp8_cuda.py:74-92)."""
    f = _fmt(fmt)
    mx = np.float32(FORMATS[f][4])
    x = np.asarray(x, dtype=np.float32)
    R, K = x.shape
    if K % BLOCK:
        raise ValueError(f"K={K} must be a multiple of {BLOCK}")
    xb = x.reshape(R, K // BLOCK, BLOCK)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore"):
        amax = np.max(np.abs(xb), axis=-1)                                # NaN propagates
        s = np.maximum(amax / mx, np.float32(1e-12)).astype(np.float32)   # NaN propagates
        nan = np.isnan(s)
        if ue8m0:
            e = np.where(np.isinf(s), 127, ceil_log2_exact(np.where(np.isfinite(s), s, 1.0)))
            e = np.clip(e, -127, 127)
            s = np.where(nan, np.float32(np.nan), np.ldexp(np.float32(1.0), e.astype(np.int32))).astype(np.float32)
            s_out = np.where(nan, 255, e + 127).astype(np.uint8)
        else:
            s_out = s
        d = (xb / s[..., None]).astype(np.float32)
        q = encode(np.clip(d, -mx, mx), f)
    q = np.where(np.isnan(d), np.uint8(0x7F), q).astype(np.uint8)
    return q.reshape(R, K), s_out


def scales_f64(s, ue8m0):
    """Scale values: UE8M0 byte -> 2^(byte-127) with 255 -> NaN (fp8_gemm_kernel.cu:22-30),
    else the fp32 value."""
    s = np.asarray(s)
    return ue8m0_decode(s).astype(np.float64) if ue8m0 else s.astype(np.float64)


def dequant(q, s, fmt, ue8m0):
    """(R, K) codes with (R, K/32) scales -> float64 values (fp8_cuda.py:141-147,
    fp8_gemm_host.cpp:114-117: decode(q) * s in double)."""
    v = decode(q, _fmt(fmt))
    return v * np.repeat(scales_f64(s, ue8m0), BLOCK, axis=1)


def gemm_ref(a, fa, sa, bt, fb, sb, ue8m0, mode, bias=None):
    """float64 reference of C = A B + bias with A (M, K) and Bt (N, K) codes
    (fp8_gemm_host.cpp:140-151): block mode dequantizes per 32-block, row/col mode scales
    rows of A by sa[m] and columns by sb[n]."""
    if mode == 0:
        A = dequant(a, sa, fa, ue8m0)
        B = dequant(bt, sb, fb, ue8m0)
    else:
        A = decode(a, _fmt(fa)) * scales_f64(sa, ue8m0).reshape(-1, 1)
        B = decode(bt, _fmt(fb)) * scales_f64(sb, ue8m0).reshape(-1, 1)
    C = A @ B.T
    if bias is not None:
        C = C + np.asarray(bias, dtype=np.float64)[None, :]
    return C


def rel_err(c, ref):
    """max |c - ref| / max |ref| (fp8_gemm_host.cpp:171-182); the reference bar is < 1e-5.
    A NaN or inf in c where ref is finite counts as an infinite error."""
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(np.asarray(c, dtype=np.float64) - ref)
    err = np.where(np.isfinite(err), err, np.inf)
    return float(np.max(err) / np.max(np.abs(ref)))


def host_case_data(M, N, K, seed=1234):
    """Inputs shaped like the reference host test's (fp8_gemm_host.cpp:90-105): normal values
    times 2^U{-4..4} per (row, 32-block) for A and per (column, 32-block) for B, normal bias.
    Returns x (M, K), w (K, N), bias (N,) as float32."""
    rng = np.random.default_rng(seed)
    KB = K // BLOCK
    ga = np.ldexp(1.0, rng.integers(-4, 5, size=(M, KB))).repeat(BLOCK, axis=1)
    x = (rng.standard_normal((M, K)) * ga).astype(np.float32)
    gb = np.ldexp(1.0, rng.integers(-4, 5, size=(N, KB))).repeat(BLOCK, axis=1)
    w = (rng.standard_normal((N, K)) * gb).astype(np.float32).T.copy()
    bias = rng.standard_normal(N).astype(np.float32)
    return x, w, bias


def quantize_whole(x, fmt, ue8m0=False):
    """One scale per row over the whole K (the row/col epilogue case of fp8_gemm_host.cpp:119-131,
    len = K); zero rows get scale 1 there (fp8_gemm_host.cpp:76)."""
    f = _fmt(fmt)
    mx = np.float32(FORMATS[f][4])
    x = np.asarray(x, dtype=np.float32)
    amax = np.max(np.abs(x), axis=1)
    s = np.where(amax > 0, amax / mx, np.float32(1.0)).astype(np.float32)
    if ue8m0:
        e = np.clip(ceil_log2_exact(s), -127, 127)
        s = np.ldexp(np.float32(1.0), e.astype(np.int32)).astype(np.float32)
        s_out = (e + 127).astype(np.uint8)
    else:
        s_out = s
    q = encode(np.clip((x / s[:, None]).astype(np.float32), -mx, mx), f)
    return q, s_out
