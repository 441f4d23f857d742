"""GPU parity of the W8A8 block-32 path (fp8_cuda: quantize_k, Fp8Weight, fp8_linear; C entry
points tfp8_w8a8_quantize / tfp8_w8a8_gemm) against the numpy oracle.

  quantizer  bit-exact codes and scales (FP32 bits, UE8M0 bytes) against w8a8_oracle.quantize_k
             for both formats, f32/f16/bf16 input, ragged row counts, K not a multiple of 128,
             and special values (zero, NaN and inf blocks, subnormal and saturating values)
  GEMM       the reference host test's six cases (tests/fp8_gemm_host.cpp:209-216) at its size
             M=128, N=96, K=512 with its bar max|C - ref| / max|ref| < 1e-5 against the float64
             reference, plus ragged M/N/K (tails of every tile and of the 128-wide K step) and a
             large case checked against torch float64 on the GPU
  fp8_linear end to end against oracle quantization + float64 GEMM, and the reference's argument
             checks (fp8_cuda.py:114-123)
"""
import numpy as np
import pytest
import torch

import fp8_cuda
from oracle import w8a8_oracle as W
from tfp8 import _ext

pytestmark = pytest.mark.gpu
FMT = {"e4m3": 0, "e5m2": 1}
HOST_CASES = [  # (name, fa, fb, mode, ue8m0)                     fp8_gemm_host.cpp:209-216
    ("E4M3 block32 FP32-scale", "e4m3", "e4m3", 0, False),
    ("E4M3 block32 UE8M0-scale", "e4m3", "e4m3", 0, True),
    ("E5M2 block32 FP32-scale", "e5m2", "e5m2", 0, False),
    ("A=E4M3 / B=E5M2 block32 UE8M0", "e4m3", "e5m2", 0, True),
    ("E4M3 per-row/col epilogue FP32", "e4m3", "e4m3", 1, False),
    ("E4M3 per-row/col epilogue UE8M0", "e4m3", "e4m3", 1, True),
]


def _gemm(a, fa, sa, bt, fb, sb, ue8m0, mode, bias, M, N, K, native=False):
    c = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    lib = _ext.require()
    rc = lib.tfp8_w8a8_gemm(a.data_ptr(), FMT[fa], sa.data_ptr(), bt.data_ptr(), FMT[fb], sb.data_ptr(),
                            int(ue8m0), mode, int(native), bias.data_ptr() if bias is not None else None, c.data_ptr(),
                            M, N, K, _ext._stream(0))
    _ext._check(rc, "tfp8_w8a8_gemm")
    torch.cuda.synchronize()
    return c


def _cuda(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _quant_case(x, fmt, ue8m0, mode):
    return W.quantize_k(x, fmt, ue8m0) if mode == 0 else W.quantize_whole(x, fmt, ue8m0)


@pytest.mark.parametrize("case", HOST_CASES, ids=[c[0] for c in HOST_CASES])
def test_host_test_cases(case):
    name, fa, fb, mode, ue8m0 = case
    M, N, K = 128, 96, 512                                     # fp8_gemm_host.cpp:208
    print(f"[w8a8] host case {name!r} M={M} N={N} K={K}", flush=True)
    x, w, bias = W.host_case_data(M, N, K)
    a, sa = _quant_case(x, fa, ue8m0, mode)
    bt, sb = _quant_case(w.T.copy(), fb, ue8m0, mode)
    ref = W.gemm_ref(a, fa, sa, bt, fb, sb, ue8m0, mode, bias)
    c = _gemm(_cuda(a), fa, _cuda(sa), _cuda(bt), fb, _cuda(sb), ue8m0, mode, _cuda(bias), M, N, K)
    rel = W.rel_err(c.cpu().numpy(), ref)
    assert rel < 1e-5, f"{name}: kernel-vs-ref rel.err {rel:.2e}"


NATIVE_TOL = 2e-4   # FP8 matrix cores: terms aligned to the largest with ~13 fraction bits


@pytest.mark.parametrize("case", HOST_CASES, ids=[c[0] for c in HOST_CASES])
def test_host_test_cases_native_fp8(case):
    """The FP8 / MX matrix-core kernel on the same six cases, to its stated tolerance (the exact
    f16 kernel meets the reference's 1e-5 on the same codes in test_host_test_cases)."""
    name, fa, fb, mode, ue8m0 = case
    M, N, K = 128, 96, 512
    print(f"[w8a8] native host case {name!r} M={M} N={N} K={K}", flush=True)
    x, w, bias = W.host_case_data(M, N, K)
    a, sa = _quant_case(x, fa, ue8m0, mode)
    bt, sb = _quant_case(w.T.copy(), fb, ue8m0, mode)
    ref = W.gemm_ref(a, fa, sa, bt, fb, sb, ue8m0, mode, bias)
    c = _gemm(_cuda(a), fa, _cuda(sa), _cuda(bt), fb, _cuda(sb), ue8m0, mode, _cuda(bias), M, N, K, native=True)
    rel = W.rel_err(c.cpu().numpy(), ref)
    assert rel < NATIVE_TOL, f"{name}: native kernel-vs-ref rel.err {rel:.2e}"


@pytest.mark.parametrize("M,N,K", [(1, 1, 32), (200, 72, 160), (257, 300, 416), (64, 520, 1056), (33, 17, 96)])
@pytest.mark.parametrize("mode,ue8m0", [(0, False), (0, True), (1, False), (1, True)])
@pytest.mark.parametrize("native", [False, True])
def test_ragged_shapes(M, N, K, mode, ue8m0, native):
    print(f"[w8a8] ragged M={M} N={N} K={K} mode={mode} ue8m0={ue8m0} native={native}", flush=True)
    x, w, bias = W.host_case_data(M, N, K, seed=M + N + K)
    a, sa = _quant_case(x, "e4m3", ue8m0, mode)
    bt, sb = _quant_case(w.T.copy(), "e5m2", ue8m0, mode)
    ref = W.gemm_ref(a, "e4m3", sa, bt, "e5m2", sb, ue8m0, mode, bias)
    tol = NATIVE_TOL if native else 1e-5
    c = _gemm(_cuda(a), "e4m3", _cuda(sa), _cuda(bt), "e5m2", _cuda(sb), ue8m0, mode, _cuda(bias), M, N, K, native)
    assert W.rel_err(c.cpu().numpy(), ref) < tol
    c0 = _gemm(_cuda(a), "e4m3", _cuda(sa), _cuda(bt), "e5m2", _cuda(sb), ue8m0, mode, None, M, N, K, native)
    assert W.rel_err(c0.cpu().numpy(), ref - bias.astype(np.float64)[None, :]) < tol


@pytest.mark.parametrize("ue8m0", [False, True])
@pytest.mark.parametrize("native", [False, True])
def test_large_against_torch_float64(ue8m0, native):
    M, N, K = 1024, 2048, 4096
    print(f"[w8a8] large M={M} N={N} K={K} ue8m0={ue8m0} native={native}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(5)
    x = torch.randn(M, K, device="cuda", generator=g)
    w = torch.randn(K, N, device="cuda", generator=g) * 0.02
    bias = torch.randn(N, device="cuda", generator=g)
    a, sa = fp8_cuda.quantize_k(x, "e4m3", ue8m0)
    wq = fp8_cuda.Fp8Weight(w, "e4m3", ue8m0)
    c = _gemm(a, "e4m3", sa, wq.qt, "e4m3", wq.st, ue8m0, 0, bias, M, N, K, native)
    A = fp8_cuda.dequant_ref(a, sa, "e4m3", ue8m0, True)
    B = fp8_cuda.dequant_ref(wq.q, wq.s, "e4m3", ue8m0, False)
    ref = A @ B + bias.double()
    rel = float((c.double() - ref).abs().max() / ref.abs().max())
    assert rel < (NATIVE_TOL if native else 1e-5), rel


@pytest.mark.parametrize("native", [False, True])
@pytest.mark.parametrize("ue8m0", [False, True])
def test_format_pairs_and_nan_scale(native, ue8m0):
    """A=E5M2 x B=E4M3 (the pair the host test does not run), and a NaN scale (UE8M0 byte 255,
    fp8_gemm_kernel.cu:8, or an f32 NaN) on one (row, block) of A: that output row is NaN, the
    others are unaffected."""
    M, N, K = 96, 80, 288
    print(f"[w8a8] e5m2 x e4m3 + NaN scale native={native} ue8m0={ue8m0}", flush=True)
    x, w, bias = W.host_case_data(M, N, K, seed=11)
    a, sa = W.quantize_k(x, "e5m2", ue8m0)
    bt, sb = W.quantize_k(w.T.copy(), "e4m3", ue8m0)
    ref = W.gemm_ref(a, "e5m2", sa, bt, "e4m3", sb, ue8m0, 0, bias)
    tol = NATIVE_TOL if native else 1e-5
    c = _gemm(_cuda(a), "e5m2", _cuda(sa), _cuda(bt), "e4m3", _cuda(sb), ue8m0, 0, _cuda(bias), M, N, K, native)
    assert W.rel_err(c.cpu().numpy(), ref) < tol
    sa_nan = sa.copy()
    sa_nan[7, 3] = 255 if ue8m0 else np.float32(np.nan)
    c = _gemm(_cuda(a), "e5m2", _cuda(sa_nan), _cuda(bt), "e4m3", _cuda(sb), ue8m0, 0, _cuda(bias), M, N, K,
              native).cpu().numpy()
    assert np.isnan(c[7]).all()
    keep = np.arange(M) != 7
    assert W.rel_err(c[keep], ref[keep]) < tol


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("ue8m0", [False, True])
@pytest.mark.parametrize("dt", [torch.float32, torch.float16, torch.bfloat16])
def test_quantizer_bit_exact(fmt, ue8m0, dt):
    R, K = 77, 416
    print(f"[w8a8] quantize R={R} K={K} fmt={fmt} ue8m0={ue8m0} dt={dt}", flush=True)
    rng = np.random.default_rng(R + K)
    g = np.ldexp(1.0, rng.integers(-30, 12, size=(R, K // 32))).repeat(32, axis=1)
    x = (rng.standard_normal((R, K)) * g).astype(np.float32)
    x[0, :32] = 0.0
    x[1, 3] = -0.0
    x[2, 40] = np.nan
    x[3, 70] = np.inf
    x[4, 100] = -np.inf
    x[5, :32] = 1e-40                                           # fp32 subnormals
    xt = torch.from_numpy(x).to(dt)
    xr = xt.float().numpy()                                     # what the kernel sees
    q, s = fp8_cuda.quantize_k(xt.cuda(), fmt, ue8m0)
    rq, rs = W.quantize_k(xr, fmt, ue8m0)
    assert np.array_equal(q.cpu().numpy(), rq)
    if ue8m0:
        assert np.array_equal(s.cpu().numpy(), rs)
    else:
        assert np.array_equal(s.cpu().numpy().view(np.uint32), rs.view(np.uint32))


def test_fp8_linear_end_to_end():
    M, K, N = 96, 640, 160
    print(f"[w8a8] fp8_linear M={M} K={K} N={N}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(9)
    for fmt, ue8m0 in (("e4m3", False), ("e4m3", True), ("e5m2", True)):
        x = torch.randn(M, K, device="cuda", generator=g).to(torch.bfloat16)
        w = torch.randn(K, N, device="cuda", generator=g) * 0.05
        bias = torch.randn(N, device="cuda", generator=g)
        wq = fp8_cuda.Fp8Weight(w, fmt, ue8m0)
        assert wq.q.shape == (K, N) and wq.s.shape == (K // 32, N)          # reference layout views
        rq, rs = W.quantize_k(w.t().contiguous().cpu().numpy(), fmt, ue8m0)
        assert np.array_equal(wq.qt.cpu().numpy(), rq)
        y = fp8_cuda.fp8_linear(x, wq, bias)
        assert y.dtype == torch.float32 and y.shape == (M, N)
        a, sa = W.quantize_k(x.float().cpu().numpy(), fmt, ue8m0)
        ref = W.gemm_ref(a, fmt, sa, rq, fmt, rs, ue8m0, 0, bias.cpu().numpy())
        assert W.rel_err(y.cpu().numpy(), ref) < 1e-5
        yn = fp8_cuda.fp8_linear(x, wq, bias, native_fp8=True)
        assert W.rel_err(yn.cpu().numpy(), ref) < NATIVE_TOL
    # activations in the other format family
    y2 = fp8_cuda.fp8_linear(x, wq, bias, act_fmt="e4m3")
    a, sa = W.quantize_k(x.float().cpu().numpy(), "e4m3", True)
    ref = W.gemm_ref(a, "e4m3", sa, wq.qt.cpu().numpy(), "e5m2", wq.st.cpu().numpy(), True, 0, bias.cpu().numpy())
    assert W.rel_err(y2.cpu().numpy(), ref) < 1e-5


def test_fp8_linear_argument_checks():
    wq = fp8_cuda.Fp8Weight(torch.randn(64, 32, device="cuda"))
    b = torch.zeros(32, device="cuda")
    with pytest.raises(ValueError, match="multiples of 32"):
        fp8_cuda.fp8_linear(torch.randn(16, 64, device="cuda"), wq, b)
    with pytest.raises(ValueError, match="multiples of 32"):
        fp8_cuda.fp8_linear(torch.randn(32, 96, device="cuda"), wq, b)
    with pytest.raises(ValueError, match="CUDA"):
        fp8_cuda.fp8_linear(torch.randn(32, 64), wq, b)
    with pytest.raises(ValueError, match="multiple of 32"):
        fp8_cuda.quantize_k(torch.randn(4, 48, device="cuda"), "e4m3")
    lib = _ext.require()
    assert lib.tfp8_w8a8_gemm(None, 0, None, None, 0, None, 0, 0, 0, None, None, 32, 32, 48, None) != 0
    assert lib.tfp8_w8a8_gemm(None, 0, None, None, 0, None, 0, 2, 0, None, None, 32, 32, 64, None) != 0
