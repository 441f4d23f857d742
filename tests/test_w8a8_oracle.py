"""Pins the W8A8 oracle (oracle/w8a8_oracle.py) and checks the host side of fp8_cuda on the CPU.

  ceil_log2_exact   closed forms with Python's exact frexp, 1 ulp either side of powers of two
  quantize_k        the reference's torch formula (fp8_cuda.py:74-92) run with torch ops on the
                    CPU: codes and FP32 scales equal everywhere; UE8M0 bytes equal except where
                    fp32 log2 rounds (identified independently); special values (NaN, inf, 0)
  dequant/gemm_ref  a brute-force triple loop with Fractions-free exact float64 sums on tiny
                    shapes; planted mistakes (transposed block scales, dropped block scale,
                    scales applied per block of the wrong operand) must fail the 1e-5 bar
  host_case_data    the FP8 quantization error against fp32 truth is what the host test reports
                    (a few percent), while kernel-vs-reference is held to 1e-5
"""
import math

import numpy as np
import pytest
import torch

from oracle import fp8_oracle as O
from oracle import w8a8_oracle as W

TORCH_DT = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}
MAXF = {"e4m3": 448.0, "e5m2": 57344.0}


def _torch_quantize_k(x, fmt, ue8m0):
    """fp8_cuda.py:74-92 with torch ops on the CPU (the reference's own formula)."""
    dt, mx = TORCH_DT[fmt], MAXF[fmt]
    R, K = x.shape
    xb = x.float().reshape(R, K // 32, 32)
    s = (xb.abs().amax(-1) / mx).clamp_min(1e-12)
    if ue8m0:
        e = torch.ceil(torch.log2(s)).clamp(-127, 127)
        s = torch.exp2(e)
        s_out = (e + 127).to(torch.uint8)
    else:
        s_out = s
    q = (xb / s[..., None]).clamp(-mx, mx).to(dt).view(torch.uint8).reshape(R, K)
    return q, s_out


def _data(R, K, seed):
    rng = np.random.default_rng(seed)
    g = np.ldexp(1.0, rng.integers(-20, 21, size=(R, K // 32))).repeat(32, axis=1)
    x = (rng.standard_normal((R, K)) * g).astype(np.float32)
    x[0, :32] = 0.0                               # all-zero block: scale clamps to 1e-12
    x[1, 5] = -0.0
    return x


def test_ceil_log2_exact_closed_forms():
    vals = []
    for k in range(-126, 128):
        p = math.ldexp(1.0, k)
        vals += [p, np.nextafter(np.float32(p), np.float32(np.inf)), np.nextafter(np.float32(p), np.float32(0))]
    vals = np.array(vals, dtype=np.float32)
    vals = vals[np.isfinite(vals) & (vals > 0)]
    got = W.ceil_log2_exact(vals)
    for v, e in zip(vals.tolist(), got.tolist()):
        m, ex = math.frexp(v)                     # exact: v = m 2^ex, 0.5 <= m < 1
        want = ex - 1 if m == 0.5 else ex
        assert e == want, (v, e, want)
        assert math.ldexp(1.0, e) >= v > math.ldexp(1.0, e - 1)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_quantize_k_fp32_scales_match_reference_formula(fmt):
    x = _data(24, 256, 1)
    q, s = W.quantize_k(x, fmt, ue8m0=False)
    tq, ts = _torch_quantize_k(torch.from_numpy(x), fmt, False)
    assert np.array_equal(q, tq.numpy())
    assert np.array_equal(s.view(np.uint32), ts.numpy().view(np.uint32))
    assert s[0, 0] == np.float32(1e-12) and np.all(q[0, :32] == 0)
    assert q[1, 5] in (0x00, 0x80)


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_quantize_k_ue8m0_matches_reference_formula_except_fp32_log2(fmt):
    x = _data(32, 512, 2)
    # blocks whose scale is a power of two, or 1 ulp above one, where fp32 log2 can round
    mx = MAXF[fmt]
    for r, k in ((2, 0), (3, 1)):
        x[r, 32 * k:32 * k + 32] = np.linspace(-0.5, 0.5, 32, dtype=np.float32)
        x[r, 32 * k + 7] = np.float32(mx * 2.0 ** -9)                        # s = 2^-9 exactly
    x[4, :32] = 0.1
    big = np.float32(mx * 2.0 ** -12)
    for _ in range(2):
        big = np.nextafter(big, np.float32(np.inf))
    x[4, 3] = big                                                            # s 1 ulp above 2^-12
    q, s = W.quantize_k(x, fmt, ue8m0=True)
    tq, ts = _torch_quantize_k(torch.from_numpy(x), fmt, True)
    tq, ts = tq.numpy(), ts.numpy()
    sf = np.maximum(np.abs(x.reshape(32, -1, 32)).max(-1) / np.float32(mx), np.float32(1e-12)).astype(np.float32)
    l2 = torch.log2(torch.from_numpy(sf)).numpy()
    rounds = (l2 == np.round(l2)) & (np.frexp(sf)[0] != 0.5)    # fp32 log2 landed on an integer
    assert rounds[4, 0] and rounds.sum() >= 1
    assert np.array_equal(s[~rounds], ts[~rounds])
    assert np.all(s[rounds].astype(int) == ts[rounds].astype(int) + 1)   # exact ceil is one higher
    blocks_ok = np.repeat(~rounds, 32, axis=1)
    assert np.array_equal(q[blocks_ok], tq[blocks_ok])
    assert s[2, 0] == 127 - 9 and s[3, 1] == 127 - 9


def test_quantize_k_special_values():
    x = np.zeros((2, 128), dtype=np.float32)
    x[0, 0:32] = np.linspace(-3, 3, 32)
    x[0, 4] = np.nan                              # NaN block
    x[0, 32:64] = 1.0
    x[0, 40] = np.inf                             # inf block
    x[1, :32] = 1e-30                             # tiny: scale 1e-12 floor
    for fmt in ("e4m3", "e5m2"):
        q, s = W.quantize_k(x, fmt, ue8m0=False)
        assert np.isnan(s[0, 0]) and np.all(q[0, :32] == 0x7F)
        assert np.isinf(s[0, 1]) and q[0, 40] == 0x7F and np.all(np.delete(q[0, 32:64], 8) == 0)
        assert s[1, 0] == np.float32(1e-12)
        qb, sb = W.quantize_k(x, fmt, ue8m0=True)
        assert sb[0, 0] == 255 and np.all(qb[0, :32] == 0x7F)
        assert sb[0, 1] == 254                    # inf scale -> 2^127
        mx = MAXF[fmt]
        top = O.encode(np.float32(mx), "e4m3fn" if fmt == "e4m3" else "e5m2")
        assert qb[0, 40] == top                   # inf / 2^127 saturates
        assert sb[1, 0] == 127 + W.ceil_log2_exact(np.float32(1e-12))


def _brute_gemm(a, fa, sa, bt, fb, sb, ue8m0, mode, bias):
    M, K = a.shape
    N = bt.shape[0]
    da = O.decode(a, W._fmt(fa))
    db = O.decode(bt, W._fmt(fb))
    ssa, ssb = W.scales_f64(sa, ue8m0), W.scales_f64(sb, ue8m0)
    C = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            acc = float(bias[n])
            for k in range(K):
                if mode == 0:
                    acc += da[m, k] * ssa[m, k // 32] * db[n, k] * ssb[n, k // 32]
                else:
                    acc += da[m, k] * db[n, k] * ssa[m] * ssb[n]
            C[m, n] = acc
    return C


@pytest.mark.parametrize("ue8m0", [False, True])
def test_gemm_ref_bruteforce_and_planted_mistakes(ue8m0):
    x, w, bias = W.host_case_data(3, 5, 96, seed=3)
    a, sa = W.quantize_k(x, "e4m3", ue8m0)
    bt, sb = W.quantize_k(w.T.copy(), "e5m2", ue8m0)
    ref = W.gemm_ref(a, "e4m3", sa, bt, "e5m2", sb, ue8m0, 0, bias)
    assert W.rel_err(_brute_gemm(a, "e4m3", sa, bt, "e5m2", sb, ue8m0, 0, bias), ref) < 1e-14
    # planted: B's block scales reversed along K, one block scale dropped, A scales on the wrong blocks
    bad = [W.gemm_ref(a, "e4m3", sa, bt, "e5m2", sb[:, ::-1], ue8m0, 0, bias),
           W.gemm_ref(a, "e4m3", sa, bt, "e5m2", np.where(np.arange(3) == 1, (127 if ue8m0 else 1), sb).astype(sb.dtype),
                      ue8m0, 0, bias),
           W.gemm_ref(a, "e4m3", np.roll(sa, 1, axis=1), bt, "e5m2", sb, ue8m0, 0, bias),
           W.gemm_ref(a, "e4m3", sa, bt, "e5m2", sb, ue8m0, 0, None),
           W.gemm_ref(a, "e5m2", sa, bt, "e5m2", sb, ue8m0, 0, bias)]
    for b in bad:
        assert W.rel_err(b, ref) > 1e-3


@pytest.mark.parametrize("ue8m0", [False, True])
def test_gemm_ref_rowcol_bruteforce(ue8m0):
    x, w, bias = W.host_case_data(4, 3, 64, seed=4)
    a, sa = W.quantize_whole(x, "e4m3", ue8m0)
    bt, sb = W.quantize_whole(w.T.copy(), "e4m3", ue8m0)
    ref = W.gemm_ref(a, "e4m3", sa, bt, "e4m3", sb, ue8m0, 1, bias)
    assert W.rel_err(_brute_gemm(a, "e4m3", sa, bt, "e4m3", sb, ue8m0, 1, bias), ref) < 1e-14
    assert W.rel_err(W.gemm_ref(a, "e4m3", sa, bt, "e4m3", sb[::-1].copy(), ue8m0, 1, bias), ref) > 1e-3


def test_host_case_quantization_error_is_fp8_sized():
    x, w, bias = W.host_case_data(128, 96, 512)
    truth = x.astype(np.float64) @ w.astype(np.float64) + bias
    for fmt, lo, hi in (("e4m3", 1e-3, 0.1), ("e5m2", 3e-3, 0.2)):
        a, sa = W.quantize_k(x, fmt)
        bt, sb = W.quantize_k(w.T.copy(), fmt)
        ref = W.gemm_ref(a, fmt, sa, bt, fmt, sb, False, 0, bias)
        assert lo < W.rel_err(ref, truth) < hi


def test_fp8_cuda_api_rejects_cpu_tensors():
    import fp8_cuda
    assert fp8_cuda.BLOCK == 32 and set(fp8_cuda.FORMATS) == {"e4m3", "e5m2"}
    with pytest.raises(ValueError, match="CUDA"):
        fp8_cuda.quantize_k(torch.zeros(2, 64), "e4m3")
    with pytest.raises(ValueError, match="CUDA"):
        fp8_cuda.Fp8Weight(torch.zeros(64, 32))
    with pytest.raises(ValueError, match="unknown"):
        fp8_cuda.quantize_k(torch.zeros(2, 64), "e3m4")
