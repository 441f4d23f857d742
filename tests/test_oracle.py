"""Pins the CPU oracle (oracle/fp8_oracle.py) before anything is checked against it.

Each oracle function is tied to something independent of its own code:
  decode / lut_f16_bits   the reference's LUT data files (tests/golden/lut_*.bin), torch's float8
                          casts, and the special values of the reference test (test_tfp8.py:37-45)
  encode                  torch's RNE float8 cast on in-range values (test_tfp8.py:48-53), an
                          exhaustive nearest-code scan at every midpoint, saturation and NaN codes
  pow2_ceil / ue8m0_*     closed forms: the fp32-log2 rounding window above each power of two
                          (from log2(1+f) = f/ln2), torch's own log2, exact powers of two
  quantize_weight         the reference's torch formula (quantize.py:15-36) run with torch ops
  dequantize_weight       exact float64 products (pow2) / one f32 rounding (non-pow2)
  activation_to_fp16      exactness invariant (test_tfp8.py:58-62) and the torch formula
  linear_ref64            a triple-loop brute force and torch float64 F.linear
  tolerance               planted mistakes (dropped bias or scale, permuted K blocks, group scale
                          off by one, wrong format, flipped sign) must fail it
"""
import hashlib
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import cpu_path
from oracle import fp8_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TORCH_DT = {"e4m3fn": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}
FMTS = ("e4m3fn", "e5m2")
LUT_SHA = {"e4m3fn": "26f6424f23eb8c679a0602789b1c0a77d61cd603245d021dd64cc7a38e7c3ed2",
           "e5m2": "463691e0517c225d73a9ac64c52c249f0eba967cc0d8ff011d754719d5683f5c"}


def _same(a, b):
    """Bitwise-equal values with NaN == NaN and the sign of zero kept (test_tfp8.py:21-26)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    both_nan = np.isnan(a) & np.isnan(b)
    eq = (a == b) & (np.signbit(a) == np.signbit(b))
    return bool((both_nan | eq).all())


@pytest.mark.parametrize("fmt", FMTS)
def test_lut_matches_reference_data_file(fmt):
    path = os.path.join(GOLDEN, f"lut_{fmt}.bin")
    raw = open(path, "rb").read()
    assert hashlib.sha256(raw).hexdigest() == LUT_SHA[fmt]
    ref = np.frombuffer(raw, dtype="<u2")
    assert np.array_equal(O.lut_f16_bits(fmt), ref)


@pytest.mark.parametrize("fmt", FMTS)
def test_decode_all_codes_match_torch(fmt):
    codes = torch.arange(256, dtype=torch.uint8)
    ref = codes.view(TORCH_DT[fmt]).float().double().numpy()
    assert _same(O.decode(np.arange(256), fmt), ref)
    # NaN codes are exactly the format's: 2 for E4M3FN, 6 for E5M2 (+-inf are separate)
    assert int(np.isnan(O.decode(np.arange(256), fmt)).sum()) == (2 if fmt == "e4m3fn" else 6)


def test_decode_special_values():
    d = lambda c, f: float(O.decode(np.array([c]), f)[0])   # noqa: E731
    assert d(0x00, "e4m3fn") == 0.0 and math.copysign(1, d(0x80, "e4m3fn")) < 0
    assert d(0x7E, "e4m3fn") == 448.0
    assert d(0x01, "e4m3fn") == 2.0 ** -9
    assert math.isnan(d(0x7F, "e4m3fn")) and math.isnan(d(0xFF, "e4m3fn"))
    assert d(0x7B, "e5m2") == 57344.0
    assert d(0x7C, "e5m2") == math.inf and d(0xFC, "e5m2") == -math.inf
    assert d(0x01, "e5m2") == 2.0 ** -16


@pytest.mark.parametrize("fmt", FMTS)
def test_encode_matches_torch_rne_in_range(fmt):
    torch.manual_seed(0)
    mx = O.FORMATS[fmt][4]
    x = torch.cat([torch.randn(20000) * mx / 8, torch.randn(2000) * 2.0 ** -10])
    x = x[x.abs() < mx]
    ref = x.to(TORCH_DT[fmt]).view(torch.uint8).numpy()
    assert np.array_equal(O.encode(x.numpy(), fmt), ref)


@pytest.mark.parametrize("fmt", FMTS)
def test_encode_saturates_and_nan(fmt):
    mx = O.FORMATS[fmt][4]
    q = O.encode(np.array([1e9, -1e9, np.inf, -np.inf, mx * 1.5, np.nan, -np.nan]), fmt)
    vals = O.decode(q[:5], fmt)
    assert vals.tolist() == [mx, -mx, mx, -mx, mx]
    nan_code = 0x7E if fmt == "e5m2" else 0x7F
    assert q[5] == nan_code and q[6] == nan_code


@pytest.mark.parametrize("fmt", FMTS)
def test_encode_midpoints_bruteforce(fmt):
    codes, vals = O._finite_table(fmt)
    mids = (vals[:-1] + vals[1:]) / 2                # exact ties (all representable in f64)
    eps = np.abs(mids) * 2.0 ** -30 + 2.0 ** -40
    probe = np.concatenate([mids, mids + eps, mids - eps, vals, [0.0, -0.0]])
    probe = np.concatenate([probe, -probe])
    got = O.encode(probe, fmt)
    want = np.array([O.bruteforce_encode(float(v), fmt) for v in probe], dtype=np.uint8)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("fmt", FMTS)
def test_encode_round_trips_every_finite_code(fmt):
    c = np.arange(256)
    v = O.decode(c, fmt)
    fin = np.isfinite(v)
    assert np.array_equal(O.encode(v[fin], fmt), c[fin].astype(np.uint8))
    assert int(fin.sum()) == (254 if fmt == "e4m3fn" else 248)


def _jmax(k):
    """Closed form of the fp32-log2 rounding: for s = 2^k (1 + j 2^-23), log2 s rounds to exactly
    k (so ceil(log2 s) = k) iff 0 < j <= floor(ln2 * 2^p), where 2^(p - 22) is the gap from k to
    the next fp32 value toward +inf (half of 2^(floor(log2|k|) - 23) below a negative power of
    two).  Derived from log2(1 + f) = f / ln2 + O(f^2), not from any log2 implementation."""
    if k == 0:
        return 0
    fl = int(math.floor(math.log2(abs(k))))
    if k < 0 and (abs(k) & (abs(k) - 1)) == 0:
        fl -= 1
    return int(math.floor(math.log(2.0) * 2.0 ** (fl - 1)))


def _edge_grid(jmax=80):
    k = np.arange(-126, 128)
    j = np.arange(0, jmax + 1)
    kk, jj = np.meshgrid(k, j, indexing="ij")
    s = np.ldexp(1.0 + jj * 2.0 ** -23, kk).astype(np.float32)
    assert np.array_equal(s.astype(np.float64), np.ldexp(1.0 + jj * 2.0 ** -23, kk))   # exact
    return kk, jj, s


def test_pow2_ceil_closed_form():
    # every exponent, the 80 values above each power of two: the closed form of the rounding
    kk, jj, s = _edge_grid()
    want = np.where((jj == 0) | (jj <= np.vectorize(_jmax)(kk)), kk, kk + 1)
    assert np.array_equal(O.ceil_log2_f32(s), want.astype(np.float32))
    assert np.array_equal(O.pow2_ceil(s), np.ldexp(np.float32(1.0), want).astype(np.float32))
    assert int((want == kk)[jj > 0].sum()) > 3000      # the window is not empty
    # torch's own fp32 log2 (an independent implementation) agrees with it everywhere here
    ts = torch.from_numpy(s)
    assert np.array_equal(torch.exp2(torch.ceil(torch.log2(ts))).numpy(), O.pow2_ceil(s))
    # away from the window: the exact power of two at or above s
    rng = np.random.default_rng(1)
    r = (rng.random(2000) * 10.0 ** rng.integers(-30, 30, 2000)).astype(np.float32)
    r = r[(r > 0) & ((r.view(np.uint32) & 0x7FFFFF) > 64)]
    got = O.pow2_ceil(r)
    for a, g in zip(r.tolist(), got.tolist()):
        m, e = math.frexp(a)
        assert g == math.ldexp(1.0, e)
    assert np.array_equal(got, O.pow2_ceil_exact(r))
    for k in (-126, -20, -7, -4, 0, 3, 60):
        p = np.float32(math.ldexp(1.0, k))
        assert O.pow2_ceil(p) == p == O.pow2_ceil_exact(p)
    # a planted mistake -- the exact ceiling -- differs from the reference rounding in the window
    assert not np.array_equal(O.pow2_ceil_exact(s), O.pow2_ceil(s))


def test_ue8m0_closed_form():
    b = np.arange(256)
    v = O.ue8m0_decode(b)
    for i in range(255):
        assert float(v[i]) == math.ldexp(1.0, i - 127)
    assert np.isnan(v[255])
    assert np.array_equal(O.ue8m0_encode(v[1:255]), b[1:255].astype(np.uint8))
    assert O.ue8m0_encode(np.float32(0.75)) == 127       # ceil(log2 0.75) = 0
    assert O.ue8m0_encode(np.float32(np.nan)) == 255


def _torch_quantize_reference(w, fmt, G, pow2):
    """The reference formula with torch ops (tfp8/quantize.py:11-36)."""
    mx = O.FORMATS[fmt][4]
    N, K = w.shape
    wg = w.float().reshape(N, K // G, G)
    amax = wg.abs().amax(-1)
    s = (amax / mx).clamp_min(torch.finfo(torch.float32).tiny)
    if pow2:
        s = torch.exp2(torch.ceil(torch.log2(s)))
    s = torch.where(amax == 0, torch.ones_like(s), s)
    q = (wg / s[..., None]).clamp(-mx, mx).to(TORCH_DT[fmt]).view(torch.uint8).reshape(N, K)
    return q.numpy(), s.numpy()


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("G", [None, 32, 128])
@pytest.mark.parametrize("pow2", [True, False])
def test_quantize_weight_matches_reference_formula(fmt, G, pow2):
    torch.manual_seed(3)
    w = torch.randn(64, 256) * 0.02
    w[3, :] = 0.0                                   # all-zero row -> scale 1
    w[5, 17] = 40.0                                 # outlier
    q, s, GG = O.quantize_weight(w.numpy(), fmt, G, pow2)
    rq, rs = _torch_quantize_reference(w, fmt, GG, pow2)
    assert np.array_equal(q, rq)
    assert np.array_equal(s, rs)


def test_quantize_weight_ue8m0_and_error_bound():
    rng = np.random.default_rng(7)
    w = (rng.laplace(0, 0.02, (32, 128))).astype(np.float32)
    q, b, G = O.quantize_weight(w, "e5m2", 32, True, "ue8m0")
    q2, s2, _ = O.quantize_weight(w, "e5m2", 32, True, "f32")
    assert b.dtype == np.uint8 and np.array_equal(q, q2)
    assert np.array_equal(O.ue8m0_decode(b), s2)
    # |w - q*s| <= half a step of the code grid (relative 2^-3 for E5M2) of the group max
    wd = O.dequantize_weight(q, b, "e5m2", 32)
    amax = np.abs(w.reshape(32, 4, 32)).max(-1).repeat(32, axis=1).reshape(32, 128)
    assert (np.abs(wd - w) <= np.maximum(np.abs(w) * 2.0 ** -3, amax * 2.0 ** -16)).all()


def test_dequantize_exact_products():
    rng = np.random.default_rng(2)
    q = rng.integers(0, 256, (16, 64)).astype(np.uint8)
    q[O.is_nan(q, "e4m3fn")] = 0
    s_pow2 = np.ldexp(np.float32(1), rng.integers(-20, 5, (16, 2))).astype(np.float32)
    exact = O.decode(q, "e4m3fn").reshape(16, 2, 32) * s_pow2.astype(np.float64)[..., None]
    assert np.array_equal(O.dequantize_weight(q, s_pow2, "e4m3fn", 32).astype(np.float64), exact.reshape(16, 64))
    s_gen = (rng.random((16, 2)) + 0.5).astype(np.float32)
    prod = (O.decode(q, "e4m3fn").reshape(16, 2, 32) * s_gen.astype(np.float64)[..., None]).astype(np.float32)
    assert np.array_equal(O.dequantize_weight(q, s_gen, "e4m3fn", 32), prod.reshape(16, 64))


def test_activation_to_fp16_exact_and_matches_torch_formula():
    torch.manual_seed(4)
    x = (torch.randn(5, 256) * 1e3).bfloat16()
    x16, xs = O.activation_to_fp16(x.float().numpy())
    assert np.all(np.log2(xs) == np.round(np.log2(xs)))
    assert np.array_equal(x16.astype(np.float32) * xs[:, None], x.float().numpy())
    # reference formula (log2-based)
    amax = x.float().abs().amax(-1)
    e = torch.ceil(torch.log2(amax)) - 8
    assert np.array_equal(torch.exp2(e).numpy(), xs)
    zero = O.activation_to_fp16(np.zeros((1, 8), np.float32))[1]
    assert zero[0] == 1.0
    # fp32 rows whose amax sits a few ULP above a power of two: e follows the fp32 log2 rounding
    kk, jj, s = _edge_grid(24)
    rows = np.zeros((s.size, 16), np.float32)
    rows[:, 3] = -s.reshape(-1)
    rows[:, 7] = s.reshape(-1) * np.float32(0.25)
    ok = s.reshape(-1) >= 2.0 ** -100
    x16, xs = O.activation_to_fp16(rows[ok])
    want = torch.exp2(torch.ceil(torch.log2(torch.from_numpy(s.reshape(-1)[ok]))) - 8).numpy()
    assert np.array_equal(xs, want)
    exact = np.ldexp(np.float32(1.0), np.ceil(np.log2(s.reshape(-1)[ok].astype(np.float64))).astype(np.int32) - 8)
    assert not np.array_equal(xs, exact.astype(np.float32))   # the window is hit


def test_linear_ref64_bruteforce_and_torch():
    rng = np.random.default_rng(5)
    q = rng.integers(0, 0x7E, (5, 32)).astype(np.uint8)
    s = (rng.random((5, 2)) + 0.5).astype(np.float32)
    x = rng.standard_normal((3, 32)).astype(np.float32)
    b = rng.standard_normal(5).astype(np.float32)
    y = O.linear_ref64(x, q, s, 16, "e4m3fn", b)
    W = O.dequantize_weight(q, s, "e4m3fn", 16)
    bf = np.array(O.bruteforce_linear(x.tolist(), W.tolist(), b.tolist()))
    assert np.allclose(y, bf, rtol=1e-12, atol=1e-12)
    t = F.linear(torch.from_numpy(x).double(), torch.from_numpy(W).double(), torch.from_numpy(b).double())
    assert np.allclose(y, t.numpy(), rtol=1e-12, atol=1e-12)


def test_tolerance_catches_planted_mistakes():
    """Plausible kernel mistakes, planted in a CPU copy of the oracle's output, must fail the bound."""
    rng = np.random.default_rng(6)
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    q, s, G = O.quantize_weight(w, "e4m3fn", 32, False)
    x = rng.standard_normal((4, 256)).astype(np.float32)
    b = (rng.standard_normal(64) * 0.1).astype(np.float32)
    ref = O.linear_ref64(x, q, s, G, "e4m3fn", b)
    tol = O.tolerance(ref, "bfloat16")
    good = ref.astype(np.float32).astype(np.float64)
    assert (np.abs(good - ref) <= tol).all()
    no_bias = O.linear_ref64(x, q, s, G, "e4m3fn", None)
    assert not (np.abs(no_bias - ref) <= tol).all()
    s_shift = np.roll(s, 1, axis=1)                  # group scale index off by one
    assert not (np.abs(O.linear_ref64(x, q, s_shift, G, "e4m3fn", b) - ref) <= tol).all()
    q_t = q.reshape(64, 8, 32)[:, ::-1, :].reshape(64, 256)   # K blocks permuted
    assert not (np.abs(O.linear_ref64(x, q_t, s, G, "e4m3fn", b) - ref) <= tol).all()
    assert not (np.abs(O.linear_ref64(x, q, s, G, "e5m2", b) - ref) <= tol).all()
    ones = np.ones_like(s)                          # scale dropped
    assert not (np.abs(O.linear_ref64(x, q, ones, G, "e4m3fn", b) - ref) <= tol).all()
    q_neg = q ^ np.uint8(0x80)                      # sign bit flipped
    assert not (np.abs(O.linear_ref64(x, q_neg, s, G, "e4m3fn", b) - ref) <= tol).all()


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("G", [None, 32])
def test_fake_quant_idempotent_pow2(fmt, G):
    """dequant(quant(.)) is a projection for power-of-two scales (test_fp8_sim.py:46-60): values already
    on the grid come back unchanged, even where the second pass picks a smaller scale."""
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((24, 128)) * 0.02).astype(np.float32)
    w[rng.random(w.shape) < 0.01] *= 20
    q, s, GG = O.quantize_weight(w, fmt, G, True)
    w1 = O.dequantize_weight(q, s, fmt, GG)
    q2, s2, _ = O.quantize_weight(w1, fmt, G, True)
    w2 = O.dequantize_weight(q2, s2, fmt, GG)
    assert np.array_equal(w1, w2)
    assert not np.array_equal(w1, w)


def test_cpu_path_matches_oracle():
    rng = np.random.default_rng(8)
    w = (rng.standard_normal((48, 128)) * 0.02).astype(np.float32)
    for fmt, G, sf in (("e4m3fn", None, "f32"), ("e5m2", 32, "ue8m0"), ("e4m3fn", 64, "f32")):
        q, s, GG = O.quantize_weight(w, fmt, G, True, sf)
        x = rng.standard_normal((6, 128)).astype(np.float32)
        ref = O.linear_ref64(x, q, s, GG, fmt, None)
        y = cpu_path.cpu_forward(torch.from_numpy(x), torch.from_numpy(q), torch.from_numpy(s), GG, fmt, None,
                                 torch.float32)
        assert (np.abs(y.double().numpy() - ref) <= O.tolerance(ref, "float32")).all()


def test_cpu_path_dequant_weight_f32_matches_oracle():
    rng = np.random.default_rng(12)
    q = rng.integers(0, 256, (24, 128)).astype(np.uint8)
    for fmt in FMTS:
        for s in (rng.random((24, 4)).astype(np.float32) + 0.25,
                  np.concatenate([rng.integers(0, 256, (23, 4)), [[0, 1, 254, 255]]]).astype(np.uint8)):
            want = O.dequantize_weight(q, s, fmt, 32)
            got = cpu_path.dequant_weight_f32(torch.from_numpy(q), torch.from_numpy(s), 32, fmt).numpy()
            same = (got == want) | (np.isnan(got) & np.isnan(want))
            assert same.all(), fmt
