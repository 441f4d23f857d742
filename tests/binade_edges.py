"""Inputs that sit a few ULP above a power of two, where the reference's fp32 log2 rounds to the
integer (tfp8/quantize.py:11-12 and :58-59): ceil(log2 s) is then k, not k + 1, for
s = 2^k (1 + j 2^-23) with 0 < j <= a small bound that grows with |k|.  Shared by the CPU and
GPU tests of quantize_weight and activation_to_fp16."""
import numpy as np

from oracle import fp8_oracle as O


def weight_rows(fmt, G=32, js=range(0, 25), ks=range(-118, 100, 3), seed=0):
    """w [N, 2G] float32: in each row, group 0's amax is fl32((2^k (1 + j 2^-23)) * max_finite), so
    its scale amax / max_finite lands on or next to the rounding window; group 1 is ordinary data."""
    mx = O.FORMATS[fmt][4]
    rng = np.random.default_rng(seed)
    rows = []
    for k in ks:
        for j in js:
            s = np.float32(np.ldexp(1.0 + j * 2.0 ** -23, k))
            amax = np.float32(np.float64(s) * mx)
            if not np.isfinite(amax) or amax == 0:
                continue
            r = (rng.standard_normal(2 * G) * 0.2).astype(np.float32)
            r[:G] = np.clip(r[:G], -0.9, 0.9) * amax
            r[rng.integers(0, G)] = amax * (1 if rng.random() < 0.5 else -1)
            r[G:] *= np.float32(np.ldexp(1.0, int(np.clip(k, -100, 100))))
            rows.append(r)
    return np.stack(rows).astype(np.float32)


def window_hits(w, fmt, G):
    """How many groups of w get a different scale from the reference rounding than from the exact
    power-of-two ceiling (i.e. fall inside the window)."""
    mx = np.float32(O.FORMATS[fmt][4])
    N, K = w.shape
    amax = np.abs(w.reshape(N, K // G, G)).max(-1)
    s = np.maximum((amax / mx).astype(np.float32), np.float32(np.finfo(np.float32).tiny))
    return int((O.pow2_ceil(s) != O.pow2_ceil_exact(s)).sum())


def activation_rows(K=64, js=range(0, 25), ks=range(-98, 120, 2)):
    """x [M, K] float32 whose row amax is 2^k (1 + j 2^-23) (sign alternating), other entries smaller."""
    rows = []
    for k in ks:
        for j in js:
            a = np.float32(np.ldexp(1.0 + j * 2.0 ** -23, k))
            r = (np.linspace(-0.9, 0.9, K) * a).astype(np.float32)
            r[(k + j) % K] = a if j % 2 == 0 else -a
            rows.append(r)
    return np.stack(rows).astype(np.float32)
