"""tfp8_linear_noalloc (the entry point that allocates nothing: its workspace is a library-owned
device scratch array) against tfp8_linear with a caller workspace: bit-identical outputs, since
both run the same kernels in the same order.  Two calls in a row, the second with a smaller input,
so the second reuses scratch the first left behind; shapes that use the scratch for split-K
partial sums and for the fp32-activation prep, the GEMV (no scratch), and the size limit."""

import pytest
import torch

from tfp8 import _ext
from tfp8.quantize import quantize_weight

pytestmark = pytest.mark.gpu


def _layer(N, K, G, fmt, sf, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(N, K, generator=g, device="cuda") * 0.02
    q, s, GG = quantize_weight(w, fmt, G, True, sf)
    b = torch.randn(N, generator=g, device="cuda") * 0.1
    return q, s, GG, b


def _args(x, q, s, G, fmt, b, y):
    M, K = x.shape
    return (x.data_ptr(), _ext.DTYPE_ID[x.dtype], M, K, q.data_ptr(), q.shape[0], s.data_ptr(), _ext.scale_kind(s),
            G, _ext.FMT_ID[fmt], b.data_ptr() if b is not None else None, y.data_ptr(), _ext.DTYPE_ID[y.dtype])


def _both(lib, x, q, s, G, fmt, b, ydt):
    M, K = x.shape
    N = q.shape[0]
    stream = torch._C._cuda_getCurrentRawStream(0)
    y_ref = torch.empty(M, N, dtype=ydt, device="cuda")
    nb = lib.tfp8_linear_workspace_size(_ext.DTYPE_ID[x.dtype], M, N, K)
    ws = torch.empty(max(nb, 1), dtype=torch.uint8, device="cuda")
    rc = lib.tfp8_linear(*_args(x, q, s, G, fmt, b, y_ref), ws.data_ptr() if nb else None, nb, stream)
    assert rc == 0, _ext.last_error()
    y = torch.full((M, N), float("nan"), dtype=ydt, device="cuda")
    rc = lib.tfp8_linear_noalloc(*_args(x, q, s, G, fmt, b, y), stream)
    assert rc == 0, lib.tfp8_last_error().decode()
    torch.cuda.synchronize()
    return y, y_ref, nb


@pytest.mark.parametrize("case", [
    # (fmt, scale kind, G, N, K, x dtype, out dtype, M first, M second)
    ("e4m3fn", "ue8m0", None, 8192, 8192, torch.float16, torch.float16, 256, 64),    # C3: split-K partials
    ("e5m2", "ue8m0", 32, 4096, 11008, torch.bfloat16, torch.bfloat16, 128, 48),     # C4 shape, group scales
    ("e4m3fn", "f32", 128, 2048, 4096, torch.float32, torch.float32, 200, 40),       # fp32 x: prep in scratch
    ("e4m3fn", "f32", 128, 14336, 4096, torch.bfloat16, torch.bfloat16, 8, 1),       # GEMV: no scratch
])
def test_noalloc_matches_workspace_entry(case):
    fmt, sf, G, N, K, xdt, ydt, m1, m2 = case
    print(f"[noalloc] {case}", flush=True)
    lib = _ext.require()
    q, s, GG, b = _layer(N, K, G, fmt, sf, N + K)
    g = torch.Generator(device="cuda").manual_seed(K)
    used = []
    for M in (m1, m2):
        x = torch.randn(M, K, generator=g, device="cuda").to(xdt)
        y, y_ref, nb = _both(lib, x, q, s, GG, fmt, b, ydt)
        used.append(nb)
        assert torch.equal(y.view(torch.uint8), y_ref.view(torch.uint8)), (case, M)
    if m1 > _ext.GEMV_MAXM:
        assert used[0] > 0          # the first call did go through the scratch
    else:
        assert used == [0, 0]


def test_noalloc_refuses_workspace_beyond_scratch():
    """fp32 activations of 4096 x 8192 need 64 MiB + 16 KiB of fp16 staging: more than the scratch,
    so the call is refused before any launch and y is untouched."""
    print("[noalloc] size limit", flush=True)
    lib = _ext.require()
    M, N, K = 4096, 256, 8192
    assert lib.tfp8_linear_workspace_size(2, M, N, K) > (64 << 20)
    q = torch.zeros(N, K, dtype=torch.uint8, device="cuda")
    s = torch.ones(N, 1, device="cuda")
    x = torch.zeros(M, K, device="cuda")
    y = torch.full((M, N), 7.0, device="cuda")
    rc = lib.tfp8_linear_noalloc(*_args(x, q, s, K, "e4m3fn", None, y), torch._C._cuda_getCurrentRawStream(0))
    assert rc == -4 and b"scratch" in lib.tfp8_last_error()
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
