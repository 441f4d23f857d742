"""GPU parity of the FP8Linear path (GEMV for M <= 8, MFMA GEMM above) against the float64
oracle, with the reference's tolerance (tests/test_tfp8.py:86-89):

    |y - ref| <= eps*|ref| + 1e-4*max|ref| + 1e-6,   eps = 2^-11 (fp16 out) or 2^-8 (bf16/fp32 out)

Cases: the reference's kernel gates (switch points, tails, ragged K, group scales x formats x
dtypes, pipeline edges, folded group scales, empty / non-contiguous / N-d input, prepared GEMV
launch state, NaN fallback) and every benchmark configuration (C1-C4) at its full size, plus the reference's
CPU dequantize-then-matmul path as a second reference.
"""

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import cpu_path
from oracle import fp8_oracle as O
from tfp8 import _ext
from tfp8.linear import FP8Linear
from tfp8.quantize import quantize_weight

pytestmark = pytest.mark.gpu
DTN = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}


def _x_eff(x, path):
    """What the kernel multiplies: x itself, except fp32 x on the GEMM path, which is fp16 with a
    power-of-two row scale (reference prep, tfp8/quantize.py:47-62)."""
    xf = x.float().cpu().numpy()
    if x.dtype == torch.float32 and path == "gemm":
        x16, xs = O.activation_to_fp16(xf)
        return x16.astype(np.float64) * xs.astype(np.float64)[:, None]
    return xf.astype(np.float64)


def _check(y, x, q, s, G, fmt, bias, out_dtype, path, label):
    ref = O.linear_ref64(_x_eff(x, path), q.cpu().numpy(), s.cpu().numpy(), G, fmt,
                         None if bias is None else bias.cpu().numpy())
    tol = O.tolerance(ref, DTN[out_dtype])
    d = np.abs(y.double().cpu().numpy() - ref)
    bad = int((~(d <= tol)).sum())
    assert bad == 0, f"{label}: {bad} mismatches, max excess {float(np.max(d - tol)):.3g}"
    return ref


def _layer(N, K, G, fmt, sf="f32", pow2=True, seed=0, wscale=0.02, bias=True):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * wscale
    q, s, GG = quantize_weight(w.cuda(), fmt, G, pow2, sf)
    b = (torch.randn(N, generator=g) * 0.1).cuda() if bias else None
    return q, s, GG, b


def _run(M, N, K, G, out_dtype, fmt="e4m3fn", bias=True, xdt=torch.bfloat16, sf="f32", pow2=True, seed=None):
    seed = M * 7 + N if seed is None else seed
    print(f"[linear] M={M} N={N} K={K} G={G} fmt={fmt} x={xdt} out={out_dtype} sf={sf} bias={bias}", flush=True)
    q, s, GG, b = _layer(N, K, G, fmt, sf, pow2, seed, bias=bias)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(seed + 1)).to(xdt).cuda()
    y = _ext.w8a16(x, q, None, s, b, out_dtype, GG, fmt)
    path = "gemv" if M <= _ext.GEMV_MAXM else "gemm"
    _check(y, x, q, s, GG, fmt, b, out_dtype, path, f"M={M} N={N} K={K} G={G} {fmt} {xdt}->{out_dtype}")


# ------------------------------------------------------------------ reference kernel gates
def test_kernel_switch_points_and_tails():
    for M in (1, 2, 3, 7, 8, 9, 15, 16, 31, 32, 127, 128, 255, 256, 300):
        _run(M, 200, 512, None, torch.float16)


def test_streaming_gemv_m1_where_pair_applies(tune):
    """M <= 3 shapes the row-pair (and 4x4x4-MFMA) GEMV would take, forced through the streaming
    GEMV instead (and M = 4 through the matrix-core decode kernel)."""
    tune(TFP8_GEMV_PAIR=0, TFP8_GEMV_QUAD=0)
    for M in (1, 2, 3, 4):
        for N, K, G in ((14336, 4096, 128), (4096, 4096, None), (998, 2048, 64)):
            _run(M, N, K, G, torch.bfloat16, seed=N + K + M)


def test_kernel_ragged_k_tail():
    for K in (528, 1040, 1152, 1168, 1184):
        for M in (1, 8, 16, 64):
            _run(M, 200, K, None, torch.float16)


def test_kernel_group_scales_formats_dtypes():
    for G in (None, 32, 128):
        for fmt in ("e4m3fn", "e5m2"):
            for od in (torch.float16, torch.bfloat16, torch.float32):
                for M in (1, 40):
                    _run(M, 128, 1024, G, od, fmt, bias=(G != 32))


def test_activation_dtypes_both_paths():
    for xdt in (torch.float16, torch.bfloat16, torch.float32):
        for M in (1, 3, 8, 9, 33, 100):
            for sf in ("f32", "ue8m0"):
                _run(M, 160, 768, 128, torch.float32, "e4m3fn", xdt=xdt, sf=sf)


def test_gemm_pipeline_edges():
    for K in (32, 64, 96, 160):
        for G in (None, 32):
            for M in (9, 64, 65, 130):
                _run(M, 72, K, G, torch.float16, bias=(G is None))


def test_group_scale_applied_per_block():
    print("[group locality]", flush=True)
    K, N = 256, 64
    g = torch.Generator().manual_seed(3)
    w = torch.randn(N, K, generator=g) * 0.02
    w[:, :128] *= 1000.0
    q, s, G = quantize_weight(w.cuda(), "e4m3fn", 128)
    x = (torch.randn(33, K, generator=g) * 1e-3).cuda()
    for M in (1, 33):
        y = _ext.w8a16(x[:M], q, None, s, None, torch.float16, G, "e4m3fn")
        ref = O.linear_ref64(x[:M].cpu().numpy(), q.cpu().numpy(), s.cpu().numpy(), G, "e4m3fn")
        assert (np.abs(y.double().cpu().numpy() - ref) / np.abs(ref).max()).max() < 2e-3


def test_gemm_group_scales_exact_fp32_partials():
    """K-group scales spanning 2^-20 (pow2) and arbitrary f32 values (checkpoint mode) are applied to
    fp32 partial sums, so the error stays at fp32-accumulation level in both cases -- tighter than
    the reference's fold-into-fp16 bound (1e-5 / 5e-4 relative to the largest output)."""
    g = torch.Generator().manual_seed(5)
    N, K, G = 96, 1024, 128
    for fmt in ("e4m3fn", "e5m2"):
        for pow2 in (True, False):
            print(f"[folded scales] fmt={fmt} pow2={pow2}", flush=True)
            codes = torch.randint(0, 256, (N, K), dtype=torch.uint8, generator=g)
            v = torch.from_numpy(O.decode(codes.numpy(), fmt))
            codes[~torch.isfinite(v)] = 0x10
            ws = torch.exp2(torch.randint(-20, 1, (N, K // G), generator=g).float()) * 1e-2
            if not pow2:
                ws = ws * (1 + torch.rand(N, K // G, generator=g))
            f = FP8Linear.from_fp8_checkpoint(codes.cuda(), ws.cuda(), bias=torch.randn(N, generator=g).cuda(),
                                              fmt=fmt)
            f.out_dtype = torch.float32
            f.nan_check = False
            for M in (16, 100):
                x = torch.randn(M, K, generator=g).bfloat16().cuda()
                ref = O.linear_ref64(x.float().cpu().numpy(), codes.numpy(), ws.numpy(), G, fmt, f.bias_f32.cpu().numpy())
                err = (np.abs(f(x).double().cpu().numpy() - ref) / np.abs(ref).max()).max()
                assert err < 1e-5, f"{fmt} pow2={pow2} M={M}: err/max {err}"
            assert f.stats["gemm"] >= 1


def test_forced_gemm_at_small_m_and_gemv_directly():
    """The MFMA GEMM at M <= 8 (gemm_prepared) and the GEMV entry point agree with the oracle."""
    q, s, G, b = _layer(136, 512, 64, "e5m2", "ue8m0", seed=21)
    for M in (1, 5, 8):
        print(f"[forced paths] M={M}", flush=True)
        x = torch.randn(M, 512, generator=torch.Generator().manual_seed(M)).half().cuda()
        y1 = _ext.gemm_prepared(x, None, q, None, s, b, torch.float32, G, "e5m2")
        _check(y1, x, q, s, G, "e5m2", b, torch.float32, "gemm", f"gemm M={M}")
        xs = torch.full((M,), 0.5, device="cuda")
        y2 = _ext.gemm_prepared(x, xs, q, None, s, b, torch.float32, G, "e5m2")
        ref = O.linear_ref64(x.float().cpu().numpy() * 0.5, q.cpu().numpy(), s.cpu().numpy(), G, "e5m2",
                             b.cpu().numpy())
        assert (np.abs(y2.double().cpu().numpy() - ref) <= O.tolerance(ref, "float32")).all()
        y3 = _ext.gemv(x, q, s, b, torch.float32, G, "e5m2")
        _check(y3, x, q, s, G, "e5m2", b, torch.float32, "gemv", f"gemv M={M}")


def test_gemv_prepared_launch_tracks_layer_state():
    print("[gemv launch state]", flush=True)
    torch.manual_seed(11)
    lin = nn.Linear(512, 200, device="cuda")
    f = FP8Linear.from_linear(lin, group_size=128)
    f.nan_check = False

    def general(x):
        return _ext.w8a16(x.reshape(-1, 512), f.qweight, None, f.weight_scale, f.bias_f32, f.out_dtype,
                          f.group_size, f.fmt)

    for xd in (torch.float16, torch.bfloat16, torch.float32):
        for M in (1, 3, 8):
            x = torch.randn(M, 512, device="cuda", dtype=xd)
            y = f(x)
            assert torch.equal(y, general(x)), (xd, M)
            _check(y, x, f.qweight, f.weight_scale, 128, "e4m3fn", f.bias_f32, f.out_dtype, "gemv", f"{xd} M={M}")
    assert len(f._bindings) == 3
    x = torch.randn(2, 3, 512, device="cuda", dtype=torch.bfloat16)
    assert torch.equal(f(x), general(x).reshape(2, 3, 200))
    x = torch.randn(4, 512, device="cuda", dtype=torch.bfloat16)
    f.out_dtype = torch.float16
    assert f(x).dtype == torch.float16 and torch.equal(f(x), general(x))
    other = FP8Linear.from_linear(nn.Linear(512, 200, device="cuda"), group_size=128)
    f.qweight = other.qweight.clone()
    f.weight_scale = other.weight_scale.clone()
    assert torch.equal(f(x), general(x))
    f.load_state_dict(other.state_dict())
    assert torch.equal(f(x), general(x))
    f.cpu()
    assert f(x.cpu()).device.type == "cpu"
    f.cuda()
    y = f(x)
    assert torch.equal(y, general(x)) and f.stats["gemv"] >= 12


def test_empty_and_noncontiguous():
    print("[empty/noncontig]", flush=True)
    f = FP8Linear.from_linear(nn.Linear(512, 128, device="cuda"))
    assert f(torch.empty(0, 512, device="cuda")).shape == (0, 128)
    x = torch.randn(512, 20, device="cuda").t()
    assert torch.allclose(f(x).float(), f(x.contiguous()).float())
    assert f(torch.randn(2, 3, 512, device="cuda")).shape == (2, 3, 128)
    assert f(torch.randn(3, 7, 512, device="cuda")).shape == (3, 7, 128)   # M=21 -> GEMM


def test_nan_fallback():
    print("[nan fallback]", flush=True)
    f = FP8Linear.from_linear(nn.Linear(512, 128, device="cuda"))
    f.out_dtype = torch.float16
    f.weight_scale.fill_(1e30)
    f(torch.randn(4, 512, device="cuda"))
    assert f.fallback is not None and "non-finite" in f.fallback_reason


def test_chunked_backend_counts_and_matches():
    """The large-M (chunked) branch, as the reference's test_chunked_formats_dtypes_and_slices
    (tests/test_tfp8.py:138-162): both formats, every output dtype, per-channel and 128-groups,
    with and without bias; then odd / ragged N with workspace_mb=0 (the reference's multi-slice
    case) against the f16-prepared activations the reference multiplies."""
    for fmt in ("e4m3fn", "e5m2"):
        for od in (torch.float16, torch.bfloat16, torch.float32):
            for G in (None, 128):
                print(f"[large-M branch] fmt={fmt} out={od} G={G}", flush=True)
                q, s, GG, b = _layer(192, 512, G, fmt, seed=len(fmt) + (G or 0), bias=G is None)
                f = FP8Linear(512, 192, bias=G is None, fmt=fmt, group_size=GG, out_dtype=od,
                              large_m_backend="chunked", device="cuda")
                f.qweight.copy_(q)
                f.weight_scale = s
                if b is not None:
                    f.bias_f32.copy_(b)
                x = torch.randn(260, 512, generator=torch.Generator().manual_seed(3)).bfloat16().cuda()
                y = f(x)
                assert y.dtype == od and f.stats["chunked"] == 1
                _check(y, x, q, s, GG, fmt, b, od, "gemm", f"chunked {fmt} {od} G={G}")
    for N, bias in ((200, True), (330, False), (77, True)):
        print(f"[large-M branch] N={N} bias={bias} workspace_mb=0", flush=True)
        torch.manual_seed(N)
        lin = nn.Linear(1024, N, bias=bias, device="cuda")
        f = FP8Linear.from_linear(lin, large_m_backend="chunked")
        f.out_dtype = torch.float16
        f.workspace_mb = 0
        x = torch.randn(300, 1024, device="cuda", dtype=torch.bfloat16)
        y = f(x)
        assert f.stats["chunked"] == 1
        _check(y, x, f.qweight, f.weight_scale, f.group_size, "e4m3fn", f.bias_f32, torch.float16, "gemm",
               f"chunked N={N}")


# ------------------------------------------------------------------ benchmark configurations C1-C4, full size
def test_config1_gemv_m1_and_cpu_path():
    """C1: M=1, K=N=4096, fp16 x ~N(0,1), W ~N(0,0.02) E4M3FN per-channel pow2 f32, no bias."""
    print("[C1] M=1 K=N=4096", flush=True)
    g = torch.Generator().manual_seed(101)
    w = torch.randn(4096, 4096, generator=g) * 0.02
    q, s, G = quantize_weight(w.cuda(), "e4m3fn", None, True)
    x = torch.randn(1, 4096, generator=g).half()
    f = FP8Linear.from_fp8_checkpoint(q, s, fmt="e4m3fn")
    f.out_dtype = torch.float16
    f.nan_check = False
    y = f(x.cuda())
    assert f.stats["gemv"] == 1
    _check(y, x, q, s, G, "e4m3fn", None, torch.float16, "gemv", "C1")
    # the reference's own CPU path (dequantize then F.linear in fp32) within the same bound
    yc = cpu_path.cpu_forward(x, q.cpu(), s.cpu(), G, "e4m3fn", None, torch.float32).double().numpy()
    d = np.abs(y.double().cpu().numpy() - yc)
    assert (d <= O.tolerance(yc, "float16")).all()


@pytest.mark.parametrize("M", [1, 2, 4, 8])
def test_config2_decode_sweep(M):
    """C2: K=4096, N=14336, bf16 x, W ~N(0,0.02) with 0.1% outliers x20, E4M3FN G=128 f32 scales
    (general amax/448 and the pow2 side check)."""
    print(f"[C2] M={M}", flush=True)
    g = torch.Generator().manual_seed(202)
    w = torch.randn(14336, 4096, generator=g) * 0.02
    w = torch.where(torch.rand(w.shape, generator=g) < 1e-3, w * 20, w)
    x = torch.randn(M, 4096, generator=g).bfloat16().cuda()
    for pow2 in (False, True):
        q, s, G = quantize_weight(w.cuda(), "e4m3fn", 128, pow2)
        y = _ext.w8a16(x, q, None, s, None, torch.bfloat16, G, "e4m3fn")
        _check(y, x, q, s, G, "e4m3fn", None, torch.bfloat16, "gemv", f"C2 M={M} pow2={pow2}")


@pytest.mark.parametrize("M", [16, 64, 256])
def test_config3_gemm(M):
    """C3: K=N=8192, fp16 x, E4M3FN W ~N(0,0.01) per-channel UE8M0, f32 bias ~N(0,0.1)."""
    print(f"[C3] M={M}", flush=True)
    g = torch.Generator().manual_seed(303)
    w = torch.randn(8192, 8192, generator=g) * 0.01
    q, s, G = quantize_weight(w.cuda(), "e4m3fn", None, True, "ue8m0")
    b = (torch.randn(8192, generator=g) * 0.1).cuda()
    x = torch.randn(M, 8192, generator=g).half().cuda()
    y = _ext.w8a16(x, q, None, s, b, torch.float16, G, "e4m3fn")
    _check(y, x, q, s, G, "e4m3fn", b, torch.float16, "gemm", f"C3 M={M}")


def test_config4_e5m2_block32_ue8m0():
    """C4: M=128, K=11008, N=4096, bf16 x rows scaled by 2^u (u in -20..20), W ~Laplace(0,0.02)
    E5M2 with G=32 UE8M0 scales; forced +-0, subnormal codes 0x01-0x03/0x81-0x83 and max codes."""
    print("[C4] M=128 K=11008 N=4096 e5m2 G32 ue8m0", flush=True)
    g = torch.Generator().manual_seed(404)
    w = torch.distributions.Laplace(0.0, 0.02).sample((4096, 11008))
    q, s, G = quantize_weight(w.cuda(), "e5m2", 32, True, "ue8m0")
    q = q.cpu()
    idx = torch.randint(0, q.numel(), (4096,), generator=g)
    special = torch.tensor([0x00, 0x80, 0x01, 0x02, 0x03, 0x81, 0x82, 0x83, 0x7B, 0xFB], dtype=torch.uint8)
    q.view(-1)[idx] = special[torch.arange(4096) % len(special)]
    q = q.cuda()
    u = torch.randint(-20, 21, (128, 1), generator=g).float()
    x = (torch.randn(128, 11008, generator=g) * torch.exp2(u)).bfloat16().cuda()
    y = _ext.w8a16(x, q, None, s, None, torch.bfloat16, G, "e5m2")
    _check(y, x, q, s, G, "e5m2", None, torch.bfloat16, "gemm", "C4")
    # the encoder side of C4: saturation of +-1e9 / +-inf and E5M2 subnormals
    t = torch.tensor([1e9, -1e9, float("inf"), -float("inf"), 2.0 ** -16, -(2.0 ** -15), 3 * 2.0 ** -16, 0.0, -0.0])
    from tfp8.formats import encode
    assert torch.equal(encode(t.cuda(), "e5m2").cpu(), torch.from_numpy(O.encode(t.numpy(), "e5m2")))


@pytest.mark.parametrize("tile", list(range(1, 14)))
def test_tiled_gemm_every_config(tile, tune):
    """Every LDS-tiled GEMM configuration (forced through the library's tuning hooks), with and
    without split-K, on ragged shapes: rows past M and N, a K tail that is not a whole K tile,
    per-channel and K-group (f32 G=32, UE8M0 G=64) scales, f16 and bf16 activations."""
    tune(TFP8_GEMM_V1=1)
    tune(TFP8_GEMM_DIRECT=0)
    tune(TFP8_GEMM_TILE=tile)
    for split in (1, 3):
        tune(TFP8_GEMM_SPLITK=split)
        _run(40, 200, 1120, None, torch.float16, xdt=torch.float16, seed=tile)
        _run(130, 72, 640, 32, torch.bfloat16, xdt=torch.bfloat16, seed=tile + 1)
        _run(257, 136, 704, 64, torch.float32, fmt="e5m2", xdt=torch.bfloat16, sf="ue8m0", seed=tile + 2)


@pytest.mark.parametrize("direct", [0, 1])
def test_split_k_workspace_contents_do_not_matter(direct, tune):
    """Split-K through the caller's workspace (fp32 partial tiles, then the reduce kernel): a
    workspace full of garbage, or one reused from the previous call, gives the same bits every
    time, within the oracle tolerance (LDS-tiled kernel and direct-load kernel)."""
    tune(TFP8_GEMM_V1=1)
    tune(TFP8_GEMM_DIRECT=direct)
    tune(TFP8_GEMM_TILE=13)
    tune(TFP8_GEMM_SPLITK=3)
    lib = _ext.require()
    M, N, K = 200, 512, 3072
    q, s, G, b = _layer(N, K, None, "e4m3fn", "ue8m0", seed=21)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(22)).half().cuda()
    nb = lib.tfp8_linear_workspace_size(_ext.DTYPE_ID[x.dtype], M, N, K)
    assert nb > 0
    ws = torch.full((nb,), 0xFF, dtype=torch.uint8, device="cuda")
    outs = []
    for rep in range(3):
        if rep == 2:
            ws.random_(0, 256)
        y = torch.empty(M, N, dtype=torch.float16, device="cuda")
        rc = lib.tfp8_linear(x.data_ptr(), _ext.DTYPE_ID[x.dtype], M, K, q.data_ptr(), N, s.data_ptr(),
                             _ext.scale_kind(s), G, _ext.FMT_ID["e4m3fn"], b.data_ptr(), y.data_ptr(),
                             _ext.DTYPE_ID[torch.float16], ws.data_ptr(), nb,
                             torch._C._cuda_getCurrentRawStream(0))
        assert rc == 0, _ext.last_error()
        outs.append(y)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    _check(outs[0], x, q, s, G, "e4m3fn", b, torch.float16, "gemm", "split-K arrival")


@pytest.mark.parametrize("M,N,K,xdt,out,fmt,sf,bias,split", [
    (129, 256, 64, torch.float16, torch.float16, "e4m3fn", "ue8m0", True, 0),     # one K step, 1 row past 128
    (200, 300, 128, torch.bfloat16, torch.bfloat16, "e5m2", "f32", False, 0),     # two steps, ragged N
    (136, 72, 192, torch.float16, torch.float32, "e4m3fn", "f32", True, 0),       # three steps, N < one tile
    (256, 1000, 2048, torch.float16, torch.float32, "e4m3fn", "f32", True, 0),
    (384, 512, 4096, torch.bfloat16, torch.bfloat16, "e4m3fn", "ue8m0", True, 3),  # uneven split (1408, 1408, 1280)
    (1000, 2048, 1024, torch.float16, torch.float16, "e5m2", "ue8m0", True, 1),
    (300, 512, 512, torch.float32, torch.float32, "e4m3fn", "f32", True, 2),      # fp32 x: f16 prep + row scales
    (640, 8192, 1024, torch.bfloat16, torch.bfloat16, "e4m3fn", "ue8m0", True, 0),  # 160 blocks of 128 x 256
])
def test_direct_gemm_shapes(M, N, K, xdt, out, fmt, sf, bias, split, tune):
    """The direct-load GEMM (M > 128, one scale per weight row): rows past M and N inside a tile,
    K of one to three steps (fewer than the LDS ring holds), even and uneven split-K, f16 / bf16 /
    fp32 activations, both formats, f32 and UE8M0 scales, every output dtype.  Grids of at most
    128 blocks of 128 x 256 take 128 x 128 tiles (every case but the last)."""
    if split:
        tune(TFP8_GEMM_SPLITK=split)
    _run(M, N, K, None, out, fmt=fmt, bias=bias, xdt=xdt, sf=sf, seed=M + K)


@pytest.mark.parametrize("M,N,K,G,sf,xdt,fmt,split", [
    (100, 520, 1088, 32, "ue8m0", torch.bfloat16, "e5m2", 0),      # UE8M0 folded into the decode, 128 x 128 tiles
    (256, 4096, 11008, 32, "ue8m0", torch.bfloat16, "e5m2", 0),    # C4's weights at M=256 (split 8, ragged last slice)
    (200, 392, 2048, 64, "f32", torch.float16, "e4m3fn", 0),       # f32 groups: fp32 partial per group
    (300, 1024, 3072, 128, "ue8m0", torch.float16, "e4m3fn", 0),   # UE8M0 groups with f16 x: partial sums
    (130, 256, 4096, 128, "f32", torch.bfloat16, "e4m3fn", 0),     # split 8, slices of 4 groups
    (150, 640, 2304, 192, "f32", torch.bfloat16, "e5m2", 5),       # slices of 512 cut groups of 192
    (200, 512, 1024, 32, "ue8m0", torch.bfloat16, "e5m2", 0),      # folded UE8M0, 128 x 128 tiles above 128 rows
])
def test_direct_gemm_group_scales(M, N, K, G, sf, xdt, fmt, split, tune):
    """K-group scales on the direct-load GEMM: UE8M0 groups folded into the decode (bf16
    activations), and f32 / UE8M0 groups with G % 64 == 0 applied to an fp32 partial sum at each
    group boundary, including split-K slices that start inside a group."""
    if split:
        tune(TFP8_GEMM_SPLITK=split)
    _run(M, N, K, G, torch.float32, fmt=fmt, xdt=xdt, sf=sf, seed=M + G)


@pytest.mark.parametrize("cfg", list(range(0, 8)))
def test_direct_gemm_every_config(cfg, tune):
    """Every direct-load GEMM configuration (block tile 32/64/128 x 128/256, 4 or 8 waves, rings of
    3 to 7 K steps), forced through the library's tuning hooks at small and large M: rows past M
    inside a tile, several row tiles, columns past N, one-step and long K slices."""
    tune(TFP8_GEMM_DIRECT_MIN_M=9)
    tune(TFP8_GEMM_DCFG=cfg)
    _run(20, 520, 64, None, torch.float16, xdt=torch.float16, sf="ue8m0", seed=cfg)
    _run(100, 392, 1088, None, torch.bfloat16, fmt="e5m2", xdt=torch.bfloat16, seed=cfg + 1)
    _run(300, 1024, 3072, None, torch.float32, xdt=torch.float16, seed=cfg + 2)


@pytest.mark.parametrize("nt,w,d", [(2, 8, 4), (2, 8, 8), (2, 4, 4), (2, 4, 8), (1, 8, 4), (1, 8, 8), (1, 4, 4), (1, 4, 8)])
def test_decode_mfma_every_config(nt, w, d, tune):
    """The matrix-core decode kernel (up to 16 rows) in every compiled configuration, forced down to
    M = 1: rows past N in the last block, a K tail that is not a whole 64-byte chunk, K ranges that
    leave some waves without work, per-channel / f32 K-group (G=64) / UE8M0 K-group (G=32) scales,
    both formats, f16 and bf16 activations, with and without bias."""
    tune(TFP8_GEMV_MFMA_MIN=1, TFP8_GEMV_PAIR=0, TFP8_GEMV_QUAD=0)
    tune(TFP8_GM_NT=nt)
    tune(TFP8_GM_W=w)
    tune(TFP8_GM_D=d)
    _run(1, 72, 720, None, torch.bfloat16, xdt=torch.bfloat16, seed=nt * 100 + w * 10 + d)   # K tail 16
    _run(5, 200, 1152, 64, torch.float16, xdt=torch.float16, seed=nt + w + d)
    _run(8, 136, 544, 32, torch.float32, fmt="e5m2", xdt=torch.bfloat16, sf="ue8m0", bias=False, seed=d)  # tail 32
    _run(3, 40, 96, None, torch.float16, xdt=torch.float16, sf="ue8m0", seed=w)
    # K a multiple of 256 x W: the transposed weight-load layout (rows past N in the last block)
    _run(6, 72, 256 * w * 2, 128, torch.bfloat16, xdt=torch.bfloat16, seed=w * d)
    _run(4, 40, 256 * w, None, torch.float16, fmt="e5m2", xdt=torch.float16, sf="ue8m0", seed=nt)
    # 9..16 rows (the GEMM entry): bf16 activations, and fp32 ones prepared to f16 with row scales
    _run(16, 136, 256 * w * 2, 64, torch.bfloat16, xdt=torch.bfloat16, seed=nt + 16)
    _run(11, 200, 1152, None, torch.float32, xdt=torch.float32, seed=d + 11)


@pytest.mark.parametrize("wpb", [1, 4, 8])
def test_row_pair_gemv_shapes(wpb, tune):
    """The row-pair GEMV (M = 1..4, K = 2048/4096/8192; at M = 1 with 4 or 8 waves per block and the
    automatic choice): per-channel and K-group (64/128/256, each lane's group scale broadcast
    inside its lane segment) scales in f32 and UE8M0, both formats, f16/bf16 activations, every
    output dtype, with and without bias, M = 3 on the 4-row kernel, N odd (a half pair at the end
    at M = 1; not taken at M > 1) and below one block."""
    tune(TFP8_GEMV_PAIR=wpb, TFP8_GEMV_QUAD=0)
    for i, (M, N, K, G, fmt, sf, xdt, out, bias) in enumerate([
            (2, 14336, 4096, 128, "e4m3fn", "f32", torch.bfloat16, torch.bfloat16, False),
            (3, 1000, 2048, 64, "e5m2", "ue8m0", torch.float16, torch.float32, True),
            (4, 4096, 4096, None, "e4m3fn", "f32", torch.float16, torch.float16, True),
            (4, 998, 8192, 256, "e5m2", "f32", torch.bfloat16, torch.float32, True),
            (2, 514, 2048, 128, "e4m3fn", "ue8m0", torch.float16, torch.float16, True),
            (2, 37, 4096, 128, "e4m3fn", "f32", torch.bfloat16, torch.bfloat16, True)]):   # N odd, M > 1: not taken
        _run(M, N, K, G, out, fmt=fmt, bias=bias, xdt=xdt, sf=sf, seed=wpb * 1000 + i)
    cases = [(14336, 4096, 128, "e4m3fn", "f32", torch.bfloat16, torch.bfloat16, False),
             (4096, 4096, None, "e4m3fn", "f32", torch.float16, torch.float16, False),
             (1001, 2048, 64, "e5m2", "ue8m0", torch.bfloat16, torch.float32, True),
             (999, 8192, 256, "e4m3fn", "f32", torch.float16, torch.float32, True),
             (37, 8192, None, "e5m2", "ue8m0", torch.bfloat16, torch.bfloat16, True),
             (514, 2048, 128, "e4m3fn", "ue8m0", torch.float16, torch.float16, True),
             (3, 4096, 128, "e5m2", "f32", torch.bfloat16, torch.float32, True)]
    for i, (N, K, G, fmt, sf, xdt, out, bias) in enumerate(cases):
        _run(1, N, K, G, out, fmt=fmt, bias=bias, xdt=xdt, sf=sf, seed=wpb * 100 + i)


def test_row_pair_gemv_partial_chunk_shapes(tune):
    """The row-pair GEMV at K other than 2048/4096/8192 (3, 5, 6, 7 chunks of 1 KB up to 4 activation
    rows, 11, 12 up to 2, 14 chunks on the streaming GEMV; the last chunk partial when K % 1024 != 0, its lanes past K reading
    zeros, x staged with zeros past K, K groups past the row reading zero scales): per-channel and
    K-group scales, f32 and UE8M0, both formats, f16/bf16 activations, N odd at M = 1; against the
    oracle, and M = 1 against the streaming GEMV it replaces for these shapes."""
    tune(TFP8_GEMV_QUAD=0)
    for i, (M, N, K, G, fmt, sf, xdt, out, bias) in enumerate([
            (1, 2048, 5632, None, "e4m3fn", "f32", torch.bfloat16, torch.bfloat16, False),   # 5.5 chunks
            (2, 1000, 5632, 128, "e5m2", "ue8m0", torch.float16, torch.float32, True),
            (4, 514, 3072, 64, "e4m3fn", "f32", torch.bfloat16, torch.float16, True),          # 3 chunks, L = 4
            (3, 998, 6144, 256, "e5m2", "f32", torch.bfloat16, torch.float32, True),
            (4, 260, 7040, 128, "e4m3fn", "ue8m0", torch.float16, torch.float16, False),       # 6.875 chunks
            (1, 4097, 11008, None, "e5m2", "ue8m0", torch.bfloat16, torch.bfloat16, True),     # 10.75 chunks, N odd
            (2, 4096, 11008, 256, "e4m3fn", "f32", torch.bfloat16, torch.float32, False),      # 43 groups of 256
            (1, 600, 12288, 256, "e5m2", "f32", torch.float16, torch.float32, True),
            (2, 1030, 14336, None, "e4m3fn", "f32", torch.bfloat16, torch.bfloat16, True),
            (1, 66, 13824, 256, "e4m3fn", "ue8m0", torch.float16, torch.float16, False)]):     # 13.5 chunks
        _run(M, N, K, G, out, fmt=fmt, bias=bias, xdt=xdt, sf=sf, seed=5000 + i)
    for K, G in ((5632, None), (11008, 256)):
        q, s, GG, b = _layer(2050, K, G, "e4m3fn", "f32", True, seed=K)
        x = torch.randn(1, K, generator=torch.Generator().manual_seed(K + 1)).bfloat16().cuda()
        outs = []
        for pair in (1, 0):
            tune(TFP8_GEMV_PAIR=pair)
            outs.append(_ext.w8a16(x, q, None, s, b, torch.float32, GG, "e4m3fn"))
        torch.cuda.synchronize()
        for y in outs:
            _check(y, x, q, s, GG, "e4m3fn", b, torch.float32, "gemv", f"pair vs streaming K={K}")
        assert torch.allclose(outs[0], outs[1], rtol=1e-5, atol=1e-5), K


def test_row_pair_gemv_chunk_tails(tune):
    """K across the row-pair GEMV's chunk boundaries: a last chunk of one lane (K = 1024 c + 16),
    of 3 and 15 lanes, K groups whose last one ends inside the tail, 1 to 4 activation rows, N odd
    at M = 1 and not a multiple of the block; chunk counts the kernel does not take (9, or 11 at
    M = 3) go to the other kernels.  Every result against the oracle."""
    tune(TFP8_GEMV_QUAD=0)
    for i, (M, N, K, G, fmt, sf) in enumerate([
            (1, 37, 2064, None, "e4m3fn", "f32"),      # 3 chunks, tail of 1 lane
            (2, 130, 3120, None, "e5m2", "ue8m0"),     # 4 chunks (not exact): other kernels
            (4, 66, 4144, None, "e4m3fn", "f32"),      # 5 chunks, tail 3 lanes
            (3, 262, 5376, 128, "e5m2", "f32"),        # 6 chunks, 42 groups of 128
            (1, 515, 6400, 256, "e4m3fn", "ue8m0"),    # 7 chunks, 25 groups of 256 (last one in the tail)
            (2, 98, 7408, None, "e4m3fn", "f32"),      # 8 chunks (not exact): other kernels
            (1, 45, 8432, None, "e5m2", "f32"),        # 9 chunks: other kernels
            (2, 1026, 10480, None, "e4m3fn", "ue8m0"), # 11 chunks, tail 15 lanes
            (3, 64, 10496, 256, "e4m3fn", "f32"),      # 11 chunks at M = 3: other kernels
            (1, 257, 12032, 256, "e5m2", "ue8m0")]):   # 12 chunks, 47 groups of 256
        _run(M, N, K, G, torch.float32, fmt=fmt, xdt=torch.bfloat16 if i % 2 else torch.float16, sf=sf,
             bias=bool(i % 3), seed=6000 + i)


def test_quad_gemv_shapes(tune):
    """The 4x4x4-MFMA GEMV, forced for every scale layout it can take and from M = 1: one scale per
    row and K-groups of 64/128/256 (group scales fetched across lanes), f32 and UE8M0 scales, both
    formats, f16/bf16 activations, every output dtype, with and without bias; one or two sets of
    four activation rows (rows past M read zeros), N not a multiple of 4 and below one block, K =
    2048 and 4096."""
    tune(TFP8_GEMV_QUAD=2, TFP8_GEMV_QUAD_MIN_M=1)
    for i, (M, N, K, G, fmt, sf, xdt, out, bias) in enumerate([
            (1, 4096, 4096, None, "e4m3fn", "f32", torch.float16, torch.float16, False),
            (2, 14336, 4096, 128, "e4m3fn", "f32", torch.bfloat16, torch.bfloat16, False),
            (3, 1001, 2048, 64, "e5m2", "ue8m0", torch.float16, torch.float32, True),
            (4, 4096, 4096, None, "e4m3fn", "f32", torch.float16, torch.float16, True),
            (5, 998, 4096, 256, "e5m2", "f32", torch.bfloat16, torch.float32, True),
            (6, 514, 2048, 128, "e4m3fn", "ue8m0", torch.float16, torch.float16, True),
            (7, 4102, 4096, None, "e5m2", "ue8m0", torch.bfloat16, torch.bfloat16, True),
            (8, 14336, 4096, 128, "e4m3fn", "f32", torch.bfloat16, torch.bfloat16, False),
            (8, 13, 2048, None, "e4m3fn", "f32", torch.float16, torch.float32, True),
            (4, 7, 4096, 64, "e5m2", "f32", torch.bfloat16, torch.float16, False)]):
        _run(M, N, K, G, out, fmt=fmt, bias=bias, xdt=xdt, sf=sf, seed=3000 + i)


def test_quad_gemv_default_routing_matches_other_kernels(tune):
    """With the default knobs the 4x4x4-MFMA GEMV takes one-scale-per-row shapes from M = 3; the same
    products through the row-pair GEMV (M = 3, 4) and the matrix-core decode kernel (M = 5..8) agree
    with it to a few f32 ulps (only the summation order differs), and all are within the oracle
    tolerance."""
    q, s, G, b = _layer(4100, 4096, None, "e4m3fn", "f32", True, seed=31)
    for M in (3, 4, 6, 8):
        x = torch.randn(M, 4096, generator=torch.Generator().manual_seed(32 + M)).half().cuda()
        outs = []
        for quad in (1, 0):
            tune(TFP8_GEMV_QUAD=quad)
            outs.append(_ext.w8a16(x, q, None, s, b, torch.float32, G, "e4m3fn"))
        torch.cuda.synchronize()
        for y in outs:
            _check(y, x, q, s, G, "e4m3fn", b, torch.float32, "gemv", f"quad routing M={M}")
        assert torch.allclose(outs[0], outs[1], rtol=1e-5, atol=1e-5), M


def test_row_pair_gemv_matches_streaming_gemv(tune):
    """The same M = 1 products through the row-pair GEMV and the streaming GEMV (which the pair
    kernel replaced for these shapes): both within the oracle tolerance and within a few f32
    ulps of each other (only the summation order differs); a 2-byte-offset output, which the
    pair store cannot take, falls back to the streaming kernel."""
    q, s, G, b = _layer(4104, 4096, 128, "e4m3fn", "f32", False, seed=5)
    x = torch.randn(1, 4096, generator=torch.Generator().manual_seed(6)).bfloat16().cuda()
    outs = []
    for pair in (0, 1):
        tune(TFP8_GEMV_PAIR=pair, TFP8_GEMV_QUAD=0)
        outs.append(_ext.w8a16(x, q, None, s, b, torch.float32, G, "e4m3fn"))
    torch.cuda.synchronize()
    for y in outs:
        _check(y, x, q, s, G, "e4m3fn", b, torch.float32, "gemv", "pair vs streaming")
    assert torch.allclose(outs[0], outs[1], rtol=1e-5, atol=1e-5)
    lib = _ext.require()
    ybuf = torch.zeros(4104 + 1, dtype=torch.bfloat16, device="cuda")
    y = ybuf[1:]
    assert y.data_ptr() % 4 == 2
    rc = lib.tfp8_gemv(x.data_ptr(), _ext.DTYPE_ID[x.dtype], 1, 4096, q.data_ptr(), 4104, s.data_ptr(), 0, G, 0,
                       b.data_ptr(), y.data_ptr(), _ext.DTYPE_ID[torch.bfloat16], torch._C._cuda_getCurrentRawStream(0))
    assert rc == 0
    _check(y.view(1, -1), x, q, s, G, "e4m3fn", b, torch.bfloat16, "gemv", "misaligned y")


@pytest.mark.parametrize("M,N,K,G,sf", [(16, 8192, 8192, None, "ue8m0"), (24, 1000, 2048, 128, "f32"),
                                        (32, 520, 4096, 32, "ue8m0"), (13, 300, 832, 64, "f32")])
def test_stream_gemm_transposed_loads_identical(M, N, K, G, sf, tune):
    """The weight-streaming GEMM's transposed weight loads (256-code chunks as 4 rows x 256 bytes,
    regrouped through LDS) against its direct operand-layout loads: bit-identical outputs (same
    operands, same order), including the K tail, rows past N and split-K."""
    print(f"[linear] stream transposed vs direct M={M} N={N} K={K} G={G} {sf}", flush=True)
    tune(TFP8_GEMV_MFMA_MAX_M=8)   # M <= 16 would take the matrix-core decode kernel
    q, s, GG, b = _layer(N, K, G, "e4m3fn", sf, True, M + N)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).half().cuda()
    outs = []
    for tl in (0, 1):
        tune(TFP8_GS_TL=tl)
        outs.append(_ext.w8a16(x, q, None, s, b, torch.float16, GG, "e4m3fn"))
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    _check(outs[1], x, q, s, GG, "e4m3fn", b, torch.float16, "gemm", "stream transposed loads")


@pytest.mark.parametrize("M,N,K,G,sf", [(4, 14336, 4096, 128, "f32"), (8, 4096, 4096, None, "ue8m0"),
                                        (6, 1000, 2048, 32, "ue8m0"), (8, 520, 4096, 64, "f32"),
                                        (16, 8192, 8192, None, "ue8m0"), (12, 14336, 4096, 128, "f32"),
                                        (7, 299, 1024, None, "f32"), (16, 2048, 5632, None, "ue8m0")])
def test_decode_mfma_transposed_loads_identical(M, N, K, G, sf, tune):
    """The decode kernel's transposed weight loads (4 rows x 256 bytes per load, regrouped through
    LDS) feed the matrix cores the same operands in the same order as the direct layout (16 rows x
    64 bytes per load): the outputs must be bit-identical.  Below N = 4096 a block owns 8 weight
    rows (half of its MFMA tile reads zeros), N = 299 ends in a partial block."""
    print(f"[linear] decode transposed vs direct M={M} N={N} K={K} G={G} {sf}", flush=True)
    tune(TFP8_GEMV_PAIR=0, TFP8_GEMV_QUAD=0)
    q, s, GG, b = _layer(N, K, G, "e4m3fn", sf, True, M + N)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).bfloat16().cuda()
    outs = []
    for tl in (0, 1):
        tune(TFP8_GM_TL=tl)
        outs.append(_ext.w8a16(x, q, None, s, b, torch.bfloat16, GG, "e4m3fn"))
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    _check(outs[1], x, q, s, GG, "e4m3fn", b, torch.bfloat16, "gemv" if M <= 8 else "gemm",
           "decode transposed loads")


def test_weight_matrix_past_2gib():
    """A weight matrix of more than 2^31 bytes (K=16384, N=132096: 2.16 GB of codes): buffer offsets
    inside every kernel are 32-bit, so the GEMV splits the launch by rows and the GEMMs address the
    weights per block.  M=1 (GEMV), M=4 and M=16 (matrix-core decode), M=16 with the decode kernel
    held to 8 rows (the weight-streaming kernel declines, the LDS-tiled kernel runs) and M=128
    (direct-load GEMM); output columns at both ends of the matrix against the float64 oracle on
    those rows."""
    K, N = 16384, 132096
    assert N * K > 2 ** 31
    print(f"[linear] N={N} K={K}: {N * K / 2 ** 30:.2f} GiB of codes", flush=True)
    g = torch.Generator(device="cuda").manual_seed(77)
    w = torch.randn(N, K, generator=g, device="cuda") * 0.02
    q, s, G = quantize_weight(w, "e4m3fn", None, True, "f32")
    del w
    torch.cuda.empty_cache()
    cols = np.r_[0:48, N - 80:N]
    qs, ss = q[cols].cpu().numpy(), s[cols].cpu().numpy()
    for M, mfma_max in ((1, 16), (4, 16), (16, 16), (16, 8), (128, 16)):
        x = (torch.randn(M, K, generator=g, device="cuda") * 0.5).bfloat16()
        with _ext.tuning(TFP8_GEMV_MFMA_MAX_M=mfma_max):
            y = _ext.w8a16(x, q, None, s, None, torch.float32, G, "e4m3fn")
        ref = O.linear_ref64(_x_eff(x, "gemv" if M <= _ext.GEMV_MAXM else "gemm"), qs, ss, G, "e4m3fn", None)
        got = y[:, cols].double().cpu().numpy()
        d = np.abs(got - ref)
        assert (d <= O.tolerance(ref, "float32")).all(), (M, float(d.max()))
    del q, s
    torch.cuda.empty_cache()


def test_concurrent_streams_match_serial():
    """The library keeps no device state between calls: the GEMV, the matrix-core decode kernel
    and split-K GEMMs (each call with its own workspace from torch's stream-ordered allocator)
    launched on two streams at once, in opposite orders and several times over, give the same bits
    as the same calls run one after another on one stream (tfp8/_ext.py:230-253 launches on the
    caller's current stream)."""
    g = torch.Generator().manual_seed(5)
    cases = []
    for M, N, K, G, sf in [(1, 4096, 4096, 128, "f32"), (8, 2048, 4096, None, "ue8m0"),
                           (256, 2048, 4096, None, "ue8m0"), (64, 1024, 8192, None, "f32"),
                           (24, 1536, 4096, 128, "f32")]:
        q, s, GG, b = _layer(N, K, G, "e4m3fn", sf, seed=M + N)
        x = torch.randn(M, K, generator=g).bfloat16().cuda()
        cases.append((x, q, s, GG, b))
    serial = [_ext.w8a16(x, q, None, s, b, torch.float32, GG, "e4m3fn") for x, q, s, GG, b in cases]
    torch.cuda.synchronize()
    streams = (torch.cuda.Stream(), torch.cuda.Stream())   # default priority
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    got = []
    for rep in range(3):
        for si, st in enumerate(streams):
            order = list(range(len(cases))) if si == 0 else list(range(len(cases)))[::-1]
            with torch.cuda.stream(st):
                for i in order:
                    x, q, s, GG, b = cases[i]
                    got.append((i, _ext.w8a16(x, q, None, s, b, torch.float32, GG, "e4m3fn")))
    torch.cuda.synchronize()
    for i, y in got:
        assert torch.equal(y, serial[i]), f"case {i}: result differs when run on two streams"


def test_misaligned_contiguous_input():
    """A contiguous input whose data does not start on a 16-byte boundary (one row sliced one
    element into its storage, and a flat buffer viewed from element 3): FP8Linear and w8a16 run it
    through an aligned copy and give the same bits as the aligned input."""
    torch.manual_seed(11)
    lin = nn.Linear(512, 192, device="cuda")
    f = FP8Linear.from_linear(lin)
    f.out_dtype = torch.float32
    for M in (1, 4, 40):
        base = torch.randn(M, 513, device="cuda").bfloat16()
        xm = base[:, 1:] if M == 1 else torch.randn(M * 512 + 3, device="cuda").bfloat16()[3:].view(M, 512)
        assert xm.is_contiguous() and xm.data_ptr() % 16
        xa = xm.clone()
        for _ in range(4):                      # past the NaN-checked calls: the decode fast path too
            got, want = f(xm), f(xa)
            assert torch.equal(got, want), f"M={M}"
        y = _ext.w8a16(xm, f.qweight, None, f.weight_scale, f.bias_f32, torch.float32, f.group_size, f.fmt)
        assert torch.equal(y, want)
