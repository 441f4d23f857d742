"""GPU parity of the elementwise kernels against the oracle: decode (all 256 codes, every output
dtype, every byte position), encode (RNE ties, saturation, NaN, every input dtype), weight
quantisation, activation prep and dequantisation. Bit-exact throughout (NaN compared as NaN)."""
import numpy as np
import pytest
import torch

import binade_edges
from oracle import fp8_oracle as O
from tfp8 import _ext
from tfp8.formats import E4M3FN, E5M2, decode, encode, lut
from tfp8.quantize import activation_to_fp16, dequantize_weight, quantize_weight

pytestmark = pytest.mark.gpu
FMTS = ("e4m3fn", "e5m2")
TDT = {"e4m3fn": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


def _same(a, b):
    a = torch.as_tensor(a).double().cpu()
    b = torch.as_tensor(b).double().cpu()
    both_nan = torch.isnan(a) & torch.isnan(b)
    eq = (a == b) & (torch.signbit(a) == torch.signbit(b))
    return bool((both_nan | eq).all())


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("odt", [torch.float32, torch.float16, torch.bfloat16])
def test_decode_all_codes_every_dtype(fmt, odt):
    print(f"[decode] fmt={fmt} out={odt}", flush=True)
    codes = torch.arange(256, dtype=torch.uint8)
    ref = torch.from_numpy(O.decode(np.arange(256), fmt))
    got = _ext.decode(codes.cuda(), fmt, odt).cpu()
    assert _same(got, ref.to(odt))
    # torch's own float8 cast on the device agrees (NaN-aware)
    assert _same(got, codes.cuda().view(TDT[fmt]).to(odt).cpu())
    # non-NaN codes are bitwise identical to the rounding of the exact value into odt
    fin = ~torch.isnan(ref)
    assert torch.equal(got[fin].view(torch.int16 if odt != torch.float32 else torch.int32),
                       ref.to(odt)[fin].view(torch.int16 if odt != torch.float32 else torch.int32))


@pytest.mark.parametrize("fmt", FMTS)
def test_decode_every_byte_position_and_lut(fmt):
    print(f"[decode offsets] fmt={fmt}", flush=True)
    base = torch.arange(256, dtype=torch.uint8).repeat(9).cuda()
    ref = torch.from_numpy(O.decode(np.arange(256), fmt)).repeat(9)
    for off in range(4):
        n = 256 * 8 + 1 + off
        got = decode(base[off:off + n], fmt).cpu()
        assert _same(got, ref[off:off + n]), off
    assert torch.equal(lut(fmt, "cuda").cpu().view(torch.int16)[~torch.isnan(ref[:256])],
                       torch.from_numpy(O.lut_f16_bits(fmt).view(np.int16))[~torch.isnan(ref[:256])])


def _encode_probe(fmt):
    torch.manual_seed(0)
    mx = O.FORMATS[fmt][4]
    codes, vals = O._finite_table(fmt)
    mids = (vals[:-1] + vals[1:]) / 2
    eps = np.abs(mids) * 2.0 ** -20
    special = np.array([0.0, -0.0, 1e9, -1e9, np.inf, -np.inf, np.nan, mx, -mx, mx * 1.03, 2.0 ** -30,
                        1e-45, -1e-45])
    probe = np.concatenate([mids, mids + eps, mids - eps, vals, special])
    probe = np.concatenate([probe, -probe])
    rnd = torch.cat([torch.randn(20000) * mx / 8, torch.randn(2000) * 2.0 ** -10]).double().numpy()
    return np.concatenate([probe, rnd])


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("xdt", [torch.float32, torch.float16, torch.bfloat16])
def test_encode_matches_oracle(fmt, xdt):
    print(f"[encode] fmt={fmt} in={xdt}", flush=True)
    x = torch.from_numpy(_encode_probe(fmt)).to(xdt)
    got = encode(x.cuda(), fmt).cpu()
    want = torch.from_numpy(O.encode(x.double().numpy(), fmt))
    assert torch.equal(got, want)
    inr = x.double().abs() < O.FORMATS[fmt][4]
    assert torch.equal(got[inr], x[inr].float().to(TDT[fmt]).view(torch.uint8))


@pytest.mark.parametrize("fmt", FMTS)
def test_encode_round_trips_all_finite_codes(fmt):
    print(f"[encode roundtrip] fmt={fmt}", flush=True)
    codes = torch.arange(256, dtype=torch.uint8).cuda()
    v = _ext.decode(codes, fmt, torch.float32)
    fin = torch.isfinite(v)
    assert torch.equal(encode(v[fin], fmt), codes[fin])


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("G", [None, 32, 128])
@pytest.mark.parametrize("sf,pow2", [("f32", True), ("f32", False), ("ue8m0", True)])
@pytest.mark.parametrize("wdt", [torch.float32, torch.bfloat16])
def test_quantize_weight_matches_oracle(fmt, G, sf, pow2, wdt):
    print(f"[quantize] fmt={fmt} G={G} sf={sf} pow2={pow2} w={wdt}", flush=True)
    torch.manual_seed(11)
    w = (torch.randn(96, 512) * 0.02).to(wdt)
    w[2] = 0
    w[5, 100] = 30.0
    q, s, GG = quantize_weight(w.cuda(), fmt, G, pow2, sf)
    oq, os_, _ = O.quantize_weight(w.float().numpy(), fmt, G, pow2, sf)
    assert torch.equal(q.cpu(), torch.from_numpy(oq))
    assert torch.equal(s.cpu(), torch.from_numpy(os_))


def test_quantize_weight_nan_group():
    print("[quantize nan]", flush=True)
    w = torch.randn(4, 64) * 0.1
    w[1, 7] = float("nan")
    q, s, _ = quantize_weight(w.cuda(), "e4m3fn", 32, True)
    oq, os_, _ = O.quantize_weight(w.numpy(), "e4m3fn", 32, True)
    assert _same(s.cpu(), torch.from_numpy(os_))
    ok = ~torch.isnan(torch.from_numpy(os_)).repeat_interleave(32, dim=1)
    assert torch.equal(q.cpu()[ok], torch.from_numpy(oq)[ok])


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("sf", ["f32", "ue8m0"])
def test_quantize_weight_binade_edges(fmt, sf):
    """Group scales a few ULP above a power of two: the kernel's power-of-two ceiling follows the
    reference's fp32 log2 rounding (tfp8/quantize.py:11-12), codes and scales bit-exact against
    the oracle, with hundreds of groups inside the rounding window."""
    print(f"[quantize binade edges] fmt={fmt} sf={sf}", flush=True)
    w = binade_edges.weight_rows(fmt)
    assert binade_edges.window_hits(w, fmt, 32) > 500
    q, s, G = quantize_weight(torch.from_numpy(w).cuda(), fmt, 32, True, sf)
    oq, os_, _ = O.quantize_weight(w, fmt, 32, True, sf)
    assert torch.equal(s.cpu(), torch.from_numpy(os_))
    assert torch.equal(q.cpu(), torch.from_numpy(oq))


def test_prepare_activations_binade_edges():
    """fp32 rows whose amax is 2^k (1 + j 2^-23): the row exponent follows the reference's fp32
    log2 rounding (tfp8/quantize.py:58-60), bit-exact against the oracle."""
    print("[prep binade edges]", flush=True)
    x = binade_edges.activation_rows()
    x16, xs = _ext.prepare_activations(torch.from_numpy(x).cuda())
    ox16, oxs = O.activation_to_fp16(x)
    assert torch.equal(xs.cpu(), torch.from_numpy(oxs))
    assert torch.equal(x16.cpu().view(torch.int16), torch.from_numpy(ox16.view(np.int16)))


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float32, torch.float16])
def test_prepare_activations_block_wide_amax(xdt):
    print(f"[prep] x={xdt}", flush=True)
    torch.manual_seed(12)
    x = torch.randn(6, 4096).to(xdt)
    x[0, 1] = 3e4
    x[1, 4095] = -5e4
    if xdt != torch.float16:
        x[2, 300] = 1e5
    x[3] = 0
    x[4] *= 1e-30 if xdt != torch.float16 else 1e-3
    x16, xs = _ext.prepare_activations(x.cuda())
    ox16, oxs = O.activation_to_fp16(x.float().numpy())
    assert torch.isfinite(x16).all()
    assert torch.equal(xs.cpu(), torch.from_numpy(oxs))
    assert torch.equal(x16.cpu().view(torch.int16), torch.from_numpy(ox16.view(np.int16)))
    if xdt == torch.bfloat16:
        a16, axs = activation_to_fp16(x.cuda())
        assert torch.equal(a16, x16) and torch.equal(axs, xs)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("sf,pow2", [("f32", False), ("ue8m0", True)])
def test_dequant_matches_oracle(fmt, sf, pow2):
    print(f"[dequant] fmt={fmt} sf={sf}", flush=True)
    torch.manual_seed(13)
    w = torch.randn(64, 256) * 0.03
    q, s, G = quantize_weight(w.cuda(), fmt, 32, pow2, sf)
    want = torch.from_numpy(O.dequantize_weight(q.cpu().numpy(), s.cpu().numpy(), fmt, G))
    assert torch.equal(dequantize_weight(q, s, fmt, G).cpu(), want)
    out16 = torch.empty(64, 256, dtype=torch.float16, device="cuda")
    _ext.dequant_into(out16, q, None, s, G, fmt)
    assert torch.equal(out16.cpu(), want.half())


def test_read_probe_reads_every_word():
    """The measurement harness's read-only probe (tfp8_read_probe) reads every 16-byte piece of the
    buffer: the XOR of its per-block results is the XOR of all 32-bit words, including buffers that
    are no multiple of the grid's stride and grids with more threads than pieces."""
    lib = _ext.library()
    g = torch.Generator().manual_seed(9)
    for nbytes, blocks in ((1 << 20, 64), (16 * 1007, 256), (48, 16)):
        print(f"[codec] read probe {nbytes} bytes, {blocks} blocks", flush=True)
        buf = torch.randint(-2 ** 31, 2 ** 31 - 1, (nbytes // 4,), dtype=torch.int32, generator=g).cuda()
        out = torch.full((blocks,), 7, dtype=torch.int32, device="cuda")
        rc = lib.tfp8_read_probe(buf.data_ptr(), nbytes, out.data_ptr(), blocks, torch.cuda.current_stream().cuda_stream)
        assert rc == 0, _ext.last_error()
        want = np.bitwise_xor.reduce(buf.cpu().numpy().view(np.uint32))
        got = np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32))
        assert got == want, (nbytes, blocks)
    assert lib.tfp8_read_probe(buf.data_ptr(), 20, out.data_ptr(), 1, None) == -1     # not a multiple of 16
