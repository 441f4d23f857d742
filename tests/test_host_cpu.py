"""CPU-side tests: the tfp8 package's CPU paths against the oracle, the module/planner API
(reference tests/test_tfp8.py:29-72, 278-319), and the C-ABI library's exports and host-side
argument validation (no kernel is launched here)."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch
import torch.nn as nn

import binade_edges
import tfp8
from oracle import fp8_oracle as O
from tfp8 import _ext
from tfp8.formats import E4M3FN, E5M2, decode, encode, lut
from tfp8.linear import FP8Linear
from tfp8.quantize import activation_to_fp16, dequantize_weight, quantize_weight

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tfp8_hip.h")
FMTS = (E4M3FN, E5M2)


def _same(a, b):
    a, b = a.float(), b.float()
    both_nan = torch.isnan(a) & torch.isnan(b)
    eq = (a == b) & (torch.signbit(a) == torch.signbit(b))
    return bool((both_nan | eq).all())


# ------------------------------------------------------------------ formats (CPU paths)
@pytest.mark.parametrize("f", FMTS, ids=lambda f: f.name)
def test_cpu_decode_and_lut_match_oracle(f):
    codes = torch.arange(256, dtype=torch.uint8)
    assert _same(decode(codes, f), torch.from_numpy(O.decode(np.arange(256), f.name)))
    assert _same(lut(f).float(), codes.view(f.torch_dtype).float())


@pytest.mark.parametrize("f", FMTS, ids=lambda f: f.name)
def test_cpu_encode_matches_oracle_and_torch(f):
    torch.manual_seed(0)
    x = torch.cat([torch.randn(20000) * f.max_finite / 8, torch.randn(2000) * 2.0 ** -10,
                   torch.tensor([1e9, -1e9, float("inf"), -float("inf"), float("nan"), 0.0, -0.0])])
    got = encode(x, f)
    assert torch.equal(got, torch.from_numpy(O.encode(x.numpy(), f.name)))
    inr = x.abs() < f.max_finite
    assert torch.equal(got[inr], x[inr].to(f.torch_dtype).view(torch.uint8))
    for dt in (torch.float16, torch.bfloat16, torch.float64):
        xd = x.to(dt)
        assert torch.equal(encode(xd, f), torch.from_numpy(O.encode(xd.double().numpy(), f.name)))


@pytest.mark.parametrize("fmt", ["e4m3fn", "e5m2"])
@pytest.mark.parametrize("G", [None, 32, 128])
@pytest.mark.parametrize("sf", ["f32", "ue8m0"])
def test_cpu_quantize_matches_oracle(fmt, G, sf):
    torch.manual_seed(1)
    w = torch.randn(40, 256) * 0.02
    w[1] = 0
    q, s, GG = quantize_weight(w, fmt, G, True, sf)
    oq, os_, _ = O.quantize_weight(w.numpy(), fmt, G, True, sf)
    assert torch.equal(q, torch.from_numpy(oq)) and torch.equal(s, torch.from_numpy(os_))
    d = dequantize_weight(q, s, fmt, GG)
    assert torch.equal(d, torch.from_numpy(O.dequantize_weight(oq, os_, fmt, GG)))


def test_cpu_quantize_nonpow2_matches_oracle():
    torch.manual_seed(2)
    w = torch.randn(24, 128) * 0.05
    q, s, G = quantize_weight(w, "e4m3fn", 32, False)
    oq, os_, _ = O.quantize_weight(w.numpy(), "e4m3fn", 32, False)
    assert torch.equal(q, torch.from_numpy(oq)) and torch.equal(s, torch.from_numpy(os_))


@pytest.mark.parametrize("fmt", ["e4m3fn", "e5m2"])
@pytest.mark.parametrize("sf", ["f32", "ue8m0"])
def test_cpu_quantize_binade_edges_match_oracle(fmt, sf):
    """Scales a few ULP above a power of two round as the reference's fp32 log2 does
    (tfp8/quantize.py:11-12) on the CPU path too."""
    w = binade_edges.weight_rows(fmt)
    assert binade_edges.window_hits(w, fmt, 32) > 500
    q, s, G = quantize_weight(torch.from_numpy(w), fmt, 32, True, sf)
    oq, os_, _ = O.quantize_weight(w, fmt, 32, True, sf)
    assert torch.equal(s, torch.from_numpy(os_)) and torch.equal(q, torch.from_numpy(oq))


def test_cpu_activation_prep_binade_edges_match_oracle():
    x = binade_edges.activation_rows()
    x16, xs = activation_to_fp16(torch.from_numpy(x))
    ox16, oxs = O.activation_to_fp16(x)
    assert torch.equal(xs, torch.from_numpy(oxs))
    assert torch.equal(x16.view(torch.int16), torch.from_numpy(ox16.view(np.int16)))


def test_activation_scaling_is_exact_power_of_two():
    x = (torch.randn(5, 256) * 1e3).bfloat16()
    x16, xs = activation_to_fp16(x)
    assert torch.all(torch.log2(xs) == torch.round(torch.log2(xs)))
    assert torch.equal((x16.float() * xs[:, None]), x.float())
    ox16, oxs = O.activation_to_fp16(x.float().numpy())
    assert torch.equal(xs, torch.from_numpy(oxs)) and torch.equal(x16, torch.from_numpy(ox16))


# ------------------------------------------------------------------ module / planner
def test_cpu_reference_path():
    lin = nn.Linear(256, 64)
    f = FP8Linear.from_linear(lin, group_size=128)
    x = torch.randn(3, 256)
    y = f(x)
    ref = x @ f.dequantized_weight().t() + lin.bias
    assert torch.allclose(y.float(), ref, atol=1e-2, rtol=1e-2)
    assert f.stats["torch"] == 1


def test_cpu_path_matches_oracle_ue8m0():
    torch.manual_seed(9)
    lin = nn.Linear(256, 96)
    f = FP8Linear.from_linear(lin, fmt="e5m2", group_size=32, scale_format="ue8m0")
    assert f.weight_scale.dtype == torch.uint8
    f.out_dtype = torch.float32
    x = torch.randn(4, 256)
    ref = O.linear_ref64(x.numpy(), f.qweight.numpy(), f.weight_scale.numpy(), 32, "e5m2", f.bias_f32.numpy())
    d = np.abs(f(x).double().numpy() - ref)
    assert (d <= O.tolerance(ref, "float32")).all()


def test_planner_policy_and_tied_weights():
    class Block(nn.Module):
        def __init__(s):
            super().__init__()
            s.q_proj, s.o_proj = nn.Linear(1024, 1024), nn.Linear(1024, 1024)
            s.gate_proj = nn.Linear(1024, 2048)
            s.input_layernorm = nn.LayerNorm(1024)
            s.lora_A = nn.Linear(1024, 8)
            s.router = nn.Linear(1024, 1024)

    class LM(nn.Module):
        def __init__(s):
            super().__init__()
            s.embed = nn.Embedding(100, 1024)
            s.layers = nn.ModuleList([Block()])
            s.lm_head = nn.Linear(1024, 100, bias=False)
            s.lm_head.weight = s.embed.weight

    m = tfp8.prepare_model(LM(), "llm", tfp8.FP8Config(profile="llm_safe"))
    owners = {d.name: d.owner for d in m._tfp8_plan}
    reasons = {d.name: d.reason for d in m._tfp8_plan}
    text = tfp8.report(m, file=open(os.devnull, "w"))
    assert owners["layers.0.q_proj"] == "tfp8" and owners["layers.0.gate_proj"] == "tfp8"
    assert owners["layers.0.lora_A"] != "tfp8" and owners["layers.0.router"] != "tfp8"
    assert owners["lm_head"] != "tfp8"
    assert m.lm_head.weight is m.embed.weight
    assert isinstance(m.layers[0].q_proj, FP8Linear)
    again = tfp8.prepare_model(m, "llm", tfp8.FP8Config())
    assert {d.name: d.owner for d in again._tfp8_plan}["layers.0.q_proj"] == "tfp8"
    assert isinstance(again.layers[0].q_proj, FP8Linear)
    assert reasons["lm_head"] == "weight shared with another module (tied)"
    assert reasons["layers.0.lora_A"] == "'lora_A' is precision-sensitive"
    assert "-- 3/6 Linear modules on tfp8" in text
    wb = tfp8.weight_bytes(m)
    assert wb["uint8"] == 1024 * 1024 * 2 + 2048 * 1024


def test_planner_ue8m0_and_groups():
    class M(nn.Module):
        def __init__(s):
            super().__init__()
            s.up_proj = nn.Linear(1024, 2048)
            s.small_mlp = nn.Linear(1024, 512)

    m = tfp8.prepare_model(M(), "llm", tfp8.FP8Config(weight_group=128, scale_format="ue8m0", fmt="e5m2"))
    assert isinstance(m.up_proj, FP8Linear) and m.up_proj.weight_scale.dtype == torch.uint8
    assert m.up_proj.weight_scale.shape == (2048, 8) and m.up_proj.fmt == "e5m2"
    assert not isinstance(m.small_mlp, FP8Linear)


def test_config_validation():
    with pytest.raises(ValueError):
        tfp8.FP8Config(profile="fast")
    with pytest.raises(NotImplementedError):
        tfp8.FP8Config(activation="fp8")
    with pytest.raises(NotImplementedError):
        tfp8.FP8Config(kv_cache="fp8")
    with pytest.raises(ValueError):
        tfp8.FP8Config(large_m_backend="cublas")
    with pytest.raises(ValueError):
        tfp8.FP8Config(scale_format="e4m3")
    assert tfp8.FP8Config(profile="image_safe").min_features == 256


def test_checkpoint_compat_mode_keeps_codes():
    q = torch.randint(0, 256, (64, 128), dtype=torch.uint8)
    q[E4M3FN.is_nan(q.int())] = 0
    s = torch.rand(64) + 0.5
    f = FP8Linear.from_fp8_checkpoint(q.view(torch.float8_e4m3fn), s, fmt="e4m3fn")
    assert torch.equal(f.qweight, q) and torch.equal(f.weight_scale[:, 0], s)
    with pytest.raises(ValueError):
        FP8Linear.from_fp8_checkpoint(q.view(torch.float8_e4m3fn), s, fmt="e5m2")
    # per-tensor (scalar) and per-K-group UE8M0 scales
    ft = FP8Linear.from_fp8_checkpoint(q, torch.tensor(0.25), fmt="e4m3fn")
    assert ft.weight_scale.shape == (64, 1) and bool((ft.weight_scale == 0.25).all())
    b = torch.randint(100, 140, (64, 4), dtype=torch.uint8)
    fg = FP8Linear.from_fp8_checkpoint(q, b, fmt="e4m3fn")
    assert fg.group_size == 32 and fg.weight_scale.dtype == torch.uint8 and torch.equal(fg.weight_scale, b)
    x = torch.randn(2, 128)
    ref = O.linear_ref64(x.numpy(), q.numpy(), b.numpy(), 32, "e4m3fn")
    assert fg.out_dtype == torch.bfloat16                    # reference default out dtype
    assert bool((np.abs(fg(x).double().numpy() - ref) <= O.tolerance(ref, "bfloat16")).all())


def test_unsupported_shapes_take_torch_path():
    f = FP8Linear(40, 16, group_size=8)     # K % 16 != 0: no kernel takes it
    assert not f._kernels_ok
    assert FP8Linear(256, 16, group_size=16)._kernels_ok is False   # G=16: GEMM needs G % 32
    assert FP8Linear(528, 16)._kernels_ok                            # K % 16 == 0, per-channel


# ------------------------------------------------------------------ C ABI
def _header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^[A-Za-z_][\w\s\*]*?\b(tfp8_\w+)\s*\(", text, re.M)))


def test_library_exports_every_header_symbol():
    names = _header_functions()
    assert len(names) == 19, names
    lib = ctypes.CDLL(_ext.lib_path())
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(_ext._SIGS) == names          # every entry point bound with argtypes
    assert _ext.library().tfp8_abi_version() == _ext.ABI_VERSION


def _header_prototypes():
    """{name: (return type, [parameter types])} from the C declarations in the header."""
    text = re.sub(r"//[^\n]*", "", open(HEADER).read())
    protos = {}
    for m in re.finditer(r"^([A-Za-z_][\w\s\*]*?)\b(tfp8_\w+)\s*\(([^)]*)\)\s*;", text, re.M):
        params = [p.strip() for p in " ".join(m.group(3).split()).split(",")]
        params = [] if params == ["void"] else params
        # a parameter's type is everything but its name
        protos[m.group(2)] = (m.group(1).strip(), [re.sub(r"\s*\b\w+$", "", p).strip() for p in params])
    return protos


def _ctypes_kind(ctype):
    if ctype == "void":
        return None
    if "*" in ctype:
        return ctypes.c_char_p if ctype.replace(" ", "") == "constchar*" else ctypes.c_void_p
    return {"int": ctypes.c_int, "int64_t": ctypes.c_int64, "size_t": ctypes.c_size_t,
            "float": ctypes.c_float}[ctype]


def test_bound_argument_kinds_match_header():
    """Every entry point is bound with exactly the argument kinds (pointer / int / int64 / size_t)
    and return kind its C declaration has, in order, so no call can pass an int where a pointer or
    a 64-bit size is expected (the bug class of the reference's launch-slot test,
    tests/test_tfp8.py:322-360, at this boundary)."""
    protos = _header_prototypes()
    assert sorted(protos) == _header_functions()
    for name, (ret, params) in protos.items():
        res, args = _ext._SIGS[name]
        assert args == [_ctypes_kind(t) for t in params], (name, params)
        assert res == _ctypes_kind(ret), (name, ret)


def test_gemm_prepared_workspace_query_covers_small_m():
    """tfp8_gemm_prepared runs the GEMM kernels at every M, so its workspace query is non-zero
    wherever they split K -- also for M <= 8, where tfp8_linear (GEMV) needs none."""
    lib = _ext.library()
    for M in range(1, 9):
        assert lib.tfp8_linear_workspace_size(0, M, 4096, 4096) == 0
        nb = lib.tfp8_gemm_prepared_workspace_size(0, M, 4096, 4096)
        assert nb >= lib.tfp8_gemm_prepared_workspace_size(0, M, 64, 64)
    assert lib.tfp8_gemm_prepared_workspace_size(0, 1, 8192, 8192) >= 0
    assert lib.tfp8_gemm_prepared_workspace_size(0, 256, 8192, 8192) == lib.tfp8_linear_workspace_size(0, 256, 8192, 8192)
    assert lib.tfp8_gemm_prepared_workspace_size(0, 0, 64, 64) == 0


def test_tuning_knobs_set_get_reset():
    """Knobs change only through the setter (the launch path never reads the environment), unknown
    names are argument errors, reset restores the load-time values, and a knob that forces split-K
    changes the workspace size the library asks for."""
    lib = _ext.library()
    base = _ext.tuning_get("TFP8_GEMM_SPLITK")
    ws0 = lib.tfp8_linear_workspace_size(0, 200, 512, 3072)
    with _ext.tuning(TFP8_GEMM_SPLITK=3, TFP8_GEMM_DIRECT=0):
        assert _ext.tuning_get("TFP8_GEMM_SPLITK") == 3 and _ext.tuning_get("TFP8_GEMM_DIRECT") == 0
        ws3 = lib.tfp8_linear_workspace_size(0, 200, 512, 3072)
    assert _ext.tuning_get("TFP8_GEMM_SPLITK") == base and _ext.tuning_get("TFP8_GEMM_DIRECT") == 1
    assert ws3 != ws0 or ws0 == 0
    os.environ["TFP8_GEMM_SPLITK"] = "5"                  # read at load only: no effect now
    try:
        assert _ext.tuning_get("TFP8_GEMM_SPLITK") == base
    finally:
        os.environ.pop("TFP8_GEMM_SPLITK")
    assert lib.tfp8_tuning_set(b"TFP8_NO_SUCH_KNOB", 1) == -1
    assert "unknown knob" in lib.tfp8_last_error().decode()
    _ext.tuning_set("TFP8_GEMV_CFG", 8)
    _ext.tuning_reset()
    assert _ext.tuning_get("TFP8_GEMV_CFG") == -1


def test_abi_argument_validation_without_gpu():
    lib = _ext.library()
    assert lib.tfp8_decode(None, -1, 0, None, 0, None) == -1
    assert b"bad n/fmt" in lib.tfp8_last_error()
    assert lib.tfp8_decode(None, 0, 0, None, 0, None) == 0          # n == 0 is a no-op
    assert lib.tfp8_encode(None, 9, 4, 0, None, None) == -1
    # K % 16
    rc = lib.tfp8_linear(None, 1, 1, 40, None, 8, None, 0, 40, 0, None, None, 1, None, 0, None)
    assert rc == -3 and b"K % 16" in lib.tfp8_last_error()
    # G neither K nor a multiple of 32 on the GEMM path
    rc = lib.tfp8_linear(None, 1, 64, 256, None, 8, None, 0, 16, 0, None, None, 1, None, 0, None)
    assert rc == -3 and b"G == K or G % 32" in lib.tfp8_last_error()
    # M > 8 with a missing workspace must be refused before launching (needs pointers first)
    assert lib.tfp8_gemv(None, 1, 9, 256, None, 8, None, 0, 256, 0, None, None, 1, None) == -1
    # null pointers with real sizes
    rc = lib.tfp8_linear(None, 1, 4, 256, None, 8, None, 0, 256, 0, None, None, 1, None, 0, None)
    assert rc == -1 and b"null pointer" in lib.tfp8_last_error()
    # misaligned x
    buf = ctypes.create_string_buffer(4096)
    base = (ctypes.addressof(buf) + 255) & ~255
    rc = lib.tfp8_linear(base + 2, 1, 4, 256, base, 8, base, 0, 256, 0, None, base, 1, None, 0, None)
    assert rc == -2
    assert lib.tfp8_quantize_weight(None, 2, 4, 100, 32, 0, 1, 0, None, None, None) == -3
    assert lib.tfp8_linear_workspace_size(2, 4, 128, 256) == 0          # GEMV needs none
    assert lib.tfp8_linear_workspace_size(2, 64, 128, 256) >= 64 * 256 * 2   # fp32 prep buffer


def test_example_ops_library_loads_and_validates_without_gpu():
    """libtfp8_llm.so (the example model's fused ops) exports its ten entry points and
    refuses arguments its kernels do not take before launching anything."""
    from tfp8.examples import llm_ops
    lib = llm_ops.library()
    for n in ("tfp8_llm_add_rmsnorm", "tfp8_llm_rope_cache", "tfp8_llm_attention", "tfp8_llm_silu_mul", "tfp8_llm_head",
              "tfp8_llm_rope_attention", "tfp8_llm_step_in", "tfp8_llm_step_out", "tfp8_llm_rope_prefill",
              "tfp8_llm_attn_prefill"):
        assert hasattr(lib, n), n
    buf = ctypes.create_string_buffer(4096)
    a = (ctypes.addressof(buf) + 255) & ~255
    assert lib.tfp8_llm_add_rmsnorm(a, None, None, a, a, 1, 12, 1e-5, None) == -1        # d % 8
    assert lib.tfp8_llm_add_rmsnorm(a + 2, None, None, a, a, 1, 16, 1e-5, None) == -1    # alignment
    assert lib.tfp8_llm_add_rmsnorm(a, None, None, a, a, 0, 16, 1e-5, None) == 0         # no rows
    assert lib.tfp8_llm_rope_cache(a, a, a, a, a, a, a, a, a, 1, 6, 4, 128, 64, 768, 512, 512, None) == -1   # H % Hkv
    assert lib.tfp8_llm_rope_cache(a, a, a, a, a, a, a, a, a, 1, 8, 4, 128, 64, 768, 512, 512, None) == -1   # ldq < H hd
    assert lib.tfp8_llm_attention(a, a, a, a, a, 2, a, 1, 4, 4, 96, 64, 1.0, None) == -1     # head dim
    assert lib.tfp8_llm_attention(a, a, a, a, a, 1, a, 1, 4, 4, 128, 65, 1.0, None) == -1    # S * 64 < L
    assert lib.tfp8_llm_silu_mul(a, a, a, 2, 16, 8, None) == -1        # row stride below the row
    assert lib.tfp8_llm_silu_mul(a, a, a, 0, 16, 16, None) == 0
    assert lib.tfp8_llm_head(a, a, a, 17, 100, 512, None) == -1          # more than 16 rows
    assert lib.tfp8_llm_head(a, a, a, 1, 100, 520, None) == -1           # K % 512
    assert lib.tfp8_llm_rope_attention(a, a, a, a, a, a, a, a, a, 2, a, 1, 8, 4, 128, 64, 512, 512, 512, 1.0,
                                       None) == -1                     # ldq < H hd
    assert lib.tfp8_llm_step_in(a, a, a, a, a, a, a, 1, 12, 64, 100, None) == -1      # d % 8
    assert lib.tfp8_llm_step_out(a, 1, 100, 99, a, a, None) == -1               # row stride below the row
    assert lib.tfp8_llm_rope_prefill(a, a, a, a, a, a, a, a, 60, 1, 8, 8, 4, 128, 64, 1024, 512, 512,
                                     None) == -1                       # start + T > L
    assert lib.tfp8_llm_rope_prefill(a, a, a, a, a, a, a, a, 0, 1, 8, 8, 4, 128, 64, 512, 512, 512,
                                     None) == -1                       # ldq < H hd
    assert lib.tfp8_llm_rope_prefill(a, a, a, a, a, a, a, a, 0, 1, 0, 8, 4, 128, 64, 1024, 512, 512, None) == 0
    assert lib.tfp8_llm_attn_prefill(a, a, a, a, 0, 1, 8, 4, 4, 64, 64, 512, 1.0, None) == -1    # head dim 64
    assert lib.tfp8_llm_attn_prefill(a, a, a, a, 0, 1, 8, 4, 4, 128, 60, 512, 1.0, None) == -1   # L % 8
    assert lib.tfp8_llm_attn_prefill(a, a, a, a, 60, 1, 8, 4, 4, 128, 64, 512, 1.0, None) == -1  # start + T > L
    assert lib.tfp8_llm_attn_prefill(a, a, a, a, 0, 1, 0, 4, 4, 128, 64, 512, 1.0, None) == 0


def test_demo_fused_projections_share_the_layers_weights():
    """The example model's decode step runs q/k/v and gate/up as one FP8Linear each: their codes and
    scales are the layers' rows concatenated, the layers' buffers become views of them (one copy;
    an in-place write to a layer reaches the fused one), and they are built once per set of buffers."""
    from tfp8 import FP8Config, prepare_model
    from tfp8.examples import demo_llm

    torch.manual_seed(0)
    model = demo_llm.Llama(dict(dim=1024, n_layers=2, n_heads=8, n_kv=8, ffn=1024, vocab=64))
    prepare_model(model, "llm", FP8Config(nan_check=False))
    ids = torch.randint(0, 64, (1, 5))
    with torch.no_grad():
        before = model(ids, model.new_cache(1, 5), 0)
    fused = model._fused_projections()
    assert len(fused) == 2 and model._fused_projections() is fused
    at, mlp = model.layers[1].self_attn, model.layers[1].mlp
    qkv, gate_up = fused[1]
    assert qkv.out_features == 3 * 1024 and gate_up.out_features == 2 * 1024
    assert at.k_proj.qweight.data_ptr() == qkv.qweight[1024:].data_ptr()
    assert mlp.up_proj.weight_scale.data_ptr() == gate_up.weight_scale[1024:].data_ptr()
    with torch.no_grad():
        assert torch.equal(model(ids, model.new_cache(1, 5), 0), before)
        y = torch.randn(2, 1024).bfloat16()
        sep = torch.cat([at.q_proj(y), at.k_proj(y), at.v_proj(y)], -1)
        assert torch.allclose(qkv(y).float(), sep.float(), rtol=1e-2, atol=1e-3)
        at.v_proj.qweight[3, 7] ^= 1
    assert qkv.qweight[2048 + 3, 7] == at.v_proj.qweight[3, 7]
    at.q_proj.qweight = at.q_proj.qweight.clone()          # a replaced buffer rebuilds the fused layers
    assert model._fused_projections() is not fused


def test_available_false_and_require_raises_without_gpu():
    if torch.cuda.is_available():
        pytest.skip("GPU present")
    assert _ext.available() is False
    with pytest.raises(RuntimeError):
        _ext.require()


@pytest.mark.parametrize("group,sf", [(None, "f32"), (32, "ue8m0")])
def test_fp8_checkpoint_roundtrip(tmp_path, group, sf):
    """save_fp8 / load_fp8: a converted model written with float8 code tensors and its scales is
    rebuilt from an unconverted model of the same architecture, with identical outputs; tied
    weights are stored once."""
    from safetensors import safe_open

    from tfp8 import FP8Config, load_fp8, prepare_model, save_fp8
    from tfp8.examples import demo_llm

    cfg = dict(dim=1024, n_layers=1, n_heads=8, n_kv=8, ffn=1024, vocab=64)
    torch.manual_seed(0)
    model = demo_llm.Llama(cfg)
    prepare_model(model, "llm", FP8Config(weight_group=group, scale_format=sf, nan_check=False))
    ids = torch.randint(0, 64, (1, 8))
    with torch.no_grad():
        want = model(ids, model.new_cache(1, 8), 0)
    path = str(tmp_path / "m.safetensors")
    save_fp8(model, path, metadata={"note": "test"})

    with safe_open(path, framework="pt") as f:
        keys = set(f.keys())
        meta = f.metadata()
        q = f.get_tensor("layers.0.mlp.up_proj.qweight")
        s = f.get_tensor("layers.0.mlp.up_proj.weight_scale")
    assert q.dtype == torch.float8_e4m3fn and q.shape == (1024, 1024)
    assert s.dtype == (torch.uint8 if sf == "ue8m0" else torch.float32)
    assert s.shape == (1024, 1024 // (group or 1024))
    assert "lm_head.weight" not in keys and meta["tfp8.alias.lm_head.weight"] == "embed.weight"
    assert meta["note"] == "test" and meta["tfp8.format"] == "1"
    assert sum(k.startswith("tfp8.layer.") for k in meta) == 7

    torch.manual_seed(1)
    fresh = demo_llm.Llama(cfg)
    load_fp8(fresh, path, nan_check=False)
    assert sum(isinstance(m, FP8Linear) for m in fresh.modules()) == 7
    assert fresh.lm_head.weight.data_ptr() == fresh.embed.weight.data_ptr()
    with torch.no_grad():
        got = fresh(ids, fresh.new_cache(1, 8), 0)
    assert torch.equal(want, got)
