"""FP8Linear: a Linear whose weight lives on the device as FP8 codes plus scales.

Public surface of the reference module (tfp8/linear.py:31-227): the constructor arguments,
`from_linear`, `from_fp8_checkpoint`, the `qweight` / `weight_scale` / `bias_f32` buffers, the
`stats` counters, the NaN watch over the first calls and the fp32 fallback it installs.

How a call runs here.  The C library (`tfp8_linear`) already picks the kernel family from M, so
the module does not need one code path per kernel: for each (activation dtype, output dtype) it
keeps a `_Binding` -- the library entry with every per-layer argument resolved to plain integers
-- and a forward is one ctypes call plus the output allocation.  The binding is rebuilt when a
buffer object is replaced (`.to()`, `.cuda()`, assignment); in-place updates keep its pointers
valid.  `stats` records which family the library ran, by the same M rules:

    M <= 8                                   "gemv"     streaming GEMV / matrix-core decode kernel
    8 < M, not (M >= large_m and chunked)    "gemm"     MFMA GEMM (decode, streaming, direct, tiled)
    M >= large_m, large_m_backend "chunked"  "chunked"  the same MFMA GEMM: on gfx950 no fp16 copy
                                                        of the weight is ever written
    CPU input, or K / G no kernel takes      "torch"    dequantize + F.linear in fp32
                                                        (the reference CPU path, linear.py:179-181)

A CUDA input whose layer the kernels take never runs the torch path: if the library is missing
the call raises.
"""
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _ext
from .formats import get_format
from .quantize import dequantize_weight, quantize_weight, scale_values

_WATCHED_CALLS = 3        # outputs checked for NaN/Inf before the check switches off


def _kernel_shape_ok(K, G):
    """What the gfx950 kernels take: K and G multiples of 16, and (for the GEMMs) one group per row
    or G a multiple of 32.  The reference probed K % 32 and G % 32 plus its NVRTC module
    (tfp8/linear.py:64-68)."""
    return K % 16 == 0 and G % 16 == 0 and (G == K or G % 32 == 0)


def _codes_u8(qweight, fmt):
    """FP8 checkpoint codes as a uint8 [N, K] view; float8 tensors must carry the declared format."""
    if qweight.dtype == torch.uint8:
        return qweight
    if qweight.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        want = get_format(fmt).torch_dtype
        if qweight.dtype != want:
            raise ValueError(f"checkpoint dtype {qweight.dtype} does not match declared fmt {fmt}")
        return qweight.view(torch.uint8)
    raise ValueError(f"checkpoint codes must be float8 or uint8, got {qweight.dtype}")


def _scale_grid(weight_scale, N, K):
    """Any checkpoint scale layout as an [N, K/G] tensor: a single value (per tensor) becomes one
    scale per row (as tfp8/linear.py:91 expands it), [N] or [N, 1] is per channel, [N, K/G] is
    per K-group.  Float scales are kept as f32, uint8 scales as UE8M0 bytes."""
    s = weight_scale if weight_scale.dtype == torch.uint8 else weight_scale.float()
    if s.numel() == 1:
        return s.reshape(1, 1).expand(N, 1)
    if s.numel() % N:
        raise ValueError(f"scale shape {tuple(weight_scale.shape)} does not match {N} output rows")
    grid = s.reshape(N, -1)
    if K % grid.shape[1]:
        raise ValueError(f"scale shape {tuple(weight_scale.shape)} does not tile K={K}")
    return grid


class _Binding:
    """tfp8_linear for one layer and one (x dtype, out dtype): everything but the activations, the
    output and the workspace fixed as integers.  Holds the layer's buffers so their storage
    outlives the pointers."""

    __slots__ = ("fn", "size_fn", "device", "dev", "q", "ws", "bias", "out_dtype", "N", "K", "xd", "yd",
                 "wargs", "wsizes")

    def __init__(self, q, ws, bias, x_dtype, out_dtype, group_size, fmt):
        lib = _ext.require()
        self.fn, self.size_fn = lib.tfp8_linear, lib.tfp8_linear_workspace_size
        self.q, self.ws, self.bias, self.out_dtype = q, ws, bias, out_dtype
        self.device, self.dev = q.device, q.get_device()
        self.N, self.K = q.shape
        self.xd, self.yd = _ext.DTYPE_ID[x_dtype], _ext.DTYPE_ID[out_dtype]
        self.wargs = (q.data_ptr(), self.N, ws.data_ptr(), _ext.scale_kind(ws), group_size, _ext.FMT_ID[fmt],
                      bias.data_ptr() if bias is not None else None)
        self.wsizes = {}

    def serves(self, q, ws, bias, out_dtype):
        return self.q is q and self.ws is ws and self.bias is bias and self.out_dtype == out_dtype

    def __call__(self, x, M, out_shape):
        y = torch.empty(out_shape, dtype=self.out_dtype, device=self.device)
        if M == 0:
            return y
        nb = 0
        if M > _ext.GEMV_MAXM:                      # the GEMV needs no workspace
            nb = self.wsizes.get(M)
            if nb is None:
                nb = self.wsizes[M] = self.size_fn(self.xd, M, self.N, self.K)
        buf = torch.empty(nb, dtype=torch.uint8, device=self.device) if nb else None
        w, N, ws, sk, G, fmt, b = self.wargs
        rc = self.fn(x.data_ptr(), self.xd, M, self.K, w, N, ws, sk, G, fmt, b, y.data_ptr(), self.yd,
                     buf.data_ptr() if buf is not None else None, nb, _ext._stream(self.dev))
        if rc:
            _ext._check(rc, "tfp8_linear")
        return y


class _CastLinear(nn.Module):
    """The fallback installed after a non-finite output: an fp32 Linear, cast to the layer's dtype."""

    def __init__(self, lin, out_dtype):
        super().__init__()
        self.lin, self.out_dtype = lin, out_dtype

    def forward(self, x):
        return self.lin(x.float()).to(self.out_dtype)


class FP8Linear(nn.Module):
    precision_owner = "tfp8"

    def __init__(self, in_features, out_features, bias=True, fmt="e4m3fn", group_size=None,
                 out_dtype=torch.bfloat16, large_m=256, large_m_backend="chunked",
                 workspace_mb=32, nan_check=True, device=None, scale_format="f32"):
        super().__init__()
        G = group_size or in_features
        if G <= 0 or in_features % G:
            raise ValueError(f"in_features={in_features} not divisible by group_size={G}")
        if scale_format not in ("f32", "ue8m0"):
            raise ValueError(f"scale_format must be 'f32' or 'ue8m0', got {scale_format!r}")
        self.in_features, self.out_features, self.group_size = in_features, out_features, G
        self.fmt = get_format(fmt).name
        self.out_dtype = out_dtype
        self.large_m, self.large_m_backend = large_m, large_m_backend
        self.workspace_mb = workspace_mb        # kept for the API; the fused GEMM needs no fp16 slices
        self.nan_check = nan_check
        self.scale_format = scale_format
        groups = in_features // G
        codes = torch.zeros(out_features, in_features, dtype=torch.uint8, device=device)
        if scale_format == "ue8m0":
            scales = torch.full((out_features, groups), 127, dtype=torch.uint8, device=device)   # 2^0
        else:
            scales = torch.ones(out_features, groups, dtype=torch.float32, device=device)
        self.register_buffer("qweight", codes)
        self.register_buffer("weight_scale", scales)
        self.register_buffer("bias_f32", torch.zeros(out_features, dtype=torch.float32, device=device)
                             if bias else None)
        self.stats = dict.fromkeys(("gemv", "gemm", "chunked", "torch", "fallback"), 0)
        self.fallback = None
        self.fallback_reason = None
        self._nan_checks = 0
        self._kernels_ok = _kernel_shape_ok(in_features, G)
        self._bindings = {}

    # ------------------------------------------------------------------ construction
    def _fill(self, codes, scales, bias):
        with torch.no_grad():
            self.qweight.copy_(codes)
            self.weight_scale.copy_(scales)
            if bias is not None:
                self.bias_f32.copy_(bias.float())
        return self

    @classmethod
    def from_linear(cls, lin: nn.Linear, fmt="e4m3fn", group_size=None, pow2_scale=True, scale_format="f32", **kw):
        """Quantize an nn.Linear (tfp8/linear.py:70-80).  The output dtype follows the weight when it
        is fp16/bf16 and is fp16 otherwise."""
        w = lin.weight.detach()
        codes, scales, G = quantize_weight(w, fmt, group_size, pow2_scale, scale_format)
        kw.setdefault("out_dtype", w.dtype if w.dtype in (torch.float16, torch.bfloat16) else torch.float16)
        layer = cls(lin.in_features, lin.out_features, lin.bias is not None, fmt, G, device=w.device,
                    scale_format=scale_format, **kw)
        return layer._fill(codes, scales, None if lin.bias is None else lin.bias.detach())

    @classmethod
    def from_fp8_checkpoint(cls, qweight, weight_scale, bias=None, fmt="e4m3fn", **kw):
        """Adopt an existing FP8 checkpoint's codes and scales unchanged (tfp8/linear.py:82-98).

        qweight: float8_e4m3fn / float8_e5m2 (matching `fmt`) or uint8 codes [N, K].
        weight_scale: one value (per tensor), [N] / [N, 1] (per channel) or [N, K/G] (per K-group);
        float scales become f32, uint8 scales are UE8M0 bytes.
        """
        codes = _codes_u8(qweight, fmt)
        N, K = codes.shape
        grid = _scale_grid(weight_scale, N, K)
        kw.setdefault("scale_format", "ue8m0" if grid.dtype == torch.uint8 else "f32")
        layer = cls(K, N, bias is not None, fmt, K // grid.shape[1], device=codes.device, **kw)
        return layer._fill(codes, grid, bias)

    def extra_repr(self):
        return (f"in={self.in_features}, out={self.out_features}, fmt={self.fmt}, "
                f"group={self.group_size}, out_dtype={self.out_dtype}, scales={self.scale_format}")

    def dequantized_weight(self):
        """fp32 [N, K] weight rebuilt from the codes and scales (never used by forward's kernels)."""
        return dequantize_weight(self.qweight, self.weight_scale, self.fmt, self.group_size)

    def scale_values(self):
        """weight_scale as float32 [N, K/G], whatever its storage."""
        return scale_values(self.weight_scale)

    # ------------------------------------------------------------------ execution
    def _binding(self, x_dtype):
        """The library call for this layer's current buffers (identity-checked through _buffers,
        which skips nn.Module.__getattr__)."""
        buf = self._buffers
        q, ws, b = buf["qweight"], buf["weight_scale"], buf.get("bias_f32")
        key = (x_dtype, self.out_dtype)
        bind = self._bindings.get(key)
        if bind is None or not bind.serves(q, ws, b, self.out_dtype):
            bind = self._bindings[key] = _Binding(q, ws, b, x_dtype, self.out_dtype, self.group_size, self.fmt)
        return bind

    def _route(self, M):
        if M <= _ext.GEMV_MAXM:
            return "gemv"
        return "chunked" if M >= self.large_m and self.large_m_backend == "chunked" else "gemm"

    def _run_torch(self, x, rows):
        self.stats["torch"] += 1
        x2 = x.reshape(rows, self.in_features)
        return F.linear(x2.float(), self.dequantized_weight(), self.bias_f32).to(self.out_dtype)

    def _run_kernels(self, x, rows, out_shape):
        if x.device != self.qweight.device:
            raise RuntimeError(f"FP8Linear on {self.qweight.device} called with an input on {x.device}")
        if x.dtype not in _ext.DTYPE_ID:
            x = x.float()
        if not x.is_contiguous() or x.data_ptr() % 16:
            x = x.contiguous() if not x.is_contiguous() else x.clone()   # 16-byte loads need an aligned start
        self.stats[self._route(rows)] += 1
        bind = self._binding(x.dtype)
        if torch.cuda.current_device() != bind.dev:
            with torch.cuda.device(bind.dev):
                return bind(x, rows, out_shape)
        return bind(x, rows, out_shape)

    def forward(self, x):
        if self.fallback is not None:
            self.stats["fallback"] += 1
            return self.fallback(x)
        K = self.in_features
        if x.shape[-1] != K:
            raise RuntimeError(f"FP8Linear expects {K} input features, got shape {tuple(x.shape)}")
        rows = x.numel() // K
        out_shape = x.shape[:-1] + (self.out_features,)
        if x.is_cuda and self._kernels_ok:
            y = self._run_kernels(x, rows, out_shape)
        else:
            y = self._run_torch(x, rows).reshape(out_shape)
        if self.nan_check and self._nan_checks < _WATCHED_CALLS:
            # A device sync per call would dominate decode, so only the first calls are checked; a
            # kernel or scale problem shows up on the first call.
            self._nan_checks += 1
            if not bool(torch.isfinite(y).all()) and bool(torch.isfinite(x).all()):
                self._back_off(f"non-finite output for input shape {tuple(x.shape)}")
                return self.forward(x)
        return y

    def _back_off(self, reason):
        """Replace the kernels by an fp32 nn.Linear built from the same codes and scales, and record
        why (reported by planner.report)."""
        lin = nn.Linear(self.in_features, self.out_features, bias=self.bias_f32 is not None,
                        device=self.qweight.device, dtype=torch.float32)
        with torch.no_grad():
            lin.weight.copy_(self.dequantized_weight())
            if self.bias_f32 is not None:
                lin.bias.copy_(self.bias_f32)
        self.fallback = _CastLinear(lin, self.out_dtype)
        self.fallback_reason = reason
