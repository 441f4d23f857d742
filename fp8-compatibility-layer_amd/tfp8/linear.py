"""FP8Linear: W8A16 Linear whose weight stays resident as FP8 (uint8 codes + f32/UE8M0 scales).

API and behaviour of the reference tfp8/linear.py:31-227. Execution paths, chosen per call by
M = number of activation rows, on a CUDA (ROCm) input:
  M <= 8           streaming GEMV (decode FP8 in registers, fp32 FMA)        -- stats["gemv"]
  8 < M            LDS-tiled MFMA GEMM (FP8 tile in LDS, decoded to f16/bf16 fragments,
                   fp32 accumulation)                                          -- stats["gemm"]
  M >= large_m     same MFMA GEMM; counted as stats["chunked"] when large_m_backend is
                   "chunked" (the reference's dequant + cuBLAS branch; on gfx950 no fp16
                   weight copy is ever materialised)
CPU input, or a layer whose K/G the kernels do not take (K % 16, G % 16, or a G that is
neither K nor a multiple of 32), runs the torch reference path (dequantize + matmul) as in
tfp8/linear.py:179-181 -- stats["torch"]. A CUDA input with the HIP library missing raises.
"""
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _ext
from .formats import get_format, lut
from .quantize import dequantize_weight, quantize_weight, scale_values


class FP8Linear(nn.Module):
    precision_owner = "tfp8"

    def __init__(self, in_features, out_features, bias=True, fmt="e4m3fn", group_size=None,
                 out_dtype=torch.bfloat16, large_m=256, large_m_backend="chunked",
                 workspace_mb=32, nan_check=True, device=None, scale_format="f32"):
        super().__init__()
        self.in_features, self.out_features = in_features, out_features
        self.fmt = get_format(fmt).name
        self.group_size = group_size or in_features
        if in_features % self.group_size:
            raise ValueError(f"in_features={in_features} not divisible by group_size={self.group_size}")
        self.out_dtype = out_dtype
        self.large_m, self.large_m_backend = large_m, large_m_backend
        self.workspace_mb, self.nan_check = workspace_mb, nan_check
        self.scale_format = scale_format
        ng = in_features // self.group_size
        sdt = torch.uint8 if scale_format == "ue8m0" else torch.float32
        self.register_buffer("qweight", torch.zeros(out_features, in_features, dtype=torch.uint8, device=device))
        self.register_buffer("weight_scale", (torch.full((out_features, ng), 127, dtype=sdt, device=device)
                                              if sdt == torch.uint8 else
                                              torch.ones(out_features, ng, dtype=sdt, device=device)))
        self.register_buffer("bias_f32", torch.zeros(out_features, dtype=torch.float32, device=device)
                             if bias else None)
        self._nan_checks = 0
        self.fallback = None        # module set when the layer had to back off (NaN/Inf output)
        self.stats = {"gemv": 0, "gemm": 0, "chunked": 0, "torch": 0, "fallback": 0}
        self._kernels_ok = self._probe_kernels()
        self._lut = lut(self.fmt, device) if device is not None and torch.device(device).type == "cpu" else None
        self._gemv = {}             # (x dtype, out dtype) -> _ext.GemvLaunch

    def _lut_for(self):
        """The fp16 decode table on this layer's device (API of tfp8/linear.py:55-62)."""
        l = self._lut
        if l is None or l.device != self.weight_scale.device:
            l = self._lut = lut(self.fmt, self.weight_scale.device)
        return l

    def _probe_kernels(self):
        """Shapes the gfx950 kernels take: K % 16, G % 16, and G == K or G % 32 (MFMA GEMM).
        The reference also required its NVRTC module here (tfp8/linear.py:64-68); on this build a
        missing library is an error at the first CUDA call instead of a silent torch path."""
        K, G = self.in_features, self.group_size
        return K % 16 == 0 and G % 16 == 0 and (G == K or G % 32 == 0)

    @classmethod
    def from_linear(cls, lin: nn.Linear, fmt="e4m3fn", group_size=None, pow2_scale=True, scale_format="f32", **kw):
        q, s, G = quantize_weight(lin.weight.data, fmt, group_size, pow2_scale, scale_format)
        m = cls(lin.in_features, lin.out_features, lin.bias is not None, fmt, G,
                out_dtype=lin.weight.dtype if lin.weight.dtype in (torch.float16, torch.bfloat16) else torch.float16,
                device=lin.weight.device, scale_format=scale_format, **kw)
        m.qweight.copy_(q)
        m.weight_scale.copy_(s)
        if lin.bias is not None:
            m.bias_f32.copy_(lin.bias.data.float())
        return m

    @classmethod
    def from_fp8_checkpoint(cls, qweight, weight_scale, bias=None, fmt="e4m3fn", **kw):
        """Compatibility mode: take an existing FP8 checkpoint's codes and scales verbatim.

        qweight: float8_e4m3fn / float8_e5m2 (must match `fmt`) or uint8 codes [N,K].
        weight_scale: a scalar (per-tensor), [N] / [N,1] (per-channel) or [N, K/G] (per-K-group);
        float scales are kept as f32, uint8 scales are UE8M0 bytes (tfp8/linear.py:82-98).
        """
        if qweight.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
            want = get_format(fmt).torch_dtype
            if qweight.dtype != want:
                raise ValueError(f"checkpoint dtype {qweight.dtype} does not match declared fmt {fmt}")
            qweight = qweight.view(torch.uint8)
        elif qweight.dtype != torch.uint8:
            raise ValueError(f"checkpoint codes must be float8 or uint8, got {qweight.dtype}")
        N, K = qweight.shape
        ue8m0 = weight_scale.dtype == torch.uint8
        sv = weight_scale if ue8m0 else weight_scale.float()
        ws = sv.reshape(N, -1) if sv.numel() > 1 else sv.reshape(1, 1).expand(N, 1)
        if K % ws.shape[1]:
            raise ValueError(f"scale shape {tuple(weight_scale.shape)} does not tile K={K}")
        G = K // ws.shape[1]
        kw.setdefault("scale_format", "ue8m0" if ue8m0 else "f32")
        m = cls(K, N, bias is not None, fmt, G, device=qweight.device, **kw)
        m.qweight.copy_(qweight)
        m.weight_scale.copy_(ws)
        if bias is not None:
            m.bias_f32.copy_(bias.float())
        return m

    def extra_repr(self):
        return (f"in={self.in_features}, out={self.out_features}, fmt={self.fmt}, "
                f"group={self.group_size}, out_dtype={self.out_dtype}, scales={self.scale_format}")

    def dequantized_weight(self):
        return dequantize_weight(self.qweight, self.weight_scale, self.fmt, self.group_size)

    def _gemv_launch(self, x_dtype):
        """Prepared GEMV launch for this layer, or None when the fast path does not apply.
        Rebuilt whenever a buffer object was replaced (`.to()`, `.cuda()`, assignment) or the output
        dtype changed; in-place updates (`load_state_dict`, `copy_`) keep the cached pointers valid."""
        b = self._buffers
        q, ws, bias = b["qweight"], b["weight_scale"], b.get("bias_f32")
        key = (x_dtype, self.out_dtype)
        p = self._gemv.get(key)
        if p is None or p.q is not q or p.ws is not ws or p.bias is not bias:
            if x_dtype not in _ext._TAG or self.out_dtype not in _ext._TAG or not q.is_cuda:
                return None
            p = self._gemv[key] = _ext.GemvLaunch(x_dtype, q, None, ws, bias, self.out_dtype,
                                                   self.group_size, self.fmt)
        return p

    def forward(self, x):
        # Decode fast path (M <= 8 rows, contiguous CUDA input, past the first NaN-checked calls):
        # only x's data pointer and M are needed, so an [B, T, K] input is neither reshaped in nor
        # out, and the output is allocated in its final shape.
        if ((self._nan_checks >= 3 or not self.nan_check) and self.fallback is None
                and self._kernels_ok and x.is_cuda and x.is_contiguous() and x.data_ptr() % 16 == 0):
            shape = x.shape
            if shape[-1] == self.in_features:
                M = x.numel() // shape[-1]
                if 0 < M <= _ext.GEMV_MAXM:
                    p = self._gemv_launch(x.dtype)
                    if p is not None and x.get_device() == p.dev and torch.cuda.current_device() == p.dev:
                        self.stats["gemv"] += 1
                        return p(x, M, shape[:-1] + (self.out_features,))
        if self.fallback is not None:
            self.stats["fallback"] += 1
            return self.fallback(x)
        shape = x.shape
        x2 = x if x.dim() == 2 else x.reshape(-1, shape[-1])
        if not x2.is_contiguous():
            x2 = x2.contiguous()
        if x2.is_cuda and x2.data_ptr() % 16:
            x2 = x2.clone()        # the kernels load x 16 bytes at a time
        M = x2.shape[0]
        if not self._kernels_ok or not x2.is_cuda:
            self.stats["torch"] += 1
            y = F.linear(x2.float(), self.dequantized_weight(), self.bias_f32).to(self.out_dtype)
        else:
            if x2.dtype not in _ext._TAG:
                x2 = x2.float()
            if M >= self.large_m and self.large_m_backend == "chunked":
                self.stats["chunked"] += 1
            else:
                self.stats["gemv" if M <= _ext.GEMV_MAXM else "gemm"] += 1
            y = None
            if 0 < M <= _ext.GEMV_MAXM:
                p = self._gemv_launch(x2.dtype)
                if p is not None and x2.get_device() == p.dev and torch.cuda.current_device() == p.dev:
                    y = p(x2, M)
            if y is None:
                y = _ext.w8a16(x2, self.qweight, None, self.weight_scale, self.bias_f32, self.out_dtype,
                               self.group_size, self.fmt)
        # A per-call device sync would dominate decode; check the first few calls (failures are
        # structural) rather than every token (tfp8/linear.py:201-207).
        if self.nan_check and self._nan_checks < 3:
            self._nan_checks += 1
            if not torch.isfinite(y).all() and torch.isfinite(x2).all():
                self._back_off(f"non-finite output for input shape {tuple(x2.shape)}")
                return self.forward(x)
        return y if x.dim() == 2 else y.reshape(*shape[:-1], self.out_features)

    def _back_off(self, reason):
        """Runtime fallback: an fp32 Linear rebuilt from the FP8 codes (same numbers), logged."""
        lin = nn.Linear(self.in_features, self.out_features, self.bias_f32 is not None,
                        device=self.qweight.device, dtype=torch.float32)
        with torch.no_grad():
            lin.weight.copy_(self.dequantized_weight())
            if self.bias_f32 is not None:
                lin.bias.copy_(self.bias_f32)
        self.fallback = _CastLinear(lin, self.out_dtype)
        self.fallback_reason = reason

    def scale_values(self):
        """weight_scale as float32 [N, K/G] whatever its storage."""
        return scale_values(self.weight_scale)


class _CastLinear(nn.Module):
    def __init__(self, lin, out_dtype):
        super().__init__()
        self.lin, self.out_dtype = lin, out_dtype

    def forward(self, x):
        return self.lin(x.float()).to(self.out_dtype)
