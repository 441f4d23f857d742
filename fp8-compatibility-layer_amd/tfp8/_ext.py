"""ctypes boundary to libtfp8_hip.so, the gfx950 kernels of the FP8Linear path.

Replaces the reference's NVRTC compile + ctypes `cuLaunchKernel` layer (tfp8/_ext.py:1-315)
with a prebuilt C-ABI HIP library: one C call per operation, device pointers from torch
tensors, launches on torch's current stream, a nonzero return turned into RuntimeError with
the library's message.  Names that callers use are kept: `available`, `last_error`, `w8a16`,
`prepare_activations`, `gemm_prepared`, `dequant_into`, `GemvLaunch`, `GEMV_MAXM`, `FMT_ID`.

Unlike the reference, CUDA tensors never fall back to a torch path when the library is
missing: `require()` raises.  `available()` still reports the state without raising.
"""
import ctypes
import os
import sys
import threading

import torch

_LIB_NAME = "libtfp8_hip.so"
_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), _LIB_NAME)

GEMV_MAXM = 8                       # tfp8/_ext.py:37 -- M <= 8 takes the GEMV
FMT_ID = {"e4m3fn": 0, "e5m2": 1}   # tfp8/_ext.py:41
DTYPE_ID = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
_TAG = DTYPE_ID                     # dtypes the kernels take (tfp8/_ext.py:160)
SCALE_F32, SCALE_UE8M0 = 0, 1
ABI_VERSION = 1

_lock = threading.Lock()
_lib = None
_error = None

_c = ctypes
_P = _c.c_void_p
_I = _c.c_int
_I64 = _c.c_int64
_SZ = _c.c_size_t

# Signatures of include/tfp8_hip.h, declared once (untyped ctypes calls are slow and unsafe).
_SIGS = {
    "tfp8_abi_version": (_I, []),
    "tfp8_last_error": (_c.c_char_p, []),
    "tfp8_decode": (_I, [_P, _I64, _I, _P, _I, _P]),
    "tfp8_encode": (_I, [_P, _I, _I64, _I, _P, _P]),
    "tfp8_quantize_weight": (_I, [_P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P]),
    "tfp8_prepare_activations": (_I, [_P, _I, _I, _I, _P, _P, _P]),
    "tfp8_dequant": (_I, [_P, _I, _I, _P, _I, _I, _I, _P, _I, _P]),
    "tfp8_linear_workspace_size": (_SZ, [_I, _I, _I, _I]),
    "tfp8_linear": (_I, [_P, _I, _I, _I, _P, _I, _P, _I, _I, _I, _P, _P, _I, _P, _SZ, _P]),
    "tfp8_linear_noalloc": (_I, [_P, _I, _I, _I, _P, _I, _P, _I, _I, _I, _P, _P, _I, _P]),
    "tfp8_gemv": (_I, [_P, _I, _I, _I, _P, _I, _P, _I, _I, _I, _P, _P, _I, _P]),
    "tfp8_gemm_prepared_workspace_size": (_SZ, [_I, _I, _I, _I]),
    "tfp8_gemm_prepared": (_I, [_P, _I, _P, _I, _I, _P, _I, _P, _I, _I, _I, _P, _P, _I, _P, _SZ, _P]),
    "tfp8_tuning_set": (_I, [_c.c_char_p, _I]),
    "tfp8_tuning_get": (_I, [_c.c_char_p, _P]),
    "tfp8_tuning_reset": (None, []),
    "tfp8_w8a8_quantize": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, _P]),
    "tfp8_w8a8_gemm": (_I, [_P, _I, _P, _P, _I, _P, _I, _I, _I, _P, _P, _I, _I, _I, _P]),
    "tfp8_read_probe": (_I, [_P, _SZ, _P, _I, _P]),
}


def lib_path():
    return _LIB_PATH


def _load():
    """Load the shared library and bind every signature. Raises on any failure."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                raise RuntimeError(f"{_LIB_PATH} not built (run fp8-compatibility-layer_amd/build_lib.py "
                                   f"or __graft_entry__.build())")
            lib = ctypes.CDLL(_LIB_PATH)
            for name, (res, args) in _SIGS.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.tfp8_abi_version() != ABI_VERSION:
                raise RuntimeError(f"{_LIB_NAME} ABI {lib.tfp8_abi_version()} != expected {ABI_VERSION}")
            _lib = lib
        return _lib


def library():
    """The loaded ctypes library (loads it on first use; no GPU needed)."""
    return _lib or _load()


def available() -> bool:
    """True when a GPU is present and the HIP library loads (tfp8/_ext.py:45-60). A load failure
    is recorded in last_error() and reported once on stderr."""
    global _error
    if not torch.cuda.is_available():
        return False
    try:
        library()
        return True
    except Exception as e:  # noqa: BLE001
        if _error is None:
            _error = e
            print(f"[tfp8] FATAL: HIP kernels unavailable: {e}", file=sys.stderr)
        return False


def last_error():
    return _error


def require():
    """The library, or RuntimeError: CUDA tensors have no other path."""
    if not torch.cuda.is_available():
        raise RuntimeError("tfp8: no GPU visible")
    try:
        return library()
    except Exception as e:  # noqa: BLE001
        raise RuntimeError(f"tfp8: HIP library unavailable for a CUDA tensor: {e}") from e


def _stream(dev: int):
    return torch._C._cuda_getCurrentRawStream(dev)


def _check(rc, name):
    if rc != 0:
        msg = _lib.tfp8_last_error().decode(errors="replace") if _lib is not None else ""
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def _dtype_id(t):
    try:
        return DTYPE_ID[t]
    except KeyError:
        raise TypeError(f"tfp8 kernels take float16/bfloat16/float32, got {t}") from None


def _aligned(x: torch.Tensor) -> torch.Tensor:
    """x itself when its data starts on a 16-byte boundary (what the kernels' 16-byte loads need),
    else an aligned copy: a contiguous view can start anywhere in its storage (e.g. one row sliced
    one element in), and the library refuses such a pointer rather than read it misaligned."""
    return x if x.data_ptr() % 16 == 0 else x.clone()


def scale_kind(ws: torch.Tensor) -> int:
    if ws.dtype == torch.float32:
        return SCALE_F32
    if ws.dtype == torch.uint8:
        return SCALE_UE8M0
    raise TypeError(f"weight_scale must be float32 or uint8 (UE8M0), got {ws.dtype}")


def _same_device(*ts):
    dev = ts[0].device
    for t in ts[1:]:
        if t is not None and t.device != dev:
            raise RuntimeError(f"tfp8: tensors on different devices ({dev} vs {t.device})")


# ------------------------------------------------------------------ codec
def decode_into(q: torch.Tensor, out: torch.Tensor, fmt) -> torch.Tensor:
    lib = require()
    _same_device(q, out)
    if q.dtype != torch.uint8 or not q.is_contiguous() or not out.is_contiguous() or out.numel() != q.numel():
        raise ValueError("decode_into: contiguous uint8 codes and a contiguous output of the same size")
    _check(lib.tfp8_decode(q.data_ptr(), q.numel(), FMT_ID[fmt], out.data_ptr(), _dtype_id(out.dtype),
                           _stream(q.get_device())), "tfp8_decode")
    return out


def decode(q: torch.Tensor, fmt, dtype=torch.float32) -> torch.Tensor:
    q = q.contiguous()
    out = torch.empty(q.shape, dtype=dtype, device=q.device)
    return decode_into(q, out, fmt)


def encode(x: torch.Tensor, fmt) -> torch.Tensor:
    lib = require()
    if x.dtype not in DTYPE_ID:
        x = x.float()
    x = x.contiguous()
    q = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    _check(lib.tfp8_encode(x.data_ptr(), _dtype_id(x.dtype), x.numel(), FMT_ID[fmt], q.data_ptr(),
                           _stream(x.get_device())), "tfp8_encode")
    return q


def quantize_weight(w: torch.Tensor, fmt, group_size, pow2_scale=True, ue8m0=False):
    """(q uint8 [N,K], scale f32 or uint8 [N,K/G]) from one kernel launch."""
    lib = require()
    if w.dtype not in DTYPE_ID:
        w = w.float()
    w = w.contiguous()
    N, K = w.shape
    G = group_size
    q = torch.empty(N, K, dtype=torch.uint8, device=w.device)
    s = torch.empty(N, K // G, dtype=torch.uint8 if ue8m0 else torch.float32, device=w.device)
    _check(lib.tfp8_quantize_weight(w.data_ptr(), _dtype_id(w.dtype), N, K, G, FMT_ID[fmt], int(bool(pow2_scale)),
                                    SCALE_UE8M0 if ue8m0 else SCALE_F32, q.data_ptr(), s.data_ptr(),
                                    _stream(w.get_device())), "tfp8_quantize_weight")
    return q, s


def prepare_activations(x):
    """(x16 fp16 [M,K], xs f32 [M]) in one kernel launch (tfp8/_ext.py:220-227). Power-of-two row
    scale from the exact exponent of the row amax."""
    lib = require()
    x = x.contiguous()
    M, K = x.shape
    x16 = torch.empty(M, K, dtype=torch.float16, device=x.device)
    xs = torch.empty(M, dtype=torch.float32, device=x.device)
    _check(lib.tfp8_prepare_activations(x.data_ptr(), _dtype_id(x.dtype), M, K, x16.data_ptr(), xs.data_ptr(),
                                        _stream(x.get_device())), "tfp8_prepare_activations")
    return x16, xs


def dequant_into(out, qweight, lut16, wscale, group_size, fmt="e4m3fn"):
    """out[n,k] = decode(q[n,k]) * scale[n, k//G] into `out` (f16/bf16/f32, [N,K]).
    `lut16` is accepted for the reference signature (tfp8/_ext.py:305) and unused: decode is
    arithmetic on gfx950."""
    lib = require()
    _same_device(out, qweight, wscale)
    N, K = qweight.shape
    if not (out.is_contiguous() and qweight.is_contiguous() and wscale.is_contiguous()):
        raise ValueError("dequant_into: contiguous tensors required")
    _check(lib.tfp8_dequant(qweight.data_ptr(), N, K, wscale.data_ptr(), scale_kind(wscale), group_size,
                            FMT_ID[fmt], out.data_ptr(), _dtype_id(out.dtype), _stream(qweight.get_device())),
           "tfp8_dequant")
    return out


# ------------------------------------------------------------------ linear
def _ptr(t):
    return t.data_ptr() if t is not None else None


def workspace_bytes(x_dtype, M, N, K) -> int:
    return library().tfp8_linear_workspace_size(_dtype_id(x_dtype), M, N, K)


def _workspace(device, nbytes):
    # Per call from torch's caching allocator: stream-ordered, so concurrent streams never share it.
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device) if nbytes else None


def w8a16(x, qweight, lut16, wscale, bias, out_dtype, group_size, fmt="e4m3fn"):
    """y = x @ dequant(qweight).T + bias  (tfp8/_ext.py:230-253).

    M <= 8   GEMV path on x in its own dtype: streaming GEMV (dot products, fp32 accumulation) up
             to 3 rows, the matrix-core decode kernel from 4
    M > 8    MFMA GEMM path (decode kernel up to 16 rows, then weight-streaming / direct-to-LDS /
             LDS-tiled by M and scale layout): f16/bf16 x directly, fp32 x via the fp16 row-scaled
             prep
    `lut16` is accepted for the reference signature and unused.
    """
    lib = require()
    M, K = x.shape
    N = qweight.shape[0]
    _same_device(x, qweight, wscale, bias)
    y = torch.empty(M, N, dtype=out_dtype, device=x.device)
    if M == 0:
        return y
    x = _aligned(x.contiguous())
    xd = _dtype_id(x.dtype)
    dev = x.get_device()
    nb = lib.tfp8_linear_workspace_size(xd, M, N, K)
    ws_buf = _workspace(x.device, nb)
    _check(lib.tfp8_linear(x.data_ptr(), xd, M, K, qweight.data_ptr(), N, wscale.data_ptr(), scale_kind(wscale),
                           group_size, FMT_ID[fmt], _ptr(bias), y.data_ptr(), _dtype_id(out_dtype),
                           _ptr(ws_buf), nb, _stream(dev)), "tfp8_linear")
    return y


def gemv(x, qweight, wscale, bias, out_dtype, group_size, fmt="e4m3fn"):
    """The GEMV alone (1 <= M <= 8)."""
    lib = require()
    M, K = x.shape
    N = qweight.shape[0]
    _same_device(x, qweight, wscale, bias)
    x = _aligned(x.contiguous())
    y = torch.empty(M, N, dtype=out_dtype, device=x.device)
    _check(lib.tfp8_gemv(x.data_ptr(), _dtype_id(x.dtype), M, K, qweight.data_ptr(), N, wscale.data_ptr(),
                         scale_kind(wscale), group_size, FMT_ID[fmt], _ptr(bias), y.data_ptr(),
                         _dtype_id(out_dtype), _stream(x.get_device())), "tfp8_gemv")
    return y


def gemm_prepared(x16, xs, qweight, lut16, wscale, bias, out_dtype, group_size, fmt="e4m3fn"):
    """The MFMA GEMM on f16/bf16 activations with an optional f32 row scale xs (tfp8/_ext.py:267-275).
    Any M >= 1 (tests force the GEMM at small M with this)."""
    lib = require()
    M, K = x16.shape
    N = qweight.shape[0]
    _same_device(x16, qweight, wscale, bias, xs)
    x16 = x16.contiguous()
    y = torch.empty(M, N, dtype=out_dtype, device=x16.device)
    if M == 0:
        return y
    nb = lib.tfp8_gemm_prepared_workspace_size(_dtype_id(x16.dtype), M, N, K)
    ws_buf = _workspace(x16.device, nb)
    _check(lib.tfp8_gemm_prepared(x16.data_ptr(), _dtype_id(x16.dtype), _ptr(xs), M, K, qweight.data_ptr(), N,
                                  wscale.data_ptr(), scale_kind(wscale), group_size, FMT_ID[fmt], _ptr(bias),
                                  y.data_ptr(), _dtype_id(out_dtype), _ptr(ws_buf), nb, _stream(x16.get_device())),
           "tfp8_gemm_prepared")
    return y


# ------------------------------------------------------------------ tuning knobs
def tuning_set(name: str, value: int) -> None:
    """Force a kernel-selection knob (TFP8_GEMV_CFG, TFP8_GEMM_SPLITK, ...; include/tfp8_hip.h) for
    every later call in this process.  Workspace sizes follow the knobs: query them afterwards."""
    _check(library().tfp8_tuning_set(name.encode(), int(value)), "tfp8_tuning_set")


def tuning_get(name: str) -> int:
    v = _c.c_int(0)
    _check(library().tfp8_tuning_get(name.encode(), _c.byref(v)), "tfp8_tuning_get")
    return v.value


def tuning_reset() -> None:
    """Every knob back to its value when the library was loaded."""
    library().tfp8_tuning_reset()


class tuning:
    """Context manager: `with _ext.tuning(TFP8_GEMM_SPLITK=3, TFP8_GEMM_TILE=13): ...` sets the knobs
    and restores the previous values on exit."""

    def __init__(self, **knobs):
        self.knobs = knobs
        self.saved = {}

    def __enter__(self):
        for k, v in self.knobs.items():
            self.saved[k] = tuning_get(k)
            tuning_set(k, v)
        return self

    def __exit__(self, *exc):
        for k, v in self.saved.items():
            tuning_set(k, v)
        return False


class GemvLaunch:
    """A GEMV launch for one layer with its static arguments bound once (tfp8/_ext.py:163-217).

    Only the activation pointer, the output pointer and M change per call. The static tensors are
    referenced here so their storage cannot be freed under the launch; FP8Linear rebuilds the
    object when any of them is replaced.
    """
    __slots__ = ("fn", "dev", "device", "q", "ws", "bias", "lut", "out_dtype", "N", "K", "args_tail", "xd", "yd")

    def __init__(self, x_dtype, qweight, lut16, wscale, bias, out_dtype, group_size, fmt):
        lib = require()
        self.fn = lib.tfp8_gemv
        self.dev = qweight.get_device()
        self.device = qweight.device
        self.N, self.K = qweight.shape
        self.xd, self.yd = _dtype_id(x_dtype), _dtype_id(out_dtype)
        self.q, self.ws, self.bias, self.lut, self.out_dtype = qweight, wscale, bias, lut16, out_dtype
        # (w, N, ws, ws_kind, G, fmt, bias) -- fixed for the layer
        self.args_tail = (qweight.data_ptr(), self.N, wscale.data_ptr(), scale_kind(wscale), group_size,
                          FMT_ID[fmt], _ptr(bias))

    def __call__(self, x, M, out_shape=None):
        """x: contiguous CUDA tensor of the bound dtype on this layer's device holding M rows of K
        (any rank: only its data pointer is used)."""
        y = torch.empty(out_shape or (M, self.N), dtype=self.out_dtype, device=self.device)
        w, N, ws, sk, G, fmt, b = self.args_tail
        rc = self.fn(x.data_ptr(), self.xd, M, self.K, w, N, ws, sk, G, fmt, b, y.data_ptr(), self.yd,
                     _stream(self.dev))
        if rc != 0:
            _check(rc, "tfp8_gemv")
        return y
