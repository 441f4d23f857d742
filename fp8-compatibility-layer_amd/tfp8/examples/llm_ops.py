"""ctypes bindings of libtfp8_llm.so, the example model's fused decode-step ops (llm_ops.hip).

Each function takes CUDA tensors, checks their shapes and dtypes, launches on torch's current
stream (so the calls record into a HIP graph under capture) and returns new output tensors.  The
library is the example model's own code; demo_llm uses it for the decode step and the prefill on
the GPU and raises if it is missing there."""
import ctypes
import math
import os

import numpy as np
import torch

_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtfp8_llm.so")
_LIB = None


def library():
    global _LIB
    if _LIB is None:
        if not os.path.exists(_PATH):
            raise RuntimeError(f"{_PATH} is not built (run __graft_entry__.build())")
        lib = ctypes.CDLL(_PATH)
        p, i, f, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_int64
        lib.tfp8_llm_add_rmsnorm.argtypes = [p, p, p, p, p, i, i, f, p]
        lib.tfp8_llm_rope_cache.argtypes = [p, p, p, p, p, p, p, p, p, i, i, i, i, i, i, i, i, p]
        lib.tfp8_llm_attention.argtypes = [p, p, p, p, p, i, p, i, i, i, i, i, f, p]
        lib.tfp8_llm_silu_mul.argtypes = [p, p, p, i, i, i64, p]
        lib.tfp8_llm_head.argtypes = [p, p, p, i, i, i, p]
        lib.tfp8_llm_rope_attention.argtypes = [p, p, p, p, p, p, p, p, p, i, p, i, i, i, i, i, i, i, i, f, p]
        lib.tfp8_llm_step_in.argtypes = [p, p, p, p, p, p, p, i, i, i, i, p]
        lib.tfp8_llm_step_out.argtypes = [p, i, i, i64, p, p, p]
        lib.tfp8_llm_rope_prefill.argtypes = [p, p, p, p, p, p, p, p, i, i, i, i, i, i, i, i, i, i, p]
        lib.tfp8_llm_attn_prefill.argtypes = [p, p, p, p, i, i, i, i, i, i, i, i, f, p]
        for fn in (lib.tfp8_llm_add_rmsnorm, lib.tfp8_llm_rope_cache, lib.tfp8_llm_attention, lib.tfp8_llm_silu_mul,
                   lib.tfp8_llm_head, lib.tfp8_llm_rope_attention, lib.tfp8_llm_step_in, lib.tfp8_llm_step_out):
            fn.restype = ctypes.c_int
        _LIB = lib
    return _LIB


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _check(rc, what):
    if rc:
        raise RuntimeError(f"{what} failed (rc={rc})")


def _bf16(t, what):
    if t.dtype != torch.bfloat16 or not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{what}: contiguous bfloat16 CUDA tensor expected, got {t.dtype} {t.device}")


def _rows(t, n, what):
    """(rows, row stride) of a bf16 CUDA tensor [..., n] whose rows are contiguous (a contiguous tensor
    or a column slice of one, such as a part of a fused projection's output)."""
    if t.dtype != torch.bfloat16 or not t.is_cuda or t.shape[-1] != n:
        raise ValueError(f"{what}: bfloat16 CUDA tensor [..., {n}] expected, got {t.dtype} {tuple(t.shape)}")
    r = t.reshape(-1, n)
    if r.data_ptr() != t.data_ptr() or (n > 1 and r.stride(1) != 1) or (r.shape[0] > 1 and r.stride(0) < n):
        raise ValueError(f"{what}: rows of {n} contiguous elements expected")
    return r.shape[0], (r.stride(0) if r.shape[0] > 1 else n)


def add_rmsnorm(x, r, weight, eps):
    """(h, y): h = x + r (bf16; h is x when r is None), y = RMSNorm(h) with `weight` (bf16 in and out,
    fp32 inside), over the last dimension."""
    _bf16(x, "x")
    _bf16(weight, "weight")
    d = x.shape[-1]
    if weight.numel() != d:
        raise ValueError(f"weight has {weight.numel()} elements, rows have {d}")
    h = x
    if r is not None:
        _bf16(r, "r")
        if r.shape != x.shape:
            raise ValueError(f"x {tuple(x.shape)} and r {tuple(r.shape)} differ")
        h = torch.empty_like(x)
    y = torch.empty_like(x)
    _check(library().tfp8_llm_add_rmsnorm(x.data_ptr(), r.data_ptr() if r is not None else None,
                                          h.data_ptr() if r is not None else None, y.data_ptr(), weight.data_ptr(),
                                          x.numel() // d, d, float(eps), _stream(x)), "add_rmsnorm")
    return h, y


def rope_cache(q, k, v, cos, sin, kt, vc, pos, n_heads, n_kv):
    """Rotary embedding of one position's q, k (bf16 [B, 1, heads * hd], rows contiguous: column slices
    of one fused projection are taken as they lie) with cos/sin (fp32 [hd / 2]), k and v written
    into the bf16 caches kt [B, n_kv, hd, L] / vc [B, n_kv, L, hd] at position pos (int64 [1] on the
    device); returns the rotated q widened to fp32 [B, n_heads, hd]."""
    B, hd, L = q.shape[0], kt.shape[2], kt.shape[3]
    (bq, ldq), (bk, ldk), (bv, ldv) = _rows(q, n_heads * hd, "q"), _rows(k, n_kv * hd, "k"), _rows(v, n_kv * hd, "v")
    if not bq == bk == bv == B:
        raise ValueError("q/k/v rows do not match the batch")
    if tuple(kt.shape) != (B, n_kv, hd, L) or tuple(vc.shape) != (B, n_kv, L, hd):
        raise ValueError(f"cache shapes {tuple(kt.shape)} / {tuple(vc.shape)}")
    _bf16(kt, "kt")
    _bf16(vc, "vc")
    for t, n in ((cos, "cos"), (sin, "sin")):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{n}: contiguous float32 expected")
    if cos.numel() != hd // 2 or sin.numel() != hd // 2 or pos.dtype != torch.int64 or pos.numel() != 1:
        raise ValueError("cos/sin need hd / 2 values and pos one int64")
    qf = torch.empty(B, n_heads, hd, dtype=torch.float32, device=q.device)
    _check(library().tfp8_llm_rope_cache(q.data_ptr(), k.data_ptr(), v.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                         qf.data_ptr(), kt.data_ptr(), vc.data_ptr(), pos.data_ptr(), B, n_heads, n_kv,
                                         hd, L, ldq, ldk, ldv, _stream(q)), "rope_cache")
    return qf


def attention(qf, kt, vc, pos, n_heads, n_kv):
    """softmax((q . k_t) / sqrt(hd), t <= pos) weighted sum of v_t for every (batch, head), over the
    caches kt [B, n_kv, hd, L] / vc [B, n_kv, L, hd] (bf16); returns bf16 [B, 1, n_heads * hd]."""
    _bf16(kt, "kt")
    _bf16(vc, "vc")
    B, hd, L = qf.shape[0], kt.shape[2], kt.shape[3]
    if tuple(qf.shape) != (B, n_heads, hd) or qf.dtype != torch.float32 or not qf.is_contiguous():
        raise ValueError(f"qf {tuple(qf.shape)} {qf.dtype}")
    S = math.ceil(L / 64)                          # chunks of at most 64 positions (one per lane)
    if S > 256:
        raise ValueError(f"cache of {L} positions: at most {256 * 64}")
    part = torch.empty(B * n_heads * S * (hd + 2), dtype=torch.float32, device=qf.device)
    out = torch.empty(B, 1, n_heads * hd, dtype=torch.bfloat16, device=qf.device)
    _check(library().tfp8_llm_attention(qf.data_ptr(), kt.data_ptr(), vc.data_ptr(), pos.data_ptr(), part.data_ptr(), S,
                                        out.data_ptr(), B, n_heads, n_kv, hd, L, float(math.sqrt(hd)), _stream(qf)),
           "attention")
    return out


def rope_attention(q, k, v, cos, sin, kt, vc, pos, n_heads, n_kv):
    """rope_cache then attention in two kernels instead of three, with the same cache contents and
    the same output bits: q, k, v bf16 [B, 1, heads * hd] rows (slices of one fused projection
    taken as they lie), cos / sin fp32 [hd / 2], the bf16 caches kt [B, n_kv, hd, L] /
    vc [B, n_kv, L, hd] written at pos (int64 [1] on the device); returns bf16 [B, 1, n_heads * hd]."""
    B, hd, L = q.shape[0], kt.shape[2], kt.shape[3]
    (bq, ldq), (bk, ldk), (bv, ldv) = _rows(q, n_heads * hd, "q"), _rows(k, n_kv * hd, "k"), _rows(v, n_kv * hd, "v")
    if not bq == bk == bv == B:
        raise ValueError("q/k/v rows do not match the batch")
    if tuple(kt.shape) != (B, n_kv, hd, L) or tuple(vc.shape) != (B, n_kv, L, hd):
        raise ValueError(f"cache shapes {tuple(kt.shape)} / {tuple(vc.shape)}")
    _bf16(kt, "kt")
    _bf16(vc, "vc")
    for t, n in ((cos, "cos"), (sin, "sin")):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{n}: contiguous float32 expected")
    if cos.numel() != hd // 2 or sin.numel() != hd // 2 or pos.dtype != torch.int64 or pos.numel() != 1:
        raise ValueError("cos/sin need hd / 2 values and pos one int64")
    S = math.ceil(L / 64)
    if S > 256:
        raise ValueError(f"cache of {L} positions: at most {256 * 64}")
    part = torch.empty(B * n_heads * S * (hd + 2), dtype=torch.float32, device=q.device)
    out = torch.empty(B, 1, n_heads * hd, dtype=torch.bfloat16, device=q.device)
    _check(library().tfp8_llm_rope_attention(q.data_ptr(), k.data_ptr(), v.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                             kt.data_ptr(), vc.data_ptr(), pos.data_ptr(), part.data_ptr(), S,
                                             out.data_ptr(), B, n_heads, n_kv, hd, L, ldq, ldk, ldv,
                                             float(math.sqrt(hd)), _stream(q)), "rope_attention")
    return out


def rope_prefill(q, k, v, cos, sin, kt, vc, start, n_heads, n_kv):
    """Rotary embedding of T positions' q, k (bf16 [B, T, heads * hd], rows contiguous: column slices
    of one fused projection are taken as they lie) with cos / sin (fp32, T * hd / 2 values, position
    major), k and v written into the bf16 caches kt [B, n_kv, hd, L] / vc [B, n_kv, L, hd] at
    positions start .. start + T - 1 (a host int); returns the rotated q as bf16 [B, n_heads, T, hd]."""
    B, T = q.shape[0], q.shape[1]
    hd, L = kt.shape[2], kt.shape[3]
    (bq, ldq), (bk, ldk), (bv, ldv) = _rows(q, n_heads * hd, "q"), _rows(k, n_kv * hd, "k"), _rows(v, n_kv * hd, "v")
    if q.dim() != 3 or not bq == bk == bv == B * T:
        raise ValueError("q/k/v rows do not match [B, T]")
    if tuple(kt.shape) != (B, n_kv, hd, L) or tuple(vc.shape) != (B, n_kv, L, hd):
        raise ValueError(f"cache shapes {tuple(kt.shape)} / {tuple(vc.shape)}")
    _bf16(kt, "kt")
    _bf16(vc, "vc")
    for t, n in ((cos, "cos"), (sin, "sin")):
        if t.dtype != torch.float32 or not t.is_contiguous() or t.numel() != T * (hd // 2):
            raise ValueError(f"{n}: contiguous float32 of T * hd / 2 values expected")
    if not 0 <= start <= L - T:
        raise ValueError(f"positions {start} .. {start + T - 1} outside a cache of {L}")
    qo = torch.empty(B, n_heads, T, hd, dtype=torch.bfloat16, device=q.device)
    _check(library().tfp8_llm_rope_prefill(q.data_ptr(), k.data_ptr(), v.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                           qo.data_ptr(), kt.data_ptr(), vc.data_ptr(), int(start), B, T, n_heads,
                                           n_kv, hd, L, ldq, ldk, ldv, _stream(q)), "rope_prefill")
    return qo


def attn_prefill(q, kt, vc, start, n_heads, n_kv):
    """Causal attention of the rotated queries q (bf16 [B, n_heads, T, 128], positions start ..
    start + T - 1) over the bf16 caches kt [B, n_kv, 128, L] / vc [B, n_kv, L, 128] (L % 8 == 0),
    positions 0 .. start + T - 1: softmax((q . k) / sqrt(128), key <= query) times v, fp32 inside;
    returns bf16 [B, T, n_heads * 128] (the rows o_proj takes)."""
    _bf16(q, "q")
    _bf16(kt, "kt")
    _bf16(vc, "vc")
    B, H, T, hd = q.shape
    L = kt.shape[3]
    if H != n_heads or hd != 128 or tuple(kt.shape) != (B, n_kv, hd, L) or tuple(vc.shape) != (B, n_kv, L, hd):
        raise ValueError(f"q {tuple(q.shape)}, caches {tuple(kt.shape)} / {tuple(vc.shape)}")
    if L % 8 or not 0 <= start <= L - T:
        raise ValueError(f"cache of {L} positions (a multiple of 8), positions {start} .. {start + T - 1}")
    out = torch.empty(B, T, H * hd, dtype=torch.bfloat16, device=q.device)
    scale = float(np.float32(1.0) / np.float32(math.sqrt(hd)))     # fp32 reciprocal of the divisor
    _check(library().tfp8_llm_attn_prefill(q.data_ptr(), kt.data_ptr(), vc.data_ptr(), out.data_ptr(), int(start), B,
                                           T, H, n_kv, hd, L, H * hd, scale, _stream(q)), "attn_prefill")
    return out


def silu_mul(g, u):
    """bf16(bf16(silu(g)) * u), elementwise over [..., n] (rows contiguous, with one row stride for
    both: separate tensors or the two halves of one fused projection); returns a new [..., n]."""
    n = g.shape[-1]
    (rg, ldg), (ru, ldu) = _rows(g, n, "g"), _rows(u, n, "u")
    if g.shape != u.shape or rg != ru or (rg > 1 and ldg != ldu):
        raise ValueError(f"g {tuple(g.shape)} and u {tuple(u.shape)} differ in shape or row stride")
    out = torch.empty(g.shape, dtype=g.dtype, device=g.device)
    _check(library().tfp8_llm_silu_mul(g.data_ptr(), u.data_ptr(), out.data_ptr(), rg, n, ldg, _stream(g)), "silu_mul")
    return out


def head(x, weight):
    """Logits fp32 [..., V] = x (bf16 [..., K], at most 16 rows) times weight (bf16 [V, K])
    transposed, with fp32 products and sums: F.linear(x.float(), weight.float()) without widening
    the weight in memory (on the matrix cores)."""
    _bf16(x, "x")
    _bf16(weight, "weight")
    V, K = weight.shape
    if x.shape[-1] != K:
        raise ValueError(f"x {tuple(x.shape)} does not match the weight {tuple(weight.shape)}")
    y = torch.empty(*x.shape[:-1], V, dtype=torch.float32, device=x.device)
    _check(library().tfp8_llm_head(x.data_ptr(), weight.data_ptr(), y.data_ptr(), x.numel() // K, V, K, _stream(x)),
           "head")
    return y


def _i64(t, what, n=None):
    if t.dtype != torch.int64 or not t.is_cuda or not t.is_contiguous() or (n is not None and t.numel() != n):
        raise ValueError(f"{what}: contiguous int64 CUDA tensor{'' if n is None else f' of {n}'} expected")


def step_in(tok, pos, inv, emb):
    """The start of a decode step in one kernel: (x, cos, sin) with x = the embedding rows of tok
    (int64 [B, 1]) as bf16 [B, 1, d] (emb bf16 [V, d]; a token outside the vocabulary gives a zero
    row), and cos / sin fp32 [hd / 2] of the angles pos.float() * inv (pos int64 [1], inv fp32)."""
    B = tok.shape[0]
    _i64(tok, "tok", B)
    _i64(pos, "pos", 1)
    _bf16(emb, "emb")
    if inv.dtype != torch.float32 or not inv.is_contiguous():
        raise ValueError("inv: contiguous float32 expected")
    V, d = emb.shape
    half = inv.numel()
    x = torch.empty(B, 1, d, dtype=torch.bfloat16, device=emb.device)
    cs = torch.empty(half, dtype=torch.float32, device=emb.device)
    sn = torch.empty(half, dtype=torch.float32, device=emb.device)
    _check(library().tfp8_llm_step_in(tok.data_ptr(), pos.data_ptr(), inv.data_ptr(), emb.data_ptr(), x.data_ptr(),
                                      cs.data_ptr(), sn.data_ptr(), B, d, half, V, _stream(emb)), "step_in")
    return x, cs, sn


def step_out(logits, tok, pos):
    """The end of a greedy decode step in one kernel: tok[b] = the index of the first maximum of
    logits[b] (fp32 [B, V], rows contiguous; NaN counts above everything, as in torch.argmax), then
    pos += 1 -- greedy(logits), tok.copy_ and pos.add_(1)."""
    if logits.dtype != torch.float32 or not logits.is_cuda or logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits: float32 CUDA tensor [B, V] with contiguous rows expected")
    B, V = logits.shape
    _i64(tok, "tok", B)
    _i64(pos, "pos", 1)
    _check(library().tfp8_llm_step_out(logits.data_ptr(), B, V, logits.stride(0), tok.data_ptr(), pos.data_ptr(),
                                       _stream(logits)), "step_out")
