"""Llama-style decoder on the FP8 W8A16 path versus native bf16 (reference tfp8/examples/demo_llm.py).

    python -m tfp8.examples.demo_llm --size c5      # 8 layers, d=2048, 16 heads, FFN 5632, vocab 32000
    python -m tfp8.examples.demo_llm --size tiny    # 2 layers, seconds

The model is built here (random N(0, 0.02) init, tied embedding / output head), converted with
prepare_model(profile="llm_safe"), and measured the way the reference demo measures it: logits
agreement with the bf16 model (cosine, relative L2, top-1), prefill and per-token decode latency,
and the FP8Linear path counters.  Layout choices for the GPU:
  * the KV cache is preallocated in the model's dtype and written in place, keys as [B, heads,
    head_dim, max_len] and values as [B, heads, max_len, head_dim], so the fused attention reads
    both as they lie (no transposed copy of the keys); the PyTorch forms widen what they read;
  * attention runs in fp32 (scores, causal mask, softmax, values);
  * the tied output head computes F.linear(x.float(), embedding.float()) (demo_llm.py:127) from
    the bf16 embedding itself on the GPU: bf16 x bf16 products are exact in fp32, so a bf16 GEMM
    with fp32 sums and fp32 output (torch.mm out_dtype) gives it in another summation order; on
    the CPU, or for other dtypes, one fp32 copy of the embedding is kept (the reference re-widens
    it on every call);
  * decoding can be replayed from one captured HIP graph (GraphDecoder): the step has static
    shapes -- the position is a device tensor that drives the rotary angles, the KV-cache write and
    the attention mask over the whole (zero-filled) cache -- and the greedy token and the position
    are updated on the device, so a token costs one graph launch instead of Python's kernel
    launches.  Prefill (static shape for a given prompt length) is captured the same way for the
    latency figure;
  * on the GPU the decode step runs the work between the FP8 linears as fused ops (llm_ops.hip:
    residual add + RMSNorm, rotary + cache write, split-sequence attention, SiLU * up, and for up
    to 16 rows the tied head straight from the bf16 embedding), with q/k/v and gate/up each as one
    FP8Linear: about 10 kernels per layer where the PyTorch form of the same step
    (decode_step(fused=False), also the CPU path) launches about 60.
"""
import argparse
import math
import statistics
import time

import torch
import torch.nn as nn
import torch.nn.functional as F

SIZES = {
    "tiny": dict(dim=1024, n_layers=2, n_heads=8, n_kv=8, ffn=2816, vocab=8192),
    "c5": dict(dim=2048, n_layers=8, n_heads=16, n_kv=16, ffn=5632, vocab=32000),
}


class RMSNorm(nn.Module):
    def __init__(self, d, eps=1e-5):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d))
        self.eps = eps

    def forward(self, x):
        xf = x.float()
        inv = torch.rsqrt(xf.square().mean(-1, keepdim=True) + self.eps)
        return (xf * inv * self.weight.float()).to(x.dtype)


def _rotary(x, cos, sin):
    """Rotate the two halves of the head dimension: x = [x1, x2] -> [x1 c - x2 s, x2 c + x1 s]."""
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h].float(), x[..., h:].float()
    return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], -1).to(x.dtype)


class Attention(nn.Module):
    def __init__(self, c):
        super().__init__()
        self.nh, self.nkv = c["n_heads"], c["n_kv"]
        self.hd = c["dim"] // c["n_heads"]
        d = c["dim"]
        self.q_proj = nn.Linear(d, self.nh * self.hd, bias=False)
        self.k_proj = nn.Linear(d, self.nkv * self.hd, bias=False)
        self.v_proj = nn.Linear(d, self.nkv * self.hd, bias=False)
        self.o_proj = nn.Linear(self.nh * self.hd, d, bias=False)

    def forward(self, x, cos, sin, cache, start):
        B, T, _ = x.shape
        q = _rotary(self.q_proj(x).view(B, T, self.nh, self.hd), cos, sin)
        k = _rotary(self.k_proj(x).view(B, T, self.nkv, self.hd), cos, sin)
        v = self.v_proj(x).view(B, T, self.nkv, self.hd)
        kt, vc = cache
        kt[:, :, :, start:start + T] = k.permute(0, 2, 3, 1)
        vc[:, :, start:start + T] = v.transpose(1, 2)
        return self.attend(q.transpose(1, 2), kt, vc, start)

    def attend(self, q, kt, vc, start):
        """Causal attention of the rotated queries q [B, H, T, hd] (positions start .. start + T - 1)
        over cache positions 0 .. start + T - 1, then o_proj; returns [B, T, dim] in q's dtype.  On
        the GPU (bf16, hd = 128, a cache length that is a multiple of 8) one flash-attention kernel
        (llm_ops.attn_prefill) computes what attend_torch does with about 15 PyTorch kernels."""
        if q.is_cuda and q.dtype == kt.dtype == torch.bfloat16 and self.hd == 128 and kt.shape[3] % 8 == 0:
            from tfp8.examples import llm_ops as ops
            return self.o_proj(ops.attn_prefill(q.contiguous(), kt, vc, start, self.nh, self.nkv))
        return self.attend_torch(q, kt, vc, start)

    def attend_torch(self, q, kt, vc, start):
        """attend as PyTorch ops: fp32 scores (bf16 q . k products with fp32 sums on the GPU), the
        causal mask, fp32 softmax and fp32 value product."""
        B, _, T, _ = q.shape
        L = start + T
        rep = self.nh // self.nkv
        vals = vc[:, :, :L].float()                                           # [B, Hkv, L, hd]
        if rep > 1:
            vals = vals.repeat_interleave(rep, 1)
        if q.is_cuda and q.dtype == torch.bfloat16 and kt.dtype == torch.bfloat16:
            # q . k of bf16 values: exact products, so a bf16 batched product with fp32 sums and fp32
            # output equals the fp32 product of the widened operands up to summation order
            keys_t = kt[:, :, :, :L]
            if rep > 1:
                keys_t = keys_t.repeat_interleave(rep, 1)
            keys_t = keys_t.reshape(B * self.nh, self.hd, L).contiguous()
            qb = q.reshape(B * self.nh, T, self.hd).contiguous()
            scores = torch.bmm(qb, keys_t, out_dtype=torch.float32).view(B, self.nh, T, L) / math.sqrt(self.hd)
        else:
            keys_t = kt[:, :, :, :L].float()                                  # [B, Hkv, hd, L]
            if rep > 1:
                keys_t = keys_t.repeat_interleave(rep, 1)
            qf = q.float().contiguous()                                       # [B, H, T, hd]
            scores = torch.matmul(qf, keys_t) / math.sqrt(self.hd)
        if T > 1:
            qpos = torch.arange(start, L, device=q.device)[:, None]
            kpos = torch.arange(L, device=q.device)[None, :]
            scores = scores.masked_fill(kpos > qpos, float("-inf"))
        o = torch.matmul(torch.softmax(scores, -1), vals)                       # [B, H, T, hd]
        return self.o_proj(o.transpose(1, 2).reshape(B, T, self.nh * self.hd).to(q.dtype))

    def forward_static(self, x, cos, sin, cache, pos, kpos):
        """One decode position with static shapes: x [B, 1, d], pos int64 [1] on the device, kpos =
        arange(max_len).  The cache row at pos is written with index_copy_ and attention covers the
        whole cache, positions past pos masked (cache rows past pos must be finite: zero-filled)."""
        B, T, _ = x.shape
        q = _rotary(self.q_proj(x).view(B, T, self.nh, self.hd), cos, sin)
        k = _rotary(self.k_proj(x).view(B, T, self.nkv, self.hd), cos, sin)
        v = self.v_proj(x).view(B, T, self.nkv, self.hd)
        kt, vc = cache
        kt.index_copy_(3, pos, k.permute(0, 2, 3, 1))
        vc.index_copy_(2, pos, v.transpose(1, 2))
        rep = self.nh // self.nkv
        keys_t, vals = kt.float(), vc.float()
        if rep > 1:
            keys_t, vals = keys_t.repeat_interleave(rep, 1), vals.repeat_interleave(rep, 1)
        qf = q.transpose(1, 2).float().contiguous()                          # [B, H, 1, hd]
        scores = torch.matmul(qf, keys_t) / math.sqrt(self.hd)
        scores = scores.masked_fill(kpos > pos, float("-inf"))
        o = torch.matmul(torch.softmax(scores, -1), vals)
        return self.o_proj(o.transpose(1, 2).reshape(B, T, self.nh * self.hd).to(x.dtype))


class MLP(nn.Module):
    def __init__(self, c):
        super().__init__()
        self.gate_proj = nn.Linear(c["dim"], c["ffn"], bias=False)
        self.up_proj = nn.Linear(c["dim"], c["ffn"], bias=False)
        self.down_proj = nn.Linear(c["ffn"], c["dim"], bias=False)

    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class Block(nn.Module):
    def __init__(self, c):
        super().__init__()
        self.input_layernorm = RMSNorm(c["dim"])
        self.self_attn = Attention(c)
        self.post_attention_layernorm = RMSNorm(c["dim"])
        self.mlp = MLP(c)

    def forward(self, x, cos, sin, cache, start):
        x = x + self.self_attn(self.input_layernorm(x), cos, sin, cache, start)
        return x + self.mlp(self.post_attention_layernorm(x))

    def forward_static(self, x, cos, sin, cache, pos, kpos):
        x = x + self.self_attn.forward_static(self.input_layernorm(x), cos, sin, cache, pos, kpos)
        return x + self.mlp(self.post_attention_layernorm(x))


class Llama(nn.Module):
    def __init__(self, c):
        super().__init__()
        self.c = c
        self.embed = nn.Embedding(c["vocab"], c["dim"])
        self.layers = nn.ModuleList(Block(c) for _ in range(c["n_layers"]))
        self.norm = RMSNorm(c["dim"])
        self.lm_head = nn.Linear(c["dim"], c["vocab"], bias=False)
        self.lm_head.weight = self.embed.weight                 # tied: the planner keeps it out of FP8
        for m in self.modules():
            if isinstance(m, (nn.Linear, nn.Embedding)):
                nn.init.normal_(m.weight, std=0.02)
        self._head32 = None

    def new_cache(self, B, max_len, zero=False):
        """Per layer (keys [B, n_kv, head_dim, max_len], values [B, n_kv, max_len, head_dim]) in the
        model's dtype."""
        c, p = self.c, self.embed.weight
        hd = c["dim"] // c["n_heads"]
        new = torch.zeros if zero else torch.empty
        return [(new(B, c["n_kv"], hd, max_len, dtype=p.dtype, device=p.device),
                 new(B, c["n_kv"], max_len, hd, dtype=p.dtype, device=p.device)) for _ in self.layers]

    def _rope(self, start, T, device):
        hd = self.c["dim"] // self.c["n_heads"]
        inv = 1.0 / (10000.0 ** (torch.arange(0, hd // 2, device=device, dtype=torch.float32) * 2.0 / hd))
        ang = torch.arange(start, start + T, device=device, dtype=torch.float32)[:, None] * inv[None, :]
        return ang.cos()[None, :, None, :], ang.sin()[None, :, None, :]

    def _logits(self, y):
        """F.linear(y.float(), embedding.float()) for the normed hidden state y [..., dim]."""
        w = self.embed.weight
        if y.is_cuda and y.dtype == torch.bfloat16 and w.dtype == torch.bfloat16:
            flat = torch.mm(y.reshape(-1, y.shape[-1]), w.t(), out_dtype=torch.float32)
            return flat.reshape(*y.shape[:-1], w.shape[0])
        if self._head32 is None or self._head32.device != y.device:
            self._head32 = w.detach().float()
        return F.linear(y.float(), self._head32)

    def _head(self, x):
        return self._logits(self.norm(x))

    def forward(self, ids, cache, start=0):
        """Logits (fp32) for every position of ids [B, T], appending to cache at `start`."""
        cos, sin = self._rope(start, ids.shape[1], ids.device)
        x = self.embed(ids)
        if x.is_cuda and x.dtype == torch.bfloat16:
            return self._forward_fused(x, cos, sin, cache, start)
        for layer, kv in zip(self.layers, cache):
            x = layer(x, cos, sin, kv, start)
        return self._head(x)

    def _forward_fused(self, x, cos, sin, cache, start):
        """forward with the work between the linears as llm_ops (one kernel each, with the PyTorch
        form's roundings, as in the decode step): residual add + RMSNorm, rotary + cache write
        (rope_prefill), SiLU * up; q/k/v and gate/up run as one fused FP8Linear each where the
        layers allow it (the same row products as the separate layers; a GEMM may sum them in
        another order).  Each block's residual adds ride in the next norm; the causal attention
        itself is Attention.attend."""
        from tfp8.examples import llm_ops as ops
        H, Hkv, ffn = self.c["n_heads"], self.c["n_kv"], self.c["ffn"]
        nq, nk = self.c["dim"], Hkv * (self.c["dim"] // H)
        cs, sn = cos.contiguous(), sin.contiguous()
        r = None
        for layer, (kt, vc), (qkv, gate_up) in zip(self.layers, cache, self._fused_projections()):
            at, mlp, n1, n2 = layer.self_attn, layer.mlp, layer.input_layernorm, layer.post_attention_layernorm
            x, y = ops.add_rmsnorm(x, r, n1.weight, n1.eps)
            if qkv is not None:
                o = qkv(y)
                q, k, v = o[..., :nq], o[..., nq:nq + nk], o[..., nq + nk:]
            else:
                q, k, v = at.q_proj(y), at.k_proj(y), at.v_proj(y)
            q = ops.rope_prefill(q, k, v, cs, sn, kt, vc, start, H, Hkv)
            x, y = ops.add_rmsnorm(x, at.attend(q, kt, vc, start), n2.weight, n2.eps)
            if gate_up is not None:
                o = gate_up(y)
                g, u = o[..., :ffn], o[..., ffn:]
            else:
                g, u = mlp.gate_proj(y), mlp.up_proj(y)
            r = mlp.down_proj(ops.silu_mul(g, u))
        _, y = ops.add_rmsnorm(x, r, self.norm.weight, self.norm.eps)
        return self._logits(y)

    def decode_step(self, tok, cache, pos, kpos, fused=None):
        """One greedy decode step with static shapes and device-resident state (capturable in a
        HIP graph): consumes tok [B, 1] at position pos (int64 [1]), returns the logits [B, 1, V],
        writes the next greedy token into tok and advances pos.  pos must be below the cache
        length: it indexes the cache write on the device (GraphDecoder checks it on the host).
        fused (default: on CUDA tensors) runs the work between the FP8 linears as the fused ops of
        llm_ops (one kernel each); fused=False runs the same step as PyTorch ops."""
        hd = self.c["dim"] // self.c["n_heads"]
        inv = self.__dict__.get("_rope_inv")             # the angles' frequencies, computed once per device
        if inv is None or inv.device != tok.device:
            inv = 1.0 / (10000.0 ** (torch.arange(0, hd // 2, device=tok.device, dtype=torch.float32) * 2.0 / hd))
            self.__dict__["_rope_inv"] = inv
        if tok.is_cuda if fused is None else fused:
            from tfp8.examples import llm_ops as ops
            x, cos, sin = ops.step_in(tok, pos, inv, self.embed.weight)     # embedding rows, rotary angles
            logits = self._decode_fused(x, cos, sin, cache, pos)
            ops.step_out(logits[:, -1], tok, pos)                           # greedy token, pos + 1
            return logits
        ang = pos.float()[:, None] * inv[None, :]
        cos, sin = ang.cos()[None, :, None, :], ang.sin()[None, :, None, :]   # [1, 1, 1, hd / 2]
        x = self.embed(tok)
        for layer, kv in zip(self.layers, cache):
            x = layer.forward_static(x, cos, sin, kv, pos, kpos)
        logits = self._head(x)
        tok.copy_(greedy(logits[:, -1]))
        pos.add_(1)
        return logits

    def _fused_projections(self):
        """Per layer (qkv, gate_up): one FP8Linear over the rows of q/k/v_proj and one over those of
        gate/up_proj, for the decode step -- the codes and scales are the separate layers' rows, so
        every output is the same row product, in two GEMV launches instead of five.  None where the
        layers are not FP8Linear of one layout.  The separate layers' buffers become views of the
        fused ones (one copy of the weights; writes into either are seen by both).  Rebuilt when a
        layer or one of its buffers is replaced; the first decode step builds them (GraphDecoder's
        warm-up steps, outside graph capture)."""
        srcs = [(l.self_attn.q_proj, l.self_attn.k_proj, l.self_attn.v_proj, l.mlp.gate_proj, l.mlp.up_proj)
                for l in self.layers]

        def key():
            return tuple((id(m), *(b.data_ptr() for b in m._buffers.values() if b is not None), id(m._parameters.get("weight")))
                         for t in srcs for m in t)
        if self.__dict__.get("_fused_key") != key():      # kept in __dict__: not registered as submodules
            self.__dict__["_fused_proj"] = [(_concat_fp8(t[:3]), _concat_fp8(t[3:])) for t in srcs]
            self.__dict__["_fused_key"] = key()
        return self.__dict__["_fused_proj"]

    def _decode_fused(self, x, cos, sin, cache, pos):
        """The layers and the head of decode_step with llm_ops between the FP8 linears: per layer
        residual add + RMSNorm, q/k/v projection (one fused FP8Linear), rotary + cache write +
        attention (one op), o_proj, residual add + RMSNorm, gate/up projection (one fused FP8Linear), SiLU * up,
        down_proj (the block's residual adds ride in the next norm)."""
        from tfp8.examples import llm_ops as ops
        H, Hkv, ffn = self.c["n_heads"], self.c["n_kv"], self.c["ffn"]
        nq, nk = self.c["dim"], Hkv * (self.c["dim"] // H)
        r = None
        for layer, (kt, vc), (qkv, gate_up) in zip(self.layers, cache, self._fused_projections()):
            at, mlp, n1, n2 = layer.self_attn, layer.mlp, layer.input_layernorm, layer.post_attention_layernorm
            x, y = ops.add_rmsnorm(x, r, n1.weight, n1.eps)
            if qkv is not None:
                o = qkv(y)
                q, k, v = o[..., :nq], o[..., nq:nq + nk], o[..., nq + nk:]
            else:
                q, k, v = at.q_proj(y), at.k_proj(y), at.v_proj(y)
            o = ops.rope_attention(q, k, v, cos, sin, kt, vc, pos, H, Hkv)
            x, y = ops.add_rmsnorm(x, at.o_proj(o), n2.weight, n2.eps)
            if gate_up is not None:
                o = gate_up(y)
                g, u = o[..., :ffn], o[..., ffn:]
            else:
                g, u = mlp.gate_proj(y), mlp.up_proj(y)
            r = mlp.down_proj(ops.silu_mul(g, u))
        _, y = ops.add_rmsnorm(x, r, self.norm.weight, self.norm.eps)
        if y.shape[0] <= 16:         # the decode-size head kernel; more rows: the bf16 GEMM
            return ops.head(y, self.embed.weight)
        return self._logits(y)


def _concat_fp8(mods):
    """One FP8Linear whose output rows are those of `mods` in order (FP8Linear layers with one input
    size, format, group size, scale storage and output dtype, no bias, not backed off), or None."""
    from tfp8.linear import FP8Linear
    f0 = mods[0]
    if not all(isinstance(f, FP8Linear) and f.fallback is None and f.bias_f32 is None
               and (f.in_features, f.fmt, f.group_size, f.scale_format, f.out_dtype)
               == (f0.in_features, f0.fmt, f0.group_size, f0.scale_format, f0.out_dtype) for f in mods):
        return None
    with torch.no_grad():
        q = torch.cat([f.qweight for f in mods])
        s = torch.cat([f.weight_scale for f in mods])
    fused = FP8Linear.from_fp8_checkpoint(q, s, None, f0.fmt, out_dtype=f0.out_dtype, nan_check=f0.nan_check)
    n0 = 0
    for f in mods:                      # the layers' buffers become row ranges of the fused ones
        n1 = n0 + f.out_features
        f.qweight, f.weight_scale = fused.qweight[n0:n1], fused.weight_scale[n0:n1]
        n0 = n1
    return fused


def greedy(logits):
    """argmax over the last dim of [B, V] logits as [B, 1], first maximum on ties (as torch.argmax).
    Two levels of per-row reductions (128-wide chunks, then the chunk maxima), so that no
    reduction spans thread blocks: such reductions clear a counter with a memset node, which has
    given wrong results on graph replays after the first."""
    B, V = logits.shape
    if V % 128:
        return logits.argmax(-1, keepdim=True)
    cmax, cidx = logits.view(B, V // 128, 128).max(-1)                      # per chunk
    c = cmax.argmax(-1, keepdim=True)                                       # first chunk holding the max
    return c * 128 + cidx.gather(1, c)


class GraphDecoder:
    """Greedy decoding replayed from one captured HIP graph (torch.cuda.CUDAGraph) per batch size:
    the graph holds the whole decode step of Llama.decode_step, its KV cache, token and position
    are static device tensors, and the prompt is prefilled eagerly into the same cache."""

    def __init__(self, model, B, max_len):
        dev = model.embed.weight.device
        self.model, self.B, self.max_len = model, B, max_len
        self.cache = model.new_cache(B, max_len, zero=True)
        self.tok = torch.zeros(B, 1, dtype=torch.long, device=dev)
        self.pos = torch.zeros(1, dtype=torch.long, device=dev)
        self.kpos = torch.arange(max_len, device=dev)
        self.graph = self.logits = None
        self.next_pos = 0          # host mirror of pos: a step writes cache row pos, so pos < max_len

    @torch.no_grad()
    def capture(self):
        # Warm-up outside the capture: FP8Linear checks its first outputs on the host, and the
        # libraries pick their kernels; then the state is cleared.
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(3):         # positions 0..2, inside the cache (reset below)
                self.model.decode_step(self.tok, self.cache, self.pos, self.kpos)
        torch.cuda.current_stream().wait_stream(s)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = self.model.decode_step(self.tok, self.cache, self.pos, self.kpos)
        self.reset()
        return self

    def reset(self):
        for kc, vc in self.cache:
            kc.zero_()
            vc.zero_()
        self.pos.zero_()
        self.tok.zero_()
        self.next_pos = 0

    def rewind(self, pos):
        """Continue decoding from position pos (cache rows from pos on are overwritten)."""
        if not 0 <= pos < self.max_len:
            raise ValueError(f"position {pos} outside the cache (max_len {self.max_len})")
        self.pos.fill_(pos)
        self.next_pos = pos

    @torch.no_grad()
    def prefill(self, prompt):
        """Eager prefill of prompt [B, T] into the cache; leaves the first greedy token in tok."""
        if prompt.shape[1] >= self.max_len:
            raise ValueError(f"prompt of {prompt.shape[1]} tokens leaves no room in the cache (max_len {self.max_len})")
        self.reset()
        logits = self.model(prompt, self.cache, 0)
        self.tok.copy_(greedy(logits[:, -1]))
        self.rewind(prompt.shape[1])
        return logits

    def step(self):
        """One decode step (one graph launch): returns the step's logits [B, 1, V] (overwritten by
        the next step) and leaves the next token in self.tok.  Raises once the cache is full: the
        step writes cache row pos, and the graph cannot check that on the device."""
        if self.next_pos >= self.max_len:
            raise RuntimeError(f"KV cache full ({self.max_len} positions)")
        self.graph.replay()
        self.next_pos += 1
        return self.logits


def build(size="c5", dtype=torch.bfloat16, device="cuda", seed=0):
    torch.manual_seed(seed)
    return Llama(dict(SIZES[size])).to(device=device, dtype=dtype)


@torch.no_grad()
def generate(model, prompt, n_new):
    """Greedy decode: prefill the prompt, then n_new single-token steps on the KV cache.
    Returns (tokens [B, n_new], prefill logits [B, T, V], step logits [B, n_new, V])."""
    B, T = prompt.shape
    cache = model.new_cache(B, T + n_new)
    logits = model(prompt, cache, 0)
    nxt = logits[:, -1].argmax(-1, keepdim=True)
    toks, steps = [nxt], [logits[:, -1]]
    for i in range(1, n_new):
        lg = model(nxt, cache, T + i - 1)[:, -1]
        nxt = lg.argmax(-1, keepdim=True)
        toks.append(nxt)
        steps.append(lg)
    return torch.cat(toks, 1), logits, torch.stack(steps, 1)


def agreement(ref, got):
    """cosine (mean over positions), relative L2 and top-1 agreement of two logit tensors."""
    r, g = ref.reshape(-1, ref.shape[-1]).float(), got.reshape(-1, got.shape[-1]).float()
    cos = F.cosine_similarity(r, g, dim=-1).mean().item()
    rel = ((g - r).norm() / r.norm()).item()
    top1 = (r.argmax(-1) == g.argmax(-1)).float().mean().item()
    return cos, rel, top1


def _median_ms(fn, n):
    ts = []
    for _ in range(n):
        torch.cuda.synchronize()
        t = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        ts.append((time.perf_counter() - t) * 1e3)
    return statistics.median(ts)


@torch.no_grad()
def timings(model, B, prompt_len, n_decode, vocab, graphs=True):
    """Eager prefill and per-token decode latency (ms); with graphs also the prefill and decode
    replayed from captured HIP graphs.  Returns (prefill, decode) or (prefill, decode,
    prefill_graph, decode_graph)."""
    ids = torch.randint(0, vocab, (B, prompt_len), device="cuda")
    cache = model.new_cache(B, prompt_len + n_decode + 8)
    for _ in range(3):
        model(ids, cache, 0)
    prefill = _median_ms(lambda: model(ids, cache, 0), 5)
    tok = ids[:, -1:]
    model(tok, cache, prompt_len)

    def steps():
        for i in range(n_decode):
            model(tok, cache, prompt_len + i)
    per_tok = _median_ms(steps, 3) / n_decode
    if not graphs:
        return prefill, per_tok
    pg = torch.cuda.CUDAGraph()
    with torch.cuda.graph(pg):
        model(ids, cache, 0)
    prefill_g = _median_ms(pg.replay, 5)
    dec = GraphDecoder(model, B, prompt_len + n_decode + 8).capture()
    dec.prefill(ids)

    def gsteps():                   # every timed run decodes the same n_decode positions
        dec.rewind(prompt_len)
        for _ in range(n_decode):
            dec.step()
    gsteps()
    per_tok_g = _median_ms(gsteps, 3) / n_decode
    return prefill, per_tok, prefill_g, per_tok_g


def run(size="c5", prompt_len=512, n_decode=128, batches=(1, 8)):
    from tfp8 import FP8Config, prepare_model
    from tfp8.linear import FP8Linear
    from tfp8.planner import weight_bytes

    c = SIZES[size]
    model = build(size)
    ids = torch.randint(0, c["vocab"], (1, prompt_len), device="cuda", generator=torch.Generator("cuda").manual_seed(1))
    with torch.no_grad():
        ref = model(ids, model.new_cache(1, prompt_len), 0)
    base_t = {}
    for B in batches:
        print(f"[demo] timing the bf16 model at B={B}", flush=True)
        base_t[B] = timings(model, B, prompt_len, n_decode, c["vocab"])
    bf16_mb = sum(weight_bytes(model).values()) / 2**20
    prepare_model(model, "llm", FP8Config(profile="llm_safe", fmt="e4m3fn", weight_group=None, nan_check=True))
    fp8_mb = sum(weight_bytes(model).values()) / 2**20
    with torch.no_grad():
        got = model(ids, model.new_cache(1, prompt_len), 0)
    cos, rel, top1 = agreement(ref, got)
    print(f"model {size}: {c}")
    print(f"weights+state bf16 {bf16_mb:.1f} MB -> fp8 {fp8_mb:.1f} MB")
    print(f"logits vs bf16: cosine {cos:.6f}  relative L2 {rel:.4f}  top-1 {100 * top1:.2f}%")
    for B in batches:
        print(f"[demo] timing the FP8 model at B={B}", flush=True)
        p, d, pg, dg = timings(model, B, prompt_len, n_decode, c["vocab"])
        pb, db, pgb, dgb = base_t[B]
        print(f"B={B}: prefill {prompt_len} tok {p:8.2f} ms (bf16 {pb:8.2f})  decode/token {d:7.3f} ms (bf16 {db:7.3f})  "
              f"-> {B * prompt_len / p * 1e3:9.0f} prefill tok/s, {B / d * 1e3:8.0f} decode tok/s")
        print(f"B={B} HIP graphs: prefill {pg:8.2f} ms (bf16 {pgb:8.2f})  decode/token {dg:7.3f} ms (bf16 {dgb:7.3f})  "
              f"-> {B * prompt_len / pg * 1e3:9.0f} prefill tok/s, {B / dg * 1e3:8.0f} decode tok/s")
    paths = {}
    for m in model.modules():
        if isinstance(m, FP8Linear):
            for k, v in m.stats.items():
                paths[k] = paths.get(k, 0) + v
    print(f"FP8Linear paths: {paths}")
    return dict(cos=cos, rel=rel, top1=top1)


@torch.no_grad()
def graph_decode(size="c5", B=1, prompt_len=512, n_decode=128):
    """Only the FP8 model's HIP-graph decode (for kernel profiles): convert, capture, prefill, then
    n_decode replayed steps; returns ms per token."""
    from tfp8 import FP8Config, prepare_model
    model = build(size)
    prepare_model(model, "llm", FP8Config(profile="llm_safe", fmt="e4m3fn"))
    ids = torch.randint(0, model.c["vocab"], (B, prompt_len), device="cuda", generator=torch.Generator("cuda").manual_seed(1))
    dec = GraphDecoder(model, B, prompt_len + n_decode).capture()
    dec.prefill(ids)
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(n_decode):
        dec.step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t) * 1e3 / n_decode
    print(f"{size} B={B}: graph decode {ms:.3f} ms per token over {n_decode} steps after a {prompt_len}-token prompt")
    return ms


def prefill_only(size="c5", B=1, prompt_len=512, reps=5):
    """Only the FP8 model's eager prefill (for kernel profiles): convert, 4 warm-up forwards (past
    the NaN-watched first calls of every layer), then `reps` timed forwards; returns ms each."""
    from tfp8 import FP8Config, prepare_model
    model = build(size)
    prepare_model(model, "llm", FP8Config(profile="llm_safe", fmt="e4m3fn"))
    ids = torch.randint(0, model.c["vocab"], (B, prompt_len), device="cuda", generator=torch.Generator("cuda").manual_seed(1))
    cache = model.new_cache(B, prompt_len + 8)
    with torch.no_grad():
        for _ in range(4):
            model(ids, cache, 0)
        torch.cuda.synchronize()
        t = time.perf_counter()
        for _ in range(reps):
            model(ids, cache, 0)
        torch.cuda.synchronize()
    ms = (time.perf_counter() - t) * 1e3 / reps
    print(f"{size} B={B}: eager prefill {ms:.3f} ms over {reps} forwards of {prompt_len} tokens")
    return ms


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--size", default="c5", choices=list(SIZES))
    ap.add_argument("--prompt-len", type=int, default=512)
    ap.add_argument("--decode", type=int, default=128)
    ap.add_argument("--graph-decode", type=int, default=None, metavar="B",
                    help="only time the FP8 model's graph decode at batch B (for kernel profiles)")
    ap.add_argument("--prefill", type=int, default=None, metavar="B",
                    help="only time the FP8 model's eager prefill at batch B (for kernel profiles)")
    a = ap.parse_args()
    if a.prefill:
        prefill_only(a.size, a.prefill, a.prompt_len)
    elif a.graph_decode:
        graph_decode(a.size, a.graph_decode, a.prompt_len, a.decode)
    else:
        run(a.size, a.prompt_len, a.decode)
