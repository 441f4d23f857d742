"""C5 end to end: the Llama-style decoder (8 layers, d=2048, 16 heads, SwiGLU 5632, vocab 32000,
random N(0, 0.02) init) converted by prepare_model to E4M3FN per-channel FP8Linear, prefilled with
512 tokens and greedily decoded for 128 at batch 1 and batch 8 (benchmark configuration C5).

Parity: the same model with every FP8Linear replaced by the reference's CPU forward arithmetic
(tfp8/linear.py:179-181: fp32 F.linear of the dequantized weight, evaluated as an fp32 GPU matmul)
is run teacher-forced over prompt + generated tokens, and every prefill and decode-step logit row
is compared.  Both models round each projection to bf16, so they differ by bf16 rounding flips
that propagate through 8 layers.  The bound is calibrated on that noise: a second reference that
only changes the fp32 summation order (each projection summed over two K halves) sets the floor,
and the FP8 model must stay within twice the floor's relative L2 and cosine distance, and within
3 points of its top-1 agreement (plus absolute bounds: cosine >= 0.999, top-1 >= 90 %).
One projection is also checked on its live inputs against the float64 oracle with the per-linear
tolerance of the other GPU tests.  Quality versus the bf16 model (the reference demo's metric,
demo_llm.py:176-185) is reported.
"""
import contextlib

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import cpu_path
from oracle import fp8_oracle as O
from tfp8 import FP8Config, prepare_model
from tfp8.examples import demo_llm
from tfp8.linear import FP8Linear

pytestmark = pytest.mark.gpu

COS_ABS, TOP1_ABS = 0.999, 0.90


class RefLinear(nn.Module):
    """The reference CPU forward of one FP8Linear, with its weight dequantized once."""

    def __init__(self, f):
        super().__init__()
        self.W = cpu_path.dequant_weight_f32(f.qweight, f.weight_scale, f.group_size, f.fmt)
        self.b = f.bias_f32
        self.out_dtype = f.out_dtype

    def forward(self, x):
        return cpu_path.ref_linear(x, self.W, self.b, self.out_dtype)


class RefLinearSplitK(RefLinear):
    """The same arithmetic with another fp32 summation order: two K halves added at the end."""

    def __init__(self, f):
        super().__init__(f)
        h = self.W.shape[1] // 2
        self.lo, self.hi = self.W[:, :h].t().contiguous(), self.W[:, h:].t().contiguous()

    def forward(self, x):
        h = self.lo.shape[0]
        xf = x.float()
        y = (xf[..., :h] @ self.lo) + (xf[..., h:] @ self.hi)
        if self.b is not None:
            y = y + self.b
        return y.to(self.out_dtype)


@contextlib.contextmanager
def swapped(model, table):
    old = {}
    for name, new in table.items():
        parent_name, leaf = name.rsplit(".", 1)
        parent = model.get_submodule(parent_name)
        old[name] = getattr(parent, leaf)
        setattr(parent, leaf, new)
    try:
        yield
    finally:
        for name, mod in old.items():
            parent_name, leaf = name.rsplit(".", 1)
            setattr(model.get_submodule(parent_name), leaf, mod)


def test_c5_prefill_and_greedy_decode():
    T, NEW = 512, 128
    model = demo_llm.build("c5")
    c = model.c
    g = torch.Generator("cuda").manual_seed(7)
    prompts = {B: torch.randint(0, c["vocab"], (B, T), device="cuda", generator=g) for B in (1, 8)}
    with torch.no_grad():
        base = model(prompts[1], model.new_cache(1, T), 0)

    prepare_model(model, "llm", FP8Config(profile="llm_safe", fmt="e4m3fn"))
    fp8 = {n: m for n, m in model.named_modules() if isinstance(m, FP8Linear)}
    assert len(fp8) == 7 * c["n_layers"]
    reasons = {d.name: d.reason for d in model._tfp8_plan}
    assert reasons["lm_head"] == "weight shared with another module (tied)"
    ref = {n: RefLinear(m) for n, m in fp8.items()}
    ref2 = {n: RefLinearSplitK(m) for n, m in fp8.items()}

    # live inputs of one projection, for the per-linear oracle check
    probe_name = "layers.5.mlp.down_proj"
    seen = []
    hook = fp8[probe_name].register_forward_hook(lambda m, i, o: seen.append((i[0].detach(), o.detach())))
    for B in (1, 8):
        print(f"[c5] B={B}: prefill {T} + greedy {NEW}", flush=True)
        toks, pre, steps = demo_llm.generate(model, prompts[B], NEW)
        full = torch.cat([prompts[B], toks[:, :-1]], 1)
        with torch.no_grad():
            with swapped(model, ref):
                rl = model(full, model.new_cache(B, full.shape[1]), 0)
            with swapped(model, ref2):
                rl2 = model(full, model.new_cache(B, full.shape[1]), 0)
        for label, sl in (("prefill", slice(0, T)), ("decode", slice(T - 1, None))):
            got = pre if label == "prefill" else steps
            fc, fr, ft = demo_llm.agreement(rl[:, sl], got)
            nc, nr, nt = demo_llm.agreement(rl[:, sl], rl2[:, sl])
            print(f"[c5] B={B} {label}: fp8 vs ref cosine {fc:.7f} rel L2 {fr:.2e} top-1 {100 * ft:.2f}% | "
                  f"noise floor cosine {nc:.7f} rel L2 {nr:.2e} top-1 {100 * nt:.2f}%", flush=True)
            assert fr <= 2 * nr + 1e-4, (B, label, fr, nr)
            assert 1 - fc <= 2 * (1 - nc) + 1e-6, (B, label, fc, nc)
            assert ft >= nt - 0.03 and ft >= TOP1_ABS and fc >= COS_ABS, (B, label, ft, nt, fc)
        if B == 1:
            cos, rel, top1 = demo_llm.agreement(base, pre)
            print(f"[c5] quality vs bf16 model (prefill, B=1): cosine {cos:.5f} rel L2 {rel:.3e} "
                  f"top-1 {100 * top1:.1f}%", flush=True)
            assert cos > 0.95   # quantization itself, reported as in the reference demo (no gate there)
    hook.remove()

    # the probe saw the B=1 prefill (M=512, GEMM), a B=1 decode step (M=1, GEMV), and the B=8 ones
    f = fp8[probe_name]
    q, s = f.qweight.cpu().numpy(), f.weight_scale.cpu().numpy()
    for x, y in (seen[0], seen[1], seen[NEW], seen[NEW + 1]):
        x2 = x.reshape(-1, x.shape[-1])[:64].float().cpu().numpy().astype(np.float64)
        y2 = y.reshape(-1, y.shape[-1])[:64].double().cpu().numpy()
        want = O.linear_ref64(x2, q, s, f.group_size, f.fmt)
        assert (np.abs(y2 - want) <= O.tolerance(want, "bfloat16")).all(), x.shape

    stats = {}
    for m in fp8.values():
        for k, v in m.stats.items():
            stats[k] = stats.get(k, 0) + v
    print(f"[c5] FP8Linear paths {stats}", flush=True)
    assert stats["gemv"] > 0 and stats["gemm"] + stats["chunked"] > 0 and stats["fallback"] == 0


def test_graph_decode_replays_match_eager():
    """GraphDecoder: the decode step captured once as a HIP graph (position and token are device
    tensors, the cache is static) and replayed.  Every replay, over two passes of the same prompt
    with host synchronizations and eager work between replays, must give the tokens and logits of
    the same static-shape step run eagerly; and the static step (attention over the whole
    zero-filled cache, masked past the position) must decode the tokens of the dynamic-shape
    forward used everywhere else."""
    model = demo_llm.build("tiny")
    prepare_model(model, "llm", FP8Config(profile="llm_safe", fmt="e4m3fn"))
    B, T, NEW = 2, 24, 12
    prompt = torch.randint(0, model.c["vocab"], (B, T), device="cuda", generator=torch.Generator("cuda").manual_seed(3))
    print(f"[graph] tiny B={B} prompt {T} decode {NEW}", flush=True)
    with torch.no_grad():
        toks_dyn, _, steps_dyn = demo_llm.generate(model, prompt, NEW + 1)
        eager = demo_llm.GraphDecoder(model, B, T + NEW + 4)
        eager.prefill(prompt)
        e_toks, e_logits = [], []
        for _ in range(NEW):
            e_logits.append(model.decode_step(eager.tok, eager.cache, eager.pos, eager.kpos)[:, -1].clone())
            e_toks.append(eager.tok.clone())
    # static step vs dynamic forward: the same tokens; the logits differ only because attention
    # sums over the longer (masked, zero-filled) cache in another fp32 order, which flips bf16
    # roundings of the projections downstream (the noise floor of the C5 test above, ~3e-3)
    assert torch.equal(torch.cat(e_toks, 1), toks_dyn[:, 1:]), "static decode step diverged from the forward"
    cos, rel, top1 = demo_llm.agreement(steps_dyn[:, 1:], torch.stack(e_logits, 1))
    print(f"[graph] static step vs forward: cosine {cos:.7f} rel L2 {rel:.2e} top-1 {100 * top1:.1f}%", flush=True)
    assert rel < 1e-2 and cos > 0.9999 and top1 == 1.0, (cos, rel, top1)

    dec = demo_llm.GraphDecoder(model, B, T + NEW + 4).capture()
    for rep in range(2):
        dec.prefill(prompt)
        tok0 = dec.tok.clone()
        for i in range(NEW):
            lg = dec.step()[:, -1].clone()
            if i % 3 == 0:
                torch.cuda.synchronize()
                _ = (lg * 2).sum().item()          # eager work and a host sync between replays
            assert torch.equal(dec.tok, e_toks[i]), (rep, i)
            torch.testing.assert_close(lg, e_logits[i], rtol=1e-5, atol=1e-6)
    print("[graph] every replay matches the eager step", flush=True)
    # the host refuses a step past the cache (the graph's cache write cannot check its position)
    assert dec.next_pos == T + NEW
    for _ in range(dec.max_len - dec.next_pos):
        dec.step()
    with pytest.raises(RuntimeError, match="KV cache full"):
        dec.step()
    with pytest.raises(ValueError):
        dec.rewind(dec.max_len)
    dec.rewind(T)                  # rows below T still hold the prompt; restart from its first token
    dec.tok.copy_(tok0)
    dec.step()
    assert torch.equal(dec.tok, e_toks[0]) and dec.next_pos == T + 1


def _bf16_ulps(a, b):
    """Distance in bf16 units in the last place between two bf16 tensors of finite values."""
    ia, ib = a.view(torch.int16).int(), b.view(torch.int16).int()
    ia = torch.where(ia < 0, -32768 - ia, ia)        # sign-magnitude -> monotonic integers
    ib = torch.where(ib < 0, -32768 - ib, ib)
    return (ia - ib).abs()


def test_llm_ops_match_pytorch_forms():
    """Each fused decode-step op (tfp8/examples/llm_ops.hip) against the PyTorch form it replaces in
    the example model: the elementwise ops with the same roundings bit for bit (residual add,
    rotary, cache write); the RMSNorm (whose fp32 row sum is ordered differently) within one bf16
    ulp; SiLU * up within one bf16 ulp (exp); attention within bf16 rounding of the fp32 result."""
    from tfp8.examples import llm_ops as ops
    g = torch.Generator("cuda").manual_seed(11)
    B, H, Hkv, hd, L, d = 3, 8, 4, 128, 300, 1024
    print(f"[llm_ops] B={B} H={H} Hkv={Hkv} hd={hd} L={L} d={d}", flush=True)

    x = torch.randn(B, 1, d, device="cuda", generator=g).bfloat16()
    r = torch.randn(B, 1, d, device="cuda", generator=g).bfloat16()
    norm = demo_llm.RMSNorm(d).cuda().bfloat16()
    norm.weight.data = (1 + 0.1 * torch.randn(d, device="cuda", generator=g)).bfloat16()
    with torch.no_grad():
        h, y = ops.add_rmsnorm(x, r, norm.weight, norm.eps)
        assert torch.equal(h, x + r)
        assert _bf16_ulps(y, norm(x + r)).max().item() <= 1
        h0, y0 = ops.add_rmsnorm(x, None, norm.weight, norm.eps)
        assert h0 is x and _bf16_ulps(y0, norm(x)).max().item() <= 1

        gg = (3 * torch.randn(B, 1, 4 * d, device="cuda", generator=g)).bfloat16()
        uu = torch.randn(B, 1, 4 * d, device="cuda", generator=g).bfloat16()
        assert _bf16_ulps(ops.silu_mul(gg, uu), torch.nn.functional.silu(gg) * uu).max().item() <= 1
        g1 = (3 * torch.randn(80, 2 * 1024, device="cuda", generator=g)).bfloat16()   # 80 rows: 8-wide form
        assert _bf16_ulps(ops.silu_mul(g1[:, :1024], g1[:, 1024:]),
                          torch.nn.functional.silu(g1[:, :1024]) * g1[:, 1024:]).max().item() <= 1

        # rotary + cache write at position p, and attention over 0..p, against the static step's
        # PyTorch ops (Attention.forward_static with the same caches)
        p = 217
        pos = torch.tensor([p], dtype=torch.long, device="cuda")
        kt = torch.randn(B, Hkv, hd, L, device="cuda", generator=g).bfloat16()
        vc = torch.randn(B, Hkv, L, hd, device="cuda", generator=g).bfloat16()
        kt2, vc2 = kt.clone(), vc.clone()
        kt0, vc0 = kt.clone(), vc.clone()           # before any write at pos
        q = torch.randn(B, 1, H * hd, device="cuda", generator=g).bfloat16()
        k = torch.randn(B, 1, Hkv * hd, device="cuda", generator=g).bfloat16()
        v = torch.randn(B, 1, Hkv * hd, device="cuda", generator=g).bfloat16()
        inv = 1.0 / (10000.0 ** (torch.arange(0, hd // 2, device="cuda", dtype=torch.float32) * 2.0 / hd))
        ang = pos.float()[:, None] * inv[None, :]
        cos, sin = ang.cos(), ang.sin()
        qf = ops.rope_cache(q, k, v, cos.reshape(-1), sin.reshape(-1), kt, vc, pos, H, Hkv)
        c4, s4 = cos[None, :, None, :], sin[None, :, None, :]
        q_ref = demo_llm._rotary(q.view(B, 1, H, hd), c4, s4)
        k_ref = demo_llm._rotary(k.view(B, 1, Hkv, hd), c4, s4)
        assert torch.equal(qf, q_ref.view(B, H, hd).float())
        kt2.index_copy_(3, pos, k_ref.permute(0, 2, 3, 1))
        vc2.index_copy_(2, pos, v.view(B, 1, Hkv, hd).transpose(1, 2))
        assert torch.equal(kt, kt2) and torch.equal(vc, vc2)
        # the same from column slices of one fused projection output, and SiLU * up from its halves
        fusedo = torch.cat([q, k, v], -1)
        kt3, vc3 = kt.clone(), vc.clone()
        qf3 = ops.rope_cache(fusedo[..., :H * hd], fusedo[..., H * hd:(H + Hkv) * hd], fusedo[..., (H + Hkv) * hd:],
                             cos.reshape(-1), sin.reshape(-1), kt3, vc3, pos, H, Hkv)
        assert torch.equal(qf3, qf) and torch.equal(kt3, kt) and torch.equal(vc3, vc)
        gu = torch.cat([gg, uu], -1)
        assert torch.equal(ops.silu_mul(gu[..., :4 * d], gu[..., 4 * d:]), ops.silu_mul(gg, uu))

        # tied head from the bf16 embedding: F.linear of the widened operands, fp32 sums reordered
        emb = (0.02 * torch.randn(1000, d, device="cuda", generator=g)).bfloat16()
        for rows in (1, 3, 4, 5, 8, 16):
            xh = torch.randn(rows, 1, d, device="cuda", generator=g).bfloat16()
            got, want = ops.head(xh, emb), torch.nn.functional.linear(xh.float(), emb.float())
            bound = 1e-5 * torch.nn.functional.linear(xh.float().abs(), emb.float().abs())
            assert got.shape == want.shape and ((got - want).abs() <= bound).all(), rows

        o = ops.attention(qf, kt, vc, pos, H, Hkv)
        rep = H // Hkv
        scores = torch.matmul(qf.view(B, H, 1, hd), kt.float().repeat_interleave(rep, 1)) / (hd ** 0.5)
        scores = scores.masked_fill(torch.arange(L, device="cuda") > pos, float("-inf"))
        o_ref32 = torch.matmul(torch.softmax(scores, -1), vc.float().repeat_interleave(rep, 1))   # [B, H, 1, hd]
        o_ref32 = o_ref32.transpose(1, 2).reshape(B, 1, H * hd)
        err = (o.float() - o_ref32).abs()
        assert (err <= 2.0 ** -8 * o_ref32.abs() + 1e-5).all(), err.max().item()

        # rotary + cache write fused into the attention kernel: the same caches and output bits
        kt4, vc4 = kt0.clone(), vc0.clone()
        o4 = ops.rope_attention(fusedo[..., :H * hd], fusedo[..., H * hd:(H + Hkv) * hd], fusedo[..., (H + Hkv) * hd:],
                                cos.reshape(-1), sin.reshape(-1), kt4, vc4, pos, H, Hkv)
        assert torch.equal(kt4, kt) and torch.equal(vc4, vc) and torch.equal(o4, o)

        # the first position (one cached row) and the last one (every row) of the cache
        for p in (0, L - 1):
            pos.fill_(p)
            o = ops.attention(qf, kt, vc, pos, H, Hkv)
            sc = torch.matmul(qf.view(B, H, 1, hd), kt.float().repeat_interleave(rep, 1)) / (hd ** 0.5)
            sc = sc.masked_fill(torch.arange(L, device="cuda") > pos, float("-inf"))
            ref = torch.matmul(torch.softmax(sc, -1), vc.float().repeat_interleave(rep, 1)).transpose(1, 2).reshape(B, 1, H * hd)
            assert ((o.float() - ref).abs() <= 2.0 ** -8 * ref.abs() + 1e-5).all(), p

        # a cache length that is a multiple of 8 takes the 16-byte-load attention kernel: positions
        # that end a chunk inside an 8-position group, one cached row, every row; and rotary + cache
        # write fused into it against the two ops
        L2 = 320
        kt5 = torch.randn(B, Hkv, hd, L2, device="cuda", generator=g).bfloat16()
        vc5 = torch.randn(B, Hkv, L2, hd, device="cuda", generator=g).bfloat16()
        for p in (0, 5, 13, 130, 317, L2 - 1):
            pos.fill_(p)
            o = ops.attention(qf, kt5, vc5, pos, H, Hkv)
            sc = torch.matmul(qf.view(B, H, 1, hd), kt5.float().repeat_interleave(rep, 1)) / (hd ** 0.5)
            sc = sc.masked_fill(torch.arange(L2, device="cuda") > pos, float("-inf"))
            ref = torch.matmul(torch.softmax(sc, -1), vc5.float().repeat_interleave(rep, 1)).transpose(1, 2).reshape(B, 1, H * hd)
            assert ((o.float() - ref).abs() <= 2.0 ** -8 * ref.abs() + 1e-5).all(), p
            ka, va, kb, vb = kt5.clone(), vc5.clone(), kt5.clone(), vc5.clone()
            qa = ops.rope_cache(q, k, v, cos.reshape(-1), sin.reshape(-1), ka, va, pos, H, Hkv)
            oa = ops.attention(qa, ka, va, pos, H, Hkv)
            ob = ops.rope_attention(q, k, v, cos.reshape(-1), sin.reshape(-1), kb, vb, pos, H, Hkv)
            assert torch.equal(ka, kb) and torch.equal(va, vb) and torch.equal(oa, ob), p


def test_rope_prefill_matches_pytorch_form():
    """rope_prefill (the prefill's rotary + cache write, one kernel) against Attention.forward's
    PyTorch form bit for bit: the rotated q in [B, H, T, hd], the rotated k and the v at cache
    positions start .. start + T - 1, every other cache position untouched; also from column slices
    of one fused projection output, with grouped and ungrouped heads and two head sizes."""
    from tfp8.examples import llm_ops as ops
    g = torch.Generator("cuda").manual_seed(13)
    for B, T, start, L, H, Hkv, hd in ((2, 37, 5, 64, 8, 4, 128), (1, 512, 0, 512, 16, 16, 128),
                                       (3, 1, 90, 100, 4, 2, 64), (2, 100, 3, 128, 4, 4, 256),
                                       (1, 20, 2, 30, 2, 1, 128)):     # L % 4 != 0: one dim a thread
        print(f"[rope_prefill] B={B} T={T} start={start} L={L} H={H} Hkv={Hkv} hd={hd}", flush=True)
        qkv = torch.randn(B, T, (H + 2 * Hkv) * hd, device="cuda", generator=g).bfloat16()
        q, k, v = qkv[..., :H * hd], qkv[..., H * hd:(H + Hkv) * hd], qkv[..., (H + Hkv) * hd:]
        kt = torch.randn(B, Hkv, hd, L, device="cuda", generator=g).bfloat16()
        vc = torch.randn(B, Hkv, L, hd, device="cuda", generator=g).bfloat16()
        kt2, vc2 = kt.clone(), vc.clone()
        inv = 1.0 / (10000.0 ** (torch.arange(0, hd // 2, device="cuda", dtype=torch.float32) * 2.0 / hd))
        ang = torch.arange(start, start + T, device="cuda", dtype=torch.float32)[:, None] * inv[None, :]
        c4, s4 = ang.cos()[None, :, None, :], ang.sin()[None, :, None, :]
        with torch.no_grad():
            qo = ops.rope_prefill(q, k, v, c4.contiguous(), s4.contiguous(), kt, vc, start, H, Hkv)
            q_ref = demo_llm._rotary(q.reshape(B, T, H, hd), c4, s4).transpose(1, 2)
            k_ref = demo_llm._rotary(k.reshape(B, T, Hkv, hd), c4, s4)
            kt2[:, :, :, start:start + T] = k_ref.permute(0, 2, 3, 1)
            vc2[:, :, start:start + T] = v.reshape(B, T, Hkv, hd).transpose(1, 2)
        assert qo.shape == (B, H, T, hd) and torch.equal(qo, q_ref)
        assert torch.equal(kt, kt2) and torch.equal(vc, vc2)


def test_attn_prefill_matches_fp32_attention():
    """attn_prefill (the prefill's causal attention as one flash-attention kernel) against the same
    attention in fp32 PyTorch ops (fp32 scores of the widened bf16 values, -inf above the diagonal,
    softmax, fp32 value product) within bf16 rounding of the fp32 result: grouped and ungrouped
    heads, query tiles that end inside a 64-row tile, a prefill that starts after cached positions,
    a single position, and cache positions past the written ones holding NaN (never read into the
    result)."""
    import math
    from tfp8.examples import llm_ops as ops
    g = torch.Generator("cuda").manual_seed(17)
    hd = 128
    for B, H, Hkv, T, start, Lc in ((2, 8, 4, 100, 0, 104), (1, 4, 4, 64, 37, 112), (3, 4, 2, 1, 90, 96),
                                    (1, 16, 16, 512, 0, 512), (2, 4, 1, 130, 7, 144)):
        print(f"[attn_prefill] B={B} H={H} Hkv={Hkv} T={T} start={start} Lc={Lc}", flush=True)
        Lw = start + T
        q = torch.randn(B, H, T, hd, device="cuda", generator=g).bfloat16()
        kt = torch.randn(B, Hkv, hd, Lc, device="cuda", generator=g).bfloat16()
        vc = torch.randn(B, Hkv, Lc, hd, device="cuda", generator=g).bfloat16()
        kt[..., Lw:] = float("nan")
        vc[:, :, Lw:] = float("nan")
        with torch.no_grad():
            o = ops.attn_prefill(q, kt, vc, start, H, Hkv)
            rep = H // Hkv
            sc = torch.matmul(q.float(), kt[..., :Lw].float().repeat_interleave(rep, 1)) / math.sqrt(hd)
            qpos = torch.arange(start, Lw, device="cuda")[:, None]
            sc = sc.masked_fill(torch.arange(Lw, device="cuda")[None, :] > qpos, float("-inf"))
            ref = torch.matmul(torch.softmax(sc, -1), vc[:, :, :Lw].float().repeat_interleave(rep, 1))
            ref = ref.transpose(1, 2).reshape(B, T, H * hd)
        assert o.shape == (B, T, H * hd) and bool(torch.isfinite(o).all())
        err = (o.float() - ref).abs()
        assert (err <= 2.0 ** -8 * ref.abs() + 1e-5).all(), err.max().item()


def test_step_in_and_step_out_match_pytorch_forms():
    """The decode step's own start and end as one kernel each, against decode_step's PyTorch ops bit
    for bit: the embedding rows of the tokens and cos / sin of pos.float() * inv (step_in); the
    greedy token (first maximum on ties, NaN above everything, as torch.argmax) with the position
    advanced by one (step_out)."""
    from tfp8.examples import llm_ops as ops
    g = torch.Generator("cuda").manual_seed(13)
    V, d, hd = 1000, 256, 128
    emb = torch.randn(V, d, device="cuda", generator=g).bfloat16()
    inv = 1.0 / (10000.0 ** (torch.arange(0, hd // 2, device="cuda", dtype=torch.float32) * 2.0 / hd))
    for B, p in ((1, 0), (3, 517), (8, 4095)):
        tok = torch.randint(0, V, (B, 1), device="cuda", generator=g)
        pos = torch.tensor([p], dtype=torch.long, device="cuda")
        x, cs, sn = ops.step_in(tok, pos, inv, emb)
        ang = pos.float()[:, None] * inv[None, :]
        assert torch.equal(x, torch.nn.functional.embedding(tok, emb))
        assert torch.equal(cs, ang.cos().reshape(-1)) and torch.equal(sn, ang.sin().reshape(-1)), p
        logits = torch.randn(B, 1, V, device="cuda", generator=g)
        if B > 1:
            logits[1, 0, 10] = logits[1, 0, 900] = logits[1].max() + 1      # tie: the first index wins
            logits[2, 0, 77] = float("nan")                                  # NaN above everything
        want = torch.stack([torch.argmax(logits[b, 0]) for b in range(B)]).view(B, 1)
        ops.step_out(logits[:, -1], tok, pos)
        assert torch.equal(tok, want) and pos.item() == p + 1, (B, tok.view(-1).tolist(), want.view(-1).tolist())
        if B > 1:
            assert tok[1, 0].item() == 10 and tok[2, 0].item() == 77
    # rows whose length is no multiple of 4 (element loads instead of 16-byte ones), ties included
    for V2 in (999, 4097):
        logits = torch.randn(2, 1, V2, device="cuda", generator=g)
        logits[0, 0, V2 - 1] = logits[0, 0, 3] = logits[0].max() + 1
        tok = torch.zeros(2, 1, dtype=torch.long, device="cuda")
        pos = torch.zeros(1, dtype=torch.long, device="cuda")
        ops.step_out(logits[:, -1], tok, pos)
        assert tok[0, 0].item() == 3 and tok[1, 0].item() == torch.argmax(logits[1, 0]).item() and pos.item() == 1


def test_fused_decode_step_matches_pytorch_step():
    """The decode step with the fused ops between the FP8 linears against the same step as PyTorch
    ops (decode_step(fused=False)): the same greedy tokens over 16 steps at B=1 and B=3, and logits
    within the bf16 rounding noise of the step (relative L2 below 1e-2, cosine above 0.9999)."""
    model = demo_llm.build("tiny")
    prepare_model(model, "llm", FP8Config(profile="llm_safe", fmt="e4m3fn"))
    for B in (1, 3):
        T, NEW = 20, 16
        print(f"[fused] tiny B={B} prompt {T} decode {NEW}", flush=True)
        prompt = torch.randint(0, model.c["vocab"], (B, T), device="cuda", generator=torch.Generator("cuda").manual_seed(B))
        runs = {}
        with torch.no_grad():
            for fused in (False, True):
                dec = demo_llm.GraphDecoder(model, B, T + NEW + 2)
                dec.prefill(prompt)
                toks, logits = [], []
                for _ in range(NEW):
                    logits.append(model.decode_step(dec.tok, dec.cache, dec.pos, dec.kpos, fused=fused)[:, -1].clone())
                    toks.append(dec.tok.clone())
                runs[fused] = (torch.cat(toks, 1), torch.stack(logits, 1))
        assert torch.equal(runs[True][0], runs[False][0])
        cos, rel, top1 = demo_llm.agreement(runs[False][1], runs[True][1])
        print(f"[fused] B={B}: cosine {cos:.7f} rel L2 {rel:.2e} top-1 {100 * top1:.1f}%", flush=True)
        assert rel < 1e-2 and cos > 0.9999 and top1 == 1.0, (B, cos, rel, top1)
