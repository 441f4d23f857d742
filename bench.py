#!/usr/bin/env python3
"""Headline benchmark of the tfp8 FP8Linear path on one MI355X.

Metric: "M=1 FP8-weight GEMV HBM GB/s (% peak); M=256 fused GEMM TFLOP/s".
`value` = GB/s of the M=1 decode GEMV on config 2 (K=4096, N=14336, bf16 activations, E4M3FN
weights ~N(0,0.02) with 0.1% x20 outliers, K-group-128 f32 scales, bf16 out): algorithmic
bytes (codes + scales + x + y, each crossing HBM once) / average kernel duration, measured with
HIP events on the stream the kernel runs on. The same line carries every other benchmark
configuration as its own roofline point (`configs`: C1 M=1, C2 M=2/4/8, C3 M=16/64/256 -- M=256
also as `gemm_m256` in TFLOP/s and MFMA fraction -- and C4), the C5 tiny-Llama prefill and
HIP-graph decode (`c5`), FP8Linear.forward's per-call time (`fp8linear_forward_call_us`), the W8A8
block-32 GEMM, and the reference's CPU forward (dequantize + F.linear in fp32, restated in
oracle/cpu_path.py) timed on every host CPU available to the process for C1, C2 M=1, C3 M=256
and C4 (`cpu_baselines`; `cpu_baseline` is the headline's).

Weights rotate over >= 512 MiB of distinct copies so the 256 MB Infinity Cache cannot serve them.
A step = one kernel launch over one batch (one copy of the layer). Synthetic data, seeded.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only gemv|gemm|c5|w8a8]
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "fp8-compatibility-layer_amd"))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0        # MI355X HBM3E
PEAK_F16_TFLOPS = 2500.0     # MI355X dense fp16/bf16 MFMA
PEAK_FP8_TFLOPS = 5000.0     # MI355X dense fp8 MFMA
ROTATE_BYTES = 512 << 20
PROFILE_TRAFFIC = os.path.join(ROOT, "profiles", "traffic_gemv_c2_m1.txt")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def c2_bytes(M):
    N, K = 14336, 4096
    return N * K + N * (K // 128) * 4 + M * K * 2 + M * N * 2


def c1_bytes(M):
    N = K = 4096
    return N * K + N * 4 + M * K * 2 + M * N * 2


def c3_bytes(M):
    N = K = 8192
    return N * K + N * 1 + N * 4 + M * K * 2 + M * N * 2


# C4: M=128, K=11008, N=4096, E5M2 codes, UE8M0 scales per 32-group, bf16 x and y, no bias.
C4_M, C4_N, C4_K = 128, 4096, 11008
C4_BYTES = C4_N * C4_K + C4_N * (C4_K // 32) + C4_M * C4_K * 2 + C4_M * C4_N * 2   # 50,364,416


def host_cpu_info():
    """CPU model, logical CPUs, CPUs this process may run on, and the cgroup CPU quota (if any)."""
    model = "?"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    quota = None
    try:
        q, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if q != "max":
            quota = int(q) / int(period)
    except (OSError, ValueError):
        pass
    return {"model": model, "logical_cpus": os.cpu_count(), "affinity": affinity, "cgroup_quota_cpus": quota}


def cpu_threads():
    """Every CPU this process can actually use: its affinity set, bounded by the cgroup quota."""
    info = host_cpu_info()
    n = info["affinity"]
    if info["cgroup_quota_cpus"]:
        n = min(n, max(1, int(info["cgroup_quota_cpus"])))
    return max(1, n)


class Layer:
    """One FP8 layer's device buffers plus prebuilt ctypes arguments for tfp8_linear."""

    def __init__(self, lib, x, q, s, sk, G, fmt_id, bias, y, ws_buf, ws_bytes):
        from tfp8 import _ext
        self.fn = lib.tfp8_linear
        M, K = x.shape
        N = q.shape[0]
        self.keep = (x, q, s, bias, y, ws_buf)
        self.args = (x.data_ptr(), _ext.DTYPE_ID[x.dtype], M, K, q.data_ptr(), N, s.data_ptr(), sk, G, fmt_id,
                     bias.data_ptr() if bias is not None else None, y.data_ptr(), _ext.DTYPE_ID[y.dtype],
                     ws_buf.data_ptr() if ws_buf is not None else None, ws_bytes)

    def __call__(self, stream):
        rc = self.fn(*self.args, stream)
        if rc:
            raise RuntimeError(f"tfp8_linear rc={rc}")


def make_layers(cfg, M, device):
    """Rotating copies of one config's layer (>= 512 MiB of weights in total)."""
    import torch

    from tfp8 import _ext
    from tfp8.quantize import quantize_weight
    lib = _ext.require()
    g = torch.Generator(device=device)
    if cfg == "c1":
        N, K, G, fmt, sf, pow2, xdt, ydt = 4096, 4096, None, "e4m3fn", "f32", True, torch.float16, torch.float16
        g.manual_seed(101)
        w = torch.randn(N, K, generator=g, device=device) * 0.02
        bias = None
    elif cfg == "c2":
        N, K, G, fmt, sf, pow2, xdt, ydt = 14336, 4096, 128, "e4m3fn", "f32", False, torch.bfloat16, torch.bfloat16
        g.manual_seed(202)
        w = torch.randn(N, K, generator=g, device=device) * 0.02
        w = torch.where(torch.rand(N, K, generator=g, device=device) < 1e-3, w * 20, w)
        bias = None
    elif cfg == "c4":
        N, K, G, fmt, sf, pow2, xdt, ydt = C4_N, C4_K, 32, "e5m2", "ue8m0", True, torch.bfloat16, torch.bfloat16
        g.manual_seed(404)
        w = torch.distributions.Laplace(0.0, 0.02).sample((N, K)).to(device)
        bias = None
    else:
        N, K, G, fmt, sf, pow2, xdt, ydt = 8192, 8192, None, "e4m3fn", "ue8m0", True, torch.float16, torch.float16
        g.manual_seed(303)
        w = torch.randn(N, K, generator=g, device=device) * 0.01
        bias = torch.randn(N, generator=g, device=device) * 0.1
    q, s, GG = quantize_weight(w, fmt, G, pow2, sf)
    del w
    x = torch.randn(M, K, generator=g, device=device)
    if cfg == "c4":   # rows scaled by 2^u, u in -20..20: a bf16 -> f16 cast would over/underflow
        x = x * torch.exp2(torch.randint(-20, 21, (M, 1), generator=g, device=device).float())
    x = x.to(xdt)
    per = q.numel() + s.numel() * s.element_size()
    copies = max(2, -(-ROTATE_BYTES // per) + 1)
    wsb = lib.tfp8_linear_workspace_size(_ext.DTYPE_ID[xdt], M, N, K)
    layers = []
    for i in range(copies):
        qi, si = (q, s) if i == 0 else (q.clone(), s.clone())
        y = torch.empty(M, N, dtype=ydt, device=device)
        wsbuf = torch.empty(wsb, dtype=torch.uint8, device=device) if wsb else None
        layers.append(Layer(lib, x, qi, si, _ext.scale_kind(si), GG, _ext.FMT_ID[fmt], bias, y, wsbuf, wsb))
    meta = dict(N=N, K=K, G=GG, fmt=fmt, scale=sf, pow2=pow2, x=str(xdt).replace("torch.", ""),
                y=str(ydt).replace("torch.", ""), copies=copies, rotate_mib=round(copies * per / 2**20, 1))
    return layers, (q, s, x, bias, GG, fmt), meta


_SLEEP_CYCLES = None


def _queue_ahead_cycles():
    """Cycles for torch.cuda._sleep to cover ~40 ms, calibrated once with events."""
    global _SLEEP_CYCLES
    if _SLEEP_CYCLES is None:
        import torch
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        torch.cuda._sleep(1_000_000)
        b.record()
        torch.cuda.synchronize()
        per_cycle = max(a.elapsed_time(b) * 1e-3 / 1e6, 1e-11)
        _SLEEP_CYCLES = int(0.04 / per_cycle)
    return _SLEEP_CYCLES


def time_layers(layers, steps, warmup):
    """Average launch duration: `steps` back-to-back launches between two events on the stream
    the kernels run on (torch's current stream). A bounded sleep kernel is queued first so the
    host has enqueued every launch before the first one starts -- the interval then holds only
    the kernels and the GPU's own dispatch gaps, not Python's launch rate."""
    import torch
    dev = torch.cuda.current_device()
    stream = torch._C._cuda_getCurrentRawStream(dev)
    R = len(layers)
    for i in range(warmup):
        layers[i % R](stream)
    cycles = _queue_ahead_cycles()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    torch.cuda._sleep(cycles)
    t0.record()
    h0 = time.perf_counter()
    for i in range(steps):
        layers[i % R](stream)
    t1.record()
    host = time.perf_counter() - h0
    torch.cuda.synchronize()
    total = t0.elapsed_time(t1) * 1e-3
    if host > 0.035:
        log(f"[bench] warning: enqueue took {host * 1e3:.1f} ms, longer than the queued sleep")
    return total / steps


def cpu_baseline(label, q, s, x, bias, G, fmt, out_dtype, nbytes, flops, rounds=7, warmup=2):
    """The reference CPU forward (oracle/cpu_path.py: dequantize to fp32, then F.linear, per call,
    as tfp8/linear.py:179-181 does) on every host CPU this process may use, timed with
    time.perf_counter: `warmup` untimed calls, then the median of `rounds` (the method of the
    reference's tests/bench_cpu_transcode.py:145-164)."""
    import torch

    from oracle import cpu_path
    th = cpu_threads()
    torch.set_num_threads(th)
    qc, sc, xc = q.cpu(), s.cpu(), x.cpu()
    bc = bias.cpu() if bias is not None else None
    table = cpu_path.lut16(fmt)
    ts = []
    for i in range(warmup + rounds):
        t = time.perf_counter()
        cpu_path.cpu_forward(xc, qc, sc, G, fmt, bc, out_dtype, table)
        ts.append(time.perf_counter() - t)
    med = statistics.median(ts[warmup:])
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "tflops": round(flops / med / 1e12, 4),
            "ms_per_call": round(med * 1e3, 2), "cores": th, "kind": "port",
            "sample": f"{label}: one full layer forward per round (weight re-dequantized each call, as the "
                      f"reference does), median of {rounds} rounds after {warmup} warm-ups"}


def forward_call_us(layer_data, M, calls=200):
    """FP8Linear.forward per Python call on this layer (tfp8/linear.py:150-208 is the reference's
    per-call path; its own figure is ~17 us at M=1, linear.py:173-176): host time per call with the
    calls enqueued back to back, and the synchronised wall time per call."""
    import torch

    from tfp8.linear import FP8Linear
    q, s, x1, bias, G, fmt = layer_data
    layer = FP8Linear.from_fp8_checkpoint(q, s, bias, fmt=fmt, out_dtype=x1.dtype)
    x = x1[:1].expand(M, -1).contiguous() if x1.shape[0] < M else x1[:M].contiguous()
    for _ in range(10):
        layer(x)
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(calls):
        layer(x)
    host = time.perf_counter() - t
    torch.cuda.synchronize()
    wall = time.perf_counter() - t
    return {"host_us": round(host / calls * 1e6, 2), "wall_us": round(wall / calls * 1e6, 2)}


def bench_c5(batches=(1, 8), prompt_len=512, n_decode=128):
    """the tiny Llama (8 layers, d=2048, 16 heads, FFN 5632, vocab 32000, random N(0,0.02)
    init), every Linear an E4M3FN per-channel FP8Linear: prefill 512 tokens, then greedy decode of
    128 tokens at B=1 and B=8, decode replayed from one captured HIP graph per token (the
    reference times the same loop eagerly, tfp8/examples/demo_llm.py:140-152, 186-200)."""
    import torch

    from tfp8 import FP8Config, prepare_model
    from tfp8.examples import demo_llm as D
    from tfp8.linear import FP8Linear
    c = D.SIZES["c5"]
    model = D.build("c5")
    prepare_model(model, "llm", FP8Config(profile="llm_safe", fmt="e4m3fn", weight_group=None, nan_check=True))
    layers = [m for m in model.modules() if isinstance(m, FP8Linear)]
    wbytes = sum(m.qweight.numel() + m.weight_scale.numel() * m.weight_scale.element_size() for m in layers)
    out = {"workload": "C5 tiny Llama, 8 layers d=2048 16 heads FFN 5632 vocab 32000, E4M3FN per-channel "
                       "FP8Linear, prefill 512 + 128 greedy decode steps, HIP-graph decode",
           "fp8_linear_layers": len(layers), "fp8_weight_bytes_per_step": wbytes}
    for B in batches:
        p, d, pg, dg = D.timings(model, B, prompt_len, n_decode, c["vocab"])
        out[f"B{B}"] = {"prefill_ms_eager": round(p, 3), "prefill_ms_graph": round(pg, 3),
                        "decode_ms_per_token_eager": round(d, 4), "decode_ms_per_token_graph": round(dg, 4),
                        "decode_tokens_per_s": round(B / dg * 1e3, 1),
                        "prefill_tokens_per_s": round(B * prompt_len / pg * 1e3, 1),
                        "fp8_weight_gbs": round(wbytes / (dg * 1e-3) / 1e9, 1),
                        "frac_of_hbm_roofline": round(wbytes / (dg * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
        log(f"[bench] C5 B={B}: {out[f'B{B}']}")
    del model
    torch.cuda.empty_cache()
    return out


def bench_w8a8(dev, steps, M=8192, N=8192, K=8192):
    """fp8_linear's GEMM (tfp8_w8a8_gemm, E4M3 x E4M3, block-32 UE8M0 and FP32 scales) on both
    matrix-core paths, and its activation quantizer, averaged over `steps` back-to-back launches
    between events on torch's current stream (same method as the GEMV)."""
    import torch

    from tfp8 import _ext
    import fp8_cuda
    lib = _ext.require()
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(M, K, device=dev, generator=g)
    w = torch.randn(N, K, device=dev, generator=g) * 0.02
    bias = torch.randn(N, device=dev, generator=g)
    c = torch.empty(M, N, device=dev)
    res = {"config": {"workload": f"W8A8 fp8_linear GEMM M={M} N={N} K={K}, E4M3 x E4M3, block-32 scales, "
                                  f"f32 bias, f32 out"}}
    fl = 2.0 * M * N * K
    for ue8m0 in (True, False):
        a_q, sa = fp8_cuda.quantize_k(x, "e4m3", ue8m0)
        bt, sb = fp8_cuda.quantize_k(w, "e4m3", ue8m0)
        for native in (False, True):
            def call(stream, native=native, a_q=a_q, sa=sa, bt=bt, sb=sb, ue8m0=ue8m0):
                rc = lib.tfp8_w8a8_gemm(a_q.data_ptr(), 0, sa.data_ptr(), bt.data_ptr(), 0, sb.data_ptr(),
                                        int(ue8m0), 0, int(native), bias.data_ptr(), c.data_ptr(), M, N, K, stream)
                if rc:
                    raise RuntimeError(f"tfp8_w8a8_gemm failed: {_ext.last_error()}")
            mean = time_layers([call], steps, 3)
            key = f"{'ue8m0' if ue8m0 else 'f32'}_{'native_fp8' if native else 'exact'}"
            peak = PEAK_FP8_TFLOPS if native else PEAK_F16_TFLOPS
            res[key] = {"us": round(mean * 1e6, 1), "tflops": round(fl / mean / 1e12, 1), "peak": peak,
                        "frac": round(fl / mean / 1e12 / peak, 4)}
            log(f"[bench] W8A8 {key}: {mean * 1e6:.1f} us -> {fl / mean / 1e12:.1f} TFLOP/s")

    def quant(stream):
        fp8_cuda.quantize_k(x, "e4m3", True)
    mq = time_layers([quant], steps, 3)
    qb = M * K * 4 + M * K + M * K // 32
    res["quantize_f32"] = {"us": round(mq * 1e6, 1), "gbs": round(qb / mq / 1e9, 1),
                           "frac": round(qb / mq / 1e9 / PEAK_HBM_GBS, 4)}
    log(f"[bench] W8A8 quantize {M}x{K} f32 -> E4M3 + UE8M0: {mq * 1e6:.1f} us -> {qb / mq / 1e9:.0f} GB/s")
    return res


def read_traffic():
    """HBM bytes per launch of the GEMV from the committed rocprofv3 --pmc summary, if present."""
    try:
        for line in open(PROFILE_TRAFFIC):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


class ReadProbe:
    """tfp8_read_probe (a read-only streaming kernel) over one buffer, launched like a Layer."""

    def __init__(self, lib, t, blocks, out):
        self.fn = lib.tfp8_read_probe
        self.keep = (t, out)
        self.args = (t.data_ptr(), t.numel() * t.element_size(), out.data_ptr(), blocks)

    def __call__(self, stream):
        rc = self.fn(*self.args, stream)
        if rc:
            raise RuntimeError(f"tfp8_read_probe rc={rc}")


def read_probe(layers, steps, warmup):
    """A plain read-only streaming kernel over the same rotating code buffers the GEMV streams, best
    of four launch shapes (256 to 2048 blocks of 512 threads): a reference rate for the GEMV's."""
    import torch
    from tfp8 import _ext
    lib = _ext.require()
    out = torch.empty(2048, dtype=torch.int32, device=layers[0].keep[1].device)
    best = None
    for blocks in (256, 512, 1024, 2048):
        probes = [ReadProbe(lib, l.keep[1], blocks, out) for l in layers]
        t = sorted(time_layers(probes, steps, warmup) for _ in range(3))[1]
        nbytes = layers[0].keep[1].numel()
        gbs = nbytes / t / 1e9
        if best is None or gbs > best["gbs"]:
            best = {"gbs": round(gbs, 1), "us": round(t * 1e6, 3), "blocks": blocks, "bytes": nbytes}
    return best


def _point(layers, nbytes, flops, steps, warmup, runs=1):
    """Average launch duration (median of `runs` timed runs) and its roofline figures."""
    ts = sorted(time_layers(layers, steps, warmup) for _ in range(runs))
    t = ts[len(ts) // 2]
    gbs, tf = nbytes / t / 1e9, flops / t / 1e12
    bound = "mfma" if flops / nbytes > PEAK_F16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9) else "hbm"
    frac = tf / PEAK_F16_TFLOPS if bound == "mfma" else gbs / PEAK_HBM_GBS
    return {"us": round(t * 1e6, 3), "gbs": round(gbs, 1), "tflops": round(tf, 2), "bound": bound,
            "frac": round(frac, 4), "algorithmic_bytes": nbytes, "flops": int(flops),
            **({"runs_us": [round(r * 1e6, 2) for r in ts]} if runs > 1 else {})}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-calls", action="store_true", help="skip the FP8Linear.forward per-call timing (its "
                    "kernels reread one weight copy, so they would mix into a kernel trace of the timed launches)")
    ap.add_argument("--only", choices=["gemv", "gemm", "w8a8", "c5"], default=None)
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run torch copies of a 256 MiB buffer (the known-size kernel that scales the "
                         "FETCH_SIZE / WRITE_SIZE counters of a rocprofv3 --pmc run)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (--gpus {a.gpus} requested). "
              f"Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if a.calibrate_copy:
        src = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("[bench] calibration: 5 copies of 268435456 bytes (read + write each)")
        return

    pts, cpu, calls, out = {}, {}, {}, {}
    gemm_steps = max(20, a.steps // 2)
    # ---------------------------------------------------------------- decode GEMVs: C2 M=1 (headline), C1, C2 sweep
    if a.only in (None, "gemv"):
        log("[bench] C2 M=1 GEMV: building rotating weights")
        layers, c2data, meta = make_layers("c2", 1, dev)
        pts["c2_m1"] = _point(layers, c2_bytes(1), 2.0 * 14336 * 4096, a.steps, a.warmup)
        log(f"[bench] C2 M=1: {pts['c2_m1']}")
        out["read_probe"] = read_probe(layers, a.steps, a.warmup)
        log(f"[bench] read-only probe over the same code buffers: {out['read_probe']}")
        out["gemv_meta"] = meta
        if not a.no_calls:
            calls["c2_m1"] = forward_call_us(c2data, 1)
        if not a.no_cpu:
            q, s_, x, bias, G, fmt = c2data
            cpu["c2_m1"] = cpu_baseline("C2 M=1 (14336x4096 E4M3FN G128, bf16 x)", q, s_, x, bias, G, fmt,
                                        torch.bfloat16, c2_bytes(1), 2.0 * 14336 * 4096)
            log(f"[bench] CPU C2 M=1: {cpu['c2_m1']}")
        del layers
        for M in (2, 4, 8):
            lm, _, _ = make_layers("c2", M, dev)
            pts[f"c2_m{M}"] = _point(lm, c2_bytes(M), 2.0 * M * 14336 * 4096, a.steps, a.warmup)
            log(f"[bench] C2 M={M}: {pts[f'c2_m{M}']}")
            del lm
        l1, c1data, _ = make_layers("c1", 1, dev)
        pts["c1_m1"] = _point(l1, c1_bytes(1), 2.0 * 4096 * 4096, a.steps, a.warmup)
        log(f"[bench] C1 M=1: {pts['c1_m1']}")
        if not a.no_calls:
            calls["c1_m1"] = forward_call_us(c1data, 1)
        if not a.no_cpu:
            q, s_, x, bias, G, fmt = c1data
            cpu["c1_m1"] = cpu_baseline("C1 M=1 (4096x4096 E4M3FN per-channel, fp16 x)", q, s_, x, bias, G, fmt,
                                        torch.float16, c1_bytes(1), 2.0 * 4096 * 4096)
            log(f"[bench] CPU C1: {cpu['c1_m1']}")
        del l1
        torch.cuda.empty_cache()

    # ---------------------------------------------------------------- GEMMs: C3 M=16/64/256, C4
    if a.only in (None, "gemm"):
        for M in (16, 64, 256):
            log(f"[bench] C3 M={M} GEMM: building rotating weights")
            lm, c3data, meta3 = make_layers("c3", M, dev)
            # median of three timed runs: single runs of the ~50 us launches vary by several percent
            pts[f"c3_m{M}"] = _point(lm, c3_bytes(M), 2.0 * M * 8192 * 8192, gemm_steps, max(5, a.warmup // 2),
                                     runs=3)
            log(f"[bench] C3 M={M}: {pts[f'c3_m{M}']}")
            if M == 16 and not a.no_calls:
                calls["c3_m16"] = forward_call_us(c3data, 16)
            if M == 256:
                out["gemm_meta"] = meta3
                if not a.no_cpu:
                    q, s_, x, bias, G, fmt = c3data
                    cpu["c3_m256"] = cpu_baseline("C3 M=256 (8192x8192 E4M3FN per-channel UE8M0, fp16 x)", q, s_, x,
                                                  bias, G, fmt, torch.float16, c3_bytes(256),
                                                  2.0 * 256 * 8192 * 8192)
                    log(f"[bench] CPU C3 M=256: {cpu['c3_m256']}")
            del lm
            torch.cuda.empty_cache()
        log("[bench] C4 M=128 GEMM (E5M2, UE8M0 32-groups): building rotating weights")
        l4, c4data, _ = make_layers("c4", C4_M, dev)
        pts["c4_m128"] = _point(l4, C4_BYTES, 2.0 * C4_M * C4_N * C4_K, gemm_steps, 5, runs=3)
        log(f"[bench] C4 M=128: {pts['c4_m128']}")
        if not a.no_cpu:
            q, s_, x, bias, G, fmt = c4data
            cpu["c4_m128"] = cpu_baseline("C4 M=128 (4096x11008 E5M2 G32 UE8M0, bf16 x)", q, s_, x, bias, G, fmt,
                                          torch.bfloat16, C4_BYTES, 2.0 * C4_M * C4_N * C4_K)
            log(f"[bench] CPU C4: {cpu['c4_m128']}")
        del l4
        torch.cuda.empty_cache()

    # ---------------------------------------------------------------- C5 tiny Llama, W8A8
    if a.only in (None, "c5"):
        out["c5"] = bench_c5()
    if a.only in (None, "w8a8"):
        out["w8a8"] = bench_w8a8(dev, max(10, a.steps // 10))

    g = pts.get("c2_m1")
    line = {
        "metric": "M=1 FP8-weight GEMV HBM GB/s (% peak); M=256 fused GEMM TFLOP/s",
        "value": g["gbs"] if g else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(g["us"] * 1e-3, 5) if g else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "C2 decode GEMV M=1: K=4096 N=14336, bf16 x, E4M3FN weights (0.1% x20 outliers), "
                               "K-group-128 f32 scales, bf16 out", **out.get("gemv_meta", {})},
    }
    if g:
        line["pct_peak_hbm"] = round(100 * g["gbs"] / PEAK_HBM_GBS, 1)
        line["roofline"] = {"bound": "hbm", "achieved": g["gbs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                            "frac": g["frac"], "traffic": read_traffic(),
                            "traffic_source": "profiles/traffic_gemv_c2_m1.txt: rocprofv3 --pmc FETCH_SIZE and "
                                              "WRITE_SIZE of this kernel on an earlier run (not measured in this run)",
                            "kernel_us": g["us"], "algorithmic_bytes": g["algorithmic_bytes"]}
        rp = out.get("read_probe")
        if rp:
            line["read_probe"] = {**rp, "frac_of_peak": round(rp["gbs"] / PEAK_HBM_GBS, 4),
                                  "gemv_over_probe": round(g["gbs"] / rp["gbs"], 4),
                                  "sample": "tfp8_read_probe: a plain read-only kernel (each block a contiguous "
                                            "share, 16 loads of 16 bytes in flight per thread) over the C2 code "
                                            "buffers the GEMV streams, rotating copies; best of 256/512/1024/2048 "
                                            "blocks"}
    if "c3_m256" in pts:
        gm = pts["c3_m256"]
        line["gemm_m256"] = {"tflops": gm["tflops"], "kernel_us": gm["us"], "runs_us": gm["runs_us"],
                             "timing": "median of 3 runs, every kernel of the call (GEMM and split-K reduce)",
                             "roofline": {"bound": "mfma", "achieved": gm["tflops"], "peak": PEAK_F16_TFLOPS,
                                          "unit": "TFLOP/s", "frac": gm["frac"]},
                             "config": {"workload": "C3 fused GEMM M=256: K=N=8192, fp16 x, E4M3FN, per-channel "
                                                    "UE8M0, f32 bias, fp16 out", **out.get("gemm_meta", {})}}
    line["configs"] = pts
    if calls:
        line["fp8linear_forward_call_us"] = calls
    if "c5" in out:
        line["c5"] = out["c5"]
    if "w8a8" in out:
        line["w8a8"] = out["w8a8"]
    if cpu:
        host = host_cpu_info()
        for v in cpu.values():
            v["cpu_model"] = host["model"]
        line["cpu_host"] = host
        line["cpu_baselines"] = cpu
    line["cpu_baseline"] = cpu.get("c2_m1")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
