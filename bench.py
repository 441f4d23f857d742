#!/usr/bin/env python3
"""Headline benchmark of the tfp8 FP8Linear path on one MI355X.

Metric: "M=1 FP8-weight GEMV HBM GB/s (% peak); M=256 fused GEMM TFLOP/s".
`value` = GB/s of the M=1 decode GEMV on config 2 (K=4096, N=14336, bf16 activations, E4M3FN
weights ~N(0,0.02) with 0.1% x20 outliers, K-group-128 f32 scales, bf16 out): algorithmic
bytes (codes + scales + x + y, each crossing HBM once) / average kernel duration, measured with
HIP events on the stream the kernel runs on. The same line carries the config-3 M=256 MFMA GEMM
(K=N=8192, fp16 x, per-channel UE8M0, f32 bias) TFLOP/s, the decode sweep M=2/4/8, and the
reference's CPU forward (dequantize + F.linear in fp32, restated in oracle/cpu_path.py) timed on
the host cores of the same box.

Weights rotate over >= 512 MiB of distinct copies so the 256 MB Infinity Cache cannot serve them.
A step = one kernel launch over one batch (one copy of the layer). Synthetic data, seeded.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only gemv|gemm]
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


def cpu_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


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


def cpu_baseline(q, s, x, bias, G, fmt, nbytes, rounds=5):
    """The reference CPU forward (oracle/cpu_path.py) on the host cores: one full C2 M=1 layer call
    per round (weight re-materialised each call, as the reference does)."""
    import torch

    from oracle import cpu_path
    th = cpu_threads()
    torch.set_num_threads(th)
    qc, sc, xc = q.cpu(), s.cpu(), x.cpu()
    bc = bias.cpu() if bias is not None else None
    table = cpu_path.lut16(fmt)
    ts = []
    for i in range(2 + rounds):
        t = time.perf_counter()
        cpu_path.cpu_forward(xc, qc, sc, G, fmt, bc, x.dtype, table)
        ts.append(time.perf_counter() - t)
    med = statistics.median(ts[2:])
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": th, "kind": "port",
            "sample": f"full C2 M=1 layer forward (14336x4096 E4M3FN G128, bf16 x), median of {rounds} "
                      f"rounds after 2 warm-ups, {med * 1e3:.1f} ms/call"}


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=["gemv", "gemm", "w8a8"], default=None)
    ap.add_argument("--sweep", action="store_true", help="also time the C2 decode sweep M=2,4,8 and C3 M=16,64")
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
    out = {}
    if a.calibrate_copy:
        src = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("[bench] calibration: 5 copies of 268435456 bytes (read + write each)")
        return

    # ---------------------------------------------------------------- C2 M=1 GEMV (headline)
    if a.only in (None, "gemv"):
        log("[bench] C2 M=1 GEMV: building rotating weights")
        layers, (q, s, x, bias, G, fmt), meta = make_layers("c2", 1, dev)
        mean = time_layers(layers, a.steps, a.warmup)
        nb = c2_bytes(1)
        gbs = nb / mean / 1e9
        log(f"[bench] C2 M=1: {mean * 1e6:.2f} us/launch -> {gbs:.1f} GB/s")
        out["gemv"] = dict(mean=mean, bytes=nb, gbs=gbs, meta=meta)
        l1, _, _ = make_layers("c1", 1, dev)
        m1 = time_layers(l1, a.steps, a.warmup)
        out["c1"] = dict(us=m1 * 1e6, gbs=c1_bytes(1) / m1 / 1e9)
        log(f"[bench] C1 M=1: {m1 * 1e6:.2f} us/launch -> {out['c1']['gbs']:.1f} GB/s")
        del l1
        if a.sweep:
            sweep = {}
            for M in (2, 4, 8):
                lm, _, _ = make_layers("c2", M, dev)
                mm = time_layers(lm, a.steps, a.warmup)
                sweep[f"M{M}"] = round(c2_bytes(M) / mm / 1e9, 1)
                log(f"[bench] C2 M={M}: {mm * 1e6:.2f} us -> {sweep[f'M{M}']} GB/s")
                del lm
            out["sweep"] = sweep
        if not a.no_cpu:
            log("[bench] CPU baseline (reference CPU forward)")
            out["cpu"] = cpu_baseline(q, s, x, bias, G, fmt, nb)
            log(f"[bench] CPU: {out['cpu']}")
        del layers
        torch.cuda.empty_cache()

    # ---------------------------------------------------------------- C3 M=256 GEMM
    if a.only in (None, "gemm"):
        log("[bench] C3 M=256 GEMM: building rotating weights")
        layers, _, meta3 = make_layers("c3", 256, dev)
        steps = max(20, a.steps // 2)
        # median of three timed runs: single runs of this ~50 us launch vary by several percent
        runs3 = sorted(time_layers(layers, steps, max(5, a.warmup // 2)) for _ in range(3))
        mean3 = runs3[1]
        fl = 2.0 * 256 * 8192 * 8192
        tf = fl / mean3 / 1e12
        log(f"[bench] C3 M=256: kernel {mean3 * 1e6:.2f} us -> {tf:.1f} TFLOP/s ({c3_bytes(256) / mean3 / 1e9:.0f} GB/s)")
        out["gemm"] = dict(mean=mean3, tflops=tf, meta=meta3, runs_us=[round(r * 1e6, 2) for r in runs3])
        gsweep = {}
        for M in ((16, 64) if a.sweep else ()):
            lm, _, _ = make_layers("c3", M, dev)
            mm = time_layers(lm, steps, 5)
            gsweep[f"M{M}"] = {"us": round(mm * 1e6, 2), "gbs": round(c3_bytes(M) / mm / 1e9, 1),
                               "tflops": round(2.0 * M * 8192 * 8192 / mm / 1e12, 1)}
            log(f"[bench] C3 M={M}: {gsweep[f'M{M}']}")
            del lm
        out["gemm_sweep"] = gsweep
        del layers
        log("[bench] C4 M=128 GEMM (E5M2, UE8M0 32-groups): building rotating weights")
        l4, _, meta4 = make_layers("c4", C4_M, dev)
        m4 = sorted(time_layers(l4, steps, 5) for _ in range(3))[1]
        out["c4"] = {"us": round(m4 * 1e6, 2), "gbs": round(C4_BYTES / m4 / 1e9, 1),
                     "tflops": round(2.0 * C4_M * C4_N * C4_K / m4 / 1e12, 1), "timing": "median of 3 runs"}
        log(f"[bench] C4 M=128: {out['c4']}")
        del l4

    # ---------------------------------------------------------------- W8A8 block-32 GEMM
    if a.only in (None, "w8a8"):
        out["w8a8"] = bench_w8a8(dev, max(10, a.steps // 10))

    g = out.get("gemv")
    line = {
        "metric": "M=1 FP8-weight GEMV HBM GB/s (% peak); M=256 fused GEMM TFLOP/s",
        "value": round(g["gbs"], 1) if g else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(g["mean"] * 1e3, 5) if g else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "C2 decode GEMV M=1: K=4096 N=14336, bf16 x, E4M3FN weights (0.1% x20 outliers), "
                               "K-group-128 f32 scales, bf16 out",
                   **({k: v for k, v in g["meta"].items()} if g else {})},
    }
    if g:
        line["pct_peak_hbm"] = round(100 * g["gbs"] / PEAK_HBM_GBS, 1)
        line["roofline"] = {"bound": "hbm", "achieved": round(g["gbs"], 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                            "frac": round(g["gbs"] / PEAK_HBM_GBS, 4), "traffic": read_traffic(),
                            "kernel_us": round(g["mean"] * 1e6, 3), "algorithmic_bytes": g["bytes"]}
        line["config1_m1"] = {"us": round(out["c1"]["us"], 2), "gbs": round(out["c1"]["gbs"], 1),
                              "frac": round(out["c1"]["gbs"] / PEAK_HBM_GBS, 4)}
        if "sweep" in out:
            line["decode_sweep_gbs"] = out["sweep"]
    if "gemm" in out:
        gm = out["gemm"]
        line["gemm_m256"] = {"tflops": round(gm["tflops"], 1), "kernel_us": round(gm["mean"] * 1e6, 2),
                             "runs_us": gm["runs_us"], "timing": "median of 3 runs, GEMM + split-K reduce",
                             "roofline": {"bound": "mfma", "achieved": round(gm["tflops"], 1),
                                          "peak": PEAK_F16_TFLOPS, "unit": "TFLOP/s",
                                          "frac": round(gm["tflops"] / PEAK_F16_TFLOPS, 4)},
                             "config": {"workload": "C3 fused GEMM M=256: K=N=8192, fp16 x, E4M3FN, per-channel "
                                                    "UE8M0, f32 bias, fp16 out", **gm["meta"]}}
        if out.get("gemm_sweep"):
            line["gemm_sweep"] = out["gemm_sweep"]
        if out.get("c4"):
            line["c4_gemm"] = out["c4"]
    if "w8a8" in out:
        line["w8a8"] = out["w8a8"]
    line["cpu_baseline"] = out.get("cpu")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
