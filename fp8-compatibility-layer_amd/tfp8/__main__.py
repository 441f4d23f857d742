"""python -m tfp8 -- report what this install can run and check the format code on it.

Same role as the reference's self-check (tfp8/__main__.py:11-38): environment, then the FP8
formats against torch's float8 casts.  Here the checks run on the GPU when the HIP library loads,
and one FP8Linear call per kernel family (GEMV, MFMA GEMM) is compared with the dequantized
fp32 product.  Exit status 1 if any check fails.
"""
import platform
import sys

import torch

from tfp8 import _ext
from tfp8.formats import E4M3FN, E5M2, decode, encode


def _environment():
    rows = [("python", f"{sys.version.split()[0]} ({platform.system()} {platform.machine()})"),
            ("torch", f"{torch.__version__}, HIP {torch.version.hip}")]
    device = "cpu"
    if torch.cuda.is_available():
        prop = torch.cuda.get_device_properties(0)
        arch = getattr(prop, "gcnArchName", "?")
        rows.append(("device", f"{prop.name} ({arch}, {prop.multi_processor_count} CUs, "
                               f"{prop.total_memory / 2 ** 30:.0f} GiB)"))
        if _ext.available():
            device = "cuda"
            rows.append(("library", f"{_ext.lib_path()} (ABI {_ext.ABI_VERSION})"))
        else:
            rows.append(("library", f"NOT LOADED: {_ext.last_error()}"))
    else:
        rows.append(("device", "no GPU: the torch CPU paths only"))
    return rows, device


def _nan_aware_equal(a, b):
    return bool(((a == b) | (torch.isnan(a) & torch.isnan(b))).all())


def _checks(device):
    """(description, passed) for each self-check on `device`."""
    out = []
    codes = torch.arange(256, dtype=torch.uint8)
    for f in (E4M3FN, E5M2):
        want = codes.view(f.torch_dtype).float()
        got = decode(codes.to(device), f).float().cpu()
        out.append((f"{f.name} decode of all 256 codes equals {f.torch_dtype}", _nan_aware_equal(got, want)))
        x = torch.randn(8192, generator=torch.Generator().manual_seed(1)) * (f.max_finite / 8)
        q = encode(x.to(device), f).cpu()
        out.append((f"{f.name} encode (RNE) equals torch's cast on in-range values",
                    torch.equal(q, x.to(f.torch_dtype).view(torch.uint8))))
    if device == "cuda":
        from tfp8.linear import FP8Linear
        g = torch.Generator().manual_seed(2)
        lin = torch.nn.Linear(1024, 320)
        with torch.no_grad():
            lin.weight.copy_(torch.randn(320, 1024, generator=g) * 0.02)
        layer = FP8Linear.from_linear(lin.to(device), group_size=128)
        layer.out_dtype = torch.float32
        w = layer.dequantized_weight()
        for rows, family in ((1, "gemv"), (64, "gemm")):
            x = torch.randn(rows, 1024, generator=g).bfloat16().to(device)
            y = layer(x)
            ref = x.float() @ w.t() + layer.bias_f32
            err = float((y - ref).abs().max() / ref.abs().max())
            out.append((f"FP8Linear M={rows} ({family} kernels) vs dequantized fp32, rel err {err:.1e}",
                        err < 1e-3 and layer.stats[family] >= 1))
    return out


def main():
    rows, device = _environment()
    print("tfp8 -- FP8 weights decoded inside MI355X (gfx950) HIP kernels\n")
    width = max(len(k) for k, _ in rows)
    for k, v in rows:
        print(f"  {k:<{width}}  {v}")
    print(f"\nself-checks on {device}")
    results = _checks(device)
    for desc, ok in results:
        print(f"  [{'ok' if ok else 'FAIL'}] {desc}")
    print("\nkernels: streaming GEMV (M <= 3), matrix-core decode (4 <= M <= 16), MFMA GEMMs above;"
          " C ABI in include/tfp8_hip.h")
    return 0 if all(ok for _, ok in results) else 1


if __name__ == "__main__":
    sys.exit(main())
