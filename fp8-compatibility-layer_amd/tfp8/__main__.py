"""python -m tfp8 : self-check and environment report (API of tfp8/__main__.py:11-38)."""
import platform
import sys

import torch

from tfp8 import _ext
from tfp8.formats import E4M3FN, E5M2, decode, encode


def _same(a, b):
    return bool(((torch.isnan(a) & torch.isnan(b)) | (a == b)).all())


def main():
    print("tfp8 -- FP8 weight layer for MI355X (gfx950 HIP kernels, W8A16)\n")
    print(f"python     {sys.version.split()[0]}  ({platform.system()} {platform.machine()})")
    print(f"torch      {torch.__version__} / HIP {torch.version.hip}")
    dev = "cpu"
    if torch.cuda.is_available():
        p = torch.cuda.get_device_properties(0)
        print(f"gpu        {p.name}  {getattr(p, 'gcnArchName', '?')}  {p.total_memory / 2**30:.1f} GB")
        ok = _ext.available()
        print(f"library    {_ext.lib_path()}  {'ok' if ok else 'UNAVAILABLE: ' + str(_ext.last_error())}")
        dev = "cuda" if ok else "cpu"
    else:
        print("gpu        none -- CPU (torch) paths only")

    print(f"\nformats (decoded on {dev})")
    codes = torch.arange(256, dtype=torch.uint8)
    for f in (E4M3FN, E5M2):
        ref = codes.view(f.torch_dtype).float()
        got = decode(codes.to(dev), f).cpu()
        print(f"  {f.name:7s} e{f.ebits}m{f.mbits} bias {f.bias:2d}  max {f.max_finite:>8.0f}  "
              f"all 256 codes decode exactly: {_same(got, ref)}")
    x = torch.randn(4096) * 100
    enc = encode(x.to(dev), E4M3FN).cpu()
    print(f"  encode RNE matches torch float8 cast: {torch.equal(enc, x.to(torch.float8_e4m3fn).view(torch.uint8))}")
    print("\nkernels: GEMV (M<=3, dwordx4 stream, in-register cvt decode, DPP reduce),"
          " matrix-core decode (4<=M<=16), MFMA GEMMs (M>16, FP8 tiles in LDS or registers,"
          " f16/bf16 MFMA, fp32 acc)")
    print("  ABI: qweight uint8[N,K], weight_scale f32|ue8m0[N,K/G], bias f32[N] -- include/tfp8_hip.h")


if __name__ == "__main__":
    main()
