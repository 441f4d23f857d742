"""Build libtfp8_hip.so (gfx950) from csrc/*.hip with hipcc: one object per source, in parallel,
then one shared library next to the Python package (tfp8/libtfp8_hip.so).  Also builds the example
model's fused decode ops, tfp8/examples/llm_ops.hip -> tfp8/examples/libtfp8_llm.so.

    python fp8-compatibility-layer_amd/build_lib.py [--jobs N]

No cmake/ninja: the library is five translation units. Objects go to _build/ (git-ignored).
"""
import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "tfp8", "libtfp8_hip.so")
EXAMPLE_SRC = os.path.join(HERE, "tfp8", "examples", "llm_ops.hip")
EXAMPLE_OUT = os.path.join(HERE, "tfp8", "examples", "libtfp8_llm.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed fp32 VALU ops are disabled for all device code (v_pk_{add,mul,fma}_f32).
FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-I", os.path.join(ROOT, "include"),
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall", "-Wno-unused-function"]


# Per-source additions.  gemv_quad.hip reads its 4x4x4 MFMA results with VALU ops every chunk; in
# the accumulator-register form the compiler gave each chunk's result its own AGPRs (up to 128 of
# them, and a v_accvgpr_read per value), so its MFMAs are built in the VGPR form.
FILE_FLAGS = {"gemv_quad.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that noise.
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    return src, obj, r.returncode, err


def build(jobs=None, verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    jobs = jobs or min(len(srcs) + 1, os.cpu_count() or 4, 8)
    with ThreadPoolExecutor(jobs) as ex:
        example = ex.submit(_compile, EXAMPLE_SRC)
        results = list(ex.map(_compile, srcs))
        example = example.result()
    bad = [(s, e) for s, _, rc, e in results if rc]
    for s, _, rc, e in results:
        if e.strip() and (verbose or rc):
            print(f"--- {os.path.basename(s)}\n{e}", file=sys.stderr)
    if bad:
        raise RuntimeError(f"hipcc failed for {[os.path.basename(s) for s, _ in bad]}")
    tmp = OUT + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *[o for _, o, _, _ in results]]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    src, obj, rc, err = example
    if rc:
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{err}")
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", EXAMPLE_OUT + ".tmp", obj],
                       capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(EXAMPLE_OUT + ".tmp", EXAMPLE_OUT)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    print(build(a.jobs, a.verbose))
