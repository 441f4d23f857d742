"""Checks on the gfx950 assembly of this library's own kernels (hipcc -S of the sources here), for
the two places where inline assembly steps outside what the compiler can check:

* the W8A8 FP32-block-scale kernel multiplies with `v_mul_f32_dpp ... row_newbcast` in inline
  assembly; a DPP read of a VGPR that a VALU instruction wrote one or two instructions earlier is a
  hazard the compiler cannot see inside the asm, so every DPP source must come from an LDS load
  (or be written at least three instructions earlier);
* the direct-to-LDS GEMM sets m0 in its `buffer_load ... lds` asm (and declares the clobber); the
  compiler must not keep anything of its own in m0 in those kernels;
* the same GEMM loads its K-group scales with inline-assembly buffer loads into VGPRs, retired by
  an explicit `s_waitcnt vmcnt`: the compiler does not know those registers fill asynchronously,
  so no instruction may read, write or copy them before that wait.

CPU only (hipcc cross-compiles for gfx950); skipped when hipcc is absent."""
import os
import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "fp8-compatibility-layer_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC) and shutil.which("hipcc") is None, reason="no hipcc")


@pytest.fixture(scope="module")
def isa(tmp_path_factory):
    out = tmp_path_factory.mktemp("isa")

    def compile_one(name):
        dst = os.path.join(out, name + ".s")
        cmd = [HIPCC, "-O3", "-std=c++17", "--offload-arch=gfx950", "--cuda-device-only", "-S",
               "-I", os.path.join(ROOT, "include"), "-I", CSRC,
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               os.path.join(CSRC, name), "-o", dst]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        return name, open(dst).read()

    with ThreadPoolExecutor(2) as ex:
        return dict(ex.map(compile_one, ["w8a8.hip", "gemm_direct.hip"]))


def _kernels(asm, pattern):
    """{kernel symbol: [instruction lines]} for the kernels whose symbol matches `pattern`."""
    out, cur = {}, None
    for line in asm.splitlines():
        m = re.match(r"^(_Z\S+):", line)
        if m:
            cur = m.group(1) if re.search(pattern, m.group(1)) else None
            if cur:
                out[cur] = []
            continue
        if cur and re.match(r"^\s+[a-z_]", line):
            out[cur].append(line.strip())
    return out


def _vgpr_dests(ins):
    op = ins.split()[0]
    if op.startswith(("s_", "buffer_store", "ds_write", "global_store")):
        return []
    first = ins[len(op):].split(",")[0].strip()
    m = re.match(r"v\[(\d+):(\d+)\]$", first)
    if m:
        return ["v%d" % i for i in range(int(m.group(1)), int(m.group(2)) + 1)]
    return [first] if re.match(r"v\d+$", first) else []


def test_w8a8_dpp_sources_not_freshly_valu_written(isa):
    ks = _kernels(isa["w8a8.hip"], "w8_f16_kernel")
    assert len(ks) == 4, "four format instantiations of the FP32-block-scale kernel"
    checked = 0
    for name, ins in ks.items():
        for i, x in enumerate(ins):
            if "_dpp" not in x.split()[0]:
                continue
            src = x.split(",")[1].strip()
            for j in range(i - 1, -1, -1):
                if src in _vgpr_dests(ins[j]):
                    op = ins[j].split()[0]
                    assert not (op.startswith("v_") and i - j - 1 < 3), f"{name}: {ins[j]!r} feeds {x!r}"
                    break
            checked += 1
    assert checked >= 4 * 64, checked   # 64 DPP multiplies per K step at least once per kernel


def test_gemm_direct_m0_only_set_by_the_dma_asm(isa):
    ks = _kernels(isa["gemm_direct.hip"], "gemm_direct_kernel")
    assert ks
    for name, ins in ks.items():
        for x in ins:
            if re.search(r"\bm0\b", x):
                assert re.match(r"s_mov_b32 m0, s\d+$", x), f"{name}: compiler use of m0: {x!r}"


def test_gemm_direct_scale_loads_untouched_until_their_wait(isa):
    ks = _kernels(isa["gemm_direct.hip"], "gemm_direct_kernel")
    checked = 0
    for name, ins in ks.items():
        for i, x in enumerate(ins):
            m = re.match(r"buffer_load_(ubyte|dword) (v\d+), ", x)
            if not m or " lds" in x:
                continue
            reg = m.group(2)
            for y in ins[i + 1:]:
                if y.startswith("s_waitcnt") and "vmcnt" in y:
                    break
                if y.startswith(("s_cbranch", "s_branch", "s_endpgm")):
                    break
                assert not re.search(r"\b%s\b" % reg, y), f"{name}: {reg} of {x!r} used before its wait: {y!r}"
            checked += 1
    assert checked >= 16, checked        # the 16 scale loads of a K-group kernel at least
