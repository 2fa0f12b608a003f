"""Register budgets of the prefill kernels (CPU: compiles the sources for gfx950 to AMD
assembly and reads each kernel's resource descriptor).

The grouped GEMM's speed depends on its row classes fitting their VGPR budgets: a
change that adds live registers makes the compiler spill to scratch memory, which cost
~15 % per call when it happened.  The bars are the spill bytes of the kept build: none
for the 16- and 64-row classes, the FP4, f32 and wide-tile GEMMs (the eight-wave form, the
default; each of its waves must stay within 256 VGPRs, two waves per SIMD); at most 32
bytes elsewhere.
"""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "micro-vllm_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"


def kernel_resources(src, tmp_path):
    out = tmp_path / (os.path.basename(src) + ".s")
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang",
                    "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only",
                    "-S", "-o", str(out), src], check=True, capture_output=True)
    text = out.read_text()
    res = {}
    for m in re.finditer(r"\.amdhsa_kernel (\S+)\n(.*?)\.end_amdhsa_kernel", text, re.S):
        body = m.group(2)
        res[m.group(1)] = (int(re.search(r"private_segment_fixed_size (\d+)", body).group(1)),
                           int(re.search(r"next_free_vgpr (\d+)", body).group(1)))
    return res


def demangle(names):
    p = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True,
                       check=True)
    return dict(zip(names, p.stdout.split("\n")))


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_gemm_classes_within_register_budget(tmp_path):
    res = kernel_resources(os.path.join(CSRC, "kern_gemm.hip"), tmp_path)
    names = demangle(list(res))
    seen = 0
    for mangled, (scratch, vgpr) in res.items():
        m = re.search(r"k_gemm<(\d), (true|false), (\d), (\d), (true|false)>", names[mangled])
        if not m:
            continue
        seen += 1
        mt = int(m.group(4))
        bar = 0 if mt in (1, 4) else 32
        assert scratch <= bar, f"{names[mangled]}: {scratch} bytes of scratch (bar {bar})"
        assert vgpr <= 256
    assert seen >= 28


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
@pytest.mark.parametrize("src,kernel", [("kern_fp4.hip", "k_gemm_fp4"),
                                        ("kern_f32.hip", "k_f32mm"),
                                        ("kern_wide.hip", "k_gemm_wide<true, 8, 4, 8>"),
                                        ("kern_wide.hip", "k_gemm_wide<false, 8, 4, 8>")])
def test_other_gemms_spill_free(tmp_path, src, kernel):
    res = kernel_resources(os.path.join(CSRC, src), tmp_path)
    names = demangle(list(res))
    hits = [(names[k], v) for k, v in res.items() if kernel in names[k]]
    assert hits
    for name, (scratch, vgpr) in hits:
        assert scratch == 0, f"{name}: {scratch} bytes of scratch"
        assert vgpr <= 256, f"{name}: {vgpr} VGPRs"
