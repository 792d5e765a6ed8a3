"""Code-generation properties the kernels' performance rests on, checked on the
CPU by compiling them to gfx950 assembly.

- bsattn_fwd.hip: the tile loop is one inline-assembly block with registers
  assigned by hand (bsattn_tile_loop.inc); the compiled kernel must carry all
  of its MFMAs, keep two waves per SIMD (at most 128 VGPRs and 128 AGPRs),
  and spill nothing to scratch around it (lane values are rebuilt per unit
  from an opaque thread index for that reason).
- bsattn_fwd.hip and qkv_proj.hip: no VGPR spills (scratch traffic) in any
  instantiation (four fused QKV forms, the plain QKV GEMM and the
  out-projection).

A different compiler release may allocate differently; a failure here says
to re-measure the kernel, not that its results are wrong.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "minimax-h3-swift_amd", "csrc")


def _asm(tmp_path, name):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not found")
    out = tmp_path / (name + ".s")
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
                    "-Xclang", "-packed-fp32-ops", f"-I{CSRC}", f"-I{os.path.join(ROOT, 'include')}",
                    "--cuda-device-only", "-S", "-o", str(out), os.path.join(CSRC, name + ".hip")],
                   check=True, capture_output=True)
    return out.read_text()


def test_attention_tile_loop_compiled_whole(tmp_path):
    asm = _asm(tmp_path, "bsattn_fwd")
    inc = open(os.path.join(CSRC, "bsattn_tile_loop.inc")).read()
    want = int(re.search(r"// \d+ lines, (\d+) MFMAs", inc).group(1))
    n = sum(1 for l in asm.splitlines() if l.strip().startswith("v_mfma_f32_32x32x16_bf16"))
    assert n == want, (n, want)
    spills = [int(x) for x in re.findall(r"\.vgpr_spill_count:\s+(\d+)", asm)]
    assert spills and max(spills) == 0, spills
    scratch = [int(x) for x in re.findall(r"\.private_segment_fixed_size:\s+(\d+)", asm)]
    assert scratch and max(scratch) == 0, scratch
    agpr = [int(x) for x in re.findall(r"\.agpr_count:\s+(\d+)", asm)]
    vgpr = [int(x) for x in re.findall(r"\.vgpr_count:\s+(\d+)", asm)]
    assert max(agpr) <= 128 and max(vgpr) <= 256, (agpr, vgpr)


def test_projection_no_vgpr_spills(tmp_path):
    asm = _asm(tmp_path, "qkv_proj")
    spills = [int(x) for x in re.findall(r"\.vgpr_spill_count:\s+(\d+)", asm)]
    assert len(spills) == 6 and max(spills) == 0, spills
