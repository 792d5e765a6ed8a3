"""Code-generation properties the kernels' performance rests on, checked on the
CPU by compiling them to gfx950 assembly.

- bsattn_fwd.hip: the tile loops feed each MFMA from LDS reads issued four
  MFMAs ahead. The compiler drops to single-buffered reads (`s_waitcnt
  lgkmcnt(0)` right before almost every MFMA, 30-40% slower) when a change
  shifts its register budget, even a change outside the loops. Today 3 of the
  80 MFMAs follow `lgkmcnt(0)` (the first reads of a phase); more than 8 means
  the pipelines collapsed.
- bsattn_fwd.hip and qkv_proj.hip: no VGPR spills (scratch traffic in the
  tile loops) in any instantiation (four fused QKV forms, the plain QKV GEMM
  and the out-projection).

A different compiler release may schedule differently; a failure here says
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


def _mfma_after_full_wait(asm):
    ins = [l.strip() for l in asm.splitlines() if l.strip() and not l.strip().startswith(";")]
    mfma = [i for i, l in enumerate(ins) if l.startswith("v_mfma")]
    return len(mfma), sum(1 for i in mfma if ins[i - 1].startswith("s_waitcnt lgkmcnt(0)"))


def test_attention_operand_pipelines_intact(tmp_path):
    asm = _asm(tmp_path, "bsattn_fwd")
    n, after_wait = _mfma_after_full_wait(asm)
    assert n == 80, n
    assert after_wait <= 8, (f"{after_wait} of {n} MFMAs wait for all LDS reads: the compiler "
                             "single-buffered the tile loops' operand reads")
    spills = [int(x) for x in re.findall(r"\.vgpr_spill_count:\s+(\d+)", asm)]
    assert spills and max(spills) == 0, spills


def test_projection_no_vgpr_spills(tmp_path):
    asm = _asm(tmp_path, "qkv_proj")
    spills = [int(x) for x in re.findall(r"\.vgpr_spill_count:\s+(\d+)", asm)]
    assert len(spills) == 6 and max(spills) == 0, spills
