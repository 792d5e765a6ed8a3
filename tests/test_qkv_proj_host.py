"""Host-side checks of the QKV projection kernel (csrc/qkv_proj.hip) that need
no GPU.

- Its launch order (csrc/tile_order.h, compiled here with g++): the 8 XCD
  lists together hold every (token tile, channel tile) exactly once, for the
  benchmark shapes and for small and ragged grids, and their lengths stay
  within two chunks of each other.
- Its hand-written HBM -> LDS loads: `buffer_load ... lds` is inline assembly,
  so the compiler's hazard padding does not see it. The GFX9/CDNA3 rule "VALU
  writes an SGPR -> VMEM reads that SGPR: 5 wait states" therefore has to
  hold by construction. Compiling the kernel to gfx950 assembly and scanning
  each such load's SGPR operands (resource and scalar offset) for a VALU
  write (e.g. `v_readlane_b32` restoring a spilled SGPR) fewer than 5 wait
  states earlier catches a register allocation that would feed a load a stale
  offset.
- Its main loop's first LDS wait: the compiler must wait only for the reads
  the first MFMA needs, not for every read in flight.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "minimax-h3-swift_amd", "csrc")

HARNESS = r"""
#include "tile_order.h"
#include <cstdio>
#include <cstdlib>
#include <set>
using h3hip::TileOrder;
int main(int argc, char** argv) {
  for (int a = 1; a + 1 < argc; a += 2) {
    const TileOrder o{std::atoi(argv[a]), std::atoi(argv[a + 1])};
    std::set<int> seen;
    long n = 0;
    int lo = 1 << 30, hi = 0;
    bool ok = true;
    for (int x = 0; x < h3hip::kOrderXcds; x++) {
      const int len = o.length(x);
      lo = len < lo ? len : lo;
      hi = len > hi ? len : hi;
      for (int p = 0; p < len; p++) {
        const int t = o.tile(x, p), tm = t >> 16, tn = t & 0xffff;
        ok &= tm >= 0 && tm < o.tiles_m && tn >= 0 && tn < o.tiles_n;
        seen.insert(t);
        n++;
      }
    }
    ok &= n == (long)o.tiles_m * o.tiles_n && (long)seen.size() == n;
    std::printf("%d %d %d %d %d\n", o.tiles_m, o.tiles_n, ok ? 1 : 0, lo, hi);
  }
  return 0;
}
"""

# (token tiles, channel tiles): cfg3 (S 31,885 -> 125 x 60 at 40 heads),
# cfg2/cfg4 (S 18,102 -> 71 x 60), the axial H3 shape (56 heads -> 84), and
# small or ragged grids (fewer tiles than XCDs, a short last chunk).
SHAPES = [(125, 60), (71, 60), (126, 84), (250, 60), (1, 3), (2, 3), (1, 2), (3, 6),
          (5, 30), (7, 2), (64, 2), (9, 9), (4, 1), (13, 7)]


def test_tile_order_covers_every_tile_once(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    src = tmp_path / "order.cpp"
    src.write_text(HARNESS)
    exe = tmp_path / "order"
    subprocess.run([gxx, "-O1", "-std=c++17", f"-I{CSRC}", str(src), "-o", str(exe)], check=True)
    args = [str(v) for s in SHAPES for v in s]
    out = subprocess.run([str(exe)] + args, check=True, capture_output=True, text=True).stdout
    rows = [list(map(int, line.split())) for line in out.strip().splitlines()]
    assert len(rows) == len(SHAPES)
    for tm, tn, ok, lo, hi in rows:
        assert ok == 1, (tm, tn)
        if tm * tn >= 8 * 8:
            assert hi - lo <= 8, (tm, tn, lo, hi)     # at most two chunks apart


def _sregs(tok):
    m = re.match(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"s(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def _dma_hazards(asm_text):
    """(loads, hazards): `buffer_load ... lds` whose resource or scalar offset
    was written by a VALU instruction fewer than 5 wait states before."""
    ins = []
    for line in asm_text.splitlines():
        s = line.strip()
        if not s or s.startswith((";", ".")) or re.match(r"^[\w.$]+:", s):
            continue
        ins.append(s.split(";")[0].strip())
    loads = hazards = 0
    for i, s in enumerate(ins):
        if not (s.startswith("buffer_load") and s.endswith(" lds")):
            continue
        loads += 1
        ops = [t.strip() for t in s.split(None, 1)[1].split(",")]
        reads = set()
        for t in ops[1:3]:
            reads |= _sregs(t.split()[0])
        waits, j = 0, i - 1
        while j >= 0 and waits < 5:
            p = ins[j]
            if p.startswith("s_nop"):
                waits += int(p.split()[1]) + 1
            else:
                if p.startswith("v_") and " " in p:
                    if _sregs(p.split(None, 1)[1].split(",")[0].strip()) & reads:
                        hazards += 1
                waits += 1
            j -= 1
    return loads, hazards


def test_dma_scan_finds_a_planted_hazard():
    """The scanner itself: a VALU write of the scalar offset right before the
    load is flagged; the same write five wait states earlier is not."""
    bad = "v_readlane_b32 s2, v255, 9\ns_mov_b32 m0, s3\ns_nop 0\nbuffer_load_dwordx4 v1, s[28:31], s2 offen lds\n"
    good = "v_readlane_b32 s2, v255, 9\ns_nop 4\nbuffer_load_dwordx4 v1, s[28:31], s2 offen lds\n"
    assert _dma_hazards(bad) == (1, 1)
    assert _dma_hazards(good) == (1, 0)


@pytest.fixture(scope="module")
def qkv_asm(tmp_path_factory):
    """gfx950 assembly of csrc/qkv_proj.hip."""
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not found")
    out = tmp_path_factory.mktemp("asm") / "qkv_proj.s"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
                    "-Xclang", "-packed-fp32-ops", f"-I{CSRC}", f"-I{os.path.join(ROOT, 'include')}",
                    "--cuda-device-only", "-S", "-o", str(out), os.path.join(CSRC, "qkv_proj.hip")],
                   check=True, capture_output=True)
    return out.read_text()


def test_qkv_proj_dma_loads_hazard_free(qkv_asm):
    loads, hazards = _dma_hazards(qkv_asm)
    assert loads > 0
    assert hazards == 0, f"{hazards} of {loads} LDS-DMA loads read an SGPR a VALU op wrote < 5 wait states earlier"


def test_main_loop_head_waits_only_for_its_operands(qkv_asm):
    """The first MFMA of each reduction step needs two operand reads issued
    early in the previous step; ten reads issued after them may still be in
    flight. A wait for (nearly) all reads at the loop head -- what the
    compiler emits when the reads before the loop come in another order than
    the loop's -- idles the matrix cores at every step."""
    lines = qkv_asm.splitlines()
    heads = [i for i, ln in enumerate(lines) if "Inner Loop Header" in ln]
    assert len(heads) == 6   # one main loop per kernel instantiation
    for i in heads:
        wait = next(re.search(r"lgkmcnt\((\d+)\)", ln) for ln in lines[i:i + 20]
                    if "s_waitcnt" in ln and "lgkmcnt" in ln)
        assert int(wait.group(1)) >= 8, lines[i:i + 12]
