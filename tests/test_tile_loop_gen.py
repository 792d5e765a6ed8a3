"""The attention tile loop is generated assembly (csrc/gen_tile_loop.py ->
csrc/bsattn_tile_loop.inc) with registers and wait states assigned by hand.
These CPU tests check that the committed include is what the generator
writes, and scan the generated instruction stream for the hazards the
hardware does not interlock and the generator must space out itself:

- a v_dot2c result read by a plain VALU instruction (dot runs on the matrix
  pipeline; a read within 4 wait states sees the old value -- this produced a
  per-row scale error in l before the gap existed);
- a v_exp_f32 result consumed by the next instruction;
- a VGPR written by VALU and read by v_permlane32_swap within 2 wait states;
- M0 written and used by an LDS DMA load in the next instruction;
- an operand-ring entry overwritten by a ds_read while the MFMA that reads it
  is the last instruction issued;
- an MFMA result read by a VALU instruction fewer than 12 wait states later
  within straight-line code;
- ds_read waits: every MFMA reading a ring entry is preceded by an
  s_waitcnt lgkmcnt(N) that leaves only later reads outstanding.
"""
import importlib.util
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "minimax-h3-swift_amd", "csrc")


@pytest.fixture(scope="module")
def gen():
    spec = importlib.util.spec_from_file_location("gen_tile_loop",
                                                  os.path.join(CSRC, "gen_tile_loop.py"))
    g = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(g)
    return g


@pytest.fixture(scope="module")
def lines(gen):
    return gen.generate()


def _regs(text):
    """Register numbers named by an operand list ('v5', 'v[4:7]', 'a[0:15]')."""
    out = set()
    text = re.sub(r"%\[\w+\]", "", text)   # named asm operands are SGPR inputs
    for kind, a, b in re.findall(r"\b([va])\[(\d+):(\d+)\]", text):
        out.update((kind, i) for i in range(int(a), int(b) + 1))
    text = re.sub(r"\b[va]\[\d+:\d+\]", "", text)
    for kind, a in re.findall(r"\b([va])(\d+)\b", text):
        out.add((kind, int(a)))
    return out


def _split(line):
    op, _, rest = line.partition(" ")
    parts = [p.strip() for p in rest.split(",")]
    return op, parts


def _wait_states(line):
    m = re.match(r"s_nop (\d+)", line)
    return int(m.group(1)) + 1 if m else 1


def _straight_segments(lines):
    """Runs of instructions without labels or branches."""
    seg = []
    for ln in lines:
        if ln.endswith(":") or ln.startswith("s_cbranch") or ln.startswith("s_branch"):
            if seg:
                yield seg
            seg = []
            continue
        seg.append(ln)
    if seg:
        yield seg


def _reads_within(seg, i, dst, states, reader):
    """True if an instruction accepted by `reader` reads a register of `dst`
    within `states` wait states after seg[i]."""
    gap = 0
    for ln in seg[i + 1:]:
        if gap >= states:
            return False
        op, parts = _split(ln)
        if reader(op) and len(parts) > 1 and _regs(",".join(parts[1:])) & dst:
            return True
        if reader(op) and op.startswith("v_dot2c") and _regs(parts[0]) & dst:
            return True
        gap += _wait_states(ln)
    return False


def test_include_is_current(gen):
    path = os.path.join(CSRC, "bsattn_tile_loop.inc")
    assert open(path).read() == gen.render(), "run python3 gen_tile_loop.py in csrc/"


def test_register_budget(gen, lines):
    text = "\n".join(lines)
    vmax = max(i for k, i in _regs(text) if k == "v")
    amax = max(i for k, i in _regs(text) if k == "a")
    # Two waves per SIMD with AGPRs in use: at most 128 of each.
    assert vmax < 128 and amax < 128, (vmax, amax)


def test_dot_results_not_read_early(lines):
    for seg in _straight_segments(lines):
        for i, ln in enumerate(seg):
            if ln.startswith("v_dot2c"):
                dst = _regs(_split(ln)[1][0])
                plain = lambda op: op.startswith("v_") and not op.startswith("v_dot2c")
                assert not _reads_within(seg, i, dst, 5, plain), ln


def test_exp_results_not_read_next(lines):
    for seg in _straight_segments(lines):
        for i, ln in enumerate(seg):
            if ln.startswith("v_exp_f32"):
                dst = _regs(_split(ln)[1][0])
                assert not _reads_within(seg, i, dst, 2, lambda op: op.startswith("v_")), ln


def test_permlane_sources_settled(lines):
    for seg in _straight_segments(lines):
        for i, ln in enumerate(seg):
            op, parts = _split(ln)
            if op.startswith("v_") and not op.startswith("v_mfma") and parts and parts[0]:
                dst = _regs(parts[0])
                if not dst or any(k == "a" for k, _ in dst):
                    continue
                assert not _reads_within(seg, i, dst, 2,
                                         lambda o: o.startswith("v_permlane")), ln


def test_m0_settled_before_lds_dma(lines):
    for a, b in zip(lines, lines[1:]):
        if a.startswith("s_add_u32 m0") or a.startswith("s_mov_b32 m0"):
            assert not (b.startswith("buffer_load") and b.endswith("lds")), (a, b)


def test_ring_entry_not_overwritten_right_after_its_mfma(gen, lines):
    ring = {("a", i) for i in range(gen.RING, gen.RING + 4 * gen.RING_N)}
    for a, b in zip(lines, lines[1:]):
        if a.startswith("v_mfma") and b.startswith("ds_read"):
            src_a = _regs(_split(a)[1][1]) & ring
            dst = _regs(_split(b)[1][0])
            assert not (src_a & dst), (a, b)


def test_mfma_results_not_read_by_valu_soon(lines):
    for seg in _straight_segments(lines):
        for i, ln in enumerate(seg):
            if ln.startswith("v_mfma"):
                dst = _regs(_split(ln)[1][0])
                valu = lambda op: op.startswith("v_") and not op.startswith("v_mfma")
                assert not _reads_within(seg, i, dst, 12, valu), ln


def test_every_ring_mfma_waits_for_its_reads(gen, lines):
    """Replays lgkmcnt: each ds_read into the ring is outstanding until a wait
    leaves fewer reads pending than were issued after it."""
    ring = {("a", i) for i in range(gen.RING, gen.RING + 4 * gen.RING_N)}
    for seg in _straight_segments(lines):
        pending = []  # register sets of outstanding ring reads, oldest first
        for ln in seg:
            op, parts = _split(ln)
            if op.startswith("ds_read") and _regs(parts[0]) & ring:
                pending.append(_regs(parts[0]))
            elif op.startswith("ds_"):
                pending.append(set())
            elif op == "s_waitcnt":
                m = re.search(r"lgkmcnt\((\d+)\)", ln)
                if m:
                    keep = int(m.group(1))
                    pending = pending[len(pending) - keep:] if keep else []
            elif op.startswith("v_mfma"):
                src_a = _regs(parts[1]) & ring
                for p in pending:
                    assert not (p & src_a), f"{ln} reads a ring entry still being loaded"


def test_column_load_early_and_collected(gen, lines):
    """The next column index (s_load into SCOL) is issued at the start of its
    block, with the block's MFMAs between it and the lgkmcnt(0) that collects
    it, and nothing reads SCOL before that wait."""
    loads = [i for i, ln in enumerate(lines) if ln.startswith("s_load_dword")]
    assert loads
    for i in loads:
        assert lines[i].split()[1].rstrip(",") == gen.SCOL
        j = next(k for k in range(i + 1, len(lines)) if "lgkmcnt(0)" in lines[k])
        between = lines[i + 1:j]
        assert sum(ln.startswith("v_mfma") for ln in between) >= 8, lines[i]
        assert not any(gen.SCOL in ln for ln in between), lines[i]
