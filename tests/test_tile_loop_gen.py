"""The attention tile loop is generated assembly (csrc/gen_tile_loop.py ->
csrc/bsattn_tile_loop.inc) with registers and wait states assigned by hand.
These CPU tests check that the committed include is what the generator
writes, and scan the generated instruction stream for the hazards the
hardware does not interlock and the generator must space out itself:

- a v_exp_f32 result consumed by the next instruction;
- a VGPR written by VALU and read by v_permlane32_swap within 2 wait states;
- M0 written and used by an LDS DMA load in the next instruction;
- an operand-ring entry overwritten by a ds_read while the MFMA that reads it
  is the last instruction issued;
- an MFMA result read by a VALU instruction fewer than 12 wait states later
  within straight-line code;
- ds_read waits: every MFMA reading a ring entry is preceded by an
  s_waitcnt lgkmcnt(N) that leaves only later reads outstanding;

and that the softmax adds every exponentiated score of a tile into the row
sum exactly once, after its exponential. Each scan is also run on a copy of
the stream with one such mistake planted, and must find it.
"""
import importlib.util
import os
import re

import numpy as np

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


def exp_read_next(lines):
    bad = []
    for seg in _straight_segments(lines):
        for i, ln in enumerate(seg):
            if ln.startswith("v_exp_f32"):
                dst = _regs(_split(ln)[1][0])
                if _reads_within(seg, i, dst, 2, lambda op: op.startswith("v_")):
                    bad.append(ln)
    return bad


def permlane_unsettled(lines):
    bad = []
    for seg in _straight_segments(lines):
        for i, ln in enumerate(seg):
            op, parts = _split(ln)
            if op.startswith("v_") and not op.startswith("v_mfma") and parts and parts[0]:
                dst = _regs(parts[0])
                if not dst or any(k == "a" for k, _ in dst):
                    continue
                if _reads_within(seg, i, dst, 2, lambda o: o.startswith("v_permlane")):
                    bad.append(ln)
    return bad


def m0_unsettled(lines):
    return [(a, b) for a, b in zip(lines, lines[1:])
            if (a.startswith("s_add_u32 m0") or a.startswith("s_mov_b32 m0"))
            and b.startswith("buffer_load") and b.endswith("lds")]


def ring_overwritten(gen, lines):
    ring = {("a", i) for i in range(gen.RING, gen.RING + 4 * gen.RING_N)}
    return [(a, b) for a, b in zip(lines, lines[1:])
            if a.startswith("v_mfma") and b.startswith("ds_read")
            and _regs(_split(a)[1][1]) & ring & _regs(_split(b)[1][0])]


def mfma_read_soon(lines):
    bad = []
    valu = lambda op: op.startswith("v_") and not op.startswith("v_mfma")
    for seg in _straight_segments(lines):
        for i, ln in enumerate(seg):
            if ln.startswith("v_mfma") and _reads_within(seg, i, _regs(_split(ln)[1][0]), 12, valu):
                bad.append(ln)
    return bad


def ring_unwaited(gen, lines):
    """Replays lgkmcnt: each ds_read into the ring is outstanding until a wait
    leaves fewer reads pending than were issued after it."""
    ring = {("a", i) for i in range(gen.RING, gen.RING + 4 * gen.RING_N)}
    bad = []
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
                if any(p & src_a for p in pending):
                    bad.append(ln)
    return bad


def row_sum_gaps(gen, ops, sb):
    """Scores of S(sb) not added into the row-sum chains (LA, LB) exactly once
    after their exponential."""
    chains = {("v", gen.LA), ("v", gen.LB)}
    x = {("v", gen.s_reg(sb, i)) for i in range(32)}
    done, added, bad = set(), {}, []
    for ln in ops:
        op, parts = _split(ln)
        if op == "v_exp_f32":
            done |= _regs(parts[0]) & x
        elif op == "v_add_f32" and _regs(parts[0]) & chains:
            for r in _regs(",".join(parts[1:])) & x:
                if r not in done:
                    bad.append(ln)
                added[r] = added.get(r, 0) + 1
    return bad + [r for r in sorted(x) if added.get(r, 0) != 1]


def _plant_after(lines, pred, extra):
    i = next(k for k, ln in enumerate(lines) if pred(ln))
    return lines[:i + 1] + [extra(lines[i])] + lines[i + 1:]


def test_exp_results_not_read_next(lines):
    assert exp_read_next(lines) == []
    dst = lambda ln: _split(ln)[1][0]
    planted = _plant_after(lines, lambda ln: ln.startswith("v_exp_f32"),
                           lambda ln: f"v_add_f32 v122, v122, {dst(ln)}")
    assert exp_read_next(planted)


def test_permlane_sources_settled(lines):
    assert permlane_unsettled(lines) == []
    i = next(k for k, ln in enumerate(lines) if ln.startswith("v_permlane"))
    src = _split(lines[i])[1][1]
    assert permlane_unsettled(lines[:i] + [f"v_mov_b32 {src}, v96"] + lines[i:])


def test_m0_settled_before_lds_dma(lines):
    assert m0_unsettled(lines) == []
    i = next(k for k, ln in enumerate(lines) if ln.startswith("buffer_load") and ln.endswith("lds"))
    assert lines[i - 1].startswith("s_nop")
    assert m0_unsettled(lines[:i - 1] + lines[i:])


def test_ring_entry_not_overwritten_right_after_its_mfma(gen, lines):
    assert ring_overwritten(gen, lines) == []
    src_a = lambda ln: _split(ln)[1][1]
    planted = _plant_after(lines, lambda ln: ln.startswith("v_mfma") and "a[9" in src_a(ln),
                           lambda ln: f"ds_read_b128 {src_a(ln)}, v98")
    assert ring_overwritten(gen, planted)


def test_mfma_results_not_read_by_valu_soon(lines):
    assert mfma_read_soon(lines) == []
    dst = lambda ln: _split(ln)[1][0]
    planted = _plant_after(lines, lambda ln: ln.startswith("v_mfma") and dst(ln).startswith("v["),
                           lambda ln: f"v_max_f32 v122, v122, v{dst(ln)[2:].split(':')[0]}")
    assert mfma_read_soon(planted)


def test_every_ring_mfma_waits_for_its_reads(gen, lines):
    assert ring_unwaited(gen, lines) == []
    # Loosen the first wait that leaves reads outstanding before a ring MFMA.
    i = next(k for k, ln in enumerate(lines)
             if re.fullmatch(r"s_waitcnt lgkmcnt\([1-9]\d*\)", ln) and lines[k + 1].startswith("v_mfma"))
    n = int(re.search(r"\((\d+)\)", lines[i]).group(1))
    planted = lines[:i] + [f"s_waitcnt lgkmcnt({n + 1})"] + lines[i + 1:]
    assert ring_unwaited(gen, planted)


def test_row_sum_adds_every_weight_once(gen):
    for sb, pb in ((0, 0), (1, 1), (0, 1), (1, 0)):
        ops = gen.softmax_ops(sb, pb)
        assert row_sum_gaps(gen, ops, sb) == []
    ops = gen.softmax_ops(0, 0)
    i = next(k for k, ln in enumerate(ops) if ln.startswith(f"v_add_f32 v{gen.LB}, v{gen.LB}, v"))
    assert row_sum_gaps(gen, ops[:i] + ops[i + 1:], 0)          # a weight left out
    j = next(k for k, ln in enumerate(ops) if ln.startswith("v_exp_f32 v0,"))
    early = f"v_add_f32 v{gen.LA}, v{gen.LA}, {_split(ops[j])[1][0]}"
    assert row_sum_gaps(gen, ops[:j] + [early] + ops[j:], 0)   # added before its exponential


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


class _Lanes:
    """A 64-lane model of the VALU/SALU subset the softmax code uses, in fp32
    (v_exp_f32 as numpy's exp2: the same function on both sides of each
    comparison below, so equalities are exact)."""

    def __init__(self, c):
        self.v = np.zeros((128, 64), dtype=np.float32)
        self.s = {}
        self.c = np.float32(c)

    def src(self, tok):
        tok = tok.strip()
        neg = tok.startswith("-")
        tok = tok.lstrip("-")
        if tok == "%[c]":
            val = np.full(64, self.c, dtype=np.float32)
        elif re.fullmatch(r"v\d+", tok):
            val = self.v[int(tok[1:])].copy()
        elif re.fullmatch(r"s\d+", tok):
            val = np.full(64, np.uint32(self.s[tok]).view(np.float32), dtype=np.float32)
        elif tok.startswith("0x"):
            val = np.full(64, np.uint32(int(tok, 16)).view(np.float32), dtype=np.float32)
        else:
            val = np.full(64, np.float32(float(tok)), dtype=np.float32)
        return -val if neg else val

    def run(self, lines):
        for ln in lines:
            op, parts = _split(ln)
            d = parts[0]
            if op in ("s_nop",):
                continue
            if op == "s_mov_b32":
                self.s[d] = int(parts[1], 16) if parts[1].startswith("0x") else int(parts[1])
                continue
            a = [self.src(p) for p in parts[1:] if not p.startswith("s[")]
            with np.errstate(over="ignore", invalid="ignore"):
                if op == "v_fma_f32":
                    r = (a[0].astype(np.float64) * a[1] + a[2]).astype(np.float32)
                elif op == "v_exp_f32":
                    r = np.exp2(a[0])
                elif op == "v_add_f32":
                    r = a[0] + a[1]
                elif op == "v_sub_f32":
                    r = a[0] - a[1]
                elif op == "v_mul_f32":
                    r = a[0] * a[1]
                elif op == "v_max_f32":
                    r = np.maximum(a[0], a[1])
                elif op == "v_max3_f32":
                    r = np.maximum(np.maximum(a[0], a[1]), a[2])
                elif op == "v_mov_b32":
                    r = a[0]
                elif op == "v_cvt_pk_bf16_f32":
                    def bf(x):
                        u = x.view(np.uint32).astype(np.uint64)
                        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
                    r = (bf(a[0]) | (bf(a[1]) << 16)).view(np.float32)
                elif op == "v_permlane32_swap_b32":
                    i, j = int(d[1:]), int(parts[1][1:])
                    hi = self.v[i, 32:].copy()
                    self.v[i, 32:] = self.v[j, :32]
                    self.v[j, :32] = hi
                    continue
                elif op in ("v_cmp_gt_f32", "v_cmp_nge_f32"):
                    m = a[0] > a[1] if op == "v_cmp_gt_f32" else ~(a[0] >= a[1])
                    self.s[d] = m
                    continue
                elif op == "v_cndmask_b32":
                    r = np.where(self.s[parts[3]], a[1], a[0])
                else:
                    raise AssertionError(f"model has no {op}")
            self.v[int(d[1:])] = r


def _softmax_state(gen, sb, seed, lift):
    rng = np.random.default_rng(seed)
    lanes = _Lanes(c=0.1275)
    scores = rng.normal(0.0, 8.0, (32, 64)).astype(np.float32)
    # m: the running max of earlier tiles, at or above this tile's max, except
    # in the lanes listed in `lift`, whose scores then exceed m by > 2^8.
    tmax = np.maximum(scores.reshape(32, 2, 32).max(axis=(0, 1)), -1e30)
    m = (np.tile(tmax, 2) * lanes.c + rng.uniform(0.0, 3.0, 64)).astype(np.float32)
    for lane in lift:
        scores[rng.integers(32), lane] = (m[lane] + 9.0 + rng.uniform(0, 4)) / lanes.c
    for i in range(32):
        lanes.v[gen.s_reg(sb, i)] = scores[i]
    lanes.v[gen.M] = m
    lanes.v[gen.L] = rng.uniform(1.0, 50.0, 64).astype(np.float32)
    return lanes


def _p_bits(lanes, gen, pb):
    return np.stack([lanes.v[gen.p_reg(pb, kc, e)].view(np.uint32)
                     for kc in range(4) for e in range(4)])


@pytest.mark.parametrize("sb, pb", [(0, 0), (1, 1), (0, 1), (1, 0)])
def test_fast_softmax_matches_full_softmax(gen, sb, pb):
    """The block end reruns the full recurrence for the whole wave when any
    lane is marked. So: every query (lanes i and i ^ 32) the full recurrence
    raises m for has a marked lane; and with no lane marked the fast path's
    weights are the full recurrence's bit for bit, its l equal to rounding,
    and the scores are still in place."""
    for seed, lift in ((1, ()), (4, ()), (2, (3, 40)), (3, tuple(range(0, 64, 5)))):
        full = _softmax_state(gen, sb, seed, lift)
        fast = _softmax_state(gen, sb, seed, lift)
        full.run(gen.softmax_ops(sb, pb))
        fast.run(gen.softmax_fast_ops(sb, pb))
        raised = full.s[gen.RAISE]
        marked = fast.s[gen.RAISE]
        pair_marked = marked | np.roll(marked, 32)
        assert np.all(pair_marked[raised]), (seed, np.nonzero(raised & ~pair_marked))
        assert raised.any() == bool(lift) and marked.any() == bool(lift)
        if lift:
            continue
        assert np.array_equal(_p_bits(full, gen, pb), _p_bits(fast, gen, pb))
        l_fast = fast.v[gen.L] + fast.v[gen.LA]          # the block end's l += LA
        np.testing.assert_allclose(l_fast, full.v[gen.L], rtol=1e-6)
        kept = _softmax_state(gen, sb, seed, lift)
        for i in range(32):
            assert np.array_equal(fast.v[gen.s_reg(sb, i)], kept.v[gen.s_reg(sb, i)])


def test_fast_softmax_test_catches_a_dropped_weight(gen):
    """The comparison above fails when the fast path leaves a weight out of l."""
    ops = gen.softmax_fast_ops(0, 0)
    i = next(k for k, ln in enumerate(ops) if ln.startswith(f"v_add_f32 v{gen.LA}, v{gen.LA}, v"))
    full = _softmax_state(gen, 0, 1, ())
    fast = _softmax_state(gen, 0, 1, ())
    full.run(gen.softmax_ops(0, 0))
    fast.run(ops[:i] + ops[i + 1:])
    assert not np.allclose(fast.v[gen.L] + fast.v[gen.LA], full.v[gen.L], rtol=1e-6)
