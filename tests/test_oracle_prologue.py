"""Pins the prologue oracle, RoPE tables and positions (CPU only).

H3RMSNorm (Modulation.swift:116-120) -> SplitHalfRoPE (DiTBlock.swift:83-103):
an independent numpy restatement must agree bit for bit with the C oracle,
and the invariants a rotation and a normalisation must satisfy hold.
"""
import numpy as np
import pytest


def numpy_mean_square(x, rot):
    """The prologue's fixed fp32 reduction order, vectorised over rows."""
    hl = rot // 16
    sj = []
    for j in range(8):
        ca = j if j < hl else 2 * hl + 2 * (j - hl)
        cb = j + hl if j < hl else ca + 1
        acc = np.zeros(x.shape[:-1], dtype=np.float32)
        for c in (ca, cb):
            for i in range(8):
                v = x[..., 8 * c + i].astype(np.float64)
                acc = (v * v + acc.astype(np.float64)).astype(np.float32)   # fma: one rounding
        sj.append(acc)
    t = [sj[0] + sj[7], sj[1] + sj[6], sj[2] + sj[5], sj[3] + sj[4]]
    return (((t[0] + t[2]) + (t[1] + t[3])) * np.float32(1.0 / 128.0))[..., None]


def numpy_reference_prologue(orc, x_bits, S, H, D, gamma_bits, eps, pos, axis, inv, rot):
    """Row-vectorised restatement with the reference's bf16 rounding points."""
    x = orc.bf16_to_f32(x_bits).reshape(S, H, D)
    g = orc.bf16_to_f32(gamma_bits)
    ms = numpy_mean_square(x, rot)
    r = (1.0 / np.sqrt((ms + np.float32(eps)).astype(np.float64))).astype(np.float32)
    y = ((x * r).astype(np.float32) * g).astype(np.float32)
    yb = orc.bf16_to_f32(orc.f32_to_bf16(y))
    half = rot // 2
    ang = (pos[:, axis].astype(np.float32) * inv[None, :]).astype(np.float32)   # [S, half]
    c = orc.bf16_to_f32(orc.f32_to_bf16(np.cos(ang.astype(np.float64)).astype(np.float32)))
    s = orc.bf16_to_f32(orc.f32_to_bf16(np.sin(ang.astype(np.float64)).astype(np.float32)))
    rb = lambda t: orc.bf16_to_f32(orc.f32_to_bf16(t.astype(np.float32)))
    a, b = yb[..., :half], yb[..., half:rot]
    c, s = c[:, None, :], s[:, None, :]
    out = yb.copy()
    out[..., :half] = rb(rb(c * a) + rb(-s * b))
    out[..., half:rot] = rb(rb(s * a) + rb(c * b))
    return orc.f32_to_bf16(out).transpose(1, 0, 2)   # [H, S, D]


def make_inputs(orc, S=37, H=3, D=128, seed=1, ld_extra=0):
    x = orc.randn_bf16((S, H * D + ld_extra), seed)
    gamma = orc.uniform_bf16((D,), seed + 1, 0.9, 1.1)
    pos = orc.positions_grid(5, 2, 4, 4)[:S]
    return x, gamma, pos


@pytest.mark.parametrize("rot,dims", [(128, (32, 48, 48)), (96, None)])
def test_c_oracle_matches_numpy_restatement(orc, rot, dims):
    S, H, D = 37, 3, 128
    x, gamma, pos = make_inputs(orc, S, H, D)
    if dims is not None:
        axis, inv = orc.rope_pairs_axes(10000.0, *dims)
    else:
        axis, inv = orc.rope_pairs_h3(np.float32(10000.0) ** (-np.arange(16, dtype=np.float32) / 16))
    got = orc.qk_norm_rope(x, H * D, S, S, H, D, gamma, 1e-6, pos, axis, inv, rot)
    want = numpy_reference_prologue(orc, x[:, :H * D], S, H, D, gamma, 1e-6, pos, axis, inv, rot)
    assert np.array_equal(got, want)


def test_position_zero_is_identity_and_tail_passes_through(orc):
    S, H, D = 16, 2, 128
    x, gamma, _ = make_inputs(orc, S, H, D)
    pos = np.zeros((S, 3), dtype=np.float32)
    axis, inv = orc.rope_pairs_h3(np.linspace(1, 0.01, 16).astype(np.float32))
    normed = orc.qk_norm_rope(x, H * D, S, S, H, D, gamma, 1e-6, pos, axis, inv, 96)
    # At position 0 every rotation is the identity: the output is bf16(y).
    xf = orc.bf16_to_f32(x).reshape(S, H, D)
    r = (1.0 / np.sqrt((numpy_mean_square(xf, 96) + np.float32(1e-6))
                       .astype(np.float64))).astype(np.float32)
    y = orc.f32_to_bf16(((xf * r).astype(np.float32) * orc.bf16_to_f32(gamma)).astype(np.float32))
    assert np.array_equal(normed, y.transpose(1, 0, 2))
    # Channels >= rot pass through bit-exactly at any position.
    pos2 = orc.positions_grid(0, 1, 4, 4)
    rotd = orc.qk_norm_rope(x, H * D, S, S, H, D, gamma, 1e-6, pos2, axis, inv, 96)
    assert np.array_equal(rotd[..., 96:], normed[..., 96:])
    assert not np.array_equal(rotd[..., :96], normed[..., :96])


def test_rotation_preserves_pair_norms_and_unit_rms(orc):
    S, H, D = 40, 2, 128
    x, _, pos = make_inputs(orc, S, H, D)
    pos = orc.positions_grid(8, 2, 4, 4)
    ones = orc.f32_to_bf16(np.ones(D, dtype=np.float32))
    axis, inv = orc.rope_pairs_axes(10000.0, 32, 48, 48)
    zero = np.zeros_like(pos)
    a = orc.bf16_to_f32(orc.qk_norm_rope(x, H * D, S, S, H, D, ones, 1e-6, zero, axis, inv, 128,
                                         orc.ROUND_FP32)).astype(np.float64)
    b = orc.bf16_to_f32(orc.qk_norm_rope(x, H * D, S, S, H, D, ones, 1e-6, pos, axis, inv, 128,
                                         orc.ROUND_FP32)).astype(np.float64)
    na = a[..., :64] ** 2 + a[..., 64:] ** 2
    nb = b[..., :64] ** 2 + b[..., 64:] ** 2
    assert np.max(np.abs(na - nb) / (na + 1e-3)) < 0.02      # bf16 store only
    rms = np.sqrt(np.mean(b ** 2, axis=-1))
    assert np.max(np.abs(rms - 1.0)) < 4e-3
    # Prefix rows sit at position 0 and are unrotated; the video rows moved.
    assert np.array_equal(a[:, :8], b[:, :8])
    assert np.mean(np.abs(a[:, 8:] - b[:, 8:])) > 0.05


def test_reference_and_fp32_roundings_are_close(orc):
    S, H, D = 64, 2, 128
    x, gamma, pos = make_inputs(orc, S, H, D)
    pos = orc.positions_grid(0, 4, 4, 4)
    axis, inv = orc.rope_pairs_axes(10000.0, 32, 48, 48)
    r = orc.bf16_to_f32(orc.qk_norm_rope(x, H * D, S, S, H, D, gamma, 1e-6, pos, axis, inv, 128))
    f = orc.bf16_to_f32(orc.qk_norm_rope(x, H * D, S, S, H, D, gamma, 1e-6, pos, axis, inv, 128,
                                         orc.ROUND_FP32))
    assert np.sqrt(np.mean((r - f) ** 2)) / np.sqrt(np.mean(f ** 2)) < 1e-2


def test_padding_rows_are_zero_and_stride_is_honoured(orc):
    S, S_pad, H, D = 20, 32, 2, 128
    x, gamma, pos = make_inputs(orc, S, H, D, ld_extra=3 * 8)
    axis, inv = orc.rope_pairs_axes(10000.0, 32, 48, 48)
    out = orc.qk_norm_rope(x, H * D + 24, S, S_pad, H, D, gamma, 1e-6, pos, axis, inv, 128)
    assert np.all(out[:, S:] == 0)
    dense = orc.qk_norm_rope(np.ascontiguousarray(x[:, :H * D]), H * D, S, S, H, D, gamma, 1e-6,
                             pos, axis, inv, 128)
    assert np.array_equal(out[:, :S], dense)


def test_rope_pair_tables(orc):
    axis, inv = orc.rope_pairs_axes(10000.0, 32, 48, 48)
    assert list(np.bincount(axis)) == [16, 24, 24]
    assert inv[0] == 1.0 and inv[16] == 1.0 and inv[40] == 1.0
    assert inv[15] == np.float32(1.0 / 10000.0 ** (30 / 32))
    assert inv[39] == np.float32(1.0 / 10000.0 ** (46 / 48))
    f = np.arange(1, 17, dtype=np.float32)
    ax3, inv3 = orc.rope_pairs_h3(f)
    assert list(ax3) == [p // 16 for p in range(48)]
    assert np.array_equal(inv3, np.tile(f, 3))


def test_positions_grid(orc):
    pos = orc.positions_grid(3, 2, 2, 3)
    assert pos.shape == (15, 3)
    assert np.all(pos[:3] == 0)
    assert list(pos[3]) == [0, 0, 0] and list(pos[3 + 6 + 4]) == [1, 1, 1]


def test_positions_packed_matches_packed_layout(orc):
    """PackedLayout at 864x480x124 (PackedLayoutTests.swift geometry): latentT
    37, audioT 207, latent 30x54 -> 15x27 patches per frame."""
    text, audio_t, lt, lh, lw = 52, 207, 37, 30, 54
    pos = orc.positions_packed(text, audio_t, lt, lh, lw)
    assert pos.shape == (52 + 414 + 37 * 405, 3)
    assert np.array_equal(pos[:52, 0], np.arange(52)) and np.all(pos[:52, 1:] == 0)
    area = np.sqrt(30.0 * 54.0)
    w_axis = [((i * ((54 / area) / 27)) + (1 - 54 / area) / 2) * 32 for i in range(27)]
    h_axis = [((i * ((30 / area) / 15)) + (1 - 30 / area) / 2) * 32 for i in range(15)]
    audio = pos[52:52 + 414]
    assert np.array_equal(audio[:207, 0], 52 + np.arange(207.0))
    assert np.all(audio[:207, 2] == w_axis[0]) and np.all(audio[207:, 2] == w_axis[-1])
    video = pos[466:].reshape(37, 15, 27, 3)
    spans = [5.0 / 3.0 * [1, 4, 4, 4, 4][k % 5] for k in range(37)]
    t = 52.0
    for k in range(37):
        assert np.all(video[k, :, :, 0] == t)
        t += spans[k]
    assert np.allclose(video[0, :, 0, 1], h_axis, rtol=0, atol=1e-12)
    assert np.allclose(video[0, 0, :, 2], w_axis, rtol=0, atol=1e-12)
    # The lattice identity (PackedLayoutTests.swift:62-81): spans cover 124 frames.
    assert sum([1, 4, 4, 4, 4][k % 5] for k in range(37)) == 124


@pytest.mark.parametrize("rot,h3", [(128, False), (96, True)])
def test_rope_table_pins(orc, rot, h3):
    """orc_rope_table (H3RoPE.rotationTable, H3Transformer.swift:62-78): the
    [[c, -s], [s, c]] structure, identity at position 0, points on the unit
    circle, REFERENCE entries = bf16 of the FP32 entries, and -- tying it to
    the pinned prologue oracle -- rotating the position-0 (unrotated) output
    of orc_qk_norm_rope with the table's entries in numpy reproduces its
    rotated output bit for bit. A swapped sign, a c/s swap or a wrong pair ->
    axis mapping fails the last check."""
    S, H, D = 37, 3, 128
    x, gamma, pos = make_inputs(orc, S, H, D, seed=5)
    pos = pos + np.float32(0.37) * (np.arange(S, dtype=np.float32)[:, None] % 5)  # non-integer too
    pos[:5] = 0.0
    if h3:
        axis, inv = orc.rope_pairs_h3((1.0 / 10000.0 ** (np.arange(16) / 16)).astype(np.float32))
    else:
        axis, inv = orc.rope_pairs_axes(10000.0, 32, 48, 48)
    axis, inv = axis[:rot // 2], inv[:rot // 2]
    half = rot // 2
    tr = orc.rope_table(pos, axis, inv, rot, orc.ROUND_REFERENCE)
    tf = orc.rope_table(pos, axis, inv, rot, orc.ROUND_FP32)
    assert tr.shape == (S, half, 4) and tr.dtype == np.uint16
    assert tf.shape == (S, half, 4) and tf.dtype == np.float32
    # Structure.
    assert np.array_equal(tr[..., 0], tr[..., 3]) and np.array_equal(tr[..., 1], tr[..., 2] ^ 0x8000)
    assert np.array_equal(tf[..., 0], tf[..., 3]) and np.array_equal(tf[..., 1], -tf[..., 2])
    # Position 0 is the identity rotation.
    assert np.all(tf[:5, :, 0] == 1.0) and np.all(tf[:5, :, 2] == 0.0)
    # Unit circle (fp32 cos and sin, each rounded once).
    c, s = tf[..., 0].astype(np.float64), tf[..., 2].astype(np.float64)
    assert np.max(np.abs(c * c + s * s - 1.0)) < 4e-7
    # REFERENCE = bf16(FP32).
    assert np.array_equal(tr, orc.f32_to_bf16(tf))
    # Tie to orc_qk_norm_rope: rotate its unrotated output with the table.
    unrot = orc.qk_norm_rope(x, H * D, S, S, H, D, gamma, 1e-6, np.zeros_like(pos), axis, inv,
                             rot, orc.ROUND_REFERENCE)
    want = orc.qk_norm_rope(x, H * D, S, S, H, D, gamma, 1e-6, pos, axis, inv, rot,
                            orc.ROUND_REFERENCE)
    a = orc.bf16_to_f32(unrot[..., :half])
    b = orc.bf16_to_f32(unrot[..., half:rot])
    tc = orc.bf16_to_f32(tr[..., 0])[None]      # [1, S, half]
    tns = orc.bf16_to_f32(tr[..., 1])[None]
    ts = orc.bf16_to_f32(tr[..., 2])[None]
    rb = lambda t: orc.bf16_to_f32(orc.f32_to_bf16(t.astype(np.float32)))
    got = unrot.copy()
    got[..., :half] = orc.f32_to_bf16(rb(rb(tc * a) + rb(tns * b)))
    got[..., half:rot] = orc.f32_to_bf16(rb(rb(ts * a) + rb(tc * b)))
    assert np.array_equal(got, want)
    # The rotation is not trivially the identity on these inputs.
    assert not np.array_equal(unrot, want)
