"""Pins the attention oracle (CPU only).

The reference pins its own oracle relationally (AxialReferenceTests.swift:41-97):
all-keys equals unmasked SDPA, the streaming recurrence equals the masked
definition for ragged key tiles, and query chunking is exact. The same checks
run here against torch's fp32 SDPA on the CPU (an independent library), plus
closed-form special cases: constant V, a single active tile, an empty row.
"""
import numpy as np
import pytest
import torch


def rel_rms(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.sqrt(np.mean((a - b) ** 2)) / np.sqrt(np.mean(b ** 2)))


def fixture(orc, prefix=7, frames=5, h=3, w=4, heads=2, d=16, seed=4, landmarks=None):
    """AxialReferenceTests.fixture (:22-33): token-level mask = tile size 1."""
    g = np.random.default_rng(seed)
    s = prefix + frames * h * w
    landmarks = [0, frames - 1] if landmarks is None else landmarks
    rule = orc.Rule(orc.RULE_AXIAL, s, tile=1, prefix_len=prefix, frames=frames, height=h,
                    width=w, landmarks=landmarks)
    q, k, v = (g.standard_normal((heads, s, d), dtype=np.float32) for _ in range(3))
    return q, k, v, rule, 1.0 / np.sqrt(d)


def torch_sdpa(q, k, v, scale, bool_mask=None):
    mask = None if bool_mask is None else torch.from_numpy(bool_mask.astype(bool))
    with torch.no_grad():
        o = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(q)[None], torch.from_numpy(k)[None], torch.from_numpy(v)[None],
            attn_mask=mask, scale=float(scale))
    return o[0].numpy()


def test_full_selection_is_dense(orc):
    q, k, v, rule, scale = fixture(orc, landmarks=list(range(5)))
    bm = orc.tile_bitmap(rule)
    assert bm.all()
    got = orc.attend_masked(q, k, v, scale, bm, tile=1)
    assert rel_rms(got, torch_sdpa(q, k, v, scale)) < 1e-6


def test_masked_matches_torch_bool_mask(orc):
    q, k, v, rule, scale = fixture(orc)
    bm = orc.tile_bitmap(rule)
    assert 0 < bm.mean() < 1
    got = orc.attend_masked(q, k, v, scale, bm, tile=1)
    assert rel_rms(got, torch_sdpa(q, k, v, scale, bm)) < 1e-6


@pytest.mark.parametrize("key_tile", [1, 7, 16, 64, 1000])
def test_streaming_matches_masked(orc, key_tile):
    q, k, v, rule, scale = fixture(orc)
    bm = orc.tile_bitmap(rule)
    want = orc.attend_masked(q, k, v, scale, bm, tile=1)
    got = orc.attend_streaming(q, k, v, scale, bm, tile=1, key_tile=key_tile)
    assert rel_rms(got, want) < 2e-6


@pytest.mark.parametrize("chunk", [1, 5, 13, 32])
def test_query_chunking_is_exact(orc, chunk):
    q, k, v, rule, scale = fixture(orc)
    bm = orc.tile_bitmap(rule)
    base = orc.attend_masked(q, k, v, scale, bm, tile=1, query_chunk=4096)
    got = orc.attend_masked(q, k, v, scale, bm, tile=1, query_chunk=chunk)
    assert rel_rms(got, base) < 1e-6


def test_tile_mask_and_ragged_sequence(orc):
    """128-token tiles over a sequence that is not a multiple of 128: the tile
    mask expands to tokens and keys past S do not exist."""
    g = np.random.default_rng(7)
    S, H, D = 300, 2, 32
    q, k, v = (g.standard_normal((H, S, D), dtype=np.float32) for _ in range(3))
    bm = np.array([[1, 0, 1], [0, 1, 0], [1, 1, 1]], dtype=np.uint8)
    tok = np.zeros((S, S), dtype=bool)
    for i in range(S):
        for j in range(S):
            tok[i, j] = bm[i // 128, j // 128]
    got = orc.attend_masked(q, k, v, 0.3, bm, tile=128)
    assert rel_rms(got, torch_sdpa(q, k, v, 0.3, tok)) < 1e-6
    got_s = orc.attend_streaming(q, k, v, 0.3, bm, tile=128, key_tile=128)
    assert rel_rms(got_s, got) < 2e-6


def test_constant_values_give_constant_output(orc):
    q, k, _, rule, scale = fixture(orc)
    v = np.full_like(q, 0.375)
    out = orc.attend_masked(q, k, v, scale, orc.tile_bitmap(rule), tile=1)
    assert np.allclose(out, 0.375, atol=1e-6)


def test_single_active_tile_is_an_exact_softmax(orc):
    g = np.random.default_rng(11)
    S, D = 512, 128
    q, k, v = (g.standard_normal((1, S, D), dtype=np.float32) for _ in range(3))
    bm = np.zeros((4, 4), dtype=np.uint8)
    bm[2, 1] = 1
    bm[0, :] = 1
    bm[1, 1] = bm[3, 3] = 1
    out = orc.attend_masked(q, k, v, 0.088, bm, tile=128)
    i = 300  # a row of q-tile 2
    s = (q[0, i].astype(np.float64) @ k[0, 128:256].T.astype(np.float64)) * 0.088
    p = np.exp(s - s.max())
    want = (p / p.sum()) @ v[0, 128:256].astype(np.float64)
    assert np.max(np.abs(out[0, i] - want)) < 1e-5


def test_empty_row_is_zero(orc):
    g = np.random.default_rng(5)
    S, D = 256, 16
    q, k, v = (g.standard_normal((1, S, D), dtype=np.float32) for _ in range(3))
    bm = np.array([[1, 1], [0, 0]], dtype=np.uint8)
    out = orc.attend_masked(q, k, v, 0.25, bm, tile=128)
    assert np.all(out[0, 128:] == 0)
    assert np.all(np.isfinite(out))
    rows = np.arange(120, 140, dtype=np.int32)
    sel = orc.attend_rows(q[0, rows], rows, k[0], v[0], 0.25, bm, tile=128)
    assert np.array_equal(sel, out[0, rows])


def test_a_planted_index_mistake_is_caught(orc):
    """A transposed tile index in the mask (bm.T instead of bm) is the kind of
    mistake the bool-mask cross-check must see."""
    q, k, v, rule, scale = fixture(orc)
    bm = orc.tile_bitmap(rule)
    wrong = orc.attend_masked(q, k, v, scale, np.ascontiguousarray(bm.T), tile=1)
    assert rel_rms(wrong, torch_sdpa(q, k, v, scale, bm)) > 1e-2
