"""TEST INFRASTRUCTURE, NOT PRODUCT CODE.

ctypes binding to ``oracle/libh3oracle.so`` (the C restatement in
``h3_oracle.c``) plus the numpy helpers the checks need. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
module, and only to check or to time the reference path on the host CPU. The
shipped library (``minimax-h3-swift_amd``) never imports it.

Parity status per function (how each is pinned; the tests live in
``tests/test_oracle_*.py``):

* ``allows``/``tile_bitmap``/``csr`` -- pinned: the reference's known-answer
  tokens (AxialReferenceTests.swift:119-143), closed-form tile counts (band
  rule: 183 tiles at 32x32), counted-vs-closed-form density
  (AxialReferenceTests.swift:145-160), brute force over token pairs.
* ``landmarks`` -- pinned: [0, 18, 36] for 37 frames, clamping and dedup
  (AxialReferenceTests.swift:176-193).
* ``attend_masked``/``attend_streaming`` -- pinned relationally as the
  reference pins its own oracle: all-keys equals torch's unmasked fp32 SDPA
  (fullSelectionIsDense), masked equals torch's boolean-mask fp32 SDPA,
  streaming equals masked for ragged key tiles, query chunking is exact.
* ``qk_norm_rope`` -- pinned by invariants (pair norms, identity at position
  0, passthrough channels bit-exact, unit RMS before gamma) and by an
  independent numpy restatement; MLX's own bf16 rounding inside RoPE is
  unpinnable without MLX (no MLX in this image), so the rounding points follow
  the fused fixture (QKFusionMetalFixture.swift:57-69).
* ``positions_packed`` -- pinned against the lattice identities of
  PackedLayoutTests.swift and hand-computed coordinates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libh3oracle.so")

RULE_DENSE, RULE_BAND, RULE_LOCAL, RULE_AXIAL = 0, 1, 2, 3
ROUND_REFERENCE, ROUND_FP32 = 0, 1

_i32p = ctypes.POINTER(ctypes.c_int32)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)


class OrcRule(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("seq_len", ctypes.c_int32),
        ("tile", ctypes.c_int32),
        ("prefix_len", ctypes.c_int32),
        ("frames", ctypes.c_int32),
        ("height", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("frame_window", ctypes.c_int32),
        ("sp_tile_h", ctypes.c_int32),
        ("sp_tile_w", ctypes.c_int32),
        ("sp_window", ctypes.c_int32),
        ("band", ctypes.c_int32),
        ("n_global_cols", ctypes.c_int32),
        ("global_cols", _i32p),
        ("n_landmarks", ctypes.c_int32),
        ("landmarks", _i32p),
    ]


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc, OpenMP)."""
    if force and os.path.exists(LIB_PATH):
        os.remove(LIB_PATH)
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.orc_allows.argtypes = [ctypes.POINTER(OrcRule), ctypes.c_int32, ctypes.c_int32]
        L.orc_landmarks.argtypes = [ctypes.c_int32, ctypes.c_int32, _i32p]
        L.orc_axial_density_closed.argtypes = [ctypes.POINTER(OrcRule)]
        L.orc_axial_density_closed.restype = ctypes.c_double
        L.orc_token_density_counted.argtypes = [ctypes.POINTER(OrcRule)]
        L.orc_token_density_counted.restype = ctypes.c_double
        L.orc_tile_bitmap.argtypes = [ctypes.POINTER(OrcRule), ctypes.c_int32, ctypes.c_int32, _u8p]
        L.orc_csr_from_bitmap.argtypes = [_u8p, ctypes.c_int32, ctypes.c_int32, _i32p, _i32p]
        L.orc_csr_from_bitmap.restype = ctypes.c_int64
        L.orc_attend_masked.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int32, ctypes.c_int32,
                                        ctypes.c_int32, ctypes.c_float, _u8p, ctypes.c_int32,
                                        ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                        ctypes.c_int32, ctypes.c_int32, _f32p]
        L.orc_attend_streaming.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int32, ctypes.c_int32,
                                           ctypes.c_int32, ctypes.c_float, _u8p, ctypes.c_int32,
                                           ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                           ctypes.c_int32, _f32p]
        L.orc_attend_masked_rows.argtypes = [_f32p, ctypes.c_int32, _i32p, _f32p, _f32p,
                                             ctypes.c_int32, ctypes.c_int32, ctypes.c_float,
                                             _u8p, ctypes.c_int32, ctypes.c_int32,
                                             ctypes.c_int32, _f32p]
        L.orc_qk_norm_rope.argtypes = [_u16p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                       ctypes.c_int32, ctypes.c_int32, _u16p, ctypes.c_float,
                                       _f32p, _i32p, _f32p, ctypes.c_int32, ctypes.c_int32,
                                       ctypes.c_int32, _u16p]
        L.orc_rope_table.argtypes = [_f32p, ctypes.c_int32, _i32p, _f32p, ctypes.c_int32,
                                     ctypes.c_int32, ctypes.c_void_p]
        L.orc_rope_pairs_axes.argtypes = [ctypes.c_double, ctypes.c_int32, ctypes.c_int32,
                                          ctypes.c_int32, _i32p, _f32p]
        L.orc_rope_pairs_h3.argtypes = [_f32p, ctypes.c_int32, _i32p, _f32p]
        L.orc_positions_grid.argtypes = [ctypes.c_int32] * 4 + [_f32p]
        L.orc_positions_packed.argtypes = [ctypes.c_int32] * 6 + [_f64p]
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    return a.ctypes.data_as(t)


# ----------------------------------------------------------------- bf16 (numpy)

def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def randn_bf16(shape, seed: int, scale: float = 1.0) -> np.ndarray:
    """Seeded N(0, scale^2) rounded to bf16 (numpy PCG64, platform-stable)."""
    g = np.random.default_rng(seed)
    return f32_to_bf16(g.standard_normal(shape, dtype=np.float32) * np.float32(scale))


_SM_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_SM_M1 = np.uint64(0xBF58476D1CE4E5B9)
_SM_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, count: int) -> np.ndarray:
    """The splitmix64 stream (Steele, Lea and Flood, "Fast splittable
    pseudorandom number generators", OOPSLA 2014): state_i = seed + (i+1)*gamma,
    each mixed by two xor-shift-multiply rounds. Integer arithmetic only."""
    with np.errstate(over="ignore"):
        x = np.uint64(seed) + (np.arange(1, count + 1, dtype=np.uint64) * _SM_GAMMA)
        x = (x ^ (x >> np.uint64(30))) * _SM_M1
        x = (x ^ (x >> np.uint64(27))) * _SM_M2
        return x ^ (x >> np.uint64(31))


def splitmix_uniform(shape, seed: int) -> np.ndarray:
    """Uniform [0, 1) doubles from the top 53 bits of splitmix64 draws."""
    n = int(np.prod(shape))
    return ((splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * 2.0 ** -53).reshape(shape)


def splitmix_normal_bf16(shape, seed: int) -> np.ndarray:
    """Bit-stable approximately N(0, 1) bf16 inputs: the Irwin-Hall sum of four
    splitmix64 uniforms, centred and scaled by sqrt(3) to unit variance, rounded
    to bf16. Every step is exact or IEEE-deterministic, so a fixture needs only
    the seed on any machine or numpy version."""
    n = int(np.prod(shape))
    u = (splitmix64(seed, 4 * n) >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    x = (u.reshape(n, 4).sum(axis=1) - 2.0) * np.sqrt(3.0)
    return f32_to_bf16(x.astype(np.float32)).reshape(shape)


def uniform_bf16(shape, seed: int, lo: float, hi: float) -> np.ndarray:
    g = np.random.default_rng(seed)
    return f32_to_bf16(g.uniform(lo, hi, size=shape).astype(np.float32))


# --------------------------------------------------------------------- topology

class Rule:
    """Python-side holder that keeps the arrays an OrcRule points into alive."""

    def __init__(self, kind: int, seq_len: int, tile: int = 128, prefix_len: int = 0,
                 frames: int = 0, height: int = 0, width: int = 0, frame_window: int = 1,
                 sp_tile=(8, 8), sp_window: int = 1, band: int = 0, global_cols=(),
                 landmarks=()):
        self.kind, self.seq_len, self.tile = kind, seq_len, tile
        self.prefix_len, self.frames, self.height, self.width = prefix_len, frames, height, width
        self.frame_window, self.sp_tile, self.sp_window, self.band = frame_window, tuple(sp_tile), sp_window, band
        self.global_cols = np.ascontiguousarray(global_cols, dtype=np.int32).reshape(-1)
        self.landmarks = np.ascontiguousarray(landmarks, dtype=np.int32).reshape(-1)
        self.c = OrcRule(kind, seq_len, tile, prefix_len, frames, height, width, frame_window,
                         self.sp_tile[0], self.sp_tile[1], sp_window, band,
                         len(self.global_cols), _p(self.global_cols, _i32p),
                         len(self.landmarks), _p(self.landmarks, _i32p))

    @property
    def n_tiles(self) -> int:
        return (self.seq_len + self.tile - 1) // self.tile


def allows(rule: Rule, q: int, k: int) -> bool:
    return bool(lib().orc_allows(ctypes.byref(rule.c), q, k))


def landmarks(frames: int, n: int) -> list[int]:
    out = np.zeros(max(frames, 2), dtype=np.int32)
    cnt = lib().orc_landmarks(frames, n, _p(out, _i32p))
    return [int(v) for v in out[:cnt]]


def axial_density_closed(rule: Rule) -> float:
    return float(lib().orc_axial_density_closed(ctypes.byref(rule.c)))


def token_density_counted(rule: Rule) -> float:
    return float(lib().orc_token_density_counted(ctypes.byref(rule.c)))


def tile_bitmap(rule: Rule) -> np.ndarray:
    n = rule.n_tiles
    out = np.zeros((n, n), dtype=np.uint8)
    lib().orc_tile_bitmap(ctypes.byref(rule.c), n, n, _p(out, _u8p))
    return out


def csr(bm: np.ndarray):
    bm = np.ascontiguousarray(bm, dtype=np.uint8)
    nq, nk = bm.shape
    nnz = int(lib().orc_csr_from_bitmap(_p(bm, _u8p), nq, nk, None, None))
    row_ptr = np.zeros(nq + 1, dtype=np.int32)
    col_idx = np.zeros(max(nnz, 1), dtype=np.int32)
    lib().orc_csr_from_bitmap(_p(bm, _u8p), nq, nk, _p(row_ptr, _i32p), _p(col_idx, _i32p))
    return row_ptr, col_idx[:nnz]


# -------------------------------------------------------------------- attention

def attend_masked(q, k, v, scale: float, bm: np.ndarray, tile: int = 128,
                  query_chunk: int = 512, q_lo: int = 0, q_hi: int | None = None,
                  threads: int = 0) -> np.ndarray:
    """AxialReference.attend on fp32 [H, S, D] (rows [q_lo, q_hi) filled)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    H, S, D = q.shape
    q_hi = S if q_hi is None else q_hi
    bm = np.ascontiguousarray(bm, dtype=np.uint8)
    out = np.zeros_like(q)
    lib().orc_attend_masked(_p(q, _f32p), _p(k, _f32p), _p(v, _f32p), H, S, D, scale,
                            _p(bm, _u8p), tile, bm.shape[1], query_chunk, q_lo, q_hi,
                            threads, _p(out, _f32p))
    return out


def attend_streaming(q, k, v, scale: float, bm: np.ndarray, tile: int = 128,
                     query_chunk: int = 512, key_tile: int = 1024, threads: int = 0) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    H, S, D = q.shape
    bm = np.ascontiguousarray(bm, dtype=np.uint8)
    out = np.zeros_like(q)
    lib().orc_attend_streaming(_p(q, _f32p), _p(k, _f32p), _p(v, _f32p), H, S, D, scale,
                               _p(bm, _u8p), tile, bm.shape[1], query_chunk, key_tile,
                               threads, _p(out, _f32p))
    return out


def attend_rows(q_rows, rows, k, v, scale: float, bm: np.ndarray, tile: int = 128,
                threads: int = 0) -> np.ndarray:
    """Masked-definition output for selected query rows of one head.

    q_rows [n, D] fp32, rows [n] indices, k/v [S, D] fp32."""
    q_rows = np.ascontiguousarray(q_rows, dtype=np.float32)
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    bm = np.ascontiguousarray(bm, dtype=np.uint8)
    S, D = k.shape
    out = np.zeros((len(rows), D), dtype=np.float32)
    lib().orc_attend_masked_rows(_p(q_rows, _f32p), len(rows), _p(rows, _i32p), _p(k, _f32p),
                                 _p(v, _f32p), S, D, scale, _p(bm, _u8p), tile, bm.shape[1],
                                 threads, _p(out, _f32p))
    return out


# --------------------------------------------------------------------- prologue

def qk_norm_rope(x: np.ndarray, ld: int, S: int, S_pad: int, H: int, D: int,
                 gamma: np.ndarray, eps: float, pos: np.ndarray, pair_axis: np.ndarray,
                 pair_inv: np.ndarray, rot: int, mode: int = ROUND_REFERENCE,
                 threads: int = 0) -> np.ndarray:
    """H3RMSNorm -> SplitHalfRoPE, token-major bf16 in (row stride ``ld``),
    head-major bf16 [H, S_pad, D] out (uint16 bit patterns)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    if (x.ndim == 2 and x.shape[1] != ld) or x.size < (S - 1) * ld + H * D:
        raise ValueError(f"x of shape {x.shape} does not hold {S} rows of stride {ld}")
    gamma = np.ascontiguousarray(gamma, dtype=np.uint16)
    pos = np.ascontiguousarray(pos, dtype=np.float32)
    pair_axis = np.ascontiguousarray(pair_axis, dtype=np.int32)
    pair_inv = np.ascontiguousarray(pair_inv, dtype=np.float32)
    out = np.zeros((H, S_pad, D), dtype=np.uint16)
    lib().orc_qk_norm_rope(_p(x, _u16p), ld, S, S_pad, H, D, _p(gamma, _u16p), eps,
                           _p(pos, _f32p), _p(pair_axis, _i32p), _p(pair_inv, _f32p), rot, mode,
                           threads, _p(out, _u16p))
    return out


def rope_table(pos: np.ndarray, pair_axis: np.ndarray, pair_inv: np.ndarray, rot: int,
               mode: int = ROUND_REFERENCE) -> np.ndarray:
    """H3RoPE.rotationTable (H3Transformer.swift:62-78): [S, rot/2, 4] entries
    (c, -s, s, c); uint16 bf16 bit patterns for REFERENCE, float32 for FP32."""
    pos = np.ascontiguousarray(pos, dtype=np.float32)
    pair_axis = np.ascontiguousarray(pair_axis, dtype=np.int32)
    pair_inv = np.ascontiguousarray(pair_inv, dtype=np.float32)
    S, half = pos.shape[0], rot // 2
    if pair_axis.size < half or pair_inv.size < half:
        raise ValueError(f"pair tables must hold rot/2 = {half} entries")
    out = np.zeros((S, half, 4), dtype=np.uint16 if mode == ROUND_REFERENCE else np.float32)
    lib().orc_rope_table(_p(pos, _f32p), S, _p(pair_axis, _i32p), _p(pair_inv, _f32p), half,
                         mode, out.ctypes.data_as(ctypes.c_void_p))
    return out


def rope_pairs_axes(theta: float, dim_t: int, dim_h: int, dim_w: int):
    n = (dim_t + dim_h + dim_w) // 2
    ax = np.zeros(n, dtype=np.int32)
    inv = np.zeros(n, dtype=np.float32)
    lib().orc_rope_pairs_axes(theta, dim_t, dim_h, dim_w, _p(ax, _i32p), _p(inv, _f32p))
    return ax, inv


def rope_pairs_h3(inv_freq: np.ndarray):
    inv_freq = np.ascontiguousarray(inv_freq, dtype=np.float32)
    n = 3 * len(inv_freq)
    ax = np.zeros(n, dtype=np.int32)
    inv = np.zeros(n, dtype=np.float32)
    lib().orc_rope_pairs_h3(_p(inv_freq, _f32p), len(inv_freq), _p(ax, _i32p), _p(inv, _f32p))
    return ax, inv


def positions_grid(prefix_len: int, frames: int, height: int, width: int) -> np.ndarray:
    out = np.zeros((prefix_len + frames * height * width, 3), dtype=np.float32)
    lib().orc_positions_grid(prefix_len, frames, height, width, _p(out, _f32p))
    return out


def positions_packed(text_tokens: int, audio_t: int, latent_t: int, latent_h: int,
                     latent_w: int, patch: int = 2) -> np.ndarray:
    n = text_tokens + 2 * audio_t + latent_t * (latent_h // patch) * (latent_w // patch)
    out = np.zeros((n, 3), dtype=np.float64)
    got = lib().orc_positions_packed(text_tokens, audio_t, latent_t, latent_h, latent_w, patch,
                                     _p(out, _f64p))
    if got != n:
        raise ValueError(f"positions_packed: geometry refused ({got})")
    return out
