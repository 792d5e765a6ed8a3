"""Mask rules (which tiles are active) and the tile plan that owns their lists.

``MaskRule`` is the Python face of ``h3hip_mask_rule``; ``TilePlan`` wraps
``h3hip_plan`` (built on the GPU, once per shape). The reference's own
topology is ``MaskRule.axial`` -- AxialTopology.allows
(Sources/H3Attention/AxialTopology.swift:128-137) -- and the rules of the
synthetic benchmark shapes are ``band`` and ``local_window``.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import _lib as L


@dataclass
class MaskRule:
    kind: int
    seq_len: int
    prefix_len: int = 0
    frames: int = 0
    height: int = 0
    width: int = 0
    frame_window: int = 1
    spatial_tile: tuple = (8, 8)
    spatial_window: int = 1
    band: int = 0
    global_cols: tuple = ()
    landmarks: tuple = ()
    bitmap: np.ndarray | None = None
    _keep: list = field(default_factory=list, repr=False, compare=False)

    # -- constructors -------------------------------------------------------
    @classmethod
    def dense(cls, seq_len: int) -> "MaskRule":
        return cls(L.RULE_DENSE, seq_len)

    @classmethod
    def band_rule(cls, seq_len: int, band: int, global_cols=(0,)) -> "MaskRule":
        return cls(L.RULE_BAND, seq_len, band=band, global_cols=tuple(global_cols))

    @classmethod
    def local_window(cls, prefix_len: int, frames: int, height: int, width: int,
                     frame_window: int = 1, spatial_tile=(8, 8), spatial_window: int = 1,
                     landmarks=()) -> "MaskRule":
        return cls(L.RULE_LOCAL, prefix_len + frames * height * width, prefix_len, frames,
                   height, width, frame_window, tuple(spatial_tile), spatial_window,
                   landmarks=tuple(landmarks))

    @classmethod
    def axial(cls, prefix_len: int, frames: int, height: int, width: int,
              landmarks=None, n_landmarks: int = 3) -> "MaskRule":
        if landmarks is None:
            landmarks = landmark_frames(frames, n_landmarks)
        return cls(L.RULE_AXIAL, prefix_len + frames * height * width, prefix_len, frames,
                   height, width, landmarks=tuple(landmarks))

    @classmethod
    def from_bitmap(cls, seq_len: int, bitmap: np.ndarray) -> "MaskRule":
        n = (seq_len + L.TILE - 1) // L.TILE
        bm = np.ascontiguousarray(bitmap, dtype=np.uint8)
        if bm.shape != (n, n):
            raise ValueError(f"bitmap must be [{n}, {n}] for seq_len {seq_len}, got {bm.shape}")
        return cls(L.RULE_BITMAP, seq_len, bitmap=bm)

    # -- properties ---------------------------------------------------------
    @property
    def n_tiles(self) -> int:
        return (self.seq_len + L.TILE - 1) // L.TILE

    @property
    def seq_pad(self) -> int:
        return self.n_tiles * L.TILE

    def to_c(self) -> L.MaskRuleC:
        cols = np.ascontiguousarray(self.global_cols, dtype=np.int32).reshape(-1)
        lms = np.ascontiguousarray(self.landmarks, dtype=np.int32).reshape(-1)
        self._keep[:] = [cols, lms, self.bitmap]
        i32p = ctypes.POINTER(ctypes.c_int32)
        return L.MaskRuleC(
            self.kind, self.seq_len, self.prefix_len, self.frames, self.height, self.width,
            self.frame_window, self.spatial_tile[0], self.spatial_tile[1], self.spatial_window,
            self.band, len(cols), cols.ctypes.data_as(i32p), len(lms), lms.ctypes.data_as(i32p),
            self.bitmap.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))
            if self.bitmap is not None else None)


def landmark_frames(frames: int, n: int = 3) -> list[int]:
    """AxialTopology's landmark placement (AxialTopology.swift:82-112)."""
    out = np.zeros(max(frames, 1), dtype=np.int32)
    cnt = L.lib().h3hip_landmarks(frames, n, out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)))
    L.check(min(cnt, 0))
    return [int(v) for v in out[:cnt]]


def axial_token_density(prefix_len: int, frames: int, height: int, width: int,
                        landmarks) -> float:
    """Token-level density of the axial topology, AxialTopology.density
    (Sources/H3Attention/AxialTopology.swift:139-170): prefix rows see all S
    keys; a video query in frame f sees the prefix, every token of frame f
    and of each landmark frame, and one token (its own position) in every
    other frame -- counted frame by frame, so the overlapping axes are never
    added twice."""
    per = height * width
    s = prefix_len + frames * per
    lm = set(int(f) for f in landmarks)
    video = 0
    for f0 in range(frames):
        full = len(lm) if f0 in lm else len(lm) + 1
        video += per * (prefix_len + per * full + (frames - full))
    return (prefix_len * s + video) / float(s * s)


def schedule(row_ptr: np.ndarray, heads: int, groups: int = 256):
    """The attention launch's persistent schedule for these CSR rows
    (h3hip_schedule): (work_ptr [groups + 1], work [heads * n_tiles]) int32;
    workgroup b runs work[work_ptr[b]:work_ptr[b + 1]], each unit
    head << 16 | q_tile. The same lists h3hip_plan_create uploads."""
    rp = np.ascontiguousarray(row_ptr, dtype=np.int32)
    n = len(rp) - 1
    work_ptr = np.zeros(groups + 1, dtype=np.int32)
    work = np.zeros(max(heads * n, 1), dtype=np.int32)
    i32p = ctypes.POINTER(ctypes.c_int32)
    L.check(L.lib().h3hip_schedule(rp.ctypes.data_as(i32p), n, heads, groups,
                                   work_ptr.ctypes.data_as(i32p), work.ctypes.data_as(i32p)))
    return work_ptr, work[:heads * n]


@dataclass
class Policy:
    """When the backend declines (AttentionContext-driven, AttentionBackend.swift:10-59)."""
    dense_first_blocks: int = 0
    dense_last_blocks: int = 0
    dense_until_progress: float = 0.0
    min_sequence_length: int = 0

    def to_c(self) -> L.PolicyC:
        return L.PolicyC(self.dense_first_blocks, self.dense_last_blocks,
                         self.dense_until_progress, self.min_sequence_length)


class TilePlan:
    """Owns an ``h3hip_plan``: CSR tile lists on host and device plus the
    attention kernel's XCD-aware schedule (each persistent workgroup's units),
    built on the current GPU."""

    def __init__(self, rule: MaskRule, heads: int, policy: Policy | None = None,
                 stream: int | None = None):
        self.rule = rule
        self.heads = heads
        self.policy = policy or Policy()
        crule = rule.to_c()
        cpol = self.policy.to_c()
        handle = ctypes.c_void_p()
        L.check(L.lib().h3hip_plan_create(ctypes.byref(crule), heads, ctypes.byref(cpol),
                                          stream, ctypes.byref(handle)))
        self.handle = handle
        s, sp, nt, hd = (ctypes.c_int32() for _ in range(4))
        nnz = ctypes.c_int64()
        L.check(L.lib().h3hip_plan_info(handle, ctypes.byref(s), ctypes.byref(sp),
                                        ctypes.byref(nt), ctypes.byref(nnz), ctypes.byref(hd)))
        self.seq_len, self.seq_pad, self.n_tiles = s.value, sp.value, nt.value
        self.nnz = nnz.value

    def tiles(self):
        """(row_ptr [n_tiles + 1], col_idx [nnz]) int32, bit-exact copies."""
        row_ptr = np.zeros(self.n_tiles + 1, dtype=np.int32)
        col_idx = np.zeros(max(self.nnz, 1), dtype=np.int32)
        i32p = ctypes.POINTER(ctypes.c_int32)
        L.check(L.lib().h3hip_plan_tiles(self.handle, row_ptr.ctypes.data_as(i32p),
                                         col_idx.ctypes.data_as(i32p)))
        return row_ptr, col_idx[:self.nnz]

    @property
    def density(self) -> float:
        return float(L.lib().h3hip_plan_density(self.handle))

    def close(self):
        if getattr(self, "handle", None) is not None and self.handle.value:
            L.lib().h3hip_plan_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
