"""The benchmark shapes and their written mask rules.

Token order is [text | audio | video] (the reference's packing with no
conditioning segments, Sources/H3Foundation/PackedSequence.swift:173-176);
everything before the video span is the prefix. S is padded to a multiple of
128.

Mask rules (fixed here once, and never tuned to a density):
  * cfg1 -- tile-level band of +-2 tiles around the diagonal plus tile column
    0 as a global column: 183 of 32x32 tiles (17.87%).
  * local window (cfg2, cfg3) -- token level, OR-reduced onto 128x128 tiles:
    a prefix (text or audio) token attends and is attended by everything; two
    video tokens attend iff their latent frames differ by at most 1 and their
    spatial tiles of 8x8 latent tokens differ by at most 1 on each axis (3x3
    spatial tiles). cfg3: 7,854 of 250^2 tiles per head (12.57%); cfg2: 3,204
    of 142^2 (15.89%). The variant with latent frame 0 also global (the
    reference's AxialTopology always keeps frame 0 as a landmark,
    AxialTopology.swift:99-111) is reported as an extra line: 9,691 (15.51%).
  * cfg4 -- every tile (the dense, no-skip path).
  * axial_h3 -- the reference's own topology (AxialTopology.allows,
    Sources/H3Attention/AxialTopology.swift:128-137) at its production shape,
    864x480x124: 746 prefix rows (text, conditioning, references, audio), a
    37x15x27 latent lattice, 56 heads, 3 landmark frames [0, 18, 36]. At
    token level that is ~15% density; OR-reduced onto 128x128 tiles it is
    10,815 of 123^2 tiles (71.5%), because a tile spans a third of a 405-token
    frame. Every relation of this topology (prefix, same frame, same in-frame
    offset, landmark frame) is unchanged by a permutation applied identically
    inside every frame, so a per-frame Morton order leaves its tiles as they
    are.
"""
from __future__ import annotations

from dataclasses import dataclass

from .topology import MaskRule

HEAD_DIM = 128
ROPE_THETA = 10000.0
ROPE_DIMS = (32, 48, 48)   # t, h, w channels -> 16 / 24 / 24 pairs, all 128 channels rotate
QK_EPS = 1e-6


@dataclass(frozen=True)
class Shape:
    name: str
    heads: int
    text: int
    audio: int
    frames: int
    height: int
    width: int
    rule: str            # "band", "local", "local_f0", "dense", "axial"

    @property
    def prefix_len(self) -> int:
        return self.text + self.audio

    @property
    def seq_len(self) -> int:
        return self.prefix_len + self.frames * self.height * self.width

    @property
    def seq_pad(self) -> int:
        return (self.seq_len + 127) // 128 * 128

    def mask_rule(self) -> MaskRule:
        if self.rule == "band":
            return MaskRule.band_rule(self.seq_len, band=2, global_cols=(0,))
        if self.rule == "dense":
            return MaskRule.dense(self.seq_len)
        if self.rule == "axial":
            return MaskRule.axial(self.prefix_len, self.frames, self.height, self.width,
                                  n_landmarks=3)
        lm = (0,) if self.rule == "local_f0" else ()
        return MaskRule.local_window(self.prefix_len, self.frames, self.height, self.width,
                                     frame_window=1, spatial_tile=(8, 8), spatial_window=1,
                                     landmarks=lm)

    def oracle_rule_kwargs(self) -> dict:
        """The same rule in the oracle's vocabulary (tests and bench only)."""
        if self.rule == "band":
            return dict(kind=1, seq_len=self.seq_len, band=2, global_cols=[0])
        if self.rule == "dense":
            return dict(kind=0, seq_len=self.seq_len)
        if self.rule == "axial":
            from .topology import landmark_frames
            return dict(kind=3, seq_len=self.seq_len, prefix_len=self.prefix_len,
                        frames=self.frames, height=self.height, width=self.width,
                        landmarks=list(landmark_frames(self.frames, 3)))
        return dict(kind=2, seq_len=self.seq_len, prefix_len=self.prefix_len,
                    frames=self.frames, height=self.height, width=self.width, frame_window=1,
                    sp_tile=(8, 8), sp_window=1,
                    landmarks=[0] if self.rule == "local_f0" else [])


CFG1 = Shape("cfg1_band_4x32x32", 4, 0, 0, 4, 32, 32, "band")
CFG2 = Shape("cfg2_864x480x7s", 40, 512, 175, 43, 15, 27, "local")
CFG3 = Shape("cfg3_1344x768x5s", 40, 512, 125, 31, 24, 42, "local")
CFG3_F0 = Shape("cfg3_1344x768x5s_frame0", 40, 512, 125, 31, 24, 42, "local_f0")
CFG4 = Shape("cfg4_dense_864x480x7s", 40, 512, 175, 43, 15, 27, "dense")
AXIAL_H3 = Shape("axial_h3_864x480x124", 56, 746, 0, 37, 15, 27, "axial")

ALL = {s.name: s for s in (CFG1, CFG2, CFG3, CFG3_F0, CFG4, AXIAL_H3)}
