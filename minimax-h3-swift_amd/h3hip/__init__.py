"""h3hip: MI355X-native DiT attention hot path (tile lists, fused Q/K
norm+RoPE prologue, block-sparse attention) behind the C ABI of
include/ch3hip.h. The compute lives in libch3hip.so; this package binds it."""
from . import _lib
from ._lib import (DECLINED, OK, OUT_HEAD_MAJOR, OUT_TOKEN_MAJOR, ROUND_FP32, ROUND_REFERENCE,
                   TILE, H3HIPError, lib, last_error)
from .topology import (MaskRule, Policy, TilePlan, axial_token_density, landmark_frames,
                       schedule)

__all__ = ["DECLINED", "OK", "OUT_HEAD_MAJOR", "OUT_TOKEN_MAJOR", "ROUND_FP32",
           "ROUND_REFERENCE", "TILE", "H3HIPError", "lib", "last_error", "MaskRule", "Policy",
           "TilePlan", "axial_token_density", "landmark_frames", "schedule"]
