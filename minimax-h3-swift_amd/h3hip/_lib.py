"""ctypes binding of libch3hip.so (declarations in include/ch3hip.h).

The library is the product; this module only loads it and declares the
signatures. Nothing here computes: if the shared object is missing the import
of any op fails loudly, there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_ROOT, "libch3hip.so")

OK, DECLINED = 0, 1
EINVAL, EHIP, ENOMEM, EDEVICE = -1, -2, -3, -4
TILE = 128

RULE_DENSE, RULE_BAND, RULE_LOCAL, RULE_AXIAL, RULE_BITMAP = 0, 1, 2, 3, 4
ROUND_REFERENCE, ROUND_FP32 = 0, 1
OUT_HEAD_MAJOR, OUT_TOKEN_MAJOR = 0, 1

_i32p = ctypes.POINTER(ctypes.c_int32)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_vp = ctypes.c_void_p


class MaskRuleC(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("seq_len", ctypes.c_int32),
        ("prefix_len", ctypes.c_int32),
        ("frames", ctypes.c_int32),
        ("height", ctypes.c_int32),
        ("width", ctypes.c_int32),
        ("frame_window", ctypes.c_int32),
        ("spatial_tile_h", ctypes.c_int32),
        ("spatial_tile_w", ctypes.c_int32),
        ("spatial_window", ctypes.c_int32),
        ("band", ctypes.c_int32),
        ("n_global_cols", ctypes.c_int32),
        ("global_cols", _i32p),
        ("n_landmarks", ctypes.c_int32),
        ("landmark_frames", _i32p),
        ("bitmap", _u8p),
    ]


class PolicyC(ctypes.Structure):
    _fields_ = [
        ("dense_first_blocks", ctypes.c_int32),
        ("dense_last_blocks", ctypes.c_int32),
        ("dense_until_progress", ctypes.c_double),
        ("min_sequence_length", ctypes.c_int32),
    ]


class AttentionContextC(ctypes.Structure):
    _fields_ = [
        ("block_index", ctypes.c_int32),
        ("block_count", ctypes.c_int32),
        ("schedule_progress", ctypes.c_double),
        ("sequence_length", ctypes.c_int32),
        ("video_start", ctypes.c_int32),
        ("video_stop", ctypes.c_int32),
    ]


class ViewC(ctypes.Structure):
    """h3hip_view: element (h, s, d) at data + h*head_stride + s*row_stride + d."""
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("head_stride", ctypes.c_int64),
        ("row_stride", ctypes.c_int64),
    ]


# Every symbol include/ch3hip.h declares, with (restype, argtypes).
SIGNATURES = {
    "h3hip_device_supported": (ctypes.c_int, [ctypes.c_int32]),
    "h3hip_last_error": (ctypes.c_char_p, []),
    "h3hip_version": (ctypes.c_char_p, []),
    "h3hip_plan_create": (ctypes.c_int, [ctypes.POINTER(MaskRuleC), ctypes.c_int32,
                                         ctypes.POINTER(PolicyC), _vp, ctypes.POINTER(_vp)]),
    "h3hip_plan_destroy": (ctypes.c_int, [_vp]),
    "h3hip_plan_info": (ctypes.c_int, [_vp, _i32p, _i32p, _i32p,
                                       ctypes.POINTER(ctypes.c_int64), _i32p]),
    "h3hip_plan_tiles": (ctypes.c_int, [_vp, _i32p, _i32p]),
    "h3hip_plan_density": (ctypes.c_double, [_vp]),
    "h3hip_schedule": (ctypes.c_int, [_i32p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                      _i32p, _i32p]),
    "h3hip_mask_from_rule": (ctypes.c_int, [ctypes.POINTER(MaskRuleC), _vp, _vp]),
    "h3hip_mask_from_rule_noalloc": (ctypes.c_int, [ctypes.POINTER(MaskRuleC), _vp, _vp]),
    "h3hip_tiles_from_mask": (ctypes.c_int, [_vp, ctypes.c_int32, ctypes.c_int32, _vp, _vp,
                                             ctypes.c_int64, ctypes.POINTER(ctypes.c_int64),
                                             _vp]),
    "h3hip_qk_norm_rope": (ctypes.c_int, [_vp, _vp, ctypes.c_int64, _vp, _vp, _vp,
                                          ctypes.c_float, _vp, _vp, _vp, ctypes.c_int32,
                                          ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                          ctypes.c_int32, ctypes.c_int32, _vp, _vp, _vp, _vp]),
    "h3hip_head_major": (ctypes.c_int, [_vp, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                        ctypes.c_int32, ctypes.c_int32, _vp, _vp]),
    "h3hip_rope_table": (ctypes.c_int, [_vp, _vp, _vp, ctypes.c_int32, ctypes.c_int32,
                                        ctypes.c_int32, _vp, _vp]),
    "h3hip_qkv_proj": (ctypes.c_int, [_vp, ctypes.c_int64, _vp, ctypes.c_int64, ctypes.c_int32,
                                      _vp, _vp, ctypes.c_float, _vp, ctypes.c_int32,
                                      ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                      ctypes.c_int32, ctypes.c_int32, _vp, _vp, _vp, _vp]),
    "h3hip_out_proj": (ctypes.c_int, [_vp, ctypes.c_int64, _vp, ctypes.c_int64, ctypes.c_int32,
                                      ctypes.c_int32, ctypes.c_int32, _vp, ctypes.c_int64, _vp]),
    "h3hip_bsattn_fwd": (ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.c_int32, ctypes.c_int32,
                                        ctypes.c_float, _vp, ctypes.c_int32, _vp]),
    "h3hip_bsattn_fwd_strided": (ctypes.c_int, [_vp, ctypes.POINTER(ViewC),
                                                ctypes.POINTER(ViewC), ctypes.POINTER(ViewC),
                                                ctypes.c_int32, ctypes.c_int32, ctypes.c_float,
                                                ctypes.POINTER(ViewC), _vp]),
    "h3hip_attend_strided": (ctypes.c_int, [_vp, ctypes.POINTER(AttentionContextC),
                                            ctypes.POINTER(ViewC), ctypes.POINTER(ViewC),
                                            ctypes.POINTER(ViewC), ctypes.c_int32,
                                            ctypes.c_int32, ctypes.c_float,
                                            ctypes.POINTER(ViewC), _vp]),
    "h3hip_attend": (ctypes.c_int, [_vp, ctypes.POINTER(AttentionContextC), _vp, _vp, _vp,
                                    ctypes.c_int32, ctypes.c_int32, ctypes.c_float, _vp, _vp]),
    "h3hip_rope_pairs_axes": (ctypes.c_int, [ctypes.c_double, ctypes.c_int32, ctypes.c_int32,
                                             ctypes.c_int32, _i32p, _f32p]),
    "h3hip_rope_pairs_h3": (ctypes.c_int, [_f32p, ctypes.c_int32, _i32p, _f32p]),
    "h3hip_positions_grid": (ctypes.c_int, [ctypes.c_int32] * 4 + [_f32p]),
    "h3hip_positions_packed": (ctypes.c_int, [ctypes.c_int32] * 6 + [_f64p]),
    "h3hip_landmarks": (ctypes.c_int, [ctypes.c_int32, ctypes.c_int32, _i32p]),
}


class H3HIPError(RuntimeError):
    """A negative status from libch3hip (invalid argument or HIP failure)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"libch3hip error {code}: {message}")
        self.code = code


_lib = None


def lib() -> ctypes.CDLL:
    """Loads the in-tree libch3hip.so, failing loudly when it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() (make -C minimax-h3-swift_amd)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    msg = lib().h3hip_last_error()
    return msg.decode() if msg else ""


def check(rc: int, allow_declined: bool = False) -> int:
    """Maps a status to Python: negative raises, DECLINED returned if allowed."""
    if rc == OK:
        return rc
    if rc == DECLINED:
        if allow_declined:
            return rc
        raise H3HIPError(rc, "declined: " + last_error())
    raise H3HIPError(rc, last_error())
