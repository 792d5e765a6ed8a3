// Device arithmetic shared by the prologue (qk_norm_rope.hip) and the fused
// projection (qkv_proj.hip), so both produce the same bits:
//   H3RMSNorm (Sources/H3Modules/Modulation.swift:116-120) and SplitHalfRoPE
//   (Sources/H3Modules/DiTBlock.swift:83-103) in the two rounding modes of
//   h3hip_qk_norm_rope (see include/ch3hip.h).
#pragma once

#include "common.h"

namespace h3hip {

// Two fp32 values -> packed bf16 (round to nearest even, v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t cvt_pk(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  const f2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, b2));
}

// Rotation table entry for one pair: (c, s), bf16-rounded for REFERENCE
// rounding (the bf16 table of H3Transformer.swift:271-273), fp32 otherwise.
struct RopeEntry {
  float c, s;
};

// The entry for angle pos[axis] * inv_freq.
template <int kMode>
__device__ __forceinline__ RopeEntry make_rope_entry(float ang) {
  float c, s;
  sincosf(ang, &s, &c);
  if (kMode == H3HIP_ROUND_REFERENCE) {
    c = round_bf16(c);
    s = round_bf16(s);
  }
  return RopeEntry{c, s};
}

// 1/sqrt(x) rounded to fp32: the hardware estimate refined by one Newton step
// in double (relative error ~1e-13 before the final rounding), i.e. the
// correctly rounded value except within ~1e-13 of an fp32 rounding midpoint.
__device__ __forceinline__ float rsqrt_rounded(float x) {
  const double xd = (double)x, r0 = (double)__builtin_amdgcn_rsqf(x);
  const double e = fma(-xd * r0, r0, 1.0);
  return (float)fma(0.5 * r0, e, r0);
}

// One RoPE pair from the normalised values ya (channel p) and yb (channel
// p + rot/2). REFERENCE: the inputs, every product and each sum are rounded
// to bf16 as MLX does on bf16 arrays; the results come back as the fp32
// values of those bf16 numbers. FP32: plain fp32. With rotate false the pair
// passes through (bf16-rounded in REFERENCE mode).
template <int kMode>
__device__ __forceinline__ void rope_pair(float ya, float yb, RopeEntry t, bool rotate,
                                          float& oa, float& ob) {
  if (kMode == H3HIP_ROUND_REFERENCE) {
    const uint32_t ab = cvt_pk(ya, yb);  // bf16(y_a) | bf16(y_b)
    const float a = bf16_lo(ab), b = bf16_hi(ab);
    const uint32_t p1 = cvt_pk(t.c * a, -t.s * b);
    const uint32_t p2 = cvt_pk(t.s * a, t.c * b);
    const float ra = bf16_lo(p1) + bf16_hi(p1);
    const float rb = bf16_lo(p2) + bf16_hi(p2);
    oa = rotate ? ra : a;
    ob = rotate ? rb : b;
  } else {
    // Two rounded products and a rounded sum, never an fma: contraction
    // would let each kernel fuse a different product and the kernels that
    // share this code would disagree in the last bit.
#pragma clang fp contract(off)
    const float ra = t.c * ya - t.s * yb;
    const float rb = t.s * ya + t.c * yb;
    oa = rotate ? ra : ya;
    ob = rotate ? rb : yb;
  }
}

__device__ __forceinline__ void unpack8(u32x4 w, float* f) {
#pragma unroll
  for (int i = 0; i < 4; i++) {
    f[2 * i] = bf16_lo(w[i]);
    f[2 * i + 1] = bf16_hi(w[i]);
  }
}

__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; i++) r[i] = cvt_pk(f[2 * i], f[2 * i + 1]);
  return r;
}

// DPP controls used by the 8-lane reduction.
constexpr int kDppHalfMirror = 0x141;   // lane j <- lane 7 - j within 8 lanes
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]

template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}

// Row arithmetic of the 8-lane row layout both kernels use for normalisation:
// lane j of an aligned 8-lane group holds two 8-channel chunks of one 128-channel
// row (chunk a in x[0..7], chunk b in x[8..15]).
//
// Mean of squares of the row in a fixed fp32 order -- each lane's 16 squares
// with fma in channel order (chunk a, then chunk b), then the 8 lane sums as
// t_j = s_j + s_{7-j}, u_j = t_j + t_{j^2}, total = u_j + u_{j^1} (DPP
// half-row mirror, quad xor 2, quad xor 1), so every lane ends with the same
// bits -- and the normalised values y = (x * r) * g.
__device__ __forceinline__ void rms_normalise(const float* x, const float* g, float eps,
                                              float* y) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; i++) s = fmaf(x[i], x[i], s);
  s = s + dpp<kDppHalfMirror>(s);
  s = s + dpp<kDppQuadXor2>(s);
  s = s + dpp<kDppQuadXor1>(s);
  const float ms = s * (1.0f / 128.0f);
  const float r = rsqrt_rounded(ms + eps);
#pragma unroll
  for (int i = 0; i < 16; i++) y[i] = (x[i] * r) * g[i];
}

// One row slice: x holds chunk a (x[0..7]) and chunk b (x[8..15]). kFull:
// every lane is a pair lane (rot == 128).
template <int kMode, bool kFull>
__device__ __forceinline__ void norm_rope(const float* x, const float* g, bool pair_lane,
                                          const RopeEntry* tab, float eps, u32x4& out_a,
                                          u32x4& out_b) {
  float y[16];
  rms_normalise(x, g, eps, y);
  const bool rotate = kFull || pair_lane;
  float oa[8], ob[8];
#pragma unroll
  for (int i = 0; i < 8; i++) rope_pair<kMode>(y[i], y[8 + i], tab[i], rotate, oa[i], ob[i]);
  out_a = pack8(oa);
  out_b = pack8(ob);
}

}  // namespace h3hip
