// Fused Q/K RMSNorm + 3D split-half RoPE + relayout to head-major.
//
// Memory-bound: every (token, head) row of Q and K is read once (256 B each)
// and written once, head-major. A workgroup owns TOKS consecutive tokens and
// all heads; it first computes the rotation table (cos, sin of pos[axis] *
// inv_freq for every pair) for its tokens into LDS -- once per token instead
// of once per (token, head, tensor) -- then 16-lane groups stream the rows,
// each lane holding 8 channels (one 16-byte load and store per tensor).
//
// Arithmetic follows H3RMSNorm (Sources/H3Modules/Modulation.swift:116-120)
// and SplitHalfRoPE (Sources/H3Modules/DiTBlock.swift:83-103):
//   r = rsqrt(mean(x^2) + eps); y = bf16((x * r) * gamma)
//   ra = bf16(bf16(c*a) + bf16(-s*b)); rb = bf16(bf16(s*a) + bf16(c*b))
// with c, s = bf16(cos/sin(pos[axis] * inv_freq)) (the bf16 rotation table of
// H3Transformer.swift:271-273). The sum of squares is accumulated in double:
// squares of bf16 values are exact, so the mean is the exactly rounded fp32
// mean whatever the reduction order; rsqrt and sin/cos are evaluated in
// double and rounded once to fp32.
#include "common.h"

namespace h3hip {

struct PrologueArgs {
  const uint16_t* __restrict__ q_in;
  const uint16_t* __restrict__ k_in;
  const uint16_t* __restrict__ v_in;
  const uint16_t* __restrict__ q_gamma;
  const uint16_t* __restrict__ k_gamma;
  const float* __restrict__ pos;
  const int32_t* __restrict__ pair_axis;
  const float* __restrict__ pair_inv;
  uint16_t* __restrict__ q_out;
  uint16_t* __restrict__ k_out;
  uint16_t* __restrict__ v_out;
  int64_t ld_in;
  float eps;
  int32_t rot, seq_len, seq_pad, heads;
};

constexpr int kTok = 4;       // tokens per workgroup
constexpr int kHeadDim = 128;
constexpr int kMaxHalf = 64;

__device__ __forceinline__ u32x4 load16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ void store16(uint16_t* p, u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}

__device__ __forceinline__ void unpack8(u32x4 w, float* f) {
#pragma unroll
  for (int i = 0; i < 4; i++) {
    f[2 * i] = bf16_lo(w[i]);
    f[2 * i + 1] = bf16_hi(w[i]);
  }
}

__device__ __forceinline__ double group16_sum(double v) {
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) v += __shfl_xor(v, off, 16);
  return v;
}

// Normalises one row slice (8 channels per lane) and applies the rotation.
// `j` is the lane's index inside its 16-lane group; channels 8j..8j+7.
template <int kMode>
__device__ __forceinline__ u32x4 norm_rope_row(u32x4 raw, const float* g, int j, int half,
                                               int rot, float eps, const float2* cs) {
  float x[8];
  unpack8(raw, x);
  double ss = 0.0;
#pragma unroll
  for (int i = 0; i < 8; i++) ss += (double)x[i] * (double)x[i];
  ss = group16_sum(ss);
  const float ms = (float)(ss / (double)kHeadDim);
  const float r = (float)(1.0 / sqrt((double)(ms + eps)));
  float y[8];
#pragma unroll
  for (int i = 0; i < 8; i++) y[i] = (x[i] * r) * g[i];

  const int hl = half >> 3;  // lanes per half
  const int src = j < hl ? j + hl : (j < 2 * hl ? j - hl : j);
  const bool is_a = j < hl, is_b = j >= hl && j < 2 * hl;
  float out[8];
  if (kMode == H3HIP_ROUND_REFERENCE) {
    u32x4 packed;
#pragma unroll
    for (int i = 0; i < 4; i++) packed[i] = pack_bf16x2(y[2 * i], y[2 * i + 1]);
    u32x4 other;
#pragma unroll
    for (int i = 0; i < 4; i++) other[i] = __shfl(packed[i], src, 16);
    float me[8], pt[8];
    unpack8(packed, me);
    unpack8(other, pt);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int p = is_a ? 8 * j + i : 8 * j + i - half;
      if (is_a) {
        const float c = cs[p].x, s = cs[p].y;
        out[i] = round_bf16(round_bf16(c * me[i]) + round_bf16(-s * pt[i]));
      } else if (is_b) {
        const float c = cs[p].x, s = cs[p].y;
        out[i] = round_bf16(round_bf16(s * pt[i]) + round_bf16(c * me[i]));
      } else {
        out[i] = me[i];
      }
    }
  } else {
    float pt[8];
#pragma unroll
    for (int i = 0; i < 8; i++) pt[i] = __shfl(y[i], src, 16);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int p = is_a ? 8 * j + i : 8 * j + i - half;
      if (is_a) {
        const float c = cs[p].x, s = cs[p].y;
        out[i] = c * y[i] - s * pt[i];
      } else if (is_b) {
        const float c = cs[p].x, s = cs[p].y;
        out[i] = s * pt[i] + c * y[i];
      } else {
        out[i] = y[i];
      }
    }
  }
  u32x4 res;
#pragma unroll
  for (int i = 0; i < 4; i++) res[i] = pack_bf16x2(out[2 * i], out[2 * i + 1]);
  return res;
}

template <int kMode>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(PrologueArgs a) {
  __shared__ float2 cs[kTok][kMaxHalf];
  const int tid = threadIdx.x;
  const int32_t s0 = blockIdx.x * kTok;
  const int half = a.rot >> 1;

  // Rotation table for this workgroup's tokens.
  for (int t = tid; t < kTok * half; t += 256) {
    const int tok = t / half, p = t - tok * half;
    const int32_t s = s0 + tok;
    float c = 1.f, sn = 0.f;
    if (s < a.seq_len) {
      const int axis = min(max(a.pair_axis[p], 0), 2);  // a bad table cannot index past pos
      const float ang = a.pos[(int64_t)s * 3 + axis] * a.pair_inv[p];
      c = (float)cos((double)ang);
      sn = (float)sin((double)ang);
      if (kMode == H3HIP_ROUND_REFERENCE) {
        c = round_bf16(c);
        sn = round_bf16(sn);
      }
    }
    cs[tok][p] = make_float2(c, sn);
  }

  const int g = tid >> 4, j = tid & 15;
  float qg[8], kg[8];
  unpack8(load16(a.q_gamma + 8 * j), qg);
  unpack8(load16(a.k_gamma + 8 * j), kg);
  __syncthreads();

  const int rows = kTok * a.heads;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  for (int rho = g; rho < rows; rho += 16) {
    const int head = rho / kTok, tok = rho - head * kTok;
    const int32_t s = s0 + tok;
    const int64_t dst = ((int64_t)head * a.seq_pad + s) * kHeadDim + 8 * j;
    if (s >= a.seq_len) {
      store16(a.q_out + dst, zero);
      store16(a.k_out + dst, zero);
      if (a.v_out) store16(a.v_out + dst, zero);
      continue;
    }
    const int64_t src = (int64_t)s * a.ld_in + (int64_t)head * kHeadDim + 8 * j;
    const u32x4 qraw = load16(a.q_in + src);
    const u32x4 kraw = load16(a.k_in + src);
    u32x4 vraw = zero;
    if (a.v_in) vraw = load16(a.v_in + src);
    store16(a.q_out + dst, norm_rope_row<kMode>(qraw, qg, j, half, a.rot, a.eps, cs[tok]));
    store16(a.k_out + dst, norm_rope_row<kMode>(kraw, kg, j, half, a.rot, a.eps, cs[tok]));
    if (a.v_in) store16(a.v_out + dst, vraw);
  }
}

}  // namespace h3hip

using namespace h3hip;

extern "C" int h3hip_qk_norm_rope(const void* q_in, const void* k_in, int64_t ld_in,
                                  const void* v_in, const void* q_gamma, const void* k_gamma,
                                  float eps, const float* pos, const int32_t* pair_axis,
                                  const float* pair_inv_freq, int32_t rot, int32_t rounding,
                                  int32_t seq_len, int32_t seq_pad, int32_t heads,
                                  int32_t head_dim, void* q_out, void* k_out, void* v_out,
                                  void* stream) {
  // The fixture's geometry guard (QKFusionMetalFixture.swift:85-95): decline
  // rather than index an unsupported row layout.
  if (head_dim != kHeadDim || rot <= 0 || rot > head_dim || rot % 16 != 0) {
    set_error("declined: head_dim %d / rot %d (needs head_dim 128, rot a multiple of 16 <= 128)",
              head_dim, rot);
    return H3HIP_DECLINED;
  }
  H3_REQUIRE(q_in && k_in && q_gamma && k_gamma && pos && pair_axis && pair_inv_freq && q_out &&
                 k_out,
             H3HIP_EINVAL, "NULL tensor argument");
  H3_REQUIRE((v_in == nullptr) == (v_out == nullptr), H3HIP_EINVAL,
             "v_in and v_out must both be set or both be NULL");
  H3_REQUIRE(seq_len > 0 && heads > 0 && seq_pad >= seq_len && seq_pad % kTok == 0, H3HIP_EINVAL,
             "bad shape: seq_len %d seq_pad %d heads %d", seq_len, seq_pad, heads);
  H3_REQUIRE(ld_in >= (int64_t)heads * head_dim && ld_in % 8 == 0, H3HIP_EINVAL,
             "ld_in %lld must be >= heads*head_dim and a multiple of 8", (long long)ld_in);
  H3_REQUIRE(rounding == H3HIP_ROUND_REFERENCE || rounding == H3HIP_ROUND_FP32, H3HIP_EINVAL,
             "unknown rounding mode %d", rounding);
  auto aligned16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  H3_REQUIRE(aligned16(q_in) && aligned16(k_in) && aligned16(q_gamma) && aligned16(k_gamma) &&
                 aligned16(q_out) && aligned16(k_out) && (!v_in || (aligned16(v_in) && aligned16(v_out))),
             H3HIP_EINVAL, "tensors must be 16-byte aligned");
  PrologueArgs a{static_cast<const uint16_t*>(q_in),   static_cast<const uint16_t*>(k_in),
                 static_cast<const uint16_t*>(v_in),   static_cast<const uint16_t*>(q_gamma),
                 static_cast<const uint16_t*>(k_gamma), pos,
                 pair_axis,                             pair_inv_freq,
                 static_cast<uint16_t*>(q_out),         static_cast<uint16_t*>(k_out),
                 static_cast<uint16_t*>(v_out),         ld_in,
                 eps,                                   rot,
                 seq_len,                               seq_pad,
                 heads};
  const dim3 grid(seq_pad / kTok);
  if (rounding == H3HIP_ROUND_REFERENCE)
    qk_norm_rope_kernel<H3HIP_ROUND_REFERENCE><<<grid, 256, 0, as_stream(stream)>>>(a);
  else
    qk_norm_rope_kernel<H3HIP_ROUND_FP32><<<grid, 256, 0, as_stream(stream)>>>(a);
  return check_launch("qk_norm_rope_kernel");
}
