// Block-sparse flash attention over 128x128 tiles, bf16 MFMA on gfx950.
//
// One workgroup (4 waves) per (head, 128-query tile) work unit, launched in
// the plan's XCD-aware order. Each wave owns 32 queries and keeps them in
// registers as the B operand of v_mfma_f32_32x32x16_bf16. Per active key tile
// the workgroup stages K (row-major) and V (transposed, V^T) in LDS, then each
// wave computes the transposed scores S^T = K Q^T, so a lane holds one
// query's scores for 32 keys: the row max and row sum are in-register
// reductions plus one exchange between the two half-waves, not a 32-lane
// shuffle tree. The exponentiated scores are already laid out as the B
// operand of O^T = V^T P^T (the 16-key chunk k of the MFMA pairs the C
// layout's register groups), so P never leaves registers.
//
// The softmax is the online recurrence of AxialReference.attendStreamingKeys
// (Sources/H3Attention/AxialReference.swift:129-171) in fp32 and base 2:
// m starts at -3e38, keys >= seq_len take the -1e30 sentinel, l and O are
// rescaled by 2^(m - m_new) per tile, and the output is O / max(l, 1e-30).
#include <cmath>

#include "common.h"
#include "plan.h"

namespace h3hip {

constexpr int kTile = 128;
constexpr int kD = 128;
// LDS row strides (bf16 elements). K rows are read 16 B at a time by 32
// consecutive rows: 272-byte rows put the 8 lanes of a phase on distinct
// banks. V^T rows are read 8 B at a time: 264-byte rows do the same for 16.
constexpr int kKStride = 136;
constexpr int kVStride = 132;

struct AttnArgs {
  const uint16_t* __restrict__ q;
  const uint16_t* __restrict__ k;
  const uint16_t* __restrict__ v;
  uint16_t* __restrict__ out;
  const int32_t* __restrict__ row_ptr;
  const int32_t* __restrict__ col_idx;
  const int32_t* __restrict__ work;
  int32_t seq_len, seq_pad, heads, out_layout;
  float scale_log2;
};

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ uint32_t half_of(uint32_t w, int hi) {
  return hi ? (w >> 16) : (w & 0xffffu);
}

__global__ __launch_bounds__(256, 2) void bsattn_fwd_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t ks[kTile * kKStride];
  __shared__ __attribute__((aligned(16))) uint16_t vt[kD * kVStride];

  const int32_t unit = a.work[blockIdx.x];
  if (unit < 0) return;
  const int head = unit >> 16, qt = unit & 0xffff;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, hh = lane >> 5;
  const size_t head_off = (size_t)head * a.seq_pad * kD;
  const uint16_t* qh = a.q + head_off;
  const uint16_t* kh = a.k + head_off;
  const uint16_t* vh = a.v + head_off;
  const int q0 = qt * kTile + wave * 32;

  // Q^T as the B operand: lane (li, hh) holds Q[q0 + li][16s + 8hh .. +7].
  bf16x8 qreg[8];
  {
    const uint16_t* qrow = qh + (size_t)(q0 + li) * kD + 8 * hh;
#pragma unroll
    for (int s = 0; s < 8; s++) qreg[s] = *reinterpret_cast<const bf16x8*>(qrow + 16 * s);
  }

  f32x16 oacc[4];
#pragma unroll
  for (int db = 0; db < 4; db++)
#pragma unroll
    for (int r = 0; r < 16; r++) oacc[db][r] = 0.f;
  float m = -3.0e38f, l = 0.f;

  const int beg = a.row_ptr[qt], end = a.row_ptr[qt + 1];
  const int k_row = tid >> 4, k_col = (tid & 15) * 8;
  const int v_d0 = (tid >> 4) * 8, v_j0 = (tid & 15) * 8;

  for (int t = beg; t < end; t++) {
    const int key0 = a.col_idx[t] * kTile;
    __syncthreads();  // the previous tile's LDS reads are done
#pragma unroll
    for (int it = 0; it < 8; it++) {
      const int row = it * 16 + k_row;
      *reinterpret_cast<u32x4*>(ks + row * kKStride + k_col) =
          ld16(kh + (size_t)(key0 + row) * kD + k_col);
    }
    {
      // 8 keys x 8 channels per thread, transposed in registers, written as
      // V^T[d0 + c][j0 .. j0 + 7]. Keys >= seq_len load as zero.
      u32x4 vr[8];
#pragma unroll
      for (int r = 0; r < 8; r++) {
        const int key = key0 + v_j0 + r;
        vr[r] = key < a.seq_len ? ld16(vh + (size_t)key * kD + v_d0) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int c = 0; c < 8; c++) {
        u32x2 w0, w1;
        w0[0] = half_of(vr[0][c >> 1], c & 1) | (half_of(vr[1][c >> 1], c & 1) << 16);
        w0[1] = half_of(vr[2][c >> 1], c & 1) | (half_of(vr[3][c >> 1], c & 1) << 16);
        w1[0] = half_of(vr[4][c >> 1], c & 1) | (half_of(vr[5][c >> 1], c & 1) << 16);
        w1[1] = half_of(vr[6][c >> 1], c & 1) | (half_of(vr[7][c >> 1], c & 1) << 16);
        uint16_t* dst = vt + (v_d0 + c) * kVStride + v_j0;
        *reinterpret_cast<u32x2*>(dst) = w0;
        *reinterpret_cast<u32x2*>(dst + 4) = w1;
      }
    }
    __syncthreads();

    // S^T[key][query] for the wave's 32 queries: 4 blocks of 32 keys.
    f32x16 sacc[4];
#pragma unroll
    for (int kb = 0; kb < 4; kb++) {
#pragma unroll
      for (int r = 0; r < 16; r++) sacc[kb][r] = 0.f;
      const uint16_t* krow = ks + (32 * kb + li) * kKStride + 8 * hh;
#pragma unroll
      for (int s = 0; s < 8; s++) {
        const bf16x8 ka = *reinterpret_cast<const bf16x8*>(krow + 16 * s);
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qreg[s], sacc[kb], 0, 0, 0);
      }
    }
    if (key0 + kTile > a.seq_len) {
#pragma unroll
      for (int kb = 0; kb < 4; kb++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int key = key0 + 32 * kb + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (key >= a.seq_len) sacc[kb][r] = -1.0e30f;
        }
    }

    float mx = -3.0e38f;
#pragma unroll
    for (int kb = 0; kb < 4; kb++)
#pragma unroll
      for (int r = 0; r < 16; r++) mx = fmaxf(mx, sacc[kb][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m, mx * a.scale_log2);
    const float alpha = __builtin_amdgcn_exp2f(m - m_new);
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < 4; kb++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const float p = __builtin_amdgcn_exp2f(fmaf(sacc[kb][r], a.scale_log2, -m_new));
        sacc[kb][r] = p;
        psum += p;
      }
    l = l * alpha + psum;
    m = m_new;
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
      for (int r = 0; r < 16; r++) oacc[db][r] *= alpha;

    // P^T as the B operand of O^T = V^T P^T: chunk kc takes registers
    // 8*(kc&1) .. +7 of key block kc>>1; element e of half-wave hh is key
    // 16kc + 8(e/4) + 4hh + e%4, so V^T supplies keys 16kc+4hh+[0,4) and
    // 16kc+8+4hh+[0,4) in the same element order.
    bf16x8 pb[8];
#pragma unroll
    for (int kc = 0; kc < 8; kc++)
#pragma unroll
      for (int e = 0; e < 8; e++) pb[kc][e] = (__bf16)sacc[kc >> 1][8 * (kc & 1) + e];
#pragma unroll
    for (int db = 0; db < 4; db++) {
      const uint16_t* vrow = vt + (32 * db + li) * kVStride + 4 * hh;
#pragma unroll
      for (int kc = 0; kc < 8; kc++) {
        const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow + 16 * kc);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 16 * kc + 8);
        const u32x4 w = {lo[0], lo[1], hi[0], hi[1]};
        const bf16x8 va = __builtin_bit_cast(bf16x8, w);
        oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[kc], oacc[db], 0, 0, 0);
      }
    }
  }

  // O^T C layout: lane (li, hh) holds query q0 + li, channels
  // 32db + 8g + 4hh + [0, 4) in registers 4g .. 4g + 3.
  const float lt = l + __shfl_xor(l, 32);
  const float inv = 1.0f / fmaxf(lt, 1.0e-30f);
  const int qi = q0 + li;
  const bool valid = qi < a.seq_len;
  uint16_t* orow = a.out_layout == H3HIP_OUT_HEAD_MAJOR
                       ? a.out + head_off + (size_t)qi * kD
                       : a.out + (size_t)qi * a.heads * kD + (size_t)head * kD;
#pragma unroll
  for (int db = 0; db < 4; db++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      u32x2 w = {0u, 0u};
      if (valid) {
        w[0] = pack_bf16x2(oacc[db][4 * g] * inv, oacc[db][4 * g + 1] * inv);
        w[1] = pack_bf16x2(oacc[db][4 * g + 2] * inv, oacc[db][4 * g + 3] * inv);
      }
      *reinterpret_cast<u32x2*>(orow + 32 * db + 8 * g + 4 * hh) = w;
    }
}

static int launch_bsattn(h3hip_plan p, const void* q, const void* k, const void* v,
                         float scale, void* out, int32_t out_layout, hipStream_t stream) {
  AttnArgs args{static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                static_cast<const uint16_t*>(v), static_cast<uint16_t*>(out),
                p->d_row_ptr, p->d_col_idx, p->d_work, p->seq_len, p->seq_pad, p->heads,
                out_layout, scale * 1.4426950408889634f};
  const unsigned grid = (unsigned)p->work.size();
  if (grid == 0) return H3HIP_OK;
  bsattn_fwd_kernel<<<grid, 256, 0, stream>>>(args);
  return check_launch("bsattn_fwd_kernel");
}

}  // namespace h3hip

using namespace h3hip;

extern "C" int h3hip_bsattn_fwd(h3hip_plan plan, const void* q, const void* k, const void* v,
                                int32_t heads, int32_t head_dim, float scale, void* out,
                                int32_t out_layout, void* stream) {
  H3_REQUIRE(plan != nullptr, H3HIP_EINVAL, "plan is NULL");
  if (head_dim != kD || heads != plan->heads) {
    set_error("declined: head_dim %d heads %d (needs head_dim 128 and the plan's %d heads)",
              head_dim, heads, plan->heads);
    return H3HIP_DECLINED;
  }
  H3_REQUIRE(q && k && v && out, H3HIP_EINVAL, "NULL tensor argument");
  auto aligned16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  H3_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out), H3HIP_EINVAL,
             "tensors must be 16-byte aligned");
  H3_REQUIRE(std::isfinite(scale) && scale > 0.f, H3HIP_EINVAL, "scale must be finite and > 0");
  H3_REQUIRE(out_layout == H3HIP_OUT_HEAD_MAJOR || out_layout == H3HIP_OUT_TOKEN_MAJOR,
             H3HIP_EINVAL, "unknown out_layout %d", out_layout);
  return launch_bsattn(plan, q, k, v, scale, out, out_layout, as_stream(stream));
}

extern "C" int h3hip_attend(h3hip_plan plan, const h3hip_attention_context* ctx, const void* q,
                            const void* k, const void* v, int32_t heads, int32_t head_dim,
                            float scale, void* out, void* stream) {
  H3_REQUIRE(plan != nullptr, H3HIP_EINVAL, "plan is NULL");
  // No context means dense: a backend that does not know its block or its
  // schedule position cannot honour its own policy
  // (Tests/H3ModulesTests/AttentionSeamTests.swift:127-137).
  if (ctx == nullptr) {
    set_error("declined: no attention context");
    return H3HIP_DECLINED;
  }
  // A plan built for another shape would attend the wrong tiles: refuse the
  // call rather than guess (AxialTopology.swift:65-77).
  if (ctx->sequence_length != plan->seq_len) {
    set_error("declined: sequence length %d, plan built for %d", ctx->sequence_length,
              plan->seq_len);
    return H3HIP_DECLINED;
  }
  if ((plan->kind == H3HIP_RULE_LOCAL || plan->kind == H3HIP_RULE_AXIAL) &&
      ctx->video_start >= 0 &&
      (ctx->video_start != plan->prefix_len || ctx->video_stop != plan->seq_len)) {
    set_error("declined: video span [%d, %d), plan built for [%d, %d)", ctx->video_start,
              ctx->video_stop, plan->prefix_len, plan->seq_len);
    return H3HIP_DECLINED;
  }
  const h3hip_policy& pol = plan->policy;
  if (ctx->block_index < pol.dense_first_blocks ||
      (pol.dense_last_blocks > 0 && ctx->block_index >= ctx->block_count - pol.dense_last_blocks) ||
      ctx->schedule_progress < pol.dense_until_progress ||
      ctx->sequence_length < pol.min_sequence_length) {
    set_error("declined by policy: block %d of %d, progress %.3f", ctx->block_index,
              ctx->block_count, ctx->schedule_progress);
    return H3HIP_DECLINED;
  }
  return h3hip_bsattn_fwd(plan, q, k, v, heads, head_dim, scale, out, H3HIP_OUT_HEAD_MAJOR,
                          stream);
}
