// Fused Q/K RMSNorm + 3D split-half RoPE + relayout to head-major.
//
// Memory-bound by design: every (token, head) row of Q and K is read once
// (256 B) and written once, head-major. A workgroup owns kTok consecutive
// tokens and all heads. It first computes the rotation table (cos, sin of
// pos[axis] * inv_freq) for its tokens into LDS -- once per token, shared by
// every head and by Q and K -- then 8-lane groups stream the rows: half of the
// groups Q, half K, each with the next row's loads in flight.
//
// Lane ownership: lane j of a row holds two 8-channel chunks, chosen so that
// each RoPE pair (p, p + rot/2) lives in one lane and the rotation needs no
// cross-lane exchange: pair lanes (8j < rot/2) hold chunks j and j + rot/16;
// the remaining lanes hold two consecutive pass-through chunks of the
// channels >= rot. Each chunk is one 16-byte load and one 16-byte store.
//
// Arithmetic follows H3RMSNorm (Sources/H3Modules/Modulation.swift:116-120)
// and SplitHalfRoPE (Sources/H3Modules/DiTBlock.swift:83-103):
//   ms = mean(x^2); r = rsqrt(ms + eps); y = (x * r) * gamma
//   REFERENCE rounding: y, the table and every RoPE product and sum are
//     rounded to bf16, as MLX computes the unfused chain on bf16 arrays:
//     ra = bf16(bf16(c*a) + bf16(-s*b)), rb = bf16(bf16(s*a) + bf16(c*b)).
//   FP32 rounding: fp32 throughout, one rounding at the store.
// The mean is an fp32 sum in a fixed order: each lane accumulates its 16
// squares with fma in channel order (chunk a, then chunk b), then the 8 lane
// sums combine as t_j = s_j + s_{7-j}, u_j = t_j + t_{j^2}, total = u_j + u_{j^1}
// (DPP half-row mirror, quad xor 2, quad xor 1); every lane ends with the same
// bits. rsqrt is refined in double and rounded once to fp32.
#include "common.h"
#include "norm_rope.h"

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

#ifndef H3HIP_PROLOGUE_TOK
#define H3HIP_PROLOGUE_TOK 4
#endif
constexpr int kTok = H3HIP_PROLOGUE_TOK;  // tokens per workgroup
constexpr int kHeadDim = 128;
constexpr int kMaxHalf = 64;
constexpr int kLanesPerRow = 8;
constexpr int kRowGroups = 256 / kLanesPerRow;

__device__ __forceinline__ u32x4 load16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
// The row streams are touched once: non-temporal loads and stores keep them
// from displacing reused lines (gamma, the table) and measure ~8% faster than
// plain ones for a pure copy on MI355X.
__device__ __forceinline__ u32x4 stream_load16(const uint16_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void store16(uint16_t* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// Workgroup: kTok tokens x all heads. Row groups of 8 lanes; the first half of
// the groups normalise Q rows, the second half K rows, each streaming its rows
// with the next row's loads issued before the current row is computed. V rows
// (when given) are copied by all groups afterwards.
template <int kMode, bool kFull>
__global__ __launch_bounds__(256, 5) void qk_norm_rope_kernel(PrologueArgs a) {
  __shared__ RopeEntry tab_lds[kTok][kMaxHalf];
  const int tid = threadIdx.x;
  const int32_t s0 = blockIdx.x * kTok;
  const int half = a.rot >> 1;

  const int grp = tid / kLanesPerRow, j = tid % kLanesPerRow;
  const int hl = half / 8;  // pair lanes per row
  const bool pair_lane = kFull || j < hl;
  const int chunk_a = pair_lane ? j : 2 * hl + 2 * (j - hl);
  const int chunk_b = pair_lane ? j + hl : chunk_a + 1;
  const int off_a = 8 * chunk_a, off_b = 8 * chunk_b;
  const int pair0 = pair_lane ? 8 * j : 0;

  constexpr int kGroupsPerTensor = kRowGroups / 2;
  const bool is_k = grp >= kGroupsPerTensor;
  const int g0 = is_k ? grp - kGroupsPerTensor : grp;
  const uint16_t* __restrict__ in = is_k ? a.k_in : a.q_in;
  uint16_t* __restrict__ out = is_k ? a.k_out : a.q_out;
  float gam[16];
  {
    const uint16_t* gsrc = is_k ? a.k_gamma : a.q_gamma;
    unpack8(load16(gsrc + off_a), gam);
    unpack8(load16(gsrc + off_b), gam + 8);
  }

  // A row group keeps one token (kGroupsPerTensor is a multiple of kTok) and
  // steps through the heads kGroupsPerTensor / kTok at a time, so both row
  // pointers advance by constants.
  static_assert(kGroupsPerTensor % kTok == 0 && kRowGroups % kTok == 0, "row groups vs tokens");
  constexpr int kHeadStep = kGroupsPerTensor / kTok;
  const int tok = g0 % kTok;
  const int32_t s = s0 + tok;
  const bool tok_valid = s < a.seq_len;
  int head = g0 / kTok;
  const uint16_t* src = in + (int64_t)s * a.ld_in + (int64_t)head * kHeadDim;
  uint16_t* dst = out + ((int64_t)head * a.seq_pad + s) * kHeadDim;
  const int64_t dst_step = (int64_t)kHeadStep * a.seq_pad * kHeadDim;
  const u32x4 zero = {0u, 0u, 0u, 0u};
  u32x4 na = zero, nb = zero;
  if (tok_valid && head < a.heads) {
    na = stream_load16(src + off_a);
    nb = stream_load16(src + off_b);
  }
  // The first row is in flight while the rotation table is computed.
  for (int t = tid; t < kTok * half; t += 256) {
    const int tk = t / half, p = t - tk * half;
    const int32_t st = s0 + tk;
    RopeEntry e{1.f, 0.f};
    if (st < a.seq_len) {
      const int axis = min(max(a.pair_axis[p], 0), 2);  // a bad table cannot index past pos
      e = make_rope_entry<kMode>(a.pos[(int64_t)st * 3 + axis] * a.pair_inv[p]);
    }
    tab_lds[tk][p] = e;
  }

  __syncthreads();

  const RopeEntry* tab = &tab_lds[tok][pair0];
  for (; head < a.heads; head += kHeadStep) {
    const u32x4 ca = na, cb = nb;
    src += kHeadStep * kHeadDim;
    if (tok_valid && head + kHeadStep < a.heads) {
      na = stream_load16(src + off_a);
      nb = stream_load16(src + off_b);
    }
    u32x4 oa = zero, ob = zero;
    if (tok_valid) {
      float x[16];
      unpack8(ca, x);
      unpack8(cb, x + 8);
      norm_rope<kMode, kFull>(x, gam, pair_lane, tab, a.eps, oa, ob);
    }
    store16(dst + off_a, oa);
    store16(dst + off_b, ob);
    dst += dst_step;
  }

  if (a.v_in) {
    // V rows: all row groups, token grp % kTok, heads kRowGroups / kTok apart.
    constexpr int kVStep = kRowGroups / kTok;
    const int vtok = grp % kTok;
    const int32_t vs = s0 + vtok;
    const bool v_valid = vs < a.seq_len;
    int vh = grp / kTok;
    const uint16_t* vsrc = a.v_in + (int64_t)vs * a.ld_in + (int64_t)vh * kHeadDim;
    uint16_t* vdst = a.v_out + ((int64_t)vh * a.seq_pad + vs) * kHeadDim;
    const int64_t vdst_step = (int64_t)kVStep * a.seq_pad * kHeadDim;
    for (; vh < a.heads; vh += kVStep) {
      u32x4 va = zero, vb = zero;
      if (v_valid) {
        va = stream_load16(vsrc + off_a);
        vb = stream_load16(vsrc + off_b);
      }
      store16(vdst + off_a, va);
      store16(vdst + off_b, vb);
      vsrc += kVStep * kHeadDim;
      vdst += vdst_step;
    }
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
                 aligned16(q_out) && aligned16(k_out) &&
                 (!v_in || (aligned16(v_in) && aligned16(v_out))),
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
  hipStream_t st = as_stream(stream);
  const bool full = rot == head_dim;
  if (rounding == H3HIP_ROUND_REFERENCE) {
    if (full)
      qk_norm_rope_kernel<H3HIP_ROUND_REFERENCE, true><<<grid, 256, 0, st>>>(a);
    else
      qk_norm_rope_kernel<H3HIP_ROUND_REFERENCE, false><<<grid, 256, 0, st>>>(a);
  } else {
    if (full)
      qk_norm_rope_kernel<H3HIP_ROUND_FP32, true><<<grid, 256, 0, st>>>(a);
    else
      qk_norm_rope_kernel<H3HIP_ROUND_FP32, false><<<grid, 256, 0, st>>>(a);
  }
  return check_launch("qk_norm_rope_kernel");
}
