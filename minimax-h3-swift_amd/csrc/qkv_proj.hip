// Fused QKV projection: the GEMM of AttentionLayer.callAsFunction
// (Sources/H3Modules/DiTBlock.swift:336-338, `matmul(x, qkvWeight.T)` split
// into Q | K | V of heads x 128 channels each) with the Q/K prologue -- per-head
// H3RMSNorm and SplitHalfRoPE (DiTBlock.swift:346-352) -- and the head-major
// relayout done in its epilogue. Q, K and V come out head-major
// [heads, seq_pad, 128], the layout the attention reads, without the token-major
// qkv ever being written and read back.
//
// GEMM: C^T[n, m] = sum_k W[n, k] x[m, k] with v_mfma_f32_32x32x16_bf16, the W
// rows as the A operand and the x rows as B. Each accumulator lane therefore
// holds one token and 16 output channels: a token's 128 channels of one head
// sit in one lane pair (lanes l and l ^ 32), so the row norm needs one exchange
// between the half-waves and every RoPE pair (p, p + rot/2) is in one lane.
//
// Workgroup: 256 tokens x 256 output channels (two heads of one of Q, K, V),
// 8 waves. Wave w owns head (w >> 2) of the tile and tokens 64 (w & 3) .. +63:
// 4 x 2 accumulators of 32 x 32. The reduction runs in steps of 64: the W and x
// tiles of a step (256 rows of 128 bytes each, 16-byte chunks XOR-swizzled so
// operand reads are conflict-free) are double-buffered in LDS and filled by
// HBM -> LDS buffer loads. Each wave issues its 8 loads for step t+1 spread
// through step t's MFMAs and drains them before the step's barrier.
//
// Epilogue (Q and K): the fp32 accumulators are rounded to bf16 (the bf16
// matmul output the reference normalises), the mean of squares is summed in
// exactly the order the prologue kernel uses, and norm and rotation use the
// same arithmetic (norm_rope.h), so the output equals h3hip_qk_norm_rope
// applied to this kernel's bf16 GEMM result, bit for bit.
#include <type_traits>

#include "common.h"
#include "norm_rope.h"

namespace h3hip {

struct ProjArgs {
  const uint16_t* __restrict__ x;        // [seq_len, hidden], row stride ldx
  const uint16_t* __restrict__ w;        // [3 * heads * 128, hidden], row stride ldw
  const uint16_t* __restrict__ q_gamma;  // [128]
  const uint16_t* __restrict__ k_gamma;
  const float* __restrict__ pos;         // [seq_len, 3]
  const int32_t* __restrict__ pair_axis;
  const float* __restrict__ pair_inv;
  uint16_t* __restrict__ q_out;          // [heads, seq_pad, 128]
  uint16_t* __restrict__ k_out;
  uint16_t* __restrict__ v_out;
  int64_t ldx, ldw;
  float eps;
  int32_t hidden, rot, seq_len, seq_pad, heads, tiles_m;
};

constexpr int kPM = 256;                  // tokens per workgroup
constexpr int kPN = 256;                  // output channels per workgroup
constexpr int kPK = 64;                   // reduction per step
constexpr int kHD = 128;                  // head_dim
constexpr int kPThreads = 512;
constexpr int kGroupM = 16;               // token tiles per launch-order group
constexpr int kTileElems = kPM * kPK;     // one operand tile (W or x) of a step
constexpr int kStageElems = 2 * kTileElems;
// s_waitcnt immediate for vmcnt(0), expcnt and lgkmcnt unconstrained (gfx9).
constexpr int kPWaitVmcnt0 = 0x0F70;
constexpr int kPBufferWord3 = 0x00020000;

typedef int i32x4p __attribute__((ext_vector_type(4)));

// 16-byte chunk c of the 128-byte row r sits at c ^ ((r >> 1) & 7): the 16
// rows of a 16-lane read phase cover both row parities x 8 chunk positions.
__device__ __forceinline__ int p_swz(int r) { return (r >> 1) & 7; }

__device__ __forceinline__ i32x4p proj_rsrc(const void* base, uint32_t bytes) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  i32x4p r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  r[1] = __builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32) & 0xffff);  // stride 0
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = kPBufferWord3;
  return r;
}

// 16 bytes per lane from a buffer into LDS at m0 + 16*lane (assembly: the
// compiler does not count it; the issuing wave drains it with vmcnt(0)). The
// s_nop is the wait state an SALU write of m0 needs before the load.
__device__ __forceinline__ void proj_dma16(const i32x4p& rsrc, uint32_t lds_addr, int voff,
                                           int soff) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds_addr)
               : "memory");
}

__device__ __forceinline__ uint32_t proj_lds_address(const uint16_t* p) {
  return (uint32_t)(size_t)((__attribute__((address_space(3))) const uint16_t*)p);
}

// kHl = rot / 16 (8-channel chunks per rotation half); kPlain: write the bf16
// GEMM result of every part unchanged (the materialised qkv, for tests).
template <int kMode, int kHl, bool kPlain>
__global__ __launch_bounds__(kPThreads, 1) void qkv_proj_kernel(ProjArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kStageElems];   // 128 KiB

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nh = wave >> 2, mq = wave & 3;
  const int li = lane & 31, hh = lane >> 5;
  // Grouped order: groups of kGroupM token tiles x all channel tiles, token
  // tile fastest, so the workgroups in flight together share a few x tiles
  // and a few W tiles in L2.
  const int inner = a.heads * kHD;
  const int tiles_n = 3 * inner / kPN;
  const int group = blockIdx.x / (kGroupM * tiles_n);
  const int first_m = group * kGroupM;
  const int gm = min(a.tiles_m - first_m, kGroupM);
  const int local = blockIdx.x - group * kGroupM * tiles_n;
  const int tm = first_m + local % gm, tn = local / gm;
  const int m0 = tm * kPM, n0 = tn * kPN;
  const int part = n0 / inner;                        // uniform over the tile
  const int head = (n0 - part * inner) / kHD + nh;    // this wave's head

  // Operand offsets within a tile (elements): A = W row nh*128 + 32nb + li,
  // B = x row 64mq + 32mb + li; chunk 2s + hh of the step's 64 columns.
  int a_row[4], b_row[2];
#pragma unroll
  for (int nb = 0; nb < 4; nb++) a_row[nb] = nh * 128 + 32 * nb + li;
#pragma unroll
  for (int mb = 0; mb < 2; mb++) b_row[mb] = 64 * mq + 32 * mb + li;
  auto operand = [&](const uint16_t* tile, int row, int s) __attribute__((always_inline)) {
    return *reinterpret_cast<const bf16x8*>(tile + row * kPK + (((2 * s + hh) ^ p_swz(row)) * 8));
  };

  // HBM -> LDS: wave w moves rows 32w .. 32w+31 of the W tile and of the x
  // tile, 8 rows per instruction (lane l: row 32w + 8i + l/8, chunk position
  // l%8 filled from the global chunk the swizzle places there).
  const i32x4p w_rsrc = proj_rsrc(a.w, (uint32_t)(3 * inner) * (uint32_t)a.ldw * 2u);
  const i32x4p x_rsrc = proj_rsrc(a.x, (uint32_t)((a.seq_len - 1) * a.ldx + a.hidden) * 2u);
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane(proj_lds_address(lds));
  const int dma_r = 32 * wave + (lane >> 3);
  int w_voff[4], x_voff[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = dma_r + 8 * i;
    const int src_chunk = (lane & 7) ^ p_swz(r);
    w_voff[i] = (n0 + r) * (int)a.ldw * 2 + src_chunk * 16;
    x_voff[i] = (m0 + r) * (int)a.ldx * 2 + src_chunk * 16;   // rows >= seq_len: out of range, read as 0
  }
  // Load i of step t (i < 4: W rows, i >= 4: x rows) into stage st.
  auto dma = [&](int t, int st, int i) __attribute__((always_inline)) {
    const int ii = i & 3;
    const uint32_t dst = lds_base + 2 * (st * kStageElems + (i >= 4 ? kTileElems : 0) +
                                         (32 * wave + 8 * ii) * kPK);
    proj_dma16(i < 4 ? w_rsrc : x_rsrc, dst, i < 4 ? w_voff[ii] : x_voff[ii], t * kPK * 2);
  };

  f32x16 acc[4][2];
#pragma unroll
  for (int nb = 0; nb < 4; nb++)
#pragma unroll
    for (int mb = 0; mb < 2; mb++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[nb][mb][r] = 0.f;

  const int steps = a.hidden / kPK;
#pragma unroll
  for (int i = 0; i < 8; i++) dma(0, 0, i);
  __builtin_amdgcn_s_waitcnt(kPWaitVmcnt0);
  __syncthreads();

  for (int t = 0; t < steps; t++) {
    const uint16_t* wt = lds + (t & 1) * kStageElems;
    const uint16_t* xt = wt + kTileElems;
    const bool more = t + 1 < steps;
    bf16x8 A[2][4], B[2][2];
#pragma unroll
    for (int nb = 0; nb < 4; nb++) A[0][nb] = operand(wt, a_row[nb], 0);
#pragma unroll
    for (int mb = 0; mb < 2; mb++) B[0][mb] = operand(xt, b_row[mb], 0);
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const int cur = s & 1;
      if (s + 1 < 4) {
#pragma unroll
        for (int nb = 0; nb < 4; nb++) A[cur ^ 1][nb] = operand(wt, a_row[nb], s + 1);
#pragma unroll
        for (int mb = 0; mb < 2; mb++) B[cur ^ 1][mb] = operand(xt, b_row[mb], s + 1);
      }
#pragma unroll
      for (int nb = 0; nb < 4; nb++) {
#pragma unroll
        for (int mb = 0; mb < 2; mb++)
          acc[nb][mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[cur][nb], B[cur][mb],
                                                                acc[nb][mb], 0, 0, 0);
        if (more && (nb & 1) == 1) dma(t + 1, (t + 1) & 1, 2 * s + (nb >> 1));
      }
    }
    __builtin_amdgcn_s_waitcnt(kPWaitVmcnt0);
    __syncthreads();
  }

  // ---- epilogue: lane (li, hh) holds token m0 + 64mq + 32mb + li, channels
  // 32nb + 8g + 4hh + e of the head in register 4g + e of acc[nb][mb].
  uint16_t* out = part == 0 ? a.q_out : part == 1 ? a.k_out : a.v_out;
  const bool norm = !kPlain && part < 2;
  const uint16_t* gamma = part == 0 ? a.q_gamma : a.k_gamma;
  constexpr int hl = kHl;
#pragma unroll
  for (int mb = 0; mb < 2; mb++) {
    const int m = m0 + 64 * mq + 32 * mb + li;
    if (m >= a.seq_pad) continue;
    const bool valid = m < a.seq_len;
    // bf16 GEMM result of this lane's 64 channels, packed: xb[nb][g][0..1].
    uint32_t xb[4][4][2];
#pragma unroll
    for (int nb = 0; nb < 4; nb++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        xb[nb][g][0] = cvt_pk(acc[nb][mb][4 * g], acc[nb][mb][4 * g + 1]);
        xb[nb][g][1] = cvt_pk(acc[nb][mb][4 * g + 2], acc[nb][mb][4 * g + 3]);
      }
    uint32_t ob[4][4][2];
    if (!norm) {
#pragma unroll
      for (int nb = 0; nb < 4; nb++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          ob[nb][g][0] = valid ? xb[nb][g][0] : 0u;
          ob[nb][g][1] = valid ? xb[nb][g][1] : 0u;
        }
    } else {
      // The partner half-wave's 64 channels: channel 8c + 4(hh^1) + e.
      uint32_t pb[4][4][2];
#pragma unroll
      for (int nb = 0; nb < 4; nb++)
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
          for (int e = 0; e < 2; e++) pb[nb][g][e] = __shfl_xor(xb[nb][g][e], 32);
      // Channel ch of the row as fp32 (its bf16 value).
      auto chan = [&](int ch) __attribute__((always_inline)) {
        const int c = ch >> 3, o = ch & 7, nb = c >> 2, g = c & 3;
        const bool mine = (o >> 2) == hh;
        const uint32_t w2 = mine ? xb[nb][g][(o & 3) >> 1] : pb[nb][g][(o & 3) >> 1];
        return (o & 1) ? bf16_hi(w2) : bf16_lo(w2);
      };
      // Mean of squares in the prologue's order: per 8-lane slot j an fma
      // chain over its chunks (a then b), then ((s0+s7)+(s2+s5)) +
      // ((s1+s6)+(s3+s4)).
      float sj[8];
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const bool pl = j < hl;
        const int ca = pl ? j : 2 * hl + 2 * (j - hl);
        const int cbk = pl ? j + hl : ca + 1;
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const float v = chan(8 * ca + i);
          s = fmaf(v, v, s);
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const float v = chan(8 * cbk + i);
          s = fmaf(v, v, s);
        }
        sj[j] = s;
      }
      const float tot = ((sj[0] + sj[7]) + (sj[2] + sj[5])) + ((sj[1] + sj[6]) + (sj[3] + sj[4]));
      const float r = rsqrt_rounded(tot * (1.0f / kHD) + a.eps);
      // Normalised values of this lane's channels, then the rotation pairs
      // (p, p + half), both in this lane.
      float y[4][4][4];
#pragma unroll
      for (int nb = 0; nb < 4; nb++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int ch0 = 32 * nb + 8 * g + 4 * hh;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const uint32_t w2 = xb[nb][g][e >> 1];
            const float xv = (e & 1) ? bf16_hi(w2) : bf16_lo(w2);
            const uint16_t gb = gamma[ch0 + e];
            y[nb][g][e] = (xv * r) * __uint_as_float((uint32_t)gb << 16);
          }
        }
      float o[4][4][4];
#pragma unroll
      for (int nb = 0; nb < 4; nb++)
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
          for (int e = 0; e < 4; e++) o[nb][g][e] = y[nb][g][e];
      const int32_t mv = valid ? m : 0;
#pragma unroll
      for (int nb = 0; nb < 4; nb++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int c = 4 * nb + g;          // chunk of channels 8c .. 8c+7
          if (c < hl) {
            // Pair chunk: partner chunk c + hl holds channel p + half.
            const int c2 = c + hl, nb2 = c2 >> 2, g2 = c2 & 3;
#pragma unroll
            for (int e = 0; e < 4; e++) {
              const int p = 8 * c + 4 * hh + e;
              const int axis = min(max(a.pair_axis[p], 0), 2);
              const RopeEntry te = valid ? make_rope_entry<kMode>(a.pos[(int64_t)mv * 3 + axis] * a.pair_inv[p])
                                         : RopeEntry{1.f, 0.f};
              rope_pair<kMode>(y[nb][g][e], y[nb2][g2][e], te, true, o[nb][g][e], o[nb2][g2][e]);
            }
          } else if (c >= 2 * hl) {
            // Pass-through channels >= rot (bf16-rounded as in the prologue).
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
              float pa, pb2;
              rope_pair<kMode>(y[nb][g][e], y[nb][g][e + 1], RopeEntry{1.f, 0.f}, false, pa, pb2);
              o[nb][g][e] = pa;
              o[nb][g][e + 1] = pb2;
            }
          }
        }
#pragma unroll
      for (int nb = 0; nb < 4; nb++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          ob[nb][g][0] = valid ? cvt_pk(o[nb][g][0], o[nb][g][1]) : 0u;
          ob[nb][g][1] = valid ? cvt_pk(o[nb][g][2], o[nb][g][3]) : 0u;
        }
    }
    uint16_t* row = out + ((int64_t)head * a.seq_pad + m) * kHD;
#pragma unroll
    for (int nb = 0; nb < 4; nb++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const u32x2 v2 = {ob[nb][g][0], ob[nb][g][1]};
        *reinterpret_cast<u32x2*>(row + 32 * nb + 8 * g + 4 * hh) = v2;
      }
  }
}

}  // namespace h3hip

using namespace h3hip;

extern "C" int h3hip_qkv_proj(const void* x, int64_t ldx, const void* w, int64_t ldw,
                              int32_t hidden, const void* q_gamma, const void* k_gamma,
                              float eps, const float* pos, const int32_t* pair_axis,
                              const float* pair_inv_freq, int32_t rot, int32_t rounding,
                              int32_t seq_len, int32_t seq_pad, int32_t heads, int32_t head_dim,
                              void* q_out, void* k_out, void* v_out, void* stream) {
  if (head_dim != kHD || (rot != 96 && rot != 128) || heads % 2 != 0 || hidden % kPK != 0) {
    set_error("declined: head_dim %d / rot %d / heads %d / hidden %d (needs head_dim 128, rot 96 "
              "or 128, an even head count, hidden a multiple of 64)",
              head_dim, rot, heads, hidden);
    return H3HIP_DECLINED;
  }
  const bool plain = q_gamma == nullptr && k_gamma == nullptr;
  H3_REQUIRE(x && w && q_out && k_out && v_out, H3HIP_EINVAL, "NULL tensor argument");
  H3_REQUIRE(plain || (q_gamma && k_gamma && pos && pair_axis && pair_inv_freq), H3HIP_EINVAL,
             "the norm/RoPE tables must all be given (or both gammas NULL for the plain GEMM)");
  H3_REQUIRE(seq_len > 0 && heads > 0 && seq_pad >= seq_len && seq_pad % 128 == 0, H3HIP_EINVAL,
             "bad shape: seq_len %d seq_pad %d heads %d", seq_len, seq_pad, heads);
  H3_REQUIRE(ldx >= hidden && ldx % 8 == 0 && ldw >= hidden && ldw % 8 == 0, H3HIP_EINVAL,
             "ldx %lld / ldw %lld must be >= hidden and multiples of 8", (long long)ldx,
             (long long)ldw);
  // 32-bit buffer offsets over x (up to the last row of the last token tile)
  // and W.
  const int tiles_m = (seq_pad + kPM - 1) / kPM;
  H3_REQUIRE((int64_t)tiles_m * kPM * ldx * 2 < ((int64_t)1 << 31) &&
                 (int64_t)3 * heads * kHD * ldw * 2 < ((int64_t)1 << 31),
             H3HIP_EINVAL, "x or W exceeds 2 GiB (32-bit buffer offsets)");
  H3_REQUIRE(rounding == H3HIP_ROUND_REFERENCE || rounding == H3HIP_ROUND_FP32, H3HIP_EINVAL,
             "unknown rounding mode %d", rounding);
  auto aligned16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  H3_REQUIRE(aligned16(x) && aligned16(w) && aligned16(q_out) && aligned16(k_out) &&
                 aligned16(v_out),
             H3HIP_EINVAL, "tensors must be 16-byte aligned");
  ProjArgs a{static_cast<const uint16_t*>(x),  static_cast<const uint16_t*>(w),
             static_cast<const uint16_t*>(q_gamma), static_cast<const uint16_t*>(k_gamma),
             pos,  pair_axis,  pair_inv_freq,
             static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_out),
             static_cast<uint16_t*>(v_out), ldx, ldw, eps, hidden, rot, seq_len, seq_pad, heads,
             tiles_m};
  const dim3 grid(tiles_m * (3 * heads * kHD / kPN));
  hipStream_t st = as_stream(stream);
  if (plain)
    qkv_proj_kernel<H3HIP_ROUND_REFERENCE, 8, true><<<grid, kPThreads, 0, st>>>(a);
  else if (rounding == H3HIP_ROUND_REFERENCE && rot == 128)
    qkv_proj_kernel<H3HIP_ROUND_REFERENCE, 8, false><<<grid, kPThreads, 0, st>>>(a);
  else if (rounding == H3HIP_ROUND_REFERENCE)
    qkv_proj_kernel<H3HIP_ROUND_REFERENCE, 6, false><<<grid, kPThreads, 0, st>>>(a);
  else if (rot == 128)
    qkv_proj_kernel<H3HIP_ROUND_FP32, 8, false><<<grid, kPThreads, 0, st>>>(a);
  else
    qkv_proj_kernel<H3HIP_ROUND_FP32, 6, false><<<grid, kPThreads, 0, st>>>(a);
  return check_launch("qkv_proj_kernel");
}
