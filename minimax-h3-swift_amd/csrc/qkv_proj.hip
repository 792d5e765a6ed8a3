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
// 8 waves, two per SIMD. Wave w owns head (w >> 2) of the tile and tokens
// 64 (w & 3) .. +63: 4 x 2 accumulators of 32 x 32. The reduction runs in steps
// of 64: the W and x tiles of a step (256 rows of 128 bytes each, 16-byte
// chunks XOR-swizzled so operand reads are conflict-free) are double-buffered
// in LDS and filled by HBM -> LDS buffer loads two steps ahead. One barrier per
// step, placed before the step's last sub-step, whose operands are already in
// registers; the loads of step t + 2 follow it, issued by one wave per SIMD
// (16 x 1 KiB each), so the other wave of the SIMD never waits on a load issue.
// The instruction order inside a sub-step is pinned with sched_barrier.
//
// Epilogue (Q and K): the fp32 accumulators are rounded to bf16 (the bf16
// matmul output the reference normalises), the mean of squares is summed in
// exactly the order the prologue kernel uses (the two half-waves each run half
// of the fixed-order chains, exchanged with permlane32_swap), the rotation
// takes its (c, s) from the render's rotation table -- the reference's
// ropeTable, built once per render by h3hip_rope_table with the prologue's own
// entry function -- and norm and rotation use the prologue's arithmetic
// (norm_rope.h). The output equals h3hip_qk_norm_rope applied to this kernel's
// bf16 GEMM result, bit for bit.
#include <type_traits>

#include "common.h"
#include "norm_rope.h"

namespace h3hip {

struct ProjArgs {
  const uint16_t* __restrict__ x;        // [seq_len, hidden], row stride ldx
  const uint16_t* __restrict__ w;        // [3 * heads * 128, hidden], row stride ldw
  const uint16_t* __restrict__ q_gamma;  // [128]
  const uint16_t* __restrict__ k_gamma;
  const void* __restrict__ table;        // [seq_len, rot/2, 2, 2]: bf16 (REFERENCE) or fp32
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
constexpr int kPWaves = 8;                // per workgroup: 2 per head x kPWaves/2 token slices
constexpr int kPThreads = 64 * kPWaves;
constexpr int kTokWave = 2 * kPM / kPWaves;   // tokens per wave
constexpr int kMB = kTokWave / 32;            // 32-token accumulator blocks per wave
constexpr int kRowsWave = kPM / kPWaves;      // rows of each operand tile a wave loads
constexpr int kLoadsTile = kRowsWave / 8;     // 1 KiB loads per operand tile per wave
constexpr int kGroupM = 4;                // token tiles per launch-order group
constexpr int kXcds = 8;
constexpr int kTileElems = kPM * kPK;     // one operand tile (W or x) of a step
constexpr int kStageElems = 2 * kTileElems;
// s_waitcnt immediate for vmcnt(0), expcnt and lgkmcnt unconstrained (gfx9).
constexpr int kPWaitVmcnt0 = 0x0F70;
// vmcnt(n), lgkmcnt and expcnt unconstrained (vmcnt bits 3:0 and 15:14).
constexpr int wait_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }
constexpr int kPWaitAll = 0x0070;         // vmcnt(0) lgkmcnt(0)
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
  const int nh = wave / (kPWaves / 2), mq = wave % (kPWaves / 2);
  const int li = lane & 31, hh = lane >> 5;
  // Tile order. Workgroup b runs on XCD b % 8 (round-robin dispatch) and
  // XCD x takes the tiles [x q + min(x, r), ...) of a grouped order (total =
  // 8 q + r), so the workgroups one XCD runs at once cover a compact block
  // of kGroupM token tiles x a few channel tiles and share their x and W
  // slices in that XCD's L2.
  const int inner = a.heads * kHD;
  const int tiles_n = 3 * inner / kPN;
  const int total = a.tiles_m * tiles_n;
  const int xcd = blockIdx.x % kXcds, slot = blockIdx.x / kXcds;
  const int tile = xcd * (total / kXcds) + min(xcd, total % kXcds) + slot;
  const int group = tile / (kGroupM * tiles_n);
  const int first_m = group * kGroupM;
  const int gm = min(a.tiles_m - first_m, kGroupM);
  const int local = tile - group * kGroupM * tiles_n;
  const int tm = first_m + local % gm, tn = local / gm;
  const int m0 = tm * kPM, n0 = tn * kPN;
  const int part = n0 / inner;                        // uniform over the tile
  const int head = (n0 - part * inner) / kHD + nh;    // this wave's head

  // Operand offsets within a tile (elements): A = W row nh*128 + 32nb + li,
  // B = x row 64mq + 32mb + li; chunk 2s + hh of the step's 64 columns.
  int a_row[4], b_row[kMB];
#pragma unroll
  for (int nb = 0; nb < 4; nb++) a_row[nb] = nh * 128 + 32 * nb + li;
#pragma unroll
  for (int mb = 0; mb < kMB; mb++) b_row[mb] = kTokWave * mq + 32 * mb + li;
  auto operand = [&](const uint16_t* tile, int row, int s) __attribute__((always_inline)) {
    return *reinterpret_cast<const bf16x8*>(tile + row * kPK + (((2 * s + hh) ^ p_swz(row)) * 8));
  };

  // HBM -> LDS: wave w moves rows 32w .. 32w+31 of the W tile and of the x
  // tile, 8 rows per instruction (lane l: row 32w + 8i + l/8, chunk position
  // l%8 filled from the global chunk the swizzle places there).
  const i32x4p w_rsrc = proj_rsrc(a.w, (uint32_t)(3 * inner) * (uint32_t)a.ldw * 2u);
  const i32x4p x_rsrc = proj_rsrc(a.x, (uint32_t)((a.seq_len - 1) * a.ldx + a.hidden) * 2u);
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane(proj_lds_address(lds));
  const int lw = wave & 3;   // loading wave: rows of waves lw and lw + 4
  int w_voff[2 * kLoadsTile], x_voff[2 * kLoadsTile];
#pragma unroll
  for (int i = 0; i < 2 * kLoadsTile; i++) {
    const int r = kRowsWave * (lw + 4 * (i >> 2)) + (lane >> 3) + 8 * (i & 3);
    const int src_chunk = (lane & 7) ^ p_swz(r);
    w_voff[i] = (n0 + r) * (int)a.ldw * 2 + src_chunk * 16;
    x_voff[i] = (m0 + r) * (int)a.ldx * 2 + src_chunk * 16;   // rows >= seq_len: out of range, read as 0
  }
  // Load i of step t (i < kLoadsTile: W rows, then x rows) into stage st.
  auto dma = [&](int t, int st, int i) __attribute__((always_inline)) {
    const bool is_x = i >= 2 * kLoadsTile;
    const int ii = is_x ? i - 2 * kLoadsTile : i;
    const uint32_t dst = lds_base + 2 * (st * kStageElems + (is_x ? kTileElems : 0) +
                                         (kRowsWave * (lw + 4 * (ii >> 2)) + 8 * (ii & 3)) * kPK);
    proj_dma16(is_x ? x_rsrc : w_rsrc, dst, is_x ? x_voff[ii] : w_voff[ii], t * kPK * 2);
  };

  f32x16 acc[4][kMB];
#pragma unroll
  for (int nb = 0; nb < 4; nb++)
#pragma unroll
    for (int mb = 0; mb < kMB; mb++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[nb][mb][r] = 0.f;

  // Stage st of the LDS ring holds step t with st = t & 1. Steps 0 and 1 are
  // loaded up front; the loads of step t + 2 are issued right after the
  // barrier inside step t, once every wave has read its last operands of
  // stage t & 1, and are drained at the barrier inside step t + 1.
  const int steps = a.hidden / kPK;
  if (wave < 4) {
#pragma unroll
    for (int i = 0; i < 4 * kLoadsTile; i++) dma(0, 0, i);
    if (steps > 1) {
#pragma unroll
      for (int i = 0; i < 4 * kLoadsTile; i++) dma(1, 1, i);
      __builtin_amdgcn_s_waitcnt(wait_vmcnt(4 * kLoadsTile));
    } else {
      __builtin_amdgcn_s_waitcnt(kPWaitVmcnt0);
    }
  }
  __syncthreads();

  bf16x8 A[2][4], B[2][kMB];
  auto read_ops = [&](int buf, const uint16_t* stage, int sub) __attribute__((always_inline)) {
#pragma unroll
    for (int nb = 0; nb < 4; nb++) A[buf][nb] = operand(stage, a_row[nb], sub);
#pragma unroll
    for (int mb = 0; mb < kMB; mb++) B[buf][mb] = operand(stage + kTileElems, b_row[mb], sub);
  };
  // Operand i of sub-step sub (i < 4: A block i, else B block i - 4).
  auto read_op = [&](int buf, const uint16_t* stage, int sub, int i) __attribute__((always_inline)) {
    if (i < 4)
      A[buf][i] = operand(stage, a_row[i], sub);
    else
      B[buf][i - 4] = operand(stage + kTileElems, b_row[i - 4], sub);
  };
  auto mfma = [&](int cur, int k) __attribute__((always_inline)) {
    const int nb = k / kMB, mb = k % kMB;
    acc[nb][mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[cur][nb], B[cur][mb], acc[nb][mb],
                                                          0, 0, 0);
  };
  constexpr int kMfmaSub = 4 * kMB;   // MFMAs per 16-deep sub-step
  constexpr int kOps = 4 + kMB;       // operand reads per sub-step
  static_assert(kMfmaSub >= 2 * kLoadsTile, "one load per MFMA of the last sub-step");
  static_assert(kMfmaSub >= kOps + 2, "reads interleave with MFMAs");
  read_ops(0, lds, 0);

  for (int t = 0; t < steps; t++) {
    const uint16_t* cur_stage = lds + (t & 1) * kStageElems;
    // Sub-steps 0..2: multiply sub-step s, one operand read of sub-step
    // s + 1 after each of its first MFMAs (the schedule is pinned: left to
    // itself the compiler moves the reads to the end of the sub-step).
#pragma unroll
    for (int s = 0; s < 3; s++) {
#pragma unroll
      for (int k = 0; k < kMfmaSub; k++) {
        mfma(s & 1, k);
        if (k < kOps) read_op((s & 1) ^ 1, cur_stage, s + 1, k);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    // This wave has read stage t & 1 and its loads of step t + 1 have landed;
    // after the barrier the same holds for every wave.
    __builtin_amdgcn_s_waitcnt(kPWaitAll);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    // Sub-step 3 (operands already in registers), one load of step t + 2 into
    // the stage just freed after each MFMA, and halfway the sub-step 0
    // operands of step t + 1. Past the last step the loads repeat the last
    // step and the reads pick up the other stage: in bounds, never used.
    const int t_load = min(t + 2, steps - 1);
#pragma unroll
    for (int k = 0; k < kMfmaSub; k++) {
      mfma(1, k);
      if (wave < 4) {
        dma(t_load, t & 1, 2 * k);
        dma(t_load, t & 1, 2 * k + 1);
      }
      if (k >= 2 && k < 2 + kOps) read_op(0, lds + ((t + 1) & 1) * kStageElems, 0, k - 2);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __builtin_amdgcn_s_waitcnt(kPWaitVmcnt0);
  // Every wave is past its last LDS read and its loads have landed: the ring
  // is free for the output transpose.
  __syncthreads();

  // ---- epilogue: lane (li, hh) holds token m0 + 64mq + 32mb + li, channels
  // 32nb + 8g + 4hh + e of the head in register 4g + e of acc[nb][mb], i.e.
  // half (hh) of each 8-channel chunk c = 4nb + g.
  uint16_t* out = part == 0 ? a.q_out : part == 1 ? a.k_out : a.v_out;
  const bool norm = !kPlain && part < 2;
  const uint16_t* gamma = part == 0 ? a.q_gamma : a.k_gamma;
  constexpr int hl = kHl;
  constexpr int half = 8 * kHl;            // rot / 2
  // Output transpose: the wave's 32 x 128 block goes through its own 8 KiB of
  // LDS, written as 8-byte slots (2c + hh) ^ li of row li (conflict-free), and
  // read back 16 bytes per lane as whole rows, so each global store writes
  // 1 KiB contiguous (4 rows of the head-major output) instead of 16-byte
  // pieces of 32 rows.
  uint16_t* blk = lds + wave * (32 * kHD);
  auto put = [&](int c, uint32_t w0, uint32_t w1) __attribute__((always_inline)) {
    const u32x2 v2 = {w0, w1};
    *reinterpret_cast<u32x2*>(blk + li * kHD + (((2 * c + hh) ^ li) * 4)) = v2;
  };
#pragma unroll
  for (int mb = 0; mb < kMB; mb++) {
    const int mrow0 = m0 + kTokWave * mq + 32 * mb;   // first row of the block (wave-uniform)
    if (mrow0 >= a.seq_pad) continue;
    const int m = mrow0 + li;
    const bool valid = m < a.seq_len;
    // bf16 GEMM result of this lane's half-chunks, packed: xb[c][0..1].
    uint32_t xb[16][2];
#pragma unroll
    for (int c = 0; c < 16; c++) {
      xb[c][0] = cvt_pk(acc[c >> 2][mb][4 * (c & 3)], acc[c >> 2][mb][4 * (c & 3) + 1]);
      xb[c][1] = cvt_pk(acc[c >> 2][mb][4 * (c & 3) + 2], acc[c >> 2][mb][4 * (c & 3) + 3]);
    }
    if (!norm) {
#pragma unroll
      for (int c = 0; c < 16; c++) put(c, valid ? xb[c][0] : 0u, valid ? xb[c][1] : 0u);
    } else {
      // Mean of squares in the prologue's order: per slot j an fma chain over
      // chunk a then chunk b, channel order within a chunk, then ((s0+s7)+(s2+s5))
      // + ((s1+s6)+(s3+s4)). The lower half-wave runs slots 0..3, the upper
      // slots 4..7: permlane32_swap(x, y) leaves the lower half-wave's word of x
      // in [0] and the lower half-wave's word of y in [0]'s upper lanes, the
      // upper half-wave's words in [1], so with x = chunk c of slot j and y =
      // chunk c' of slot j + 4 every lane gets channels 0..3 of its chunk in
      // [0] and 4..7 in [1] -- one swap per word for both half-waves.
      auto pair_sq = [&](int c, int c2, float acc_s) __attribute__((always_inline)) {
        const auto w0 = __builtin_amdgcn_permlane32_swap(xb[c][0], xb[c2][0], false, false);
        const auto w1 = __builtin_amdgcn_permlane32_swap(xb[c][1], xb[c2][1], false, false);
        const uint32_t wd[4] = {w0[0], w1[0], w0[1], w1[1]};
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const float v0 = bf16_lo(wd[q]), v1 = bf16_hi(wd[q]);
          acc_s = fmaf(v0, v0, acc_s);
          acc_s = fmaf(v1, v1, acc_s);
        }
        return acc_s;
      };
      auto slot_a = [&](int j) { return j < hl ? j : 2 * hl + 2 * (j - hl); };
      auto slot_b = [&](int j) { return j < hl ? j + hl : 2 * hl + 2 * (j - hl) + 1; };
      float sj[8];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        // This lane's slot: j (lower half-wave) or j + 4 (upper).
        const float mine =
            pair_sq(slot_b(j), slot_b(j + 4), pair_sq(slot_a(j), slot_a(j + 4), 0.f));
        const auto both = __builtin_amdgcn_permlane32_swap(__float_as_uint(mine),
                                                           __float_as_uint(mine), false, false);
        sj[j] = __uint_as_float(both[0]);
        sj[j + 4] = __uint_as_float(both[1]);
      }
      const float tot = ((sj[0] + sj[7]) + (sj[2] + sj[5])) + ((sj[1] + sj[6]) + (sj[3] + sj[4]));
      const float r = rsqrt_rounded(tot * (1.0f / kHD) + a.eps);
      // Normalised values of this lane's half-chunk c: (x r) gamma.
      auto norm4 = [&](int c, float y[4]) __attribute__((always_inline)) {
        const u32x2 g2 = *reinterpret_cast<const u32x2*>(gamma + 8 * c + 4 * hh);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const uint32_t xw = xb[c][e >> 1], gw = g2[e >> 1];
          const float xv = (e & 1) ? bf16_hi(xw) : bf16_lo(xw);
          const float gv = (e & 1) ? bf16_hi(gw) : bf16_lo(gw);
          y[e] = (xv * r) * gv;
        }
      };
      auto store4 = [&](int c, const float o[4]) __attribute__((always_inline)) {
        put(c, valid ? cvt_pk(o[0], o[1]) : 0u, valid ? cvt_pk(o[2], o[3]) : 0u);
      };
      // Table row of this token (row 0 for padding rows, whose output is zero).
      const int64_t trow = (int64_t)(valid ? m : 0) * half;
#pragma unroll
      for (int c = 0; c < hl; c++) {
        // Pairs p = 8c + 4hh + e rotate channels p (chunk c) and p + rot/2
        // (chunk c + hl), both in this lane.
        RopeEntry te[4];
        if (kMode == H3HIP_ROUND_REFERENCE) {
          const u32x4* tp = reinterpret_cast<const u32x4*>(
              static_cast<const uint16_t*>(a.table) + (trow + 8 * c + 4 * hh) * 4);
          const u32x4 t01 = tp[0], t23 = tp[1];   // (c, -s, s, c) bf16 of pairs e
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const u32x4& tv = e < 2 ? t01 : t23;
            const int o = 2 * (e & 1);
            te[e] = RopeEntry{bf16_lo(tv[o]), bf16_lo(tv[o + 1])};
          }
        } else {
          const f32x4* tp = reinterpret_cast<const f32x4*>(a.table) + trow + 8 * c + 4 * hh;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const f32x4 tv = tp[e];
            te[e] = RopeEntry{tv[0], tv[2]};
          }
        }
        float ya[4], yb[4], oa[4], ob[4];
        norm4(c, ya);
        norm4(c + hl, yb);
#pragma unroll
        for (int e = 0; e < 4; e++) rope_pair<kMode>(ya[e], yb[e], te[e], true, oa[e], ob[e]);
        store4(c, oa);
        store4(c + hl, ob);
      }
      // Channels >= rot pass through (bf16-rounded as in the prologue).
#pragma unroll
      for (int c = 2 * hl; c < 16; c++) {
        float y[4], o[4];
        norm4(c, y);
        rope_pair<kMode>(y[0], y[1], RopeEntry{1.f, 0.f}, false, o[0], o[1]);
        rope_pair<kMode>(y[2], y[3], RopeEntry{1.f, 0.f}, false, o[2], o[3]);
        store4(c, o);
      }
    }
    // Row r = 4i + lane / 16, chunk k = lane % 16: slots 2k, 2k + 1 sit at
    // (2k ^ r) and (2k + 1) ^ r, i.e. the 16-byte word at 2k ^ (r & 30) with
    // its halves swapped when r is odd.
    uint16_t* dst = out + ((int64_t)head * a.seq_pad + mrow0) * kHD;
    const int k = lane & 15;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int r = 4 * i + (lane >> 4);
      u32x4 v = *reinterpret_cast<const u32x4*>(blk + r * kHD + ((2 * k) ^ (r & 30)) * 4);
      if (r & 1) v = u32x4{v[2], v[3], v[0], v[1]};
      if (mrow0 + r < a.seq_pad) *reinterpret_cast<u32x4*>(dst + r * kHD + 8 * k) = v;
    }
  }
}

}  // namespace h3hip

using namespace h3hip;

extern "C" int h3hip_qkv_proj(const void* x, int64_t ldx, const void* w, int64_t ldw,
                              int32_t hidden, const void* q_gamma, const void* k_gamma,
                              float eps, const void* rope_table, int32_t rot, int32_t rounding,
                              int32_t seq_len, int32_t seq_pad, int32_t heads, int32_t head_dim,
                              void* q_out, void* k_out, void* v_out, void* stream) {
  // hidden <= 0 is an invalid shape, not an unsupported one (0 and negative
  // multiples of 64 would pass the decline test below, and a negative hidden
  // wraps the x buffer's byte range).
  H3_REQUIRE(hidden > 0, H3HIP_EINVAL, "hidden must be positive (got %d)", hidden);
  if (head_dim != kHD || (rot != 96 && rot != 128) || heads % 2 != 0 || hidden % kPK != 0) {
    set_error("declined: head_dim %d / rot %d / heads %d / hidden %d (needs head_dim 128, rot 96 "
              "or 128, an even head count, hidden a multiple of 64)",
              head_dim, rot, heads, hidden);
    return H3HIP_DECLINED;
  }
  const bool plain = q_gamma == nullptr && k_gamma == nullptr;
  H3_REQUIRE(x && w && q_out && k_out && v_out, H3HIP_EINVAL, "NULL tensor argument");
  H3_REQUIRE(plain || (q_gamma && k_gamma && rope_table), H3HIP_EINVAL,
             "gammas and the rotation table must all be given (or both gammas NULL for the "
             "plain GEMM)");
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
                 aligned16(v_out) && (plain || (aligned16(rope_table) && aligned16(q_gamma) &&
                                                aligned16(k_gamma))),
             H3HIP_EINVAL, "tensors must be 16-byte aligned");
  ProjArgs a{static_cast<const uint16_t*>(x),  static_cast<const uint16_t*>(w),
             static_cast<const uint16_t*>(q_gamma), static_cast<const uint16_t*>(k_gamma),
             rope_table,
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
