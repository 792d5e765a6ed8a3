// Fused QKV projection: the GEMM of AttentionLayer.callAsFunction
// (Sources/H3Modules/DiTBlock.swift:336-338, `matmul(x, qkvWeight.T)` split
// into Q | K | V of heads x 128 channels each) with the Q/K prologue -- per-head
// H3RMSNorm and SplitHalfRoPE (DiTBlock.swift:346-352) -- and the head-major
// relayout done in its epilogue. Q, K and V come out head-major
// [heads, seq_pad, 128], the layout the attention reads, without the token-major
// qkv ever being written and read back.
//
// GEMM: C^T[n, m] = sum_k W[n, k] x[m, k] with v_mfma_f32_16x16x32_bf16, the W
// rows as the A operand and the x rows as B. At random bf16 operands the chip
// runs this GEMM at its power limit, and the 16 x 16 x 32 form does about 11%
// more FLOPs per joule than the 32 x 32 x 16 form (sustained-MFMA measurement
// on MI355X: 2.00 against 1.80 PFLOP/s; equal at zero operands).
//
// Workgroup: 256 tokens x 256 output channels (two heads of one of Q, K, V),
// 8 waves, two per SIMD. Wave w owns head (w >> 2) of the tile and tokens
// 64 (w & 3) .. +63: 8 x 4 accumulators of 16 x 16. The reduction runs in steps
// of 64: the W and x tiles of a step (256 rows of 128 bytes each, 16-byte
// chunks XOR-swizzled so operand reads are conflict-free) are double-buffered
// in LDS and filled by HBM -> LDS buffer loads two steps ahead. A step is two
// 32-deep sub-steps of 32 MFMAs; the operands of the next sub-step are read
// while the current one multiplies (x operands double-buffered, each W operand
// re-read into its register right after its last MFMA). One barrier per step,
// before the second sub-step, whose operands are then in registers; the loads
// of step t + 2 follow it, issued by one wave per SIMD (16 x 1 KiB each), so
// the other wave of the SIMD never waits on a load issue. The instruction
// order is pinned with sched_barrier.
//
// Epilogue: the fp32 accumulators are rounded to bf16 (the bf16 matmul output
// the reference normalises) and written as token rows to the wave's own 8 KiB
// of LDS. Each row is then read back in the prologue kernel's 8-lane row layout
// and, for Q and K, normalised and rotated by the same device code the
// prologue runs (norm_rope.h), with (c, s) from the render's rotation table --
// the reference's ropeTable, built once per render by h3hip_rope_table with
// the prologue's own entry function. The output therefore equals
// h3hip_qk_norm_rope applied to this kernel's bf16 GEMM result, bit for bit.
// Rows are stored whole: 8 consecutive head-major rows (2 KiB) per pass.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "norm_rope.h"
#include "tile_order.h"

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
  // Out-projection mode: n_out output channels, written token-major into
  // q_out with row stride ldo.
  int32_t n_out;
  int64_t ldo;
};

constexpr int kPM = 256;                  // tokens per workgroup
constexpr int kPN = 256;                  // output channels per workgroup
constexpr int kPK = 64;                   // reduction per step
constexpr int kHD = 128;                  // head_dim
constexpr int kPWaves = 8;                // per workgroup: 2 per head x kPWaves/2 token slices
constexpr int kPThreads = 64 * kPWaves;
constexpr int kTokWave = 2 * kPM / kPWaves;   // tokens per wave
constexpr int kMB = kTokWave / 16;            // 16-token accumulator blocks per wave
constexpr int kNB = kHD / 16;                 // 16-channel accumulator blocks per wave
constexpr int kRowsWave = kPM / kPWaves;      // rows of each operand tile a wave loads
constexpr int kLoadsTile = kRowsWave / 8;     // 1 KiB loads per operand tile per wave
constexpr int kLoadsStep = 4 * kLoadsTile;    // loads per step of a loading wave
constexpr int kXcds = kOrderXcds;
constexpr int kTileElems = kPM * kPK;     // one operand tile (W or x) of a step
constexpr int kStageElems = 2 * kTileElems;
constexpr int kMfmaSub = kNB * kMB;       // MFMAs per 32-deep sub-step
// s_waitcnt immediate for vmcnt(0), expcnt and lgkmcnt unconstrained (gfx9).
constexpr int kPWaitVmcnt0 = 0x0F70;
// vmcnt(n), lgkmcnt and expcnt unconstrained (vmcnt bits 3:0 and 15:14).
constexpr int wait_vmcnt(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0F70; }
constexpr int kPWaitAll = 0x0070;         // vmcnt(0) lgkmcnt(0)
constexpr int kPBufferWord3 = 0x00020000;
static_assert(kMfmaSub == 2 * kLoadsStep, "one load per two MFMAs of the second sub-step");

typedef int i32x4p __attribute__((ext_vector_type(4)));

// 16-byte chunk c of the 128-byte operand row r sits at c ^ ((r >> 1) & 7):
// the 16 rows of a 16-lane read phase cover both row parities x 8 chunk
// positions. Rows 16 apart share the swizzle.
__device__ __forceinline__ int p_swz(int r) { return (r >> 1) & 7; }

// 16-byte chunk c of the 256-byte epilogue row r sits at c ^ e_swz(r): the
// 16 rows one accumulator write covers hit 16 distinct positions (every 8-byte
// slot of a bank window once per 32 lanes), and rows r, r ^ 1 map the chunks
// 0..7 onto complementary halves, so the 2 rows x 8 lanes of a 16-lane read
// phase are conflict-free.
__device__ __forceinline__ int e_swz(int r) { return ((r & 1) << 3) | ((r >> 1) & 7); }

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
// GEMM result of every part unchanged (the materialised qkv, for tests);
// kOut: the out-projection, a plain GEMM of n_out channels written
// token-major [seq_len, n_out] (row stride ldo) instead of head-major parts.
template <int kMode, int kHl, bool kPlain, bool kOut = false>
__global__ __launch_bounds__(kPThreads, 1) void qkv_proj_kernel(ProjArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * kStageElems];   // 128 KiB

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nh = wave / (kPWaves / 2), mq = wave % (kPWaves / 2);
  // v_mfma_f32_16x16x32_bf16 layout: lane (g = lane/16, lr = lane%16) holds
  // row lr of an A block and column lr of a B block at k = 8g .. 8g + 7, and
  // rows 4g .. 4g + 3 of column lr of the 16 x 16 result.
  const int lr = lane & 15, g = lane >> 4;
  // Tile order (TileOrder). Workgroup b runs on XCD b % 8 (round-robin
  // dispatch), as that XCD's (b / 8)-th workgroup; the grid is 8 x the longest
  // XCD list, and a workgroup past its XCD's list has no tile.
  const int inner = a.heads * kHD;
  const int n_total = kOut ? a.n_out : 3 * inner;
  const int tiles_n = n_total / kPN;
  const TileOrder order{a.tiles_m, tiles_n};
  const int xcd = blockIdx.x % kXcds, slot = blockIdx.x / kXcds;
  if (slot >= order.length(xcd)) return;
  const int tile = order.tile(xcd, slot);
  const int m0 = (tile >> 16) * kPM, n0 = (tile & 0xffff) * kPN;
  const int part = kOut ? 0 : n0 / inner;                   // uniform over the tile
  const int head = kOut ? 0 : (n0 - part * inner) / kHD + nh;   // this wave's head

  // Operand offsets within a stage (elements). A block nb = W row
  // nh*128 + 16nb + lr, B block mb = x row 64mq + 16mb + lr; sub-step u reads
  // chunk 4u + g of the step's 8. The block index is an immediate offset.
  const int a_row0 = nh * kHD + lr, b_row0 = kTokWave * mq + lr;
  int a_off[2], b_off[2];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    a_off[u] = a_row0 * kPK + (((4 * u + g) ^ p_swz(a_row0)) * 8);
    b_off[u] = kTileElems + b_row0 * kPK + (((4 * u + g) ^ p_swz(b_row0)) * 8);
  }
  auto operand = [&](const uint16_t* stage, int off, int blk) __attribute__((always_inline)) {
    return *reinterpret_cast<const bf16x8*>(stage + off + blk * 16 * kPK);
  };

  // HBM -> LDS by one wave per SIMD: loading wave lw (waves 0-3) moves rows
  // 32 lw .. 32 lw + 31 and 32 (lw + 4) .. + 31 of the W tile and of the x
  // tile, 8 rows per instruction (lane l: row + 8i + l/8, chunk position l%8
  // filled from the global chunk the swizzle places there).
  const i32x4p w_rsrc = proj_rsrc(a.w, (uint32_t)n_total * (uint32_t)a.ldw * 2u);
  const i32x4p x_rsrc = proj_rsrc(a.x, (uint32_t)((a.seq_len - 1) * a.ldx + a.hidden) * 2u);
  const uint32_t lds_base = __builtin_amdgcn_readfirstlane(proj_lds_address(lds));
  const int lw = wave & 3;   // loading wave: rows of waves lw and lw + 4
  // Load ii of a tile covers row r(ii) = 32 lw + 128 (ii >> 2) + 8 (ii & 3) +
  // lane / 8; rows 16 apart share the chunk swizzle, so the source chunk
  // depends on ii only through ii & 1. x offsets stay whole in the lane offset,
  // which the hardware range-checks (rows >= seq_len read as 0); every W row
  // of the tile exists, so W's row step goes into the scalar offset and two
  // lane offsets serve its eight loads.
  int w_voff[2], x_voff[2 * kLoadsTile];
#pragma unroll
  for (int i = 0; i < 2 * kLoadsTile; i++) {
    const int r = kRowsWave * (lw + 4 * (i >> 2)) + (lane >> 3) + 8 * (i & 3);
    const int src_chunk = (lane & 7) ^ p_swz(r);
    if (i < 2) w_voff[i] = (n0 + r) * (int)a.ldw * 2 + src_chunk * 16;
    x_voff[i] = (m0 + r) * (int)a.ldx * 2 + src_chunk * 16;
  }
  // Load i of step t (i < 2 kLoadsTile: W rows, then x rows) into stage st.
  auto dma = [&](int t, int st, int i) __attribute__((always_inline)) {
    const bool is_x = i >= 2 * kLoadsTile;
    const int ii = is_x ? i - 2 * kLoadsTile : i;
    const uint32_t dst = lds_base + 2 * (st * kStageElems + (is_x ? kTileElems : 0) +
                                         (kRowsWave * (lw + 4 * (ii >> 2)) + 8 * (ii & 3)) * kPK);
    if (is_x)
      proj_dma16(x_rsrc, dst, x_voff[ii], t * kPK * 2);
    else
      proj_dma16(w_rsrc, dst, w_voff[ii & 1],
                 t * kPK * 2 + (8 * (ii & 2) + 4 * kRowsWave * (ii >> 2)) * (int)a.ldw * 2);
  };

  f32x4 acc[kNB][kMB];
#pragma unroll
  for (int nb = 0; nb < kNB; nb++)
#pragma unroll
    for (int mb = 0; mb < kMB; mb++) acc[nb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Stage st of the LDS ring holds step t with st = t & 1. Steps 0 and 1 are
  // loaded up front; the loads of step t + 2 are issued right after the
  // barrier inside step t, once every wave has read its last operands of
  // stage t & 1, and are drained at the barrier inside step t + 1.
  const int steps = a.hidden / kPK;
  if (wave < 4) {
#pragma unroll
    for (int i = 0; i < kLoadsStep; i++) dma(0, 0, i);
    if (steps > 1) {
#pragma unroll
      for (int i = 0; i < kLoadsStep; i++) dma(1, 1, i);
      __builtin_amdgcn_s_waitcnt(wait_vmcnt(kLoadsStep));
    } else {
      __builtin_amdgcn_s_waitcnt(kPWaitVmcnt0);
    }
  }
  __syncthreads();

  // A: the W operands of the current sub-step, each replaced by the next
  // sub-step's right after its last MFMA. B: the x operands, double-buffered
  // (buffer u for sub-step u).
  bf16x8 A[kNB], B[2][kMB];

  // MFMA k of a sub-step: block (nb, mb) = (k / kMB, k % kMB), W-major, so W
  // operand nb is free after MFMA kMB nb + kMB - 1.
  auto mfma = [&](int u, int k) __attribute__((always_inline)) {
    const int nb = k / kMB, mb = k % kMB;
    acc[nb][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[nb], B[u][mb], acc[nb][mb], 0, 0, 0);
  };
  // Reads of sub-step u' (from stage) after MFMA k: x operand k/2 at even k
  // < 2 kMB, W operand nb after the last MFMA of nb.
  auto reads_after = [&](int k, const uint16_t* stage, int u2) __attribute__((always_inline)) {
    if (k < 2 * kMB && (k & 1) == 0) B[u2][k >> 1] = operand(stage, b_off[u2], k >> 1);
    if (k % kMB == kMB - 1) A[k / kMB] = operand(stage, a_off[u2], k / kMB);
  };
  // Step 0's first-sub-step operands, read in the order the loop reads them:
  // the compiler's LDS waits at the loop head then count the same reads on
  // both entry paths. Read in any other order, its merged wait at the loop
  // head is for every read before the first MFMA of each step.
#pragma unroll
  for (int k = 0; k < kMfmaSub; k++) {
    reads_after(k, lds, 0);
    __builtin_amdgcn_sched_barrier(0);
  }

  for (int t = 0; t < steps; t++) {
    const uint16_t* cur_stage = lds + (t & 1) * kStageElems;
    const uint16_t* next_stage = lds + ((t + 1) & 1) * kStageElems;
    // Sub-step 0, reading sub-step 1's operands from the same stage.
#pragma unroll
    for (int k = 0; k < kMfmaSub; k++) {
      mfma(0, k);
      reads_after(k, cur_stage, 1);
      __builtin_amdgcn_sched_barrier(0);
    }
    // This wave has read stage t & 1 and its loads of step t + 1 have landed;
    // after the barrier the same holds for every wave.
    __builtin_amdgcn_s_waitcnt(kPWaitAll);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    // Sub-step 1, one load of step t + 2 into the stage just freed after every
    // second MFMA, and the reads of step t + 1's sub-step 0. Past the last
    // step the loads repeat the last step and the reads pick up the other
    // stage: in bounds, never used.
    const int t_load = min(t + 2, steps - 1);
#pragma unroll
    for (int k = 0; k < kMfmaSub; k++) {
      mfma(1, k);
      if (wave < 4 && (k & 1)) dma(t_load, t & 1, k >> 1);
      reads_after(k, next_stage, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __builtin_amdgcn_s_waitcnt(kPWaitVmcnt0);
  // Every wave is past its last LDS read and its loads have landed: the ring
  // is free for the epilogue rows.
  __syncthreads();

  // ---- epilogue. Accumulator (nb, mb) of lane (g, lr): channels
  // 16nb + 4g .. +3 of token m0 + 64mq + 16mb + lr.
  uint16_t* out = part == 0 ? a.q_out : part == 1 ? a.k_out : a.v_out;
  const bool norm = !kPlain && !kOut && part < 2;
  constexpr bool kFull = kHl == 8;          // rot == 128
  constexpr int kHalf = 8 * kHl;            // rot / 2
  // The prologue's row layout: lane j of 8-lane group rg holds chunks
  // (chunk_a, chunk_b) of row rg, each RoPE pair (p, p + rot/2) in one lane.
  const int j = lane & 7, rg = lane >> 3;
  const bool pair_lane = kFull || j < kHl;
  const int chunk_a = pair_lane ? j : 2 * kHl + 2 * (j - kHl);
  const int chunk_b = pair_lane ? j + kHl : chunk_a + 1;
  float gam[16];
  if (norm) {
    const uint16_t* gsrc = part == 0 ? a.q_gamma : a.k_gamma;
    unpack8(*reinterpret_cast<const u32x4*>(gsrc + 8 * chunk_a), gam);
    unpack8(*reinterpret_cast<const u32x4*>(gsrc + 8 * chunk_b), gam + 8);
  }
  // The wave's 32-row x 128-channel staging block.
  uint16_t* blk = lds + wave * (32 * kHD);
#pragma unroll
  for (int mp = 0; mp < kMB / 2; mp++) {
    const int mrow0 = m0 + kTokWave * mq + 32 * mp;   // first row of the block (wave-uniform)
    if (mrow0 >= a.seq_pad) continue;
    // bf16 GEMM result -> rows: row 16h + lr, 8-byte slot 4nb + g.
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
      for (int nb = 0; nb < kNB; nb++) {
        const f32x4& c = acc[nb][2 * mp + h];
        const int r = 16 * h + lr;
        const u32x2 v2 = {cvt_pk(c[0], c[1]), cvt_pk(c[2], c[3])};
        *reinterpret_cast<u32x2*>(blk + r * kHD + (((4 * nb + g) ^ (2 * e_swz(r))) * 4)) = v2;
      }
    // Rows back in the row layout, 8 rows per pass.
#pragma unroll
    for (int pass = 0; pass < 4; pass++) {
      const int r = 8 * pass + rg, m = mrow0 + r;
      const u32x4 ca = *reinterpret_cast<const u32x4*>(blk + r * kHD + ((chunk_a ^ e_swz(r)) * 8));
      const u32x4 cb = *reinterpret_cast<const u32x4*>(blk + r * kHD + ((chunk_b ^ e_swz(r)) * 8));
      const bool valid = m < a.seq_len;
      u32x4 oa = {0u, 0u, 0u, 0u}, ob = {0u, 0u, 0u, 0u};
      if (valid) {
        if (norm) {
          // This lane's pairs 8j .. 8j + 7 (pair lanes) from token m's table row.
          RopeEntry tab[8];
          if (pair_lane) {
            if (kMode == H3HIP_ROUND_REFERENCE) {
              const u32x4* tp = reinterpret_cast<const u32x4*>(
                  static_cast<const uint16_t*>(a.table) + ((int64_t)m * kHalf + 8 * j) * 4);
#pragma unroll
              for (int q = 0; q < 4; q++) {
                const u32x4 tv = tp[q];   // (c, -s, s, c) bf16 of pairs 2q, 2q + 1
                tab[2 * q] = RopeEntry{bf16_lo(tv[0]), bf16_lo(tv[1])};
                tab[2 * q + 1] = RopeEntry{bf16_lo(tv[2]), bf16_lo(tv[3])};
              }
            } else {
              const f32x4* tp = reinterpret_cast<const f32x4*>(a.table) + (int64_t)m * kHalf + 8 * j;
#pragma unroll
              for (int e = 0; e < 8; e++) {
                const f32x4 tv = tp[e];
                tab[e] = RopeEntry{tv[0], tv[2]};
              }
            }
          } else {
#pragma unroll
            for (int e = 0; e < 8; e++) tab[e] = RopeEntry{1.f, 0.f};
          }
          float xv[16];
          unpack8(ca, xv);
          unpack8(cb, xv + 8);
          norm_rope<kMode, kFull>(xv, gam, pair_lane, tab, a.eps, oa, ob);
        } else {
          oa = ca;
          ob = cb;
        }
      }
      if (kOut) {
        // Token-major: row m's 256 bytes of channels n0 + 128 nh .. + 127.
        if (valid) {
          uint16_t* dst = a.q_out + (int64_t)m * a.ldo + n0 + nh * kHD;
          *reinterpret_cast<u32x4*>(dst + 8 * chunk_a) = oa;
          *reinterpret_cast<u32x4*>(dst + 8 * chunk_b) = ob;
        }
      } else if (m < a.seq_pad) {
        uint16_t* dst = out + ((int64_t)head * a.seq_pad + m) * kHD;
        *reinterpret_cast<u32x4*>(dst + 8 * chunk_a) = oa;
        *reinterpret_cast<u32x4*>(dst + 8 * chunk_b) = ob;
      }
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
             tiles_m, 0, 0};
  // 8 x the longest XCD list of the tile order (a few empty workgroups when
  // the lists differ in length).
  const TileOrder order{tiles_m, 3 * heads * kHD / kPN};
  int longest = 0;
  for (int xcd = 0; xcd < kXcds; xcd++) longest = std::max(longest, order.length(xcd));
  const dim3 grid(kXcds * longest);
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

extern "C" int h3hip_out_proj(const void* x, int64_t ldx, const void* w, int64_t ldw,
                              int32_t in_features, int32_t out_features, int32_t seq_len,
                              void* y, int64_t ldy, void* stream) {
  H3_REQUIRE(in_features > 0 && out_features > 0 && seq_len > 0, H3HIP_EINVAL,
             "bad shape: in_features %d out_features %d seq_len %d", in_features, out_features,
             seq_len);
  if (in_features % kPK != 0 || out_features % kPN != 0) {
    set_error("declined: in_features %d / out_features %d (needs multiples of 64 and 256)",
              in_features, out_features);
    return H3HIP_DECLINED;
  }
  H3_REQUIRE(x && w && y, H3HIP_EINVAL, "NULL tensor argument");
  H3_REQUIRE(ldx >= in_features && ldx % 8 == 0 && ldw >= in_features && ldw % 8 == 0 &&
                 ldy >= out_features && ldy % 8 == 0,
             H3HIP_EINVAL, "ldx %lld / ldw %lld / ldy %lld must cover a row and be multiples of 8",
             (long long)ldx, (long long)ldw, (long long)ldy);
  const int tiles_m = (seq_len + kPM - 1) / kPM;
  H3_REQUIRE((int64_t)tiles_m * kPM * ldx * 2 < ((int64_t)1 << 31) &&
                 (int64_t)out_features * ldw * 2 < ((int64_t)1 << 31),
             H3HIP_EINVAL, "x or W exceeds 2 GiB (32-bit buffer offsets)");
  auto aligned16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  H3_REQUIRE(aligned16(x) && aligned16(w) && aligned16(y), H3HIP_EINVAL,
             "tensors must be 16-byte aligned");
  ProjArgs a{static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w), nullptr, nullptr,
             nullptr, static_cast<uint16_t*>(y), nullptr, nullptr, ldx, ldw, 0.f, in_features,
             128, seq_len, tiles_m * kPM, 1, tiles_m, out_features, ldy};
  const TileOrder order{tiles_m, out_features / kPN};
  int longest = 0;
  for (int xcd = 0; xcd < kXcds; xcd++) longest = std::max(longest, order.length(xcd));
  qkv_proj_kernel<H3HIP_ROUND_REFERENCE, 8, true, true>
      <<<dim3(kXcds * longest), kPThreads, 0, as_stream(stream)>>>(a);
  return check_launch("qkv_proj_kernel (out-projection)");
}
