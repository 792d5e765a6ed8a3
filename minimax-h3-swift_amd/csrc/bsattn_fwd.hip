// Block-sparse flash attention over 128x128 tiles, bf16 MFMA on gfx950.
//
// Persistent workgroups of 8 waves, one per CU, each running the (head,
// 128-query tile) work units that the plan's XCD-aware schedule gives it, one
// after another; the next unit's first K tile and its Q tile load while the
// current one merges and stores its output. Waves w and w+4
// own the same 32 queries (the B operand of v_mfma_f32_32x32x16_bf16, kept in
// registers) and split every key tile in two 64-key halves, each keeping its
// own online-softmax state; the halves are merged exactly at the end. The two
// waves of a pair share a SIMD and run a ping-pong schedule (see the kernel),
// so one's softmax overlaps the other's MFMAs.
//
// Each wave computes transposed scores S^T = K Q^T, so a lane holds one
// query's scores and the row max/sum are in-register reductions plus one
// exchange between half-waves. The exponentiated scores are already the B
// operand of O^T = V^T P^T; the A operand V^T is read from the row-major V
// tile with ds_read_b64_tr_b16, whose 16-lane transpose hands lane i column
// c0+i of four consecutive rows.
//
// The softmax is the online recurrence of AxialReference.attendStreamingKeys
// (Sources/H3Attention/AxialReference.swift:129-171) in fp32 and base 2:
// m starts at -3e38 and l and O are rescaled by 2^(m - m_new) when the
// running max moves. Padding keys (>= seq_len, which the reference's unpadded
// arrays do not have) score -inf, not the reference's finite -1e30 mask
// sentinel: their weight is then exactly 0 whatever m is, and a 64-key half
// made only of padding leaves m where it was. (With a finite sentinel that
// half would raise m to round(-1e30 * c), and 2^(-1e30 * c - m) is 2 to the
// power of the product's rounding residual, which can be +1e21: an infinite
// weight times a zeroed V row is NaN.)
// The rescale is lazy: m is only raised when a tile's max exceeds it by more
// than 2^8, which keeps every exponentiated score <= 256 and changes nothing
// in exact arithmetic (numerator and denominator share m). l sums the bf16-rounded
// weights that O accumulates, so both sides of the quotient see the same
// weights. The output is O / max(l, 1e-30).
#include <cmath>

#include "common.h"
#include "plan.h"

namespace h3hip {

constexpr int kTile = 128;
constexpr int kD = 128;
constexpr int kThreads = 512;
constexpr int kSlot = kTile * kD;                   // one K or V tile, unpadded
constexpr float kRescaleSlack = 8.0f;              // log2 units
// s_waitcnt immediate for vmcnt(0) with expcnt and lgkmcnt left unconstrained
// (gfx9 encoding: vmcnt[3:0] bits 3:0, expcnt bits 6:4, lgkmcnt bits 11:8,
// vmcnt[5:4] bits 15:14).
constexpr int kWaitVmcnt0 = 0x0F70;
// Buffer resource word 3 for raw (untyped, unswizzled) buffer loads on gfx9:
// DATA_FORMAT = 32 bits, everything else zero.
constexpr int kBufferWord3 = 0x00020000;
// Instruction classes for __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;

// Each tensor is a [heads, rows, 128] view: element (h, s, d) at
// base + h*head_stride + s*row_stride + d. Only rows < seq_len of q, k and v
// are read; rows < out_rows of out are written (zero past seq_len).
struct AttnArgs {
  const uint16_t* __restrict__ q;
  const uint16_t* __restrict__ k;
  const uint16_t* __restrict__ v;
  uint16_t* __restrict__ out;
  const int32_t* __restrict__ row_ptr;
  const int32_t* __restrict__ col_idx;
  const int32_t* __restrict__ work_ptr;  // [groups + 1]
  const int32_t* __restrict__ work;
  int64_t q_hs, k_hs, v_hs, o_hs;  // head strides (elements)
  int32_t q_rs, k_rs, v_rs, o_rs;  // row strides (elements)
  int32_t seq_len, out_rows;
  float scale_log2;
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(1))) void global_void;
typedef __attribute__((address_space(3))) void lds_void;

// LDS tiles are unpadded 256-byte rows whose 16-byte chunks are XOR-swizzled
// so the operand reads hit 64 distinct banks per phase:
//   K: chunk c of row r sits at c ^ (r & 15) -- 16 consecutive rows read at
//      one chunk (ds_read_b128) land on 16 different chunk positions;
//   V: chunk c of row r sits at c ^ (4*(r & 3) + ((r >> 2) & 3)) -- the
//      transpose load reads 4 consecutive rows x 4 consecutive chunks per
//      32-lane phase, which this maps onto all 16 chunk positions.
__device__ __forceinline__ int k_swz(int r) { return r & 15; }
__device__ __forceinline__ int v_swz(int r) { return 4 * (r & 3) + ((r >> 2) & 3); }

// Eight bf16 of V^T for the A operand: two transpose loads of 4 rows each.
__device__ __forceinline__ bf16x8 vt_operand(const uint16_t* p0, const uint16_t* p1) {
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p0));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p1));
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x8 w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8, w);
}

// max(x[i], x[i ^ 32]) in every lane, without going through LDS.
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ bf16x8 to_bf16x8(const f32x16& s, int base) {
  typedef float f32x8 __attribute__((ext_vector_type(8)));
  const f32x8 v = {s[base], s[base + 1], s[base + 2], s[base + 3],
                   s[base + 4], s[base + 5], s[base + 6], s[base + 7]};
  return __builtin_convertvector(v, bf16x8);
}

// A unit's first K tile and its Q tile, HBM -> LDS, issued by one half of the
// workgroup (wave w moves rows 32(w&3) .. +31 of each, 4 rows per instruction,
// chunks K-swizzled) into K slot 0 and the Q slot. Buffer resources bound the
// rows at seq_len, so no row past it is fetched; Q rows past seq_len are
// replaced by zeros when they are read.
__device__ __forceinline__ void load_unit_start(const AttnArgs& a, uint16_t* lds, int32_t unit,
                                                int qg, int lane) {
  const int head = unit >> 16, qt = unit & 0xffff;
  const int dma_row = 32 * qg + (lane >> 4);
  auto tile = [&](const uint16_t* base, int rs2, int row0, uint16_t* slot)
      __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)base, 0, (a.seq_len - 1) * rs2 + kD * 2, kBufferWord3);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int row = dma_row + 4 * i;
      const int voff = (row0 + row) * rs2 + (((lane & 15) ^ k_swz(row)) * 16);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsrc, (lds_void*)(slot + (32 * qg + 4 * i) * kD), 16, voff, 0, 0, 0);
    }
  };
  tile(a.q + head * a.q_hs, a.q_rs * 2, qt * kTile, lds + 4 * kSlot);
  const int beg = a.row_ptr[qt];
  if (a.row_ptr[qt + 1] > beg) {
    const int32_t first_col =
        *((const __attribute__((address_space(4))) int32_t*)(a.col_idx) + beg);
    tile(a.k + head * a.k_hs, a.k_rs * 2, first_col * kTile, lds);
  }
}

// Workgroup: 8 waves, one (head, 128-query tile) unit at a time. Wave w owns
// queries 32*(w&3) .. +31 and key half (w>>2) (keys 64*(w>>2) .. +63) of
// every tile.
//
// Ping-pong schedule. Each wave alternates an MFMA phase M_j -- the scores
// S(j) = K(j) Q^T of tile j and the product O += V(j-1)^T P(j-1) of the
// previous tile -- with a VALU phase V_j -- the online softmax of S(j) into
// P(j). Waves 4-7 run one phase behind waves 0-3, and every phase ends in a
// workgroup barrier, so on each SIMD one wave of the pair is issuing MFMAs
// while the other is in its softmax.
//
// Data movement is direct HBM -> LDS (global_load_lds, no registers), issued
// only by the waves in their softmax phase, which drain it before the phase
// barrier: waves 4-7 load K(j+1) in phase 2j, waves 0-3 load V(j) in phase
// 2j+1, and both are consumed from phase 2j+2 on. K(j+1) replaces K(j-1) and
// V(j) replaces V(j-2), both last read before phase 2j. The MFMA waves thus
// never have a load in flight, and their LDS operand reads wait for nothing.
__global__ __launch_bounds__(kThreads, 1) void bsattn_fwd_kernel(AttnArgs a) {
  // Slots: K(j) at (j & 1) * kSlot, V(j) at (2 + (j & 1)) * kSlot, the unit's
  // Q tile at 4 * kSlot; 160 KiB.
  __shared__ __attribute__((aligned(16))) uint16_t lds[5 * kSlot];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform, in an SGPR
  const int qg = wave & 3, half = wave >> 2;
  const float c = a.scale_log2;
  const int k_rs2 = a.k_rs * 2, v_rs2 = a.v_rs * 2;

  // The workgroup's units, one after another (the plan's static schedule).
  // Waves 4-7 load each unit's K(0) and Q while the previous unit merges and
  // stores its output; the first unit's here.
  const int u_beg = a.work_ptr[blockIdx.x], u_end = a.work_ptr[blockIdx.x + 1];
  if (half == 1 && u_beg < u_end) load_unit_start(a, lds, a.work[u_beg], qg, threadIdx.x & 63);
  for (int iu = u_beg; iu < u_end; iu++) {
    // Lane-derived offsets are rebuilt for each unit from an opaque copy of the
    // thread index: hoisted out of the unit loop they would hold registers that
    // the operand pipelines of the inner loops need.
    int tid;
    asm volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"(threadIdx.x));
    const int lane = tid & 63;
    const int li = lane & 31, hh = lane >> 5;
    // K operand offsets: block b row half*64 + 32b + li, chunk 2s + hh.
    int k_off[8];
#pragma unroll
    for (int s = 0; s < 8; s++) k_off[s] = (half * 64 + li) * kD + (((2 * s + hh) ^ k_swz(li)) * 8);
    // V^T operand offsets: lane (g = lane/16, m = lane%16) points at row
    // half*64 + 16kc + 8p + 4(g/2) + m/4, element 32db + 16(g%2) + 4(m%4).
    const int g = lane >> 4, mm = lane & 15;
    int v_off[2][4];
#pragma unroll
    for (int p = 0; p < 2; p++)
#pragma unroll
      for (int db = 0; db < 4; db++) {
        const int row = half * 64 + 8 * p + 4 * (g >> 1) + (mm >> 2);
        const int chunk = 4 * db + 2 * (g & 1) + ((mm & 3) >> 1);
        v_off[p][db] = row * kD + ((chunk ^ v_swz(row)) * 8) + 4 * (mm & 1);
      }
    const int dma_row = 32 * qg + (lane >> 4);

    const int32_t unit = a.work[iu];
    const int head = unit >> 16, qt = unit & 0xffff;
    const int q0 = qt * kTile + qg * 32;

    // The unit's K(0) and Q have landed (the loading waves wait for their own
    // loads), and the previous unit's merge buffers have been read.
    if (half == 1) __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    __syncthreads();

    // Q^T as the B operand, from the Q slot: lane (li, hh) holds
    // Q[q0 + li][16s + 8hh .. +7]; query rows past seq_len are zero.
    bf16x8 qreg[8];
    {
      const bool q_valid = q0 + li < a.seq_len;
      const uint16_t* qrow = lds + 4 * kSlot + (qg * 32 + li) * kD;
#pragma unroll
      for (int s = 0; s < 8; s++) {
        const bf16x8 x = *reinterpret_cast<const bf16x8*>(qrow + (((2 * s + hh) ^ k_swz(li)) * 8));
        qreg[s] = q_valid ? x : bf16x8{};
      }
    }

    // HBM -> LDS by one half of the workgroup, as buffer loads (a per-head
    // resource bounded at row seq_len, 32-bit lane offsets): wave w moves rows
    // 32(w&3) .. +31 of a tile, 4 rows per instruction; lane l fills chunk
    // position l%16 of row 32(w&3) + 4i + l/16 from the global chunk that the
    // swizzle places there. The whole offset is in the lane offset, which the
    // hardware range-checks, so rows at or past seq_len are never fetched.
    const __amdgpu_buffer_rsrc_t k_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.k + head * a.k_hs), 0, (a.seq_len - 1) * k_rs2 + kD * 2, kBufferWord3);
    const __amdgpu_buffer_rsrc_t v_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.v + head * a.v_hs), 0, (a.seq_len - 1) * v_rs2 + kD * 2, kBufferWord3);
    auto dma = [&](__amdgpu_buffer_rsrc_t rsrc, int key0, uint16_t* slot,
                   bool v_layout) __attribute__((always_inline)) {
      const int rs2 = v_layout ? v_rs2 : k_rs2;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const int row = dma_row + 4 * i;
        const int swz = v_layout ? v_swz(row) : k_swz(row);
        const int voff = (key0 + row) * rs2 + (((lane & 15) ^ swz) * 16);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsrc, (lds_void*)(slot + (32 * qg + 4 * i) * kD), 16, voff, 0, 0, 0);
      }
    };

    f32x16 oacc[4];
#pragma unroll
    for (int db = 0; db < 4; db++)
#pragma unroll
      for (int r = 0; r < 16; r++) oacc[db][r] = 0.f;
    float m = -3.0e38f, l = 0.f;
    f32x16 sacc[2];
    bf16x8 pb[4];

    const int beg = a.row_ptr[qt], n = a.row_ptr[qt + 1] - beg;
    // Column indices through the constant address space: scalar loads.
    const __attribute__((address_space(4))) int32_t* cols =
        (const __attribute__((address_space(4))) int32_t*)(a.col_idx) + beg;

    // M_j: S(j) = K(j) Q^T and O += V(j-1)^T P(j-1).
    auto m_phase = [&](int j) __attribute__((always_inline)) {
      if (j < n) {
        const uint16_t* kb = lds + (j & 1) * kSlot;
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
          for (int r = 0; r < 16; r++) sacc[b][r] = 0.f;
#pragma unroll
        for (int s = 0; s < 8; s++) {
#pragma unroll
          for (int b = 0; b < 2; b++) {
            const bf16x8 ka = *reinterpret_cast<const bf16x8*>(kb + k_off[s] + b * 32 * kD);
            sacc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, qreg[s], sacc[b], 0, 0, 0);
          }
        }
        // Operand reads run four MFMAs ahead of their use.
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 4, 0);
#pragma unroll
        for (int i = 0; i < 12; i++) {
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 4, 0);
      }
      if (j >= 1) {
        const uint16_t* vb = lds + (2 + ((j - 1) & 1)) * kSlot;
#pragma unroll
        for (int kc = 0; kc < 4; kc++)
#pragma unroll
          for (int db = 0; db < 4; db++) {
            const bf16x8 va = vt_operand(vb + v_off[0][db] + 16 * kc * kD,
                                         vb + v_off[1][db] + 16 * kc * kD);
            oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[kc], oacc[db], 0, 0, 0);
          }
        // Each V^T operand is two transpose reads; keep four operands in flight.
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 8, 0);
#pragma unroll
        for (int i = 0; i < 12; i++) {
          __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
          __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 4, 0);
      }
    };

    // V_j: online softmax of S(j) into P(j) (bf16 B operands).
    auto v_phase = [&](int j) __attribute__((always_inline)) {
      const int key0 = cols[j] * kTile;
      if (key0 + kTile > a.seq_len) {
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
          for (int r = 0; r < 16; r++) {
            const int key = key0 + half * 64 + 32 * b + 8 * (r >> 2) + 4 * hh + (r & 3);
            if (key >= a.seq_len) sacc[b][r] = -__builtin_inff();
          }
      }
      float mx = -3.0e38f;
#pragma unroll
      for (int b = 0; b < 2; b++)
#pragma unroll
        for (int r = 0; r < 16; r++) mx = fmaxf(mx, sacc[b][r]);
      mx = max_xor32(mx);
      const float m_cand = fmaxf(m, mx * c);
      const bool raise = m_cand > m + kRescaleSlack;
      if (__builtin_amdgcn_ballot_w64(raise) != 0) {
        const float m_new = raise ? m_cand : m;
        const float alpha = __builtin_amdgcn_exp2f(m - m_new);
        m = m_new;
        l *= alpha;
#pragma unroll
        for (int db = 0; db < 4; db++)
#pragma unroll
          for (int r = 0; r < 16; r++) oacc[db][r] *= alpha;
      }
#pragma unroll
      for (int b = 0; b < 2; b++)
#pragma unroll
        for (int r = 0; r < 16; r++) sacc[b][r] = __builtin_amdgcn_exp2f(fmaf(sacc[b][r], c, -m));
      // Chunk kc of P^T: registers 8*(kc&1) .. +7 of block kc>>1; element e of
      // half-wave hh is key 16kc + 8(e/4) + 4hh + e%4, matching the rows the
      // two transpose loads of the V^T operand fetch.
#pragma unroll
      for (int kc = 0; kc < 4; kc++) pb[kc] = to_bf16x8(sacc[kc >> 1], 8 * (kc & 1));
      // The row sum of the bf16 P that O accumulates: pairs dotted with (1, 1),
      // so numerator and denominator use the same rounded weights.
      typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
      const bf16x2 ones = {(__bf16)1.0f, (__bf16)1.0f};
      float ps[2] = {0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < 4; kc++)
#pragma unroll
        for (int i = 0; i < 4; i++)
          ps[kc & 1] = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{pb[kc][2 * i], pb[kc][2 * i + 1]},
                                                       ones, ps[kc & 1], false);
      l += ps[0] + ps[1];
    };

    if (n > 0) {
      // Each half runs its own loop of two phases per tile (2n + 2 phases and
      // barriers in all), so neither loop merges the other role's state.
      if (half == 0) {
        for (int j = 0; j <= n; j++) {
          m_phase(j);                                       // phase 2j
          __syncthreads();
          if (j < n) {                                      // phase 2j + 1
            const int key0 = cols[j] * kTile;
            uint16_t* vb = lds + (2 + (j & 1)) * kSlot;
            dma(v_rsrc, key0, vb, true);
            v_phase(j);
            __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
            // Rows past seq_len of a ragged tile are zeroed after they land, so
            // padding never reaches P V (0 * NaN would).
            if (key0 + kTile > a.seq_len) {
#pragma unroll
              for (int i = 0; i < 8; i++) {
                const int row = dma_row + 4 * i;
                if (key0 + row >= a.seq_len)
                  *reinterpret_cast<u32x4*>(vb + row * kD + (lane & 15) * 8) =
                      u32x4{0u, 0u, 0u, 0u};
              }
            }
          }
          __syncthreads();
        }
      } else {
        for (int j = 0; j <= n; j++) {
          if (j + 1 < n) dma(k_rsrc, cols[j + 1] * kTile, lds + ((j + 1) & 1) * kSlot, false);
          if (j >= 1) v_phase(j - 1);                       // phase 2j
          __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
          __syncthreads();
          m_phase(j);                                       // phase 2j + 1
          __syncthreads();
        }
      }
    }

    // Merge the two key halves of each query (exact: rescale both to the larger
    // m). Waves 4-7 leave (O, m, l) in LDS -- O in the two V slots, m and l in
    // K slot 1 -- then, while waves 0-3 merge and store, start the next unit's
    // K(0) and Q loads into K slot 0 and the Q slot, which no wave reads any
    // more in this unit.
    const float lt = l + __shfl_xor(l, 32);
    float* xo = reinterpret_cast<float*>(lds + 2 * kSlot) + qg * 64 * 64;
    float* xm = reinterpret_cast<float*>(lds + kSlot);
    float* xl = xm + 4 * 64;
    if (half == 1) {
#pragma unroll
      for (int db = 0; db < 4; db++)
#pragma unroll
        for (int r = 0; r < 16; r++) xo[(db * 16 + r) * 64 + lane] = oacc[db][r];
      xm[qg * 64 + lane] = m;
      xl[qg * 64 + lane] = lt;
    }
    __syncthreads();
    if (half == 1 && iu + 1 < u_end) load_unit_start(a, lds, a.work[iu + 1], qg, lane);
    if (half == 0) {
    const float m1 = xm[qg * 64 + lane], l1 = xl[qg * 64 + lane];
    const float mmax = fmaxf(m, m1);
    const float f0 = __builtin_amdgcn_exp2f(m - mmax), f1 = __builtin_amdgcn_exp2f(m1 - mmax);
    const float inv = 1.0f / fmaxf(lt * f0 + l1 * f1, 1.0e-30f);
    const float s0 = f0 * inv, s1 = f1 * inv;

    // O^T C layout: lane (li, hh) holds query q0 + li, channels
    // 32db + 8g + 4hh + [0, 4) in registers 4g .. 4g + 3.
    const int qi = q0 + li;
    const bool valid = qi < a.seq_len;
    if (qi < a.out_rows) {
      uint16_t* orow = a.out + head * a.o_hs + (int64_t)qi * a.o_rs;
#pragma unroll
      for (int db = 0; db < 4; db++)
#pragma unroll
        for (int gg = 0; gg < 4; gg++) {
          float o[4];
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int r = 4 * gg + e;
            o[e] = oacc[db][r] * s0 + xo[(db * 16 + r) * 64 + lane] * s1;
          }
          u32x2 w = {0u, 0u};
          if (valid) {
            w[0] = pack_bf16x2(o[0], o[1]);
            w[1] = pack_bf16x2(o[2], o[3]);
          }
          *reinterpret_cast<u32x2*>(orow + 32 * db + 8 * gg + 4 * hh) = w;
        }
    }
    }
  }
}

// One [heads, rows, 128] view of a caller tensor (strides in elements).
struct View {
  const void* ptr;
  int64_t head_stride, row_stride;
};

static int launch_bsattn(h3hip_plan p, const View& q, const View& k, const View& v,
                         const View& o, int32_t out_rows, float scale, hipStream_t stream) {
  AttnArgs args{static_cast<const uint16_t*>(q.ptr),
                static_cast<const uint16_t*>(k.ptr),
                static_cast<const uint16_t*>(v.ptr),
                static_cast<uint16_t*>(const_cast<void*>(o.ptr)),
                p->d_row_ptr,
                p->d_col_idx,
                p->d_work_ptr,
                p->d_work,
                q.head_stride,
                k.head_stride,
                v.head_stride,
                o.head_stride,
                (int32_t)q.row_stride,
                (int32_t)k.row_stride,
                (int32_t)v.row_stride,
                (int32_t)o.row_stride,
                p->seq_len,
                out_rows,
                scale * 1.4426950408889634f};
  const unsigned grid = (unsigned)p->groups;
  if (p->work.empty()) return H3HIP_OK;
  bsattn_fwd_kernel<<<grid, kThreads, 0, stream>>>(args);
  return check_launch("bsattn_fwd_kernel");
}

// Checks shared by both entry points; H3HIP_OK or the code to return.
static int check_attention_call(h3hip_plan plan, int32_t heads, int32_t head_dim, float scale) {
  H3_REQUIRE(plan != nullptr, H3HIP_EINVAL, "plan is NULL");
  if (head_dim != kD || heads != plan->heads) {
    set_error("declined: head_dim %d heads %d (needs head_dim 128 and the plan's %d heads)",
              head_dim, heads, plan->heads);
    return H3HIP_DECLINED;
  }
  H3_REQUIRE(std::isfinite(scale) && scale > 0.f, H3HIP_EINVAL, "scale must be finite and > 0");
  return H3HIP_OK;
}

}  // namespace h3hip

using namespace h3hip;

extern "C" int h3hip_bsattn_fwd(h3hip_plan plan, const void* q, const void* k, const void* v,
                                int32_t heads, int32_t head_dim, float scale, void* out,
                                int32_t out_layout, void* stream) {
  const int rc = check_attention_call(plan, heads, head_dim, scale);
  if (rc != H3HIP_OK) return rc;
  H3_REQUIRE(q && k && v && out, H3HIP_EINVAL, "NULL tensor argument");
  auto aligned16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  H3_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out), H3HIP_EINVAL,
             "tensors must be 16-byte aligned");
  H3_REQUIRE(out_layout == H3HIP_OUT_HEAD_MAJOR || out_layout == H3HIP_OUT_TOKEN_MAJOR,
             H3HIP_EINVAL, "unknown out_layout %d", out_layout);
  const int64_t hm = (int64_t)plan->seq_pad * kD;
  const View o = out_layout == H3HIP_OUT_HEAD_MAJOR
                     ? View{out, hm, kD}
                     : View{out, kD, (int64_t)plan->heads * kD};
  return launch_bsattn(plan, View{q, hm, kD}, View{k, hm, kD}, View{v, hm, kD}, o,
                       plan->seq_pad, scale, as_stream(stream));
}

extern "C" int h3hip_bsattn_fwd_strided(h3hip_plan plan, const h3hip_view* q,
                                        const h3hip_view* k, const h3hip_view* v,
                                        int32_t heads, int32_t head_dim, float scale,
                                        const h3hip_view* out, void* stream) {
  const int rc = check_attention_call(plan, heads, head_dim, scale);
  if (rc != H3HIP_OK) return rc;
  H3_REQUIRE(q && k && v && out, H3HIP_EINVAL, "NULL view argument");
  const h3hip_view* views[4] = {q, k, v, out};
  const char* names[4] = {"q", "k", "v", "out"};
  for (int i = 0; i < 4; i++) {
    const h3hip_view& t = *views[i];
    H3_REQUIRE(t.data != nullptr, H3HIP_EINVAL, "%s: NULL data", names[i]);
    H3_REQUIRE((reinterpret_cast<uintptr_t>(t.data) & 15u) == 0, H3HIP_EINVAL,
               "%s: data must be 16-byte aligned", names[i]);
    H3_REQUIRE(t.head_stride >= 0 && t.head_stride % 8 == 0, H3HIP_EINVAL,
               "%s: head_stride %lld must be a non-negative multiple of 8", names[i],
               (long long)t.head_stride);
    H3_REQUIRE(t.row_stride >= kD && t.row_stride % 8 == 0 && t.row_stride <= INT32_MAX,
               H3HIP_EINVAL, "%s: row_stride %lld must be a multiple of 8 and >= %d", names[i],
               (long long)t.row_stride, kD);
  }
  // Q, K and V are fetched with 32-bit offsets from each head's base.
  for (int i = 0; i < 3; i++)
    H3_REQUIRE((int64_t)plan->seq_pad * views[i]->row_stride * 2 < ((int64_t)1 << 31),
               H3HIP_EINVAL, "%s: seq_pad x row_stride exceeds 32-bit offsets", names[i]);
  auto as_view = [](const h3hip_view* t) { return View{t->data, t->head_stride, t->row_stride}; };
  return launch_bsattn(plan, as_view(q), as_view(k), as_view(v), as_view(out), plan->seq_len,
                       scale, as_stream(stream));
}

// The decline policy of H3AttentionBackend.attend (AttentionBackend.swift:123-127)
// with its AttentionContext: H3HIP_OK to run, H3HIP_DECLINED (caller runs
// dense) or an error.
static int attend_policy(h3hip_plan plan, const h3hip_attention_context* ctx) {
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
  return H3HIP_OK;
}

extern "C" int h3hip_attend(h3hip_plan plan, const h3hip_attention_context* ctx, const void* q,
                            const void* k, const void* v, int32_t heads, int32_t head_dim,
                            float scale, void* out, void* stream) {
  const int rc = attend_policy(plan, ctx);
  if (rc != H3HIP_OK) return rc;
  return h3hip_bsattn_fwd(plan, q, k, v, heads, head_dim, scale, out, H3HIP_OUT_HEAD_MAJOR,
                          stream);
}

extern "C" int h3hip_attend_strided(h3hip_plan plan, const h3hip_attention_context* ctx,
                                    const h3hip_view* q, const h3hip_view* k,
                                    const h3hip_view* v, int32_t heads, int32_t head_dim,
                                    float scale, const h3hip_view* out, void* stream) {
  const int rc = attend_policy(plan, ctx);
  if (rc != H3HIP_OK) return rc;
  return h3hip_bsattn_fwd_strided(plan, q, k, v, heads, head_dim, scale, out, stream);
}
