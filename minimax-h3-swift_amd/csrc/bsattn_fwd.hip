// Block-sparse flash attention over 128x128 tiles, bf16 MFMA on gfx950.
//
// Persistent workgroups of 8 waves (two per SIMD), one per CU, each running
// the (head, 128-query tile) work units that the plan's XCD-aware schedule
// gives it, one after another; the next unit's first K tile and its Q tile
// load while the current one merges and stores its output. Wave w owns
// queries 32(w&3) .. +31 -- the B operand of v_mfma_f32_32x32x16_bf16 -- and
// key half w>>2 (keys 64(w>>2) .. +63) of every 128-key tile, keeping its own
// online-softmax state; the two key halves of each query are merged exactly
// at the end of the unit.
//
// The tile loop of a unit is one inline-assembly block (bsattn_tile_loop.inc,
// written by gen_tile_loop.py) with every register assigned by hand: O, Q^T
// and a six-entry operand ring in AGPRs (LDS reads land there directly),
// scores and weights double-buffered in VGPRs. In iteration j one instruction
// stream carries the scores of tile j+1, the product with the weights of tile
// j-1, the softmax of tile j and the wave's share of the HBM -> LDS loads of
// K(j+2) and V(j), so each wave's VALU work runs beside its own MFMAs and the
// partner wave on its SIMD fills the issue slots it leaves; one barrier per
// tile orders the loads against the LDS reads.
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
// in exact arithmetic (numerator and denominator share m). After a row's
// first tile the loop takes the row max only when it may matter: it weighs
// a tile at the current m first, and reruns the full step (max, raise,
// alpha, weights) when the weights of a lane sum past 2^8 or to NaN. l sums the fp32
// weights, as the reference's recurrence does; O accumulates their bf16
// roundings, the P operand of the P V product. The output is O / max(l, 1e-30).
#include <cmath>

#include "common.h"
#include "plan.h"
#include "bsattn_tile_loop.inc"

namespace h3hip {

constexpr int kTile = 128;
constexpr int kD = 128;
constexpr int kWaves = H3_TILE_LOOP_WAVES;
constexpr int kThreads = 64 * kWaves;
constexpr int kRowsPerWave = H3_TILE_LOOP_ROWS_PER_WAVE;  // of each tile a wave loads
static_assert(kWaves == 8 && kRowsPerWave * kWaves == kTile, "tile loop layout");
constexpr int kSlot = kTile * kD;                   // one K or V tile, unpadded (elements)
// LDS byte layout: K slots 0 and 1, V slots 0 and 1, the unit's Q tile.
constexpr uint32_t kKSlot0 = 0, kVSlot0 = 65536, kQSlot = 131072;
// s_waitcnt immediate for vmcnt(0) with expcnt and lgkmcnt left unconstrained
// (gfx9 encoding: vmcnt[3:0] bits 3:0, expcnt bits 6:4, lgkmcnt bits 11:8,
// vmcnt[5:4] bits 15:14).
constexpr int kWaitVmcnt0 = 0x0F70;
// Buffer resource word 3 for raw (untyped, unswizzled) buffer loads on gfx9:
// DATA_FORMAT = 32 bits, everything else zero.
constexpr int kBufferWord3 = 0x00020000;

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
  const int32_t* __restrict__ unit_desc;  // [units][kUnitDescInts], in work order
  int64_t q_hs, k_hs, v_hs, o_hs;  // head strides (elements)
  int32_t q_rs, k_rs, v_rs, o_rs;  // row strides (elements)
  int32_t seq_len, out_rows;
  float scale_log2;
};

typedef __attribute__((address_space(3))) void lds_void;
typedef float f32x32 __attribute__((ext_vector_type(32)));

// LDS tiles are unpadded 256-byte rows whose 16-byte chunks are XOR-swizzled
// so the operand reads hit 64 distinct banks per phase:
//   K and Q: chunk c of row r sits at c ^ (r & 15) -- 16 consecutive rows read
//      at one chunk (ds_read_b128) land on 16 different chunk positions;
//   V: chunk c of row r sits at c ^ (4*(r & 3) + ((r >> 2) & 3)) -- the
//      transpose load reads 4 consecutive rows x 4 consecutive chunks per
//      32-lane phase, which this maps onto all 16 chunk positions.
__host__ __device__ __forceinline__ int k_swz(int r) { return r & 15; }
__host__ __device__ __forceinline__ int v_swz(int r) { return 4 * (r & 3) + ((r >> 2) & 3); }

// Workgroup barrier ordering this wave's LDS accesses only (not its
// outstanding global loads and stores, which __syncthreads would also wait for).
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// A unit's first K tile and its Q tile, HBM -> LDS: wave w moves rows
// kRowsPerWave*w .. + kRowsPerWave-1 of each, 4 rows per instruction, chunks
// K-swizzled, into K slot 0 and the Q slot. Buffer resources bound the rows
// at seq_len, so no row past it is fetched; query rows past it only feed
// output rows that are stored as zeros.
// Unit iu's descriptor (plan.h: unit, col_idx index, n, c0, c1, c2, ragged),
// through the scalar cache.
__device__ __forceinline__ const __attribute__((address_space(4))) int32_t* unit_desc(
    const AttnArgs& a, int iu) {
  return (const __attribute__((address_space(4))) int32_t*)(a.unit_desc) + kUnitDescInts * iu;
}

__device__ __forceinline__ void load_unit_start(const AttnArgs& a, uint16_t* lds, int iu,
                                                int wave, int lane) {
  const auto* d = unit_desc(a, iu);
  const int32_t unit = d[0];
  const int head = unit >> 16, qt = unit & 0xffff;
  const int dma_row = kRowsPerWave * wave + (lane >> 4);
  auto tile = [&](const uint16_t* base, int rs2, int row0, uint16_t* slot)
      __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)base, 0, (a.seq_len - 1) * rs2 + kD * 2, kBufferWord3);
#pragma unroll
    for (int i = 0; i < kRowsPerWave / 4; i++) {
      const int row = dma_row + 4 * i;
      const int voff = (row0 + row) * rs2 + (((lane & 15) ^ k_swz(row)) * 16);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsrc, (lds_void*)(slot + (kRowsPerWave * wave + 4 * i) * kD), 16, voff, 0, 0, 0);
    }
  };
  tile(a.q + head * a.q_hs, a.q_rs * 2, qt * kTile, lds + kQSlot / 2);
  if (d[2] > 0) tile(a.k + head * a.k_hs, a.k_rs * 2, d[3] * kTile, lds + kKSlot0 / 2);
}

__global__ __launch_bounds__(kThreads, 1) void bsattn_fwd_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[5 * kSlot];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform, in an SGPR
  const int qg = wave & 3, kh = wave >> 2;
  const int k_rs2 = a.k_rs * 2, v_rs2 = a.v_rs * 2;
  const uint32_t base = lds_addr(lds);

  const int u_beg = a.work_ptr[blockIdx.x], u_end = a.work_ptr[blockIdx.x + 1];
  if (u_beg < u_end) load_unit_start(a, lds, u_beg, wave, threadIdx.x & 63);
  // Lane address offsets of the tile loop (bytes), the same for every unit:
  // computed once; the tile loop takes them as inputs and leaves them intact.
  const int lane0 = threadIdx.x & 63, li0 = lane0 & 31, hh0 = lane0 >> 5;
  int ka[8], va[8], dk[kRowsPerWave / 4], dv[kRowsPerWave / 4];
#pragma unroll
  for (int s = 0; s < 8; s++)
    ka[s] = base + kKSlot0 + 2 * ((kh * 64 + li0) * kD + (((2 * s + hh0) ^ k_swz(li0)) * 8));
  const int g = lane0 >> 4, mm = lane0 & 15;
#pragma unroll
  for (int p = 0; p < 2; p++)
#pragma unroll
    for (int db = 0; db < 4; db++) {
      const int row = kh * 64 + 8 * p + 4 * (g >> 1) + (mm >> 2);
      const int chunk = 4 * db + 2 * (g & 1) + ((mm & 3) >> 1);
      va[4 * p + db] =
          base + kVSlot0 + 2 * (row * kD + ((chunk ^ v_swz(row)) * 8) + 4 * (mm & 1));
    }
#pragma unroll
  for (int i = 0; i < kRowsPerWave / 4; i++) {
    const int row = kRowsPerWave * wave + 4 * i + (lane0 >> 4);
    // Less 1024 i: the tile loop's loads add it back as their
    // instruction offset, which also steps their LDS address.
    dk[i] = row * k_rs2 + (((lane0 & 15) ^ k_swz(row)) * 16) - 1024 * i;
    dv[i] = row * v_rs2 + (((lane0 & 15) ^ v_swz(row)) * 16) - 1024 * i;
  }
  // The first unit's K(0) and Q have landed (later units wait in the merge).
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  for (int iu = u_beg; iu < u_end; iu++) {
    // Lane-derived values are rebuilt for each unit from an opaque copy of the
    // thread index: hoisted out of the unit loop they would stay live across
    // the tile loop, which leaves no VGPRs to hold them.
    int tid;
    asm volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"(threadIdx.x));
    const int lane = tid & 63, li = lane & 31, hh = lane >> 5;
    const auto* desc = unit_desc(a, iu);
    const int32_t unit = desc[0];
    const int head = unit >> 16, qt = unit & 0xffff;
    const int q0 = qt * kTile + qg * 32;
    const int beg = desc[1], n = desc[2];

    // The unit's K(0) and Q have landed (each wave waited for its own loads
    // before its output stores) and the previous unit's merge buffers have
    // been read. The output stores stay in flight: loads return in order, so
    // the tile loop's counted waits only grow stronger for them.
    lds_barrier();

    f32x32 o01, o23;  // O(0), O(1) and O(2), O(3): 16 accumulators each
    float m, l;
    if (n > 0) {

      const int keyoff = kh * 64 + 4 * hh, lane16 = 16 * lane;
      const int rowb = kRowsPerWave * wave + (lane >> 4);

      // Scalar operands of the tile loop, made wave-uniform explicitly so they
      // are SGPRs.
      auto u = [](uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); };
      const uint32_t c0 = u(desc[3]), c1 = u(desc[4]), c2 = u(desc[5]), ragged = u(desc[6]);
      const uint64_t colp = (uint64_t)(uintptr_t)(a.col_idx + beg);
      const uint64_t kbp = (uint64_t)(uintptr_t)(a.k + head * a.k_hs);
      const uint64_t vbp = (uint64_t)(uintptr_t)(a.v + head * a.v_hs);
      const uint32_t krec = u((uint32_t)((a.seq_len - 1) * k_rs2 + kD * 2));
      const uint32_t vrec = u((uint32_t)((a.seq_len - 1) * v_rs2 + kD * 2));
      const uint32_t m0k = u(base + kKSlot0 + 256u * kRowsPerWave * wave);
      const uint32_t m0v = u(base + kVSlot0 + 256u * kRowsPerWave * wave);
      const uint32_t qoff = u(kQSlot - kKSlot0 + 256u * 32u * qg - 256u * 64u * kh);
      const uint32_t nn = u(n), seq = u(a.seq_len), k128 = u(k_rs2 * kTile), v128 = u(v_rs2 * kTile);
      const uint32_t cbits = u(__float_as_uint(a.scale_log2));
      asm volatile(H3_TILE_LOOP_ASM
                   : "=&{a[0:31]}"(o01), "=&{a[32:63]}"(o23), "=&{v96}"(m), "=&{v97}"(l)
                   : "{v98}"(ka[0]), "{v99}"(ka[1]), "{v100}"(ka[2]), "{v101}"(ka[3]),
                     "{v102}"(ka[4]), "{v103}"(ka[5]), "{v104}"(ka[6]), "{v105}"(ka[7]),
                     "{v106}"(va[0]), "{v107}"(va[1]), "{v108}"(va[2]), "{v109}"(va[3]),
                     "{v110}"(va[4]), "{v111}"(va[5]), "{v112}"(va[6]), "{v113}"(va[7]),
                     "{v114}"(dk[0]), "{v115}"(dk[1]), "{v116}"(dk[2]), "{v117}"(dk[3]),
                     "{v118}"(dv[0]), "{v119}"(dv[1]), "{v120}"(dv[2]), "{v121}"(dv[3]),
                     "{a120}"(keyoff), "{a121}"(lane16), "{a122}"(rowb),
                     [n] "s"(nn), [c0] "s"(c0), [c1] "s"(c1), [c2] "s"(c2),
                     [colp_lo] "s"(u((uint32_t)colp)), [colp_hi] "s"(u((uint32_t)(colp >> 32))),
                     [kb_lo] "s"(u((uint32_t)kbp)), [kb_hi] "s"(u((uint32_t)(kbp >> 32))),
                     [vb_lo] "s"(u((uint32_t)vbp)), [vb_hi] "s"(u((uint32_t)(vbp >> 32))),
                     [krec] "s"(krec), [vrec] "s"(vrec), [kstep] "s"(k128), [vstep] "s"(v128),
                     [c] "s"(cbits), [m0k] "s"(m0k), [m0v] "s"(m0v), [qoff] "s"(qoff),
                     [seq] "s"(seq), [ragged] "s"(ragged)
                   : H3_TILE_LOOP_CLOBBERS);
    } else {
      // A row with no active tile: its output is zero.
      o01 = f32x32{};
      o23 = f32x32{};
      m = -3.0e38f;
      l = 0.f;
    }

    // Lane values again, from a fresh opaque copy: kept from before the tile
    // loop they would be spilled across it.
    asm volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"(threadIdx.x));
    const int lane2 = tid & 63, li2 = lane2 & 31, hh2 = lane2 >> 5;
    // The next unit's K(0) and Q go into K slot 0 and the Q slot, which no
    // wave reads once its tile loop has passed the last tile's barrier.
    if (iu + 1 < u_end) load_unit_start(a, lds, iu + 1, wave, lane2);
    // Every wave's last V reads are done: the V slots are free. An LDS-only
    // barrier: __syncthreads would also wait for the loads just issued, whose
    // HBM latency the merge is there to cover (the next unit waits for them).
    lds_barrier();

    // Merge of the two key halves (exact: both rescaled to the larger m).
    // Wave (qg, kh) finalises channel blocks 2kh, 2kh+1 of its 32 queries and
    // hands the partner wave (qg, 1-kh) its O of the partner's blocks, 8 KiB
    // per wave in V slot 0, with m and l in K slot 1.
    // l summed with the other half-wave's (the same queries' other 32 keys).
    const auto lsw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l),
                                                      false, false);
    const float lt = __uint_as_float(lsw[0]) + __uint_as_float(lsw[1]);
    float* xo = reinterpret_cast<float*>(lds + kVSlot0 / 2);
    float* xml = reinterpret_cast<float*>(lds + kSlot);
    // The wave keeps channel blocks 2kh, 2kh+1 (keep) and gives the other
    // two (give); block 2i + b is register 16b + r of o01 (i = 0) or o23.
    auto merge = [&](const f32x32& keep, const f32x32& give, int kb0)
                     __attribute__((always_inline)) {
      float* mine = xo + wave * 2048;
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int r4 = 0; r4 < 4; r4++) {
          const int r = 16 * i + 4 * r4;
          const f32x4 w = {give[r], give[r + 1], give[r + 2], give[r + 3]};
          *reinterpret_cast<f32x4*>(mine + ((4 * i + r4) * 64 + lane2) * 4) = w;
        }
      xml[wave * 128 + lane2] = m;
      xml[wave * 128 + 64 + lane2] = lt;
      lds_barrier();
      const int pw = wave ^ 4;
      const float* theirs = xo + pw * 2048;
      const float mp = xml[pw * 128 + lane2], ltp = xml[pw * 128 + 64 + lane2];
      const float mmax = fmaxf(m, mp);
      const float f0 = __builtin_amdgcn_exp2f(m - mmax), f1 = __builtin_amdgcn_exp2f(mp - mmax);
      const float inv = 1.0f / fmaxf(lt * f0 + ltp * f1, 1.0e-30f);
      const float s0 = f0 * inv, s1 = f1 * inv;
      // O^T C layout: lane (li, hh) holds query q0 + li, channels
      // 32db + 8gg + 4hh + [0, 4) in registers 16db + 4gg .. +3.
      const int qi = q0 + li2;
      const bool valid = qi < a.seq_len;
      // This wave's loads of the next unit are done before its output
      // stores are issued, so that the next unit waits for no store.
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      if (qi < a.out_rows) {
        uint16_t* orow = a.out + head * a.o_hs + (int64_t)qi * a.o_rs;
#pragma unroll
        for (int i = 0; i < 2; i++) {
          const int db = kb0 + i;
#pragma unroll
          for (int gg = 0; gg < 4; gg++) {
            const f32x4 t =
                *reinterpret_cast<const f32x4*>(theirs + ((4 * i + gg) * 64 + lane2) * 4);
            float ov[4];
#pragma unroll
            for (int e = 0; e < 4; e++) ov[e] = keep[16 * i + 4 * gg + e] * s0 + t[e] * s1;
            u32x2 w = {0u, 0u};
            if (valid) {
              w[0] = pack_bf16x2(ov[0], ov[1]);
              w[1] = pack_bf16x2(ov[2], ov[3]);
            }
            *reinterpret_cast<u32x2*>(orow + 32 * db + 8 * gg + 4 * hh2) = w;
          }
        }
      }
    };
    if (kh == 0)
      merge(o01, o23, 0);
    else
      merge(o23, o01, 2);
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
                p->d_unit_desc,
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
