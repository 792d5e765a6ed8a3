// Same-run hardware ceilings for bench.py: not part of the attention path and not
// linked into libch3hip.so.
//
//  * h3probe_mfma: a sustained stream of one MFMA shape on every CU (8 waves per
//    CU, operands in registers, no memory traffic inside the loop). Its rate on
//    random bf16 operands is what the chip sustains for that shape under its
//    power limit; on zero operands, close to the clock-limited rate.
//  * h3probe_stream: HBM streams of a given byte count (read-only, write-only,
//    read+write), with the grid and the per-thread unroll as parameters so
//    bench.py can sweep them and keep the best.
//  * h3probe_relayout: the prologue's token-major -> head-major layout change
//    without arithmetic, in several thread mappings.
//  * h3probe_issue: cycles per iteration (the shader clock, s_memtime) of an
//    MFMA stream with softmax-like VALU work between its MFMAs, two waves per
//    SIMD: how much of each kind of instruction the matrix cores absorb. The
//    attention kernel's row sum chose v_add_f32 over v_dot2c from it.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 512;
constexpr int kVar = 4;  // distinct operand registers per wave

// Every wave keeps four independent accumulator chains busy; the chains'
// operands rotate over kVar register sets so consecutive MFMAs read different
// registers. `ops` holds 2 * kVar bf16x8 per thread of the grid.
template <int kShape>
__global__ __launch_bounds__(kThreads, 1) void mfma_stream(const bf16x8* __restrict__ ops,
                                                           int iters, float* __restrict__ sink) {
  const int gid = blockIdx.x * kThreads + threadIdx.x;
  bf16x8 a[kVar], b[kVar];
#pragma unroll
  for (int v = 0; v < kVar; v++) {
    a[v] = ops[gid * 2 * kVar + v];
    b[v] = ops[gid * 2 * kVar + kVar + v];
  }
  float s = 0.f;
  if (kShape == 0) {
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int i = 0; i < iters; i++) {
#pragma unroll
      for (int v = 0; v < kVar; v++) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[v], b[v], c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[(v + 1) % kVar], b[v], c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[v], b[(v + 1) % kVar], c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[(v + 2) % kVar], b[(v + 3) % kVar], c3,
                                                     0, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < 16; j++) s += c0[j] + c1[j] + c2[j] + c3[j];
  } else if (kShape == 2) {
    // The same stream with the accumulators in the AGPR file: the MFMA is
    // written out so its C/D operands are tied to AGPRs.
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int i = 0; i < iters; i++) {
#pragma unroll
      for (int v = 0; v < kVar; v++) {
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c0) : "v"(a[v]), "v"(b[v]));
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
                     : "+a"(c1) : "v"(a[(v + 1) % kVar]), "v"(b[v]));
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
                     : "+a"(c2) : "v"(a[v]), "v"(b[(v + 1) % kVar]));
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0"
                     : "+a"(c3) : "v"(a[(v + 2) % kVar]), "v"(b[(v + 3) % kVar]));
      }
    }
    // The last MFMAs' results are read by VALU code below: wait out their
    // latency before the accumulators are read.
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+a"(c0), "+a"(c1), "+a"(c2), "+a"(c3));
#pragma unroll
    for (int j = 0; j < 16; j++) s += c0[j] + c1[j] + c2[j] + c3[j];
  } else if (kShape == 3) {
    f32x4 c[8] = {};
    for (int i = 0; i < iters; i++) {
#pragma unroll
      for (int v = 0; v < kVar; v++)
#pragma unroll
        for (int k = 0; k < 8; k++)
          asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                       : "+a"(c[k]) : "v"(a[(v + k) % kVar]), "v"(b[(v + (k >> 1)) % kVar]));
    }
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7"
                 : "+a"(c[0]), "+a"(c[1]), "+a"(c[2]), "+a"(c[3]), "+a"(c[4]), "+a"(c[5]),
                   "+a"(c[6]), "+a"(c[7]));
#pragma unroll
    for (int k = 0; k < 8; k++) s += c[k][0] + c[k][1] + c[k][2] + c[k][3];
  } else {
    // Twice the instructions of half the FLOPs each: eight f32x4 chains.
    f32x4 c[8] = {};
    for (int i = 0; i < iters; i++) {
#pragma unroll
      for (int v = 0; v < kVar; v++)
#pragma unroll
        for (int k = 0; k < 8; k++)
          c[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[(v + k) % kVar],
                                                         b[(v + (k >> 1)) % kVar], c[k], 0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < 8; k++) s += c[k][0] + c[k][1] + c[k][2] + c[k][3];
  }
  // A data-dependent store the compiler cannot remove; it fires for no input
  // bench.py passes (finite operands never sum to exactly this value).
  if (s == 1234.5f) sink[gid] = s;
}

// Read-only stream: each thread XOR-folds kUnroll 16-byte chunks per grid
// stride and writes one word per block.
template <int kUnroll>
__global__ __launch_bounds__(256) void read_stream(const u32x4* __restrict__ src, int64_t n,
                                                   uint32_t* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * 256 * kUnroll;
  uint32_t acc = 0;
  for (int64_t base = (int64_t)blockIdx.x * 256 * kUnroll + threadIdx.x; base < n;
       base += stride) {
    u32x4 x[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      const int64_t i = base + (int64_t)u * 256;
      x[u] = i < n ? __builtin_nontemporal_load(src + i) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; u++) acc ^= x[u][0] ^ x[u][1] ^ x[u][2] ^ x[u][3];
  }
  __shared__ uint32_t red[256];
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t r = 0;
    for (int i = 0; i < 256; i++) r ^= red[i];
    sink[blockIdx.x] = r;
  }
}

// Write-only stream of a constant pattern.
template <int kUnroll>
__global__ __launch_bounds__(256) void write_stream(u32x4* __restrict__ dst, int64_t n,
                                                    uint32_t pattern) {
  const int64_t stride = (int64_t)gridDim.x * 256 * kUnroll;
  const u32x4 w = {pattern, pattern, pattern, pattern};
  for (int64_t base = (int64_t)blockIdx.x * 256 * kUnroll + threadIdx.x; base < n;
       base += stride) {
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      const int64_t i = base + (int64_t)u * 256;
      if (i < n) __builtin_nontemporal_store(w, dst + i);
    }
  }
}

// Read+write stream: a plain copy.
template <int kUnroll>
__global__ __launch_bounds__(256) void copy_stream(const u32x4* __restrict__ src,
                                                   u32x4* __restrict__ dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * 256 * kUnroll;
  for (int64_t base = (int64_t)blockIdx.x * 256 * kUnroll + threadIdx.x; base < n;
       base += stride) {
    u32x4 x[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      const int64_t i = base + (int64_t)u * 256;
      x[u] = i < n ? __builtin_nontemporal_load(src + i) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; u++) {
      const int64_t i = base + (int64_t)u * 256;
      if (i < n) __builtin_nontemporal_store(x[u], dst + i);
    }
  }
}

// Token-major [rows, heads * 128] -> head-major [heads, rows_pad, 128] (bf16):
// the prologue's layout change with no arithmetic. 16 lanes per 256-byte row
// (one 16-byte chunk each). kMap 0: consecutive row groups take consecutive
// tokens of one head (contiguous writes); 1: consecutive heads of one token
// (contiguous reads); 2: a wave's four rows are 2 tokens x 2 heads. kTok
// tokens per workgroup, kU rows in flight per thread; tokens >= rows are
// written as zeros.
// kNt: non-temporal loads and stores (1) or the default cache policy (0),
// which lets L2 gather the scattered head-major rows before they go out.
template <int kTok, int kU, int kThr, int kMap, int kNt = 1>
__global__ __launch_bounds__(kThr) void relayout_stream(const u32x4* __restrict__ in,
                                                       u32x4* __restrict__ out, int rows,
                                                       int rows_pad, int heads) {
  constexpr int kG = kThr / 16;
  const int g = threadIdx.x >> 4, c = threadIdx.x & 15;
  const int s0 = blockIdx.x * kTok;
  const int total = kTok * heads;
  for (int p0 = 0; p0 < total; p0 += kU * kG) {
    u32x4 x[kU];
    int tok[kU], hd[kU];
#pragma unroll
    for (int u = 0; u < kU; u++) {
      const int r = p0 + u * kG + g;
      if (kMap == 0) {
        hd[u] = r / kTok;
        tok[u] = r % kTok;
      } else if (kMap == 1) {
        tok[u] = r / heads;
        hd[u] = r % heads;
      } else {
        const int blk = r >> 2, q = r & 3;
        tok[u] = 2 * (blk % (kTok / 2)) + (q & 1);
        hd[u] = 2 * (blk / (kTok / 2)) + (q >> 1);
      }
      const int s = s0 + tok[u];
      const u32x4* src = in + ((int64_t)s * heads + hd[u]) * 16 + c;
      x[u] = (r < total && s < rows && hd[u] < heads)
                 ? (kNt ? __builtin_nontemporal_load(src) : *src)
                 : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kU; u++) {
      const int r = p0 + u * kG + g;
      const int s = s0 + tok[u];
      if (r < total && s < rows_pad && hd[u] < heads)
      {
        u32x4* dst = out + ((int64_t)hd[u] * rows_pad + s) * 16 + c;
        if (kNt)
          __builtin_nontemporal_store(x[u], dst);
        else
          *dst = x[u];
      }
    }
  }
}

int launch_status() {
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// Issue mixes. One iteration: four independent v_mfma_f32_32x32x16_bf16
// (operands v[0:15], accumulators a[0:63]), each followed by the mix's
// instructions. The VALU work reads v[0:15] and writes v[16:49], which
// nothing reads back within the loop, so the mixes differ only in what they
// issue:
//   0  MFMAs alone;
//   1  + per MFMA v_fma_f32, v_max3_f32, v_exp_f32 (the softmax's shape:
//      about 3.5 non-sum VALU instructions per MFMA in the attention loop);
//   2  mix 1 + a v_dot2c_f32_bf16 after every second MFMA (the row sum over
//      packed bf16 weights: 16 per 32 MFMAs);
//   3  mix 1 + a v_add_f32 after every MFMA (the row sum over fp32 weights:
//      32 per 32 MFMAs);
//   4  mix 1 + one v_mfma_f32_4x4x4bf16_1k per four MFMAs (a row sum on the
//      matrix cores: 8 per 32 MFMAs).
#define H3P_MF0 "v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]\n"
#define H3P_MF1 "v_mfma_f32_32x32x16_bf16 a[16:31], v[8:11], v[12:15], a[16:31]\n"
#define H3P_MF2 "v_mfma_f32_32x32x16_bf16 a[32:47], v[0:3], v[12:15], a[32:47]\n"
#define H3P_MF3 "v_mfma_f32_32x32x16_bf16 a[48:63], v[8:11], v[4:7], a[48:63]\n"
#define H3P_SMX(a, b, c) \
  "v_fma_f32 v" #a ", v1, v2, v3\n v_max3_f32 v" #b ", v4, v5, v6\n v_exp_f32 v" #c ", v7\n"
#define H3P_SM0 H3P_SMX(16, 17, 18)
#define H3P_SM1 H3P_SMX(19, 20, 21)
#define H3P_SM2 H3P_SMX(22, 23, 24)
#define H3P_SM3 H3P_SMX(25, 26, 27)
#define H3P_DOT(d) "v_dot2c_f32_bf16 v" #d ", v8, v9\n"
#define H3P_ADD(d) "v_add_f32 v" #d ", v10, v11\n"
#define H3P_M4 "v_mfma_f32_4x4x4bf16_1k a[64:67], v[12:13], v[14:15], a[64:67]\n"
#define H3P_CLOBBERS                                                                          \
  "v16", "v17", "v18", "v19", "v20", "v21", "v22", "v23", "v24", "v25", "v26", "v27", "v28",  \
      "v29", "v30", "v31", "v32", "v33", "a0", "a1", "a2", "a3", "a4", "a5", "a6", "a7", "a8",  \
      "a9", "a10", "a11", "a12", "a13", "a14", "a15", "a16", "a17", "a18", "a19", "a20", "a21", \
      "a22", "a23", "a24", "a25", "a26", "a27", "a28", "a29", "a30", "a31", "a32", "a33", "a34", \
      "a35", "a36", "a37", "a38", "a39", "a40", "a41", "a42", "a43", "a44", "a45", "a46", "a47", \
      "a48", "a49", "a50", "a51", "a52", "a53", "a54", "a55", "a56", "a57", "a58", "a59", "a60", \
      "a61", "a62", "a63", "a64", "a65", "a66", "a67"

template <int kMix>
__global__ __launch_bounds__(kThreads, 1) void issue_mix(const u32x4* __restrict__ ops,
                                                         int iters,
                                                         unsigned long long* __restrict__ cycles) {
  const int gid = blockIdx.x * kThreads + threadIdx.x;
  const u32x4 x0 = ops[4 * gid], x1 = ops[4 * gid + 1], x2 = ops[4 * gid + 2],
              x3 = ops[4 * gid + 3];
  // Random operands into v[0:15], accumulators cleared.
  asm volatile(
      "v_mov_b32 v0, %0\n v_mov_b32 v1, %1\n v_mov_b32 v2, %2\n v_mov_b32 v3, %3\n"
      "v_mov_b32 v4, %4\n v_mov_b32 v5, %5\n v_mov_b32 v6, %6\n v_mov_b32 v7, %7\n"
      "v_mov_b32 v8, %8\n v_mov_b32 v9, %9\n v_mov_b32 v10, %10\n v_mov_b32 v11, %11\n"
      "v_mov_b32 v12, %12\n v_mov_b32 v13, %13\n v_mov_b32 v14, %14\n v_mov_b32 v15, %15"
      :
      : "v"(x0[0]), "v"(x0[1]), "v"(x0[2]), "v"(x0[3]), "v"(x1[0]), "v"(x1[1]), "v"(x1[2]),
        "v"(x1[3]), "v"(x2[0]), "v"(x2[1]), "v"(x2[2]), "v"(x2[3]), "v"(x3[0]), "v"(x3[1]),
        "v"(x3[2]), "v"(x3[3])
      : "v0", "v1", "v2", "v3", "v4", "v5", "v6", "v7", "v8", "v9", "v10", "v11", "v12", "v13",
        "v14", "v15");
  asm volatile(
      "v_accvgpr_write_b32 a0, 0\n v_accvgpr_write_b32 a1, 0\n v_accvgpr_write_b32 a2, 0\n v_accvgpr_write_b32 a3, 0\n"
      "v_accvgpr_write_b32 a4, 0\n v_accvgpr_write_b32 a5, 0\n v_accvgpr_write_b32 a6, 0\n v_accvgpr_write_b32 a7, 0\n"
      "v_accvgpr_write_b32 a8, 0\n v_accvgpr_write_b32 a9, 0\n v_accvgpr_write_b32 a10, 0\n v_accvgpr_write_b32 a11, 0\n"
      "v_accvgpr_write_b32 a12, 0\n v_accvgpr_write_b32 a13, 0\n v_accvgpr_write_b32 a14, 0\n v_accvgpr_write_b32 a15, 0\n"
      "v_accvgpr_write_b32 a16, 0\n v_accvgpr_write_b32 a17, 0\n v_accvgpr_write_b32 a18, 0\n v_accvgpr_write_b32 a19, 0\n"
      "v_accvgpr_write_b32 a20, 0\n v_accvgpr_write_b32 a21, 0\n v_accvgpr_write_b32 a22, 0\n v_accvgpr_write_b32 a23, 0\n"
      "v_accvgpr_write_b32 a24, 0\n v_accvgpr_write_b32 a25, 0\n v_accvgpr_write_b32 a26, 0\n v_accvgpr_write_b32 a27, 0\n"
      "v_accvgpr_write_b32 a28, 0\n v_accvgpr_write_b32 a29, 0\n v_accvgpr_write_b32 a30, 0\n v_accvgpr_write_b32 a31, 0\n"
      "v_accvgpr_write_b32 a32, 0\n v_accvgpr_write_b32 a33, 0\n v_accvgpr_write_b32 a34, 0\n v_accvgpr_write_b32 a35, 0\n"
      "v_accvgpr_write_b32 a36, 0\n v_accvgpr_write_b32 a37, 0\n v_accvgpr_write_b32 a38, 0\n v_accvgpr_write_b32 a39, 0\n"
      "v_accvgpr_write_b32 a40, 0\n v_accvgpr_write_b32 a41, 0\n v_accvgpr_write_b32 a42, 0\n v_accvgpr_write_b32 a43, 0\n"
      "v_accvgpr_write_b32 a44, 0\n v_accvgpr_write_b32 a45, 0\n v_accvgpr_write_b32 a46, 0\n v_accvgpr_write_b32 a47, 0\n"
      "v_accvgpr_write_b32 a48, 0\n v_accvgpr_write_b32 a49, 0\n v_accvgpr_write_b32 a50, 0\n v_accvgpr_write_b32 a51, 0\n"
      "v_accvgpr_write_b32 a52, 0\n v_accvgpr_write_b32 a53, 0\n v_accvgpr_write_b32 a54, 0\n v_accvgpr_write_b32 a55, 0\n"
      "v_accvgpr_write_b32 a56, 0\n v_accvgpr_write_b32 a57, 0\n v_accvgpr_write_b32 a58, 0\n v_accvgpr_write_b32 a59, 0\n"
      "v_accvgpr_write_b32 a60, 0\n v_accvgpr_write_b32 a61, 0\n v_accvgpr_write_b32 a62, 0\n v_accvgpr_write_b32 a63, 0\n"
      "v_accvgpr_write_b32 a64, 0\n v_accvgpr_write_b32 a65, 0\n v_accvgpr_write_b32 a66, 0\n v_accvgpr_write_b32 a67, 0\n"
      ::: H3P_CLOBBERS);
  __syncthreads();
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int i = 0; i < iters; i++) {
    if constexpr (kMix == 0) {
      asm volatile(H3P_MF0 H3P_MF1 H3P_MF2 H3P_MF3 ::: H3P_CLOBBERS);
    } else if constexpr (kMix == 1) {
      asm volatile(H3P_MF0 H3P_SM0 H3P_MF1 H3P_SM1 H3P_MF2 H3P_SM2 H3P_MF3 H3P_SM3 ::: H3P_CLOBBERS);
    } else if constexpr (kMix == 2) {
      asm volatile(H3P_MF0 H3P_SM0 H3P_DOT(28) H3P_MF1 H3P_SM1 H3P_MF2 H3P_SM2 H3P_DOT(29)
                   H3P_MF3 H3P_SM3 ::: H3P_CLOBBERS);
    } else if constexpr (kMix == 3) {
      asm volatile(H3P_MF0 H3P_SM0 H3P_ADD(30) H3P_MF1 H3P_SM1 H3P_ADD(31) H3P_MF2 H3P_SM2
                   H3P_ADD(32) H3P_MF3 H3P_SM3 H3P_ADD(33) ::: H3P_CLOBBERS);
    } else {
      asm volatile(H3P_MF0 H3P_SM0 H3P_M4 H3P_MF1 H3P_SM1 H3P_MF2 H3P_SM2 H3P_MF3
                   H3P_SM3 ::: H3P_CLOBBERS);
    }
  }
  // Let the last MFMAs and dots drain before the clock is read again.
  asm volatile("s_nop 15\n s_nop 15\n s_nop 15\n s_nop 15" ::: "memory");
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  if ((threadIdx.x & 63) == 0) cycles[blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6)] = t1 - t0;
}

}  // namespace

extern "C" {

// Operand buffer size in bytes for `blocks` workgroups.
int64_t h3probe_mfma_operand_bytes(int32_t blocks) {
  return (int64_t)blocks * kThreads * 2 * kVar * 16;
}

// FLOPs of one h3probe_mfma launch (both shapes do the same FLOPs per iteration).
double h3probe_mfma_flops(int32_t blocks, int32_t iters) {
  return (double)blocks * (kThreads / 64) * iters * kVar * 4 * 32768.0;
}

// shape 0: v_mfma_f32_32x32x16_bf16, 1: v_mfma_f32_16x16x32_bf16, with VGPR
// accumulators; 2 and 3: the same shapes with AGPR accumulators. `ops` holds
// h3probe_mfma_operand_bytes(blocks) bytes, `sink` blocks * 512 floats.
// Returns 0, -1 on a bad argument, -2 on a launch failure.
int h3probe_mfma(int32_t shape, const void* ops, int32_t blocks, int32_t iters, void* sink,
                 void* stream) {
  if (shape < 0 || shape > 3 || !ops || !sink || blocks <= 0 || iters <= 0) return -1;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // 96 KiB of dynamic LDS keeps one workgroup per CU, as in the attention kernel.
  const int lds = 96 * 1024;
  const void* fn = shape == 0   ? (const void*)mfma_stream<0>
                   : shape == 1 ? (const void*)mfma_stream<1>
                   : shape == 2 ? (const void*)mfma_stream<2>
                                : (const void*)mfma_stream<3>;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess)
    return -2;
  const bf16x8* o = static_cast<const bf16x8*>(ops);
  float* sk = static_cast<float*>(sink);
  switch (shape) {
    case 0: mfma_stream<0><<<blocks, kThreads, lds, s>>>(o, iters, sk); break;
    case 1: mfma_stream<1><<<blocks, kThreads, lds, s>>>(o, iters, sk); break;
    case 2: mfma_stream<2><<<blocks, kThreads, lds, s>>>(o, iters, sk); break;
    default: mfma_stream<3><<<blocks, kThreads, lds, s>>>(o, iters, sk); break;
  }
  return launch_status();
}

// kind 0: read `bytes` from src (sink: blocks words); 1: write `bytes` to dst;
// 2: copy `bytes` from src to dst. bytes a multiple of 16, buffers 16-byte
// aligned; unroll 1, 2, 4 or 8; blocks of 256 threads.
int h3probe_stream(int32_t kind, const void* src, void* dst, int64_t bytes, int32_t blocks,
                   int32_t unroll, void* sink, void* stream) {
  if (bytes <= 0 || bytes % 16 || blocks <= 0) return -1;
  if (unroll != 1 && unroll != 2 && unroll != 4 && unroll != 8) return -1;
  if ((kind == 0 || kind == 2) && (!src || (reinterpret_cast<uintptr_t>(src) & 15))) return -1;
  if ((kind == 1 || kind == 2) && (!dst || (reinterpret_cast<uintptr_t>(dst) & 15))) return -1;
  if (kind == 0 && !sink) return -1;
  if (kind < 0 || kind > 2) return -1;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int64_t n = bytes / 16;
  const u32x4* in = static_cast<const u32x4*>(src);
  u32x4* out = static_cast<u32x4*>(dst);
  uint32_t* sk = static_cast<uint32_t*>(sink);
#define H3PROBE_DISPATCH(U)                                                   \
  case U:                                                                     \
    if (kind == 0) read_stream<U><<<blocks, 256, 0, s>>>(in, n, sk);          \
    else if (kind == 1) write_stream<U><<<blocks, 256, 0, s>>>(out, n, 0x3f803f80u); \
    else copy_stream<U><<<blocks, 256, 0, s>>>(in, out, n);                   \
    break;
  switch (unroll) {
    H3PROBE_DISPATCH(1)
    H3PROBE_DISPATCH(2)
    H3PROBE_DISPATCH(4)
    H3PROBE_DISPATCH(8)
  }
#undef H3PROBE_DISPATCH
  return launch_status();
}

// The prologue's relayout without arithmetic: in [rows, heads * 128] bf16
// token-major, out [heads, rows_pad, 128] head-major (rows_pad a multiple of
// 32). variant: 0 tokens-fastest 8 tokens x 5 rows in flight x 512 threads,
// 1 tokens-fastest 2 x 5 x 256, 2 tokens-fastest 4 x 4 x 256, 3 heads-fastest
// 4 x 4 x 256, 4 2x2 blocks 4 x 5 x 512; with the default cache policy
// instead of non-temporal: 5 tokens-fastest 8x5x512, 6 4x4x256, 7 16x5x512,
// 9 32x5x512; 8 tokens-fastest 16x5x512 non-temporal.
int h3probe_relayout(int32_t variant, const void* in, void* out, int32_t rows, int32_t rows_pad,
                     int32_t heads, void* stream) {
  if (!in || !out || rows <= 0 || rows_pad < rows || rows_pad % 32 || heads <= 0 || heads % 2)
    return -1;
  if ((reinterpret_cast<uintptr_t>(in) & 15) || (reinterpret_cast<uintptr_t>(out) & 15)) return -1;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const u32x4* i4 = static_cast<const u32x4*>(in);
  u32x4* o4 = static_cast<u32x4*>(out);
  switch (variant) {
    case 0: relayout_stream<8, 5, 512, 0><<<rows_pad / 8, 512, 0, s>>>(i4, o4, rows, rows_pad, heads); break;
    case 1: relayout_stream<2, 5, 256, 0><<<rows_pad / 2, 256, 0, s>>>(i4, o4, rows, rows_pad, heads); break;
    case 2: relayout_stream<4, 4, 256, 0><<<rows_pad / 4, 256, 0, s>>>(i4, o4, rows, rows_pad, heads); break;
    case 3: relayout_stream<4, 4, 256, 1><<<rows_pad / 4, 256, 0, s>>>(i4, o4, rows, rows_pad, heads); break;
    case 4: relayout_stream<4, 5, 512, 2><<<rows_pad / 4, 512, 0, s>>>(i4, o4, rows, rows_pad, heads); break;
    case 5: relayout_stream<8, 5, 512, 0, 0><<<rows_pad / 8, 512, 0, s>>>(i4, o4, rows, rows_pad, heads); break;
    case 6: relayout_stream<4, 4, 256, 0, 0><<<rows_pad / 4, 256, 0, s>>>(i4, o4, rows, rows_pad, heads); break;
    case 7: relayout_stream<16, 5, 512, 0, 0><<<rows_pad / 16, 512, 0, s>>>(i4, o4, rows, rows_pad, heads); break;
    case 8: relayout_stream<16, 5, 512, 0, 1><<<rows_pad / 16, 512, 0, s>>>(i4, o4, rows, rows_pad, heads); break;
    case 9: relayout_stream<32, 5, 512, 0, 0><<<rows_pad / 32, 512, 0, s>>>(i4, o4, rows, rows_pad, heads); break;
    default: return -1;
  }
  return launch_status();
}

// Operand buffer size in bytes of h3probe_issue for `blocks` workgroups.
int64_t h3probe_issue_operand_bytes(int32_t blocks) { return (int64_t)blocks * kThreads * 64; }

// Issue mix `mix` (0..4, see issue_mix) on `blocks` workgroups of 8 waves (one
// per CU), `iters` iterations; `ops` holds h3probe_issue_operand_bytes(blocks)
// random bytes, `cycles` receives blocks * 8 shader-clock counts, one per
// wave. Returns 0, -1 on a bad argument, -2 on a launch failure.
int h3probe_issue(int32_t mix, const void* ops, int32_t blocks, int32_t iters, void* cycles,
                  void* stream) {
  if (mix < 0 || mix > 4 || !ops || !cycles || blocks <= 0 || iters <= 0) return -1;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const u32x4* o = static_cast<const u32x4*>(ops);
  unsigned long long* c = static_cast<unsigned long long*>(cycles);
  switch (mix) {
    case 0: issue_mix<0><<<blocks, kThreads, 0, s>>>(o, iters, c); break;
    case 1: issue_mix<1><<<blocks, kThreads, 0, s>>>(o, iters, c); break;
    case 2: issue_mix<2><<<blocks, kThreads, 0, s>>>(o, iters, c); break;
    case 3: issue_mix<3><<<blocks, kThreads, 0, s>>>(o, iters, c); break;
    default: issue_mix<4><<<blocks, kThreads, 0, s>>>(o, iters, c); break;
  }
  return launch_status();
}

}  // extern "C"
