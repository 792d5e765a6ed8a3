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

}  // extern "C"
