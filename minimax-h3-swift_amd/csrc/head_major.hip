// Token-major [S, heads * 128] -> head-major [heads, seq_pad, 128] copy.
//
// What AttentionLayer.sdpa's transposes (Sources/H3Modules/DiTBlock.swift:297-300,
// `v.transposed(1, 0, 2)` of the [S, heads, headDim] projection) become when
// they are materialised: each (token, head) row of 256 bytes moves once, rows
// seq_len .. seq_pad of the output are zeroed. The attention reads V in place
// and the prologue relays Q and K itself, so the layer step does not call this;
// it serves callers that want head-major V for h3hip_bsattn_fwd, and it is the
// pure-data-movement ceiling of the prologue's layout change (same bytes, no
// arithmetic).
//
// HBM-bound. A workgroup owns kTok consecutive tokens and all heads; a row is
// 16 lanes x 16 bytes, and the 16 rows a wave moves per instruction are kTok
// consecutive tokens of 16 / kTok heads, so every store instruction writes
// kTok x 256 contiguous bytes of each head. Measured on MI355X over a sweep of
// tokens per workgroup (2..32), lanes per row (8, 16), row order (heads or
// tokens innermost) and loads in flight (1, 2, 4), this mapping moves the
// most bytes per second; 8 lanes per row (two chunks per lane) is ~25% slower.
#include "common.h"

namespace h3hip {

namespace {

constexpr int kTok = 4;          // tokens per workgroup
constexpr int kLanes = 16;       // lanes per 256-byte row
constexpr int kRowsPerPass = 256 / kLanes;
constexpr int kInFlight = 2;     // rows in flight per lane

struct HeadMajorArgs {
  const uint16_t* __restrict__ in;
  uint16_t* __restrict__ out;
  int64_t ld_in;
  int32_t seq_len, seq_pad, heads;
};

__device__ __forceinline__ u32x4 stream_load16(const uint16_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void stream_store16(uint16_t* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

__global__ __launch_bounds__(256) void head_major_kernel(HeadMajorArgs a) {
  const int lane = threadIdx.x % kLanes, r0 = threadIdx.x / kLanes;
  const int32_t s0 = blockIdx.x * kTok;
  const int rows = kTok * a.heads;
  for (int base = 0; base < rows; base += kRowsPerPass * kInFlight) {
    u32x4 v[kInFlight];
    uint16_t* dst[kInFlight];
#pragma unroll
    for (int u = 0; u < kInFlight; u++) {
      const int r = base + u * kRowsPerPass + r0;
      const int tok = r % kTok, head = r / kTok;
      const int32_t s = s0 + tok;
      dst[u] = nullptr;
      v[u] = u32x4{0u, 0u, 0u, 0u};
      if (r < rows && s < a.seq_pad) {
        dst[u] = a.out + ((int64_t)head * a.seq_pad + s) * 128 + lane * 8;
        if (s < a.seq_len) v[u] = stream_load16(a.in + (int64_t)s * a.ld_in + head * 128 + lane * 8);
      }
    }
#pragma unroll
    for (int u = 0; u < kInFlight; u++)
      if (dst[u] != nullptr) stream_store16(dst[u], v[u]);
  }
}

}  // namespace

}  // namespace h3hip

using namespace h3hip;

extern "C" int h3hip_head_major(const void* in, int64_t ld_in, int32_t seq_len, int32_t seq_pad,
                                int32_t heads, int32_t head_dim, void* out, void* stream) {
  if (head_dim != 128) {
    set_error("declined: head_dim %d (needs 128)", head_dim);
    return H3HIP_DECLINED;
  }
  H3_REQUIRE(in != nullptr && out != nullptr, H3HIP_EINVAL, "NULL tensor argument");
  H3_REQUIRE(seq_len > 0 && heads > 0 && seq_pad >= seq_len && seq_pad % 128 == 0, H3HIP_EINVAL,
             "bad shape: seq_len %d seq_pad %d heads %d", seq_len, seq_pad, heads);
  H3_REQUIRE(ld_in >= (int64_t)heads * 128 && ld_in % 8 == 0, H3HIP_EINVAL,
             "ld_in %lld must be >= heads * 128 and a multiple of 8", (long long)ld_in);
  H3_REQUIRE((reinterpret_cast<uintptr_t>(in) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(out) & 15u) == 0,
             H3HIP_EINVAL, "tensors must be 16-byte aligned");
  HeadMajorArgs a{static_cast<const uint16_t*>(in), static_cast<uint16_t*>(out), ld_in, seq_len,
                  seq_pad, heads};
  const unsigned grid = (unsigned)(seq_pad / kTok);
  head_major_kernel<<<grid, 256, 0, as_stream(stream)>>>(a);
  return check_launch("head_major_kernel");
}
