// The RoPE rotation table of a render: H3RoPE.rotationTable(H3RoPE.angles(pos,
// inv_freq)) (Sources/H3Modules/H3Transformer.swift:62-78), built once per
// render by prepareRender (:271-273) and passed to every layer's
// AttentionLayer.callAsFunction(_:ropeTable:) (Sources/H3Modules/DiTBlock.swift:336).
// Per token s and pair p the 2x2 block [[c, -s], [s, c]] stored row-major as
// (c, -s, s, c): [seq_len, rot/2, 2, 2], bf16 for REFERENCE rounding (the
// reference's `.asType(computeDType)` table), fp32 for FP32 rounding.
//
// The entries come from make_rope_entry, the function the prologue kernel
// evaluates on the fly, so a layer that rotates with this table produces the
// prologue's bits.
#include "common.h"
#include "norm_rope.h"

namespace h3hip {

template <int kMode>
__global__ __launch_bounds__(256) void rope_table_kernel(const float* __restrict__ pos,
                                                         const int32_t* __restrict__ pair_axis,
                                                         const float* __restrict__ pair_inv,
                                                         int32_t half, int64_t n, void* table) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  const int64_t s = e / half;
  const int p = (int)(e - s * half);
  const int axis = min(max(pair_axis[p], 0), 2);
  const RopeEntry t = make_rope_entry<kMode>(pos[s * 3 + axis] * pair_inv[p]);
  if (kMode == H3HIP_ROUND_REFERENCE) {
    const u32x2 v = {cvt_pk(t.c, -t.s), cvt_pk(t.s, t.c)};
    reinterpret_cast<u32x2*>(table)[e] = v;
  } else {
    const f32x4 v = {t.c, -t.s, t.s, t.c};
    reinterpret_cast<f32x4*>(table)[e] = v;
  }
}

}  // namespace h3hip

using namespace h3hip;

extern "C" int h3hip_rope_table(const float* pos, const int32_t* pair_axis,
                                const float* pair_inv_freq, int32_t rot, int32_t rounding,
                                int32_t seq_len, void* table, void* stream) {
  H3_REQUIRE(pos && pair_axis && pair_inv_freq && table, H3HIP_EINVAL, "NULL argument");
  H3_REQUIRE(rot > 0 && rot % 2 == 0 && seq_len > 0, H3HIP_EINVAL, "bad rot %d / seq_len %d",
             rot, seq_len);
  H3_REQUIRE(rounding == H3HIP_ROUND_REFERENCE || rounding == H3HIP_ROUND_FP32, H3HIP_EINVAL,
             "unknown rounding mode %d", rounding);
  H3_REQUIRE((reinterpret_cast<uintptr_t>(table) & 15u) == 0, H3HIP_EINVAL,
             "table must be 16-byte aligned");
  const int32_t half = rot / 2;
  const int64_t n = (int64_t)seq_len * half;
  const dim3 grid((unsigned)((n + 255) / 256));
  hipStream_t st = as_stream(stream);
  if (rounding == H3HIP_ROUND_REFERENCE)
    rope_table_kernel<H3HIP_ROUND_REFERENCE><<<grid, 256, 0, st>>>(pos, pair_axis, pair_inv_freq,
                                                                  half, n, table);
  else
    rope_table_kernel<H3HIP_ROUND_FP32><<<grid, 256, 0, st>>>(pos, pair_axis, pair_inv_freq, half,
                                                             n, table);
  return check_launch("rope_table_kernel");
}
