// Shared internals of libch3hip: error reporting, bf16 helpers, vector types.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/ch3hip.h"

namespace h3hip {

// Thread-local last error; the ABI is re-entrant per thread.
void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

#define H3_HIP_CHECK(expr)                                                             \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess) {                                                            \
      ::h3hip::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, \
                         __LINE__);                                                    \
      return H3HIP_EHIP;                                                               \
    }                                                                                  \
  } while (0)

#define H3_REQUIRE(cond, code, ...)      \
  do {                                   \
    if (!(cond)) {                       \
      ::h3hip::set_error(__VA_ARGS__);   \
      return (code);                     \
    }                                    \
  } while (0)

// Checks the launch that was just enqueued.
int check_launch(const char* what);

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 bits, round to nearest even (inputs here are finite).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ float round_bf16(float f) {
  return __uint_as_float(f32_to_bf16_bits(f) << 16);
}
// Two floats to packed bf16 (lo in bits 0-15), round to nearest even: on gfx950
// one v_cvt_pk_bf16_f32, the same rounding as f32_to_bf16_bits for finite
// values (NaN stays NaN here; f32_to_bf16_bits can carry a NaN's low bits
// into the sign).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

}  // namespace h3hip
