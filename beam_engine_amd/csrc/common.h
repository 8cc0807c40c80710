// Shared device/host helpers for the beam_engine_amd HIP library (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <cstdio>
#include <string>

#include "../../include/beam_engine_amd.h"

namespace be {

// ---------------------------------------------------------------- errors
// Last error message of the calling host thread, returned by be_last_error().
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);

#define BE_HIP_CHECK(expr)                                                         \
  do {                                                                             \
    hipError_t _e = (expr);                                                        \
    if (_e != hipSuccess)                                                          \
      return ::be::fail(BE_ERR_HIP, "%s failed: %s (%s:%d)", #expr,              \
                        hipGetErrorString(_e), __FILE__, __LINE__);                \
  } while (0)

#define BE_REQUIRE(cond, ...)                                                      \
  do {                                                                             \
    if (!(cond)) return ::be::fail(BE_ERR_INVALID, __VA_ARGS__);                   \
  } while (0)

// ---------------------------------------------------------------- scalar types
// Storage types are plain 16-bit patterns; arithmetic is always fp32.
struct bf16_t { uint16_t v; };
struct f16_t { _Float16 v; };

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return __uint_as_float(((uint32_t)x.v) << 16); }
__device__ __forceinline__ float to_f32(f16_t x) { return (float)x.v; }

// Round-to-nearest-even float -> bf16 (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16_t from_f32<bf16_t>(float x) { return bf16_t{f32_to_bf16_bits(x)}; }
template <> __device__ __forceinline__ f16_t from_f32<f16_t>(float x) { return f16_t{(_Float16)x}; }

// ---------------------------------------------------------------- wave64 reductions
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

inline size_t dtype_size(int dt) { return dt == BE_F32 ? 4 : 2; }

}  // namespace be
