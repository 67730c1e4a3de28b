// Shared helpers for the gfx950 LatentMoE kernels: status codes, the
// thread-local error string, bf16 bit conversions and launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/lmoe.h"

namespace lmoe {

// ---- error reporting -------------------------------------------------------
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);

#define LMOE_CHECK_ARG(cond, ...)                       \
  do {                                                  \
    if (!(cond)) return ::lmoe::fail(LMOE_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define LMOE_CHECK_SUPPORTED(cond, ...)                 \
  do {                                                  \
    if (!(cond)) return ::lmoe::fail(LMOE_ERR_UNSUPPORTED, __VA_ARGS__); \
  } while (0)

#define LMOE_CHECK_LAUNCH(name)                                                   \
  do {                                                                            \
    hipError_t _e = hipGetLastError();                                            \
    if (_e != hipSuccess)                                                         \
      return ::lmoe::fail(LMOE_ERR_HIP, "%s: launch failed: %s", name, hipGetErrorString(_e)); \
  } while (0)

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---- bf16 ------------------------------------------------------------------
// bf16 values are carried as uint16_t bit patterns in memory.

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even f32 -> bf16 (NaN stays a quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Load one element of either dtype as f32.
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i, int dtype) {
  return dtype == LMOE_BF16 ? bf16_to_f32(static_cast<const uint16_t*>(p)[i])
                            : static_cast<const float*>(p)[i];
}

// Round f32 to the storage dtype and return the stored value as f32.
__device__ __forceinline__ float round_to(float f, int dtype) {
  return dtype == LMOE_BF16 ? round_bf16(f) : f;
}

__device__ __forceinline__ void store_from_f32(void* p, int64_t i, float v, int dtype) {
  if (dtype == LMOE_BF16)
    static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
  else
    static_cast<float*>(p)[i] = v;
}

inline int dtype_size(int dtype) { return dtype == LMOE_BF16 ? 2 : 4; }

inline bool valid_dtype(int dtype) { return dtype == LMOE_BF16 || dtype == LMOE_F32; }

}  // namespace lmoe
