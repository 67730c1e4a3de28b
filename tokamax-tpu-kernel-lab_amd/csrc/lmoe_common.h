// Shared helpers for the gfx950 LatentMoE kernels: status codes, the
// thread-local error string, bf16 bit conversions and launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <initializer_list>

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

// A buffer of these (non-negative) dimensions has at most 2^48 elements --
// beyond any device's memory, so every entry point refuses larger sizes, and
// every index and byte offset computed from accepted sizes fits in int64.
// The product is formed with overflow checks; a zero dimension makes the
// buffer empty.
constexpr int64_t kMaxElems = int64_t{1} << 48;
inline bool extent_ok(std::initializer_list<int64_t> dims) {
  bool empty = false;
  for (int64_t d : dims) {
    if (d < 0) return false;
    empty = empty || d == 0;
  }
  if (empty) return true;
  int64_t n = 1;
  for (int64_t d : dims)
    if (__builtin_mul_overflow(n, d, &n) || n > kMaxElems) return false;
  return true;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---- bf16 ------------------------------------------------------------------
// bf16 values are carried as uint16_t bit patterns in memory.

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even f32 -> bf16 with the hardware conversion
// (v_cvt_pk_bf16_f32; NaN stays a quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
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

// ---- wave-wide (64-lane) primitives on DPP row shifts / row broadcasts ----
// Each is six dependent DPP steps (no LDS traffic); lanes whose DPP source
// falls outside the row take the operation's identity.

// Saturating add of non-negative 32-bit counts (cap <= 2^31).
__device__ __forceinline__ uint32_t sat_add(uint32_t a, uint32_t b, uint32_t cap) {
  const uint32_t s = a + b;
  return s < cap ? s : cap;
}

// Inclusive prefix sum over the wave, saturating at cap.
__device__ __forceinline__ uint32_t wave_scan_sat(uint32_t x, uint32_t cap) {
  x = sat_add(x, __builtin_amdgcn_update_dpp(0u, x, 0x111, 0xf, 0xf, false), cap);  // row_shr:1
  x = sat_add(x, __builtin_amdgcn_update_dpp(0u, x, 0x112, 0xf, 0xf, false), cap);  // row_shr:2
  x = sat_add(x, __builtin_amdgcn_update_dpp(0u, x, 0x114, 0xf, 0xf, false), cap);  // row_shr:4
  x = sat_add(x, __builtin_amdgcn_update_dpp(0u, x, 0x118, 0xf, 0xf, false), cap);  // row_shr:8
  x = sat_add(x, __builtin_amdgcn_update_dpp(0u, x, 0x142, 0xa, 0xf, false), cap);  // row_bcast:15
  x = sat_add(x, __builtin_amdgcn_update_dpp(0u, x, 0x143, 0xc, 0xf, false), cap);  // row_bcast:31
  return x;
}

// Wave-wide maximum / minimum of unsigned 32-bit values (uniform result):
// an inclusive max (min) scan whose last lane holds the answer.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0u, x, 0x111, 0xf, 0xf, false)));
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0u, x, 0x112, 0xf, 0xf, false)));
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0u, x, 0x114, 0xf, 0xf, false)));
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0u, x, 0x118, 0xf, 0xf, false)));
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0u, x, 0x142, 0xa, 0xf, false)));
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0u, x, 0x143, 0xc, 0xf, false)));
  return __builtin_amdgcn_readlane(x, 63);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
  constexpr uint32_t kId = 0xffffffffu;
  x = min(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(kId, x, 0x111, 0xf, 0xf, false)));
  x = min(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(kId, x, 0x112, 0xf, 0xf, false)));
  x = min(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(kId, x, 0x114, 0xf, 0xf, false)));
  x = min(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(kId, x, 0x118, 0xf, 0xf, false)));
  x = min(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(kId, x, 0x142, 0xa, 0xf, false)));
  x = min(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(kId, x, 0x143, 0xc, 0xf, false)));
  return __builtin_amdgcn_readlane(x, 63);
}

}  // namespace lmoe
