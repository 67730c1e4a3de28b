// Adjacent elementwise stages of the layer: RMSNorm (ref.py:286-293), SiTU-GLU
// on separate gate/up tensors (ref.py:296-310) and the residual add
// (ref.py:435).  All in f32 internally with explicit rounding to the storage
// dtype, no FMA contraction (the reference rounds each op).
#include "gemm_tile.h"

namespace lmoe {
namespace {

// One 64-lane wave per row (4 rows per block): each lane reads VEC
// consecutive elements per pass (16-byte loads for bf16 / f32 with VEC 8 / 4),
// f32 sum of squares per lane, then a wave tree sum.
template <int VEC>
__device__ __forceinline__ void load_row_vec(const void* p, int64_t i, int dt, float* v) {
  if constexpr (VEC == 1) {
    v[0] = load_as_f32(p, i, dt);
  } else if (dt == LMOE_BF16) {
    const uint4 raw = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int j = 0; j < VEC / 2; ++j) {
      v[2 * j] = __uint_as_float(w[j] << 16);
      v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int j = 0; j < VEC; j += 4) {
      const float4 f = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i + j);
      v[j] = f.x;
      v[j + 1] = f.y;
      v[j + 2] = f.z;
      v[j + 3] = f.w;
    }
  }
}

template <int VEC>
__global__ __launch_bounds__(256) void rms_norm_kernel(const void* __restrict__ x,
                                                       const void* __restrict__ scale, int64_t rows,
                                                       int64_t n, float eps, int dt, void* __restrict__ out) {
  const int lane = threadIdx.x % 64;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / 64;
  if (row >= rows) return;
  float ss = 0.0f;
  for (int64_t c0 = static_cast<int64_t>(lane) * VEC; c0 < n; c0 += 64 * VEC) {
    float v[VEC];
    load_row_vec<VEC>(x, row * n + c0, dt, v);
#pragma unroll
    for (int j = 0; j < VEC; ++j) ss = __fadd_rn(ss, __fmul_rn(v[j], v[j]));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss = __fadd_rn(ss, __shfl_xor(ss, off, 64));
  const float var = __fdiv_rn(ss, static_cast<float>(n));
  const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(var, eps)));
  for (int64_t c0 = static_cast<int64_t>(lane) * VEC; c0 < n; c0 += 64 * VEC) {
    float v[VEC], sc[VEC];
    load_row_vec<VEC>(x, row * n + c0, dt, v);
    load_row_vec<VEC>(scale, c0, dt, sc);
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float normed = round_to(__fmul_rn(v[j], inv), dt);
      store_from_f32(out, row * n + c0 + j, __fmul_rn(normed, sc[j]), dt);
    }
  }
}

__global__ __launch_bounds__(256) void situ_kernel(const void* __restrict__ g, const void* __restrict__ u,
                                                   int64_t count, float beta, float beta_lin, int dt,
                                                   void* __restrict__ out) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    store_from_f32(out, i, gemm::situ(load_as_f32(g, i, dt), load_as_f32(u, i, dt), beta, beta_lin), dt);
}

__global__ __launch_bounds__(256) void add_kernel(const void* __restrict__ a, const void* __restrict__ b,
                                                  int64_t count, int dt, void* __restrict__ out) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    store_from_f32(out, i, __fadd_rn(load_as_f32(a, i, dt), load_as_f32(b, i, dt)), dt);
}

// out (rows, cols) contiguous = cast(x) with x rows ld elements apart.  Fast
// path f32 -> bf16 with 4 elements per thread (16-byte load, 8-byte store).
__global__ __launch_bounds__(256) void cast_rows_f32_bf16x4(const float* __restrict__ x, int64_t rows,
                                                            int64_t cols, int64_t ld, uint16_t* __restrict__ out) {
  const int64_t q = cols / 4;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < rows * q;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / q, c = (i % q) * 4;
    const float4 v = *reinterpret_cast<const float4*>(x + r * ld + c);
    *reinterpret_cast<uint2*>(out + r * cols + c) = uint2{gemm::pack_bf16x2(v.x, v.y), gemm::pack_bf16x2(v.z, v.w)};
  }
}

__global__ __launch_bounds__(256) void cast_rows_kernel(const void* __restrict__ x, int xdt, int64_t rows,
                                                        int64_t cols, int64_t ld, void* __restrict__ out, int odt) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < rows * cols;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / cols, c = i % cols;
    store_from_f32(out, i, load_as_f32(x, r * ld + c, xdt), odt);
  }
}

unsigned grid_for(int64_t count) {
  const int64_t b = ceil_div(count, 256);
  return static_cast<unsigned>(b < 262144 ? (b > 0 ? b : 1) : 262144);
}

}  // namespace
}  // namespace lmoe

using namespace lmoe;

extern "C" int lmoe_rms_norm(const void* x, const void* scale, int64_t rows, int64_t n, float eps,
                             int dtype, void* out, void* stream) {
  LMOE_CHECK_ARG(rows >= 0 && n > 0 && valid_dtype(dtype), "rms_norm: bad arguments");
  LMOE_CHECK_SUPPORTED(rows < (1ll << 33) && extent_ok({rows, n}), "rms_norm: too many rows");
  if (rows == 0) return LMOE_OK;
  LMOE_CHECK_ARG(x && scale && out, "rms_norm: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned blocks = static_cast<unsigned>(ceil_div(rows, 4));
  const bool a16 = aligned(x, 16) && aligned(scale, 16);
  if (dtype == LMOE_BF16 && n % 8 == 0 && a16)
    rms_norm_kernel<8><<<blocks, 256, 0, st>>>(x, scale, rows, n, eps, dtype, out);
  else if (dtype == LMOE_F32 && n % 4 == 0 && a16)
    rms_norm_kernel<4><<<blocks, 256, 0, st>>>(x, scale, rows, n, eps, dtype, out);
  else
    rms_norm_kernel<1><<<blocks, 256, 0, st>>>(x, scale, rows, n, eps, dtype, out);
  LMOE_CHECK_LAUNCH("rms_norm");
  return LMOE_OK;
}

extern "C" int lmoe_situ_and_mul(const void* gate, const void* up, int64_t count, float beta,
                                 float beta_lin, int dtype, void* out, void* stream) {
  LMOE_CHECK_ARG(count >= 0 && valid_dtype(dtype), "situ_and_mul: bad arguments");
  LMOE_CHECK_SUPPORTED(extent_ok({count}), "situ_and_mul: sizes beyond device memory");
  if (count == 0) return LMOE_OK;
  LMOE_CHECK_ARG(gate && up && out, "situ_and_mul: null pointer");
  situ_kernel<<<grid_for(count), 256, 0, static_cast<hipStream_t>(stream)>>>(gate, up, count, beta,
                                                                            beta_lin, dtype, out);
  LMOE_CHECK_LAUNCH("situ_and_mul");
  return LMOE_OK;
}

extern "C" int lmoe_add(const void* a, const void* b, int64_t count, int dtype, void* out, void* stream) {
  LMOE_CHECK_ARG(count >= 0 && valid_dtype(dtype), "add: bad arguments");
  LMOE_CHECK_SUPPORTED(extent_ok({count}), "add: sizes beyond device memory");
  if (count == 0) return LMOE_OK;
  LMOE_CHECK_ARG(a && b && out, "add: null pointer");
  add_kernel<<<grid_for(count), 256, 0, static_cast<hipStream_t>(stream)>>>(a, b, count, dtype, out);
  LMOE_CHECK_LAUNCH("add");
  return LMOE_OK;
}

extern "C" int lmoe_cast_rows(const void* x, int x_dtype, int64_t rows, int64_t cols, int64_t ld, void* out,
                              int out_dtype, void* stream) {
  LMOE_CHECK_ARG(rows >= 0 && cols >= 0 && ld >= cols && valid_dtype(x_dtype) && valid_dtype(out_dtype),
                 "cast_rows: bad arguments");
  LMOE_CHECK_SUPPORTED(extent_ok({rows, ld}), "cast_rows: sizes beyond device memory");
  if (rows == 0 || cols == 0) return LMOE_OK;
  LMOE_CHECK_ARG(x && out, "cast_rows: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (x_dtype == LMOE_F32 && out_dtype == LMOE_BF16 && cols % 4 == 0 && ld % 4 == 0 && aligned(x, 16) &&
      aligned(out, 8)) {
    cast_rows_f32_bf16x4<<<grid_for(rows * cols / 4), 256, 0, st>>>(static_cast<const float*>(x), rows, cols, ld,
                                                                      static_cast<uint16_t*>(out));
  } else {
    cast_rows_kernel<<<grid_for(rows * cols), 256, 0, st>>>(x, x_dtype, rows, cols, ld, out, out_dtype);
  }
  LMOE_CHECK_LAUNCH("cast_rows");
  return LMOE_OK;
}

namespace lmoe {
namespace {

// Batched transpose out[g][c][r] = in[g][r][c] through a 64x64 LDS tile
// (one padding element per row: the column reads hit distinct banks).
template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(const T* __restrict__ in, int64_t R, int64_t C,
                                                        T* __restrict__ out) {
  __shared__ T tile[64][65];
  const int64_t g = blockIdx.z;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64, c0 = static_cast<int64_t>(blockIdx.x) * 64;
  const T* src = in + g * R * C;
  T* dst = out + g * R * C;
  const int tx = threadIdx.x % 64, ty = threadIdx.x / 64;
  for (int i = ty; i < 64; i += 4) {
    const int64_t r = r0 + i, c = c0 + tx;
    if (r < R && c < C) tile[i][tx] = src[r * C + c];
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int64_t c = c0 + i, r = r0 + tx;
    if (r < R && c < C) dst[c * R + r] = tile[tx][i];
  }
}

// The same for 2-byte elements with R % 4 == 0 and C % 4 == 0: 8-byte loads
// of 4 consecutive columns and 8-byte stores of 4 consecutive rows.
__global__ __launch_bounds__(256) void transpose16x4_kernel(const uint16_t* __restrict__ in, int64_t R, int64_t C,
                                                            uint16_t* __restrict__ out) {
  __shared__ uint16_t tile[64][68];
  const int64_t g = blockIdx.z;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64, c0 = static_cast<int64_t>(blockIdx.x) * 64;
  const uint16_t* src = in + g * R * C;
  uint16_t* dst = out + g * R * C;
  const int tq = threadIdx.x % 16, ty = threadIdx.x / 16;
  for (int i = ty; i < 64; i += 16) {
    const int64_t r = r0 + i, c = c0 + 4 * tq;
    if (r < R && c < C) {
      const uint2 v = *reinterpret_cast<const uint2*>(src + r * C + c);
      tile[i][4 * tq] = static_cast<uint16_t>(v.x);
      tile[i][4 * tq + 1] = static_cast<uint16_t>(v.x >> 16);
      tile[i][4 * tq + 2] = static_cast<uint16_t>(v.y);
      tile[i][4 * tq + 3] = static_cast<uint16_t>(v.y >> 16);
    }
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 16) {
    const int64_t c = c0 + i, r = r0 + 4 * tq;
    if (c < C && r < R) {
      const uint32_t lo = tile[4 * tq][i] | (static_cast<uint32_t>(tile[4 * tq + 1][i]) << 16);
      const uint32_t hi = tile[4 * tq + 2][i] | (static_cast<uint32_t>(tile[4 * tq + 3][i]) << 16);
      *reinterpret_cast<uint2*>(dst + c * R + r) = uint2{lo, hi};
    }
  }
}

}  // namespace
}  // namespace lmoe

extern "C" int lmoe_transpose(const void* in, int64_t G, int64_t R, int64_t C, int elem_bytes, void* out,
                              void* stream) {
  using namespace lmoe;
  LMOE_CHECK_ARG(G >= 0 && R >= 0 && C >= 0, "transpose: bad sizes");
  LMOE_CHECK_ARG(elem_bytes == 2 || elem_bytes == 4, "transpose: elem_bytes %d", elem_bytes);
  LMOE_CHECK_SUPPORTED(G < 65536, "transpose: G=%lld batches", (long long)G);
  LMOE_CHECK_SUPPORTED(extent_ok({G, R, C}) && ceil_div(R, 64) < 65536 && ceil_div(C, 64) < (1ll << 31),
                       "transpose: sizes beyond device memory or the grid (R=%lld C=%lld)", (long long)R, (long long)C);
  if (G * R * C == 0) return LMOE_OK;
  LMOE_CHECK_ARG(in && out && in != out, "transpose: null or aliased pointer");
  const dim3 grid(static_cast<unsigned>(ceil_div(C, 64)), static_cast<unsigned>(ceil_div(R, 64)),
                  static_cast<unsigned>(G));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (elem_bytes == 2 && R % 4 == 0 && C % 4 == 0 && aligned(in, 8) && aligned(out, 8))
    transpose16x4_kernel<<<grid, 256, 0, st>>>(static_cast<const uint16_t*>(in), R, C, static_cast<uint16_t*>(out));
  else if (elem_bytes == 2)
    transpose_kernel<uint16_t><<<grid, 256, 0, st>>>(static_cast<const uint16_t*>(in), R, C, static_cast<uint16_t*>(out));
  else
    transpose_kernel<uint32_t><<<grid, 256, 0, st>>>(static_cast<const uint32_t*>(in), R, C, static_cast<uint32_t*>(out));
  LMOE_CHECK_LAUNCH("transpose");
  return LMOE_OK;
}
