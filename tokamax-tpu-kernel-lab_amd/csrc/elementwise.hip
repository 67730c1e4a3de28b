// Adjacent elementwise stages of the layer: RMSNorm (ref.py:286-293), SiTU-GLU
// on separate gate/up tensors (ref.py:296-310) and the residual add
// (ref.py:435).  All in f32 internally with explicit rounding to the storage
// dtype, no FMA contraction (the reference rounds each op).
#include "gemm_tile.h"

namespace lmoe {
namespace {

// One block per row; block-wide f32 sum of squares.
__global__ __launch_bounds__(256) void rms_norm_kernel(const void* __restrict__ x,
                                                       const void* __restrict__ scale, int64_t n,
                                                       float eps, int dt, void* __restrict__ out) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  float ss = 0.0f;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    const float v = load_as_f32(x, row * n + i, dt);
    ss = __fadd_rn(ss, __fmul_rn(v, v));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss = __fadd_rn(ss, __shfl_xor(ss, off, 64));
  if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = ss;
  __syncthreads();
  const float tot = __fadd_rn(__fadd_rn(red[0], red[1]), __fadd_rn(red[2], red[3]));
  const float var = __fdiv_rn(tot, static_cast<float>(n));
  const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(var, eps)));
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    const float v = load_as_f32(x, row * n + i, dt);
    const float normed = round_to(__fmul_rn(v, inv), dt);
    store_from_f32(out, row * n + i, __fmul_rn(normed, load_as_f32(scale, i, dt)), dt);
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
  LMOE_CHECK_SUPPORTED(rows < (1ll << 31), "rms_norm: too many rows");
  if (rows == 0) return LMOE_OK;
  rms_norm_kernel<<<static_cast<unsigned>(rows), 256, 0, static_cast<hipStream_t>(stream)>>>(
      x, scale, n, eps, dtype, out);
  LMOE_CHECK_LAUNCH("rms_norm");
  return LMOE_OK;
}

extern "C" int lmoe_situ_and_mul(const void* gate, const void* up, int64_t count, float beta,
                                 float beta_lin, int dtype, void* out, void* stream) {
  LMOE_CHECK_ARG(count >= 0 && valid_dtype(dtype), "situ_and_mul: bad arguments");
  if (count == 0) return LMOE_OK;
  situ_kernel<<<grid_for(count), 256, 0, static_cast<hipStream_t>(stream)>>>(gate, up, count, beta,
                                                                            beta_lin, dtype, out);
  LMOE_CHECK_LAUNCH("situ_and_mul");
  return LMOE_OK;
}

extern "C" int lmoe_add(const void* a, const void* b, int64_t count, int dtype, void* out, void* stream) {
  LMOE_CHECK_ARG(count >= 0 && valid_dtype(dtype), "add: bad arguments");
  if (count == 0) return LMOE_OK;
  add_kernel<<<grid_for(count), 256, 0, static_cast<hipStream_t>(stream)>>>(a, b, count, dtype, out);
  LMOE_CHECK_LAUNCH("add");
  return LMOE_OK;
}
