// fp32 grouped GEMM (tokamax.ragged_dot on f32 operands with
// precision=HIGHEST, trg.py:150-163): full-precision FMA on the vector ALUs.
// Used for the fp32 golden bundles and the fp32 config; the bf16 path is the
// MFMA kernel in gemm_bf16.hip.  64x64 tiles, 16 x 16 threads, 4 x 4 outputs
// per thread, K staged through LDS 16 at a time.
#include "gemm_tile.h"

namespace lmoe {
namespace gemm {
namespace {

constexpr int kFT = 64;
constexpr int kFK = 16;

__global__ __launch_bounds__(256) void grouped_gemm_f32_kernel(const float* __restrict__ lhs,
                                                               const float* __restrict__ rhs,
                                                               int layout, Params p) {
  __shared__ float As[kFK][kFT + 1];
  __shared__ float Bs[kFK][kFT + 1];
  __shared__ TileInfo s_tile;
  const int tid = threadIdx.x;
  if (tid < 64) {
    TileInfo ti = locate_tile<kFT>(p.group_sizes, p.G, p.M, p.zero_group, blockIdx.y);
    if (tid == 0) s_tile = ti;
  }
  __syncthreads();
  const TileInfo tile = s_tile;
  if (tile.group < 0) return;
  const int64_t K = p.K, N = p.N, g = tile.group;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kFT;
  const int tx = tid % 16, ty = tid / 16;
  float acc[4][4] = {};
  if (!tile.zero) {
    for (int64_t k0 = 0; k0 < K; k0 += kFK) {
      for (int i = tid; i < kFT * kFK; i += 256) {
        const int r = i / kFK, kk = i % kFK;
        const int64_t k = k0 + kk;
        As[kk][r] = (r < tile.rows && k < K) ? lhs[(tile.row0 + r) * K + k] : 0.0f;
        const int c = i % kFT, kb = i / kFT;
        const int64_t kb2 = k0 + kb, n = n0 + c;
        float bv = 0.0f;
        if (kb2 < K && n < N)
          bv = layout == kGKN ? rhs[(g * K + kb2) * N + n] : rhs[(g * N + n) * K + kb2];
        Bs[kb][c] = bv;
      }
      __syncthreads();
#pragma unroll
      for (int kk = 0; kk < kFK; ++kk) {
        float a[4], b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
      }
      __syncthreads();
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = ty * 4 + i;
    if (r >= tile.rows) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + tx * 4 + j;
      if (n < N) store_from_f32(p.out, (tile.row0 + r) * N + n, acc[i][j], p.out_dtype);
    }
  }
}

}  // namespace

int run_f32(const Params& p, int layout, hipStream_t st, const char* name) {
  const int64_t ntiles = ceil_div(p.N, kFT);
  const int64_t mtiles = ceil_div(p.M, kFT) + p.G + 1;
  if (p.M == 0 || p.N == 0) return LMOE_OK;
  LMOE_CHECK_SUPPORTED(ntiles < (1ll << 31) && mtiles < 65536, "%s: grid too large", name);
  grouped_gemm_f32_kernel<<<dim3(static_cast<unsigned>(ntiles), static_cast<unsigned>(mtiles)), 256, 0,
                            st>>>(static_cast<const float*>(static_cast<const void*>(p.lhs)),
                                  static_cast<const float*>(p.rhs), layout, p);
  LMOE_CHECK_LAUNCH(name);
  return LMOE_OK;
}

}  // namespace gemm
}  // namespace lmoe
