// C-ABI entry points of the grouped GEMMs and the MXFP4 dequantisation.
#include "gemm_tile.h"

namespace lmoe {
namespace gemm {
int run_bf16(const Params& p, int layout, int epi, hipStream_t st, const char* name);
int run_f32(const Params& p, int layout, hipStream_t st, const char* name);
int run_dma(const Params& p, int layout, int epi, hipStream_t st, const char* name);
int run_dma_splitk(const Params& p, int layout, int epi, int64_t k_split, float* ws, hipStream_t st,
                   const char* name);
int tile_mxfp4(const uint8_t* packed, const uint8_t* scale, int64_t G, int64_t N, int64_t K, uint8_t* packed_out,
               uint8_t* scale_out, hipStream_t st);

namespace {

// Dequantise one packed byte per thread pair: thread handles 16 packed bytes
// (32 values) when the scale group is 32, else one byte.
__global__ __launch_bounds__(256) void mxfp4_dequant_kernel(const uint8_t* __restrict__ packed,
                                                            const uint8_t* __restrict__ scale,
                                                            int64_t rows, int64_t K, int64_t gs,
                                                            void* __restrict__ out, int odt) {
  const int64_t kh = K / 2;
  const int64_t total = rows * kh;
  const int64_t ng = K / gs;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t r = i / kh, j = i % kh;
    const uint32_t byte = packed[i];
    const int64_t k = 2 * j;
    const uint32_t s0 = scale[r * ng + k / gs];
    const uint32_t s1 = scale[r * ng + (k + 1) / gs];
    uint32_t b0, b1;
    if (s0 == s1) {
      const uint32_t both = dequant_byte(byte, s0);
      b0 = both & 0xffffu;
      b1 = both >> 16;
    } else {
      b0 = fp4_to_bf16_bits(byte & 15u, e8m0_to_float(s0));
      b1 = fp4_to_bf16_bits(byte >> 4, e8m0_to_float(s1));
    }
    if (odt == LMOE_BF16) {
      reinterpret_cast<uint32_t*>(out)[i] = b0 | (b1 << 16);
    } else {
      float* o = static_cast<float*>(out) + r * K + k;
      o[0] = __uint_as_float(b0 << 16);
      o[1] = __uint_as_float(b1 << 16);
    }
  }
}

int check_common(const void* lhs, const void* rhs, const int32_t* gs, int64_t M, int64_t K,
                 int64_t N, int64_t G, int zero_group, const void* out, const char* name) {
  LMOE_CHECK_ARG(M >= 0 && K > 0 && N > 0 && G > 0, "%s: bad sizes M=%lld K=%lld N=%lld G=%lld", name,
                 (long long)M, (long long)K, (long long)N, (long long)G);
  LMOE_CHECK_ARG(zero_group >= -1 && zero_group < G, "%s: bad zero_group %d", name, zero_group);
  LMOE_CHECK_SUPPORTED(extent_ok({M, K}) && extent_ok({G, K, N}) && extent_ok({M, N}),
                       "%s: sizes beyond device memory (M=%lld K=%lld N=%lld G=%lld)", name, (long long)M,
                       (long long)K, (long long)N, (long long)G);
  LMOE_CHECK_ARG(M == 0 || (lhs && rhs && gs && out), "%s: null pointer", name);
  LMOE_CHECK_SUPPORTED(M < (1ll << 31), "%s: M=%lld rows (the tile scan counts rows in 32 bits)", name, (long long)M);
  return LMOE_OK;
}

}  // namespace
}  // namespace gemm
}  // namespace lmoe

using namespace lmoe;
using namespace lmoe::gemm;

extern "C" int lmoe_ragged_dot(const void* lhs, int lhs_dtype, const void* rhs, int rhs_layout,
                               const int32_t* group_sizes, int64_t M, int64_t K, int64_t N,
                               int64_t G, int zero_group, void* out, int out_dtype, void* stream) {
  const char* name = "ragged_dot";
  int rc = check_common(lhs, rhs, group_sizes, M, K, N, G, zero_group, out, name);
  if (rc) return rc;
  LMOE_CHECK_ARG(valid_dtype(lhs_dtype) && valid_dtype(out_dtype), "%s: bad dtype", name);
  LMOE_CHECK_ARG(rhs_layout == LMOE_RHS_GKN || rhs_layout == LMOE_RHS_GNK, "%s: bad layout %d", name,
                 rhs_layout);
  Params p{static_cast<const uint16_t*>(lhs), rhs, nullptr, group_sizes, M, K, N, G, zero_group,
           out, out_dtype, 0.f, 0.f, 0};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (lhs_dtype == LMOE_F32) return run_f32(p, rhs_layout == LMOE_RHS_GKN ? kGKN : kGNK, st, name);
  LMOE_CHECK_SUPPORTED(K % 8 == 0 && N % 8 == 0, "%s: bf16 needs K %% 8 == 0 and N %% 8 == 0 (K=%lld N=%lld)",
                       name, (long long)K, (long long)N);
  LMOE_CHECK_SUPPORTED(aligned(lhs, 16) && aligned(rhs, 16), "%s: lhs/rhs must be 16-byte aligned", name);
  return run_bf16(p, rhs_layout == LMOE_RHS_GKN ? kGKN : kGNK, kEpiNone, st, name);
}

extern "C" int lmoe_ragged_dot_gateup_situ(const void* lhs, const void* rhs_gu, int rhs_layout,
                                           const int32_t* group_sizes, int64_t M, int64_t K,
                                           int64_t I, int64_t G, int zero_group, float beta,
                                           float beta_lin, int round_before_act, void* out,
                                           void* stream) {
  const char* name = "ragged_dot_gateup_situ";
  int rc = check_common(lhs, rhs_gu, group_sizes, M, K, 2 * I, G, zero_group, out, name);
  if (rc) return rc;
  LMOE_CHECK_ARG(rhs_layout == LMOE_RHS_GKN || rhs_layout == LMOE_RHS_GNK, "%s: bad layout %d", name,
                 rhs_layout);
  LMOE_CHECK_SUPPORTED(K % 8 == 0 && I % 8 == 0, "%s: needs K %% 8 == 0 and I %% 8 == 0", name);
  LMOE_CHECK_SUPPORTED(aligned(lhs, 16) && aligned(rhs_gu, 16), "%s: lhs/rhs must be 16-byte aligned", name);
  Params p{static_cast<const uint16_t*>(lhs), rhs_gu, nullptr, group_sizes, M, K, 2 * I, G, zero_group,
           out, LMOE_BF16, beta, beta_lin, round_before_act};
  return run_bf16(p, rhs_layout == LMOE_RHS_GKN ? kGKN : kGNK, kEpiSitu,
                  static_cast<hipStream_t>(stream), name);
}

extern "C" int lmoe_ragged_dot_fp8_scaled(const void* lhs, const uint8_t* rhs_q, const float* rhs_scale,
                                          int64_t block_size, const int32_t* group_sizes, int64_t M, int64_t K,
                                          int64_t N, int64_t G, int zero_group, int epilogue, float beta,
                                          float beta_lin, void* out, void* stream) {
  const char* name = "ragged_dot_fp8_scaled";
  int rc = check_common(lhs, rhs_q, group_sizes, M, K, N, G, zero_group, out, name);
  if (rc) return rc;
  LMOE_CHECK_ARG(rhs_scale || M == 0, "%s: null scale", name);
  LMOE_CHECK_ARG(epilogue == LMOE_EPI_NONE || epilogue == LMOE_EPI_SITU, "%s: bad epilogue", name);
  LMOE_CHECK_ARG(block_size > 0 && K % block_size == 0, "%s: block_size %lld must divide K=%lld", name,
                 (long long)block_size, (long long)K);
  LMOE_CHECK_SUPPORTED(block_size % 4 == 0, "%s: block_size %% 4 == 0 (got %lld)", name, (long long)block_size);
  LMOE_CHECK_SUPPORTED(K % 8 == 0 && N % (epilogue == LMOE_EPI_SITU ? 16 : 8) == 0,
                       "%s: needs K %% 8 == 0 and N %% %d == 0 (K=%lld N=%lld)", name,
                       epilogue == LMOE_EPI_SITU ? 16 : 8, (long long)K, (long long)N);
  LMOE_CHECK_SUPPORTED(aligned(lhs, 16) && aligned(rhs_q, 8) && aligned(rhs_scale, 16) && aligned(out, 4),
                       "%s: lhs 16-, rhs 8-, scale 16-byte aligned", name);
  Params p{static_cast<const uint16_t*>(lhs), rhs_q, nullptr, group_sizes, M, K, N, G, zero_group,
           out, LMOE_BF16, beta, beta_lin, 1};
  p.scale_f32 = rhs_scale;
  p.scale_block = block_size;
  return run_bf16(p, kFP8GKN, epilogue == LMOE_EPI_SITU ? kEpiSitu : kEpiNone, static_cast<hipStream_t>(stream),
                  name);
}

extern "C" int lmoe_ragged_dot_mxfp4(const void* lhs, const uint8_t* w_packed, const uint8_t* w_scale,
                                     const int32_t* group_sizes, int64_t M, int64_t K, int64_t N,
                                     int64_t G, int zero_group, int mode, int epilogue, float beta,
                                     float beta_lin, void* out, void* stream) {
  const char* name = "ragged_dot_mxfp4";
  const int skip_zero_rows = (mode & LMOE_MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS) != 0;
  mode &= ~LMOE_MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS;
  int rc = check_common(lhs, w_packed, group_sizes, M, K, N, G, zero_group, out, name);
  if (rc) return rc;
  LMOE_CHECK_ARG(w_scale || M == 0, "%s: null scale", name);
  LMOE_CHECK_ARG(epilogue == LMOE_EPI_NONE || epilogue == LMOE_EPI_SITU, "%s: bad epilogue", name);
  LMOE_CHECK_SUPPORTED(K % 64 == 0, "%s: needs K %% 64 == 0 (K=%lld)", name, (long long)K);
  LMOE_CHECK_SUPPORTED(N % (epilogue == LMOE_EPI_SITU ? 16 : 8) == 0, "%s: N=%lld", name, (long long)N);
  LMOE_CHECK_SUPPORTED(aligned(lhs, 16) && aligned(w_packed, 16), "%s: 16-byte alignment", name);
  Params p{static_cast<const uint16_t*>(lhs), w_packed, w_scale, group_sizes, M, K, N, G, zero_group,
           out, LMOE_BF16, beta, beta_lin, 1};
  p.skip_zero_rows = skip_zero_rows;
  const int epi = epilogue == LMOE_EPI_SITU ? kEpiSitu : kEpiNone;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (mode == LMOE_MXFP4_LDS_DEQUANT) return run_bf16(p, kMXFP4, epi, st, name);
  if (mode == LMOE_MXFP4_LDS_DEQUANT_TILED) {
    LMOE_CHECK_SUPPORTED(aligned(w_scale, 16), "%s: tiled scales must be 16-byte aligned", name);
    // w_packed (G, K/64, N, 32) and w_scale (G, K/64, N, 2) from lmoe_mxfp4_tile
    return M == 0 ? LMOE_OK : run_dma(p, kMXFP4, epi, st, name);
  }
  if (mode == LMOE_MXFP4_SCALED_MFMA)
    return fail(LMOE_ERR_UNSUPPORTED,
                "%s: the scaled-MFMA path takes MXFP8 activations: lmoe_quantize_mxfp8 + lmoe_ragged_dot_mxfp8_mxfp4",
                name);
  return fail(LMOE_ERR_INVALID, "%s: bad mode %d", name, mode);
}

extern "C" int lmoe_ragged_dot_mxfp4_rows(const void* lhs, int64_t lhs_rows, const int32_t* row_index,
                                          const uint8_t* w_packed, const uint8_t* w_scale,
                                          const int32_t* group_sizes, int64_t M, int64_t K, int64_t N, int64_t G,
                                          int zero_group, int mode, int epilogue, float beta, float beta_lin,
                                          void* out, void* stream) {
  const char* name = "ragged_dot_mxfp4_rows";
  const int skip_zero_rows = (mode & LMOE_MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS) != 0;
  mode &= ~LMOE_MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS;
  int rc = check_common(lhs, w_packed, group_sizes, M, K, N, G, zero_group, out, name);
  if (rc) return rc;
  LMOE_CHECK_ARG(w_scale || M == 0, "%s: null scale", name);
  LMOE_CHECK_ARG(row_index || M == 0, "%s: null row index", name);
  LMOE_CHECK_ARG(lhs_rows > 0 || M == 0, "%s: lhs_rows=%lld", name, (long long)lhs_rows);
  LMOE_CHECK_ARG(epilogue == LMOE_EPI_NONE || epilogue == LMOE_EPI_SITU, "%s: bad epilogue", name);
  LMOE_CHECK_SUPPORTED(mode == LMOE_MXFP4_LDS_DEQUANT_TILED, "%s: tiled weights only (mode %d)", name, mode);
  LMOE_CHECK_SUPPORTED(K % 64 == 0, "%s: needs K %% 64 == 0 (K=%lld)", name, (long long)K);
  LMOE_CHECK_SUPPORTED(N % (epilogue == LMOE_EPI_SITU ? 16 : 8) == 0, "%s: N=%lld", name, (long long)N);
  LMOE_CHECK_SUPPORTED(aligned(lhs, 16) && aligned(w_packed, 16) && aligned(w_scale, 16), "%s: 16-byte alignment",
                       name);
  // per-lane DMA offsets are 32-bit: any row of lhs
  LMOE_CHECK_SUPPORTED(lhs_rows <= 65536 && extent_ok({lhs_rows, K}) && lhs_rows * K * 2 < (1ll << 32),
                       "%s: lhs too large (%lld rows)", name, (long long)lhs_rows);
  if (M == 0) return LMOE_OK;
  Params p{static_cast<const uint16_t*>(lhs), w_packed, w_scale, group_sizes, M, K, N, G, zero_group,
           out, LMOE_BF16, beta, beta_lin, 1};
  p.skip_zero_rows = skip_zero_rows;
  p.a_index = row_index;
  p.a_rows = lhs_rows;
  return run_dma(p, kMXFP4, epilogue == LMOE_EPI_SITU ? kEpiSitu : kEpiNone, static_cast<hipStream_t>(stream), name);
}

extern "C" int lmoe_ragged_dot_mxfp4_splitk(const void* lhs, const uint8_t* w_packed, const uint8_t* w_scale,
                                            const int32_t* group_sizes, int64_t M, int64_t K, int64_t N, int64_t G,
                                            int zero_group, int64_t k_split, float* workspace,
                                            int64_t workspace_bytes, int epilogue, float beta, float beta_lin,
                                            void* out, void* stream) {
  const char* name = "ragged_dot_mxfp4_splitk";
  int rc = check_common(lhs, w_packed, group_sizes, M, K, N, G, zero_group, out, name);
  if (rc) return rc;
  LMOE_CHECK_ARG(w_scale || M == 0, "%s: null scale", name);
  LMOE_CHECK_ARG(epilogue == LMOE_EPI_NONE || epilogue == LMOE_EPI_SITU, "%s: bad epilogue", name);
  LMOE_CHECK_SUPPORTED(K % 64 == 0, "%s: needs K %% 64 == 0 (K=%lld)", name, (long long)K);
  LMOE_CHECK_SUPPORTED(N % (epilogue == LMOE_EPI_SITU ? 16 : 8) == 0, "%s: N=%lld", name, (long long)N);
  LMOE_CHECK_ARG(k_split >= 1 && k_split <= K / 64, "%s: k_split=%lld outside [1, K/64=%lld]", name,
                 (long long)k_split, (long long)(K / 64));
  if (M == 0) return LMOE_OK;
  LMOE_CHECK_SUPPORTED(aligned(lhs, 16) && aligned(w_packed, 16) && aligned(w_scale, 16),
                       "%s: 16-byte alignment", name);
  // no empty K range: k_split ranges of ceil(steps / k_split) steps
  const int64_t steps = K / 64, per = ceil_div(steps, k_split), splits = ceil_div(steps, per);
  Params p{static_cast<const uint16_t*>(lhs), w_packed, w_scale, group_sizes, M, K, N, G, zero_group,
           out, LMOE_BF16, beta, beta_lin, 1};
  const int epi = epilogue == LMOE_EPI_SITU ? kEpiSitu : kEpiNone;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (splits == 1) return run_dma(p, kMXFP4, epi, st, name);
  LMOE_CHECK_ARG(workspace && aligned(workspace, 16), "%s: workspace must be non-null and 16-byte aligned", name);
  LMOE_CHECK_SUPPORTED(extent_ok({splits, M, N}), "%s: partial planes beyond device memory", name);
  LMOE_CHECK_ARG(workspace_bytes >= splits * M * N * 4, "%s: workspace %lld bytes < %lld (k_split * M * N * 4)",
                 name, (long long)workspace_bytes, (long long)(splits * M * N * 4));
  return run_dma_splitk(p, kMXFP4, epi, splits, workspace, st, name);
}

extern "C" int lmoe_mxfp4_dequant(const uint8_t* packed, const uint8_t* scale, int64_t batch,
                                  int64_t N, int64_t K, int64_t group_size, void* out, int out_dtype,
                                  void* stream) {
  const char* name = "mxfp4_dequant";
  LMOE_CHECK_ARG(batch >= 0 && N >= 0 && K > 0 && K % 2 == 0 && group_size > 0 && K % group_size == 0,
                 "%s: bad sizes N=%lld K=%lld gs=%lld", name, (long long)N, (long long)K,
                 (long long)group_size);
  LMOE_CHECK_ARG(valid_dtype(out_dtype), "%s: bad dtype", name);
  LMOE_CHECK_SUPPORTED(extent_ok({batch, N, K}), "%s: sizes beyond device memory", name);
  const int64_t rows = batch * N;
  if (rows == 0) return LMOE_OK;
  LMOE_CHECK_ARG(packed && scale && out, "%s: null pointer", name);
  LMOE_CHECK_SUPPORTED(out_dtype == LMOE_F32 || aligned(out, 4), "%s: out alignment", name);
  const int64_t total = rows * (K / 2);
  const int64_t blocks64 = ceil_div(total, 256);
  const unsigned blocks = static_cast<unsigned>(blocks64 < 65536 * 4 ? blocks64 : 65536 * 4);
  mxfp4_dequant_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(packed, scale, rows, K,
                                                                             group_size, out, out_dtype);
  LMOE_CHECK_LAUNCH(name);
  return LMOE_OK;
}

extern "C" int lmoe_mxfp4_tile(const uint8_t* packed, const uint8_t* scale, int64_t G, int64_t N, int64_t K,
                               uint8_t* packed_out, uint8_t* scale_out, void* stream) {
  const char* name = "mxfp4_tile";
  LMOE_CHECK_ARG(G >= 0 && N >= 0 && K > 0, "%s: bad sizes", name);
  LMOE_CHECK_SUPPORTED(K % 64 == 0, "%s: needs K %% 64 == 0 (K=%lld)", name, (long long)K);
  LMOE_CHECK_SUPPORTED(extent_ok({G, N, K}), "%s: sizes beyond device memory", name);
  if (G * N == 0) return LMOE_OK;
  LMOE_CHECK_ARG(packed && scale && packed_out && scale_out, "%s: null pointer", name);
  LMOE_CHECK_SUPPORTED(aligned(packed, 16) && aligned(packed_out, 16), "%s: packed buffers must be 16-byte aligned",
                       name);
  return tile_mxfp4(packed, scale, G, N, K, packed_out, scale_out, static_cast<hipStream_t>(stream));
}
