// MXFP8 activations x MXFP4 weights on gfx950's block-scaled MFMA
// (v_mfma_scale_f32_16x16x128_f8f6f4): the native scaled-MFMA path.
//
// Activations are quantised once to OCP MX E4M3 with one E8M0 scale per 32
// elements along K (quantize_mxfp8_kernel), so the GEMM reads 1 byte per
// activation instead of 2 and the weights enter the MFMA still packed: no
// per-element conversion in the main loop at all.
//
// Operand lane layouts of the 16x16x128 MFMA (established by one-hot probes on
// the device):
//   A (E4M3, 8 dwords): lane l holds row l%16; with g = l/16, bytes 0..15 are
//     k = 16g .. 16g+15 and bytes 16..31 are k = 64+16g .. 64+16g+15.
//   B (E2M1, 4 dwords): lane l holds column l%16, k = 32g .. 32g+31, low
//     nibble first.
//   Scales: lane (row or column, g) supplies the E8M0 byte of k-block g
//     (k = 32g .. 32g+31), for A and B alike.
//   D: lane l holds column l%16, rows 4*(l/16) .. +3.
//
// Pipeline: as the bf16 DMA kernel (gemm_dma.hip) -- an NS-deep LDS ring filled
// by global_load_lds, one vmcnt wait + s_barrier per 128-wide k step.  Per step
// and block: A codes BM x 128 B (rows XOR-swizzled in 16-byte chunks), A scales
// BM x 4 B (one dword DMA lane per row), B = the two 64-k records of the
// k-step-major MXFP4 layout (lmoe_mxfp4_tile), B scales 2 x BN x 2 B.

#include "dma_util.h"
#include "gemm_tile.h"

namespace lmoe {
namespace gemm {
namespace {

using namespace lmoe::dma;

typedef int v8i_t __attribute__((ext_vector_type(8)));

constexpr int kXK = 128;  // K per pipeline step (one scaled MFMA deep)

// ---- activation quantiser ---------------------------------------------------
// One thread per (row, 32-element block): shared exponent floor(log2(max|x|))
// - 8 over the block's finite values (E4M3 emax = 8), clamped to [-127, 127];
// elements x * 2^-e clamped to +-448 and converted round-to-nearest-even by
// the hardware (v_cvt_pk_fp8_f32, OCP E4M3); NaN -> 0x7F.  Scales go to the
// k-step-major (K/128, M4, 4) layout, M4 = roundup(M, 4), pad rows 0.
template <typename T>
__global__ __launch_bounds__(256) void quantize_mxfp8_kernel(const T* __restrict__ x, int64_t M, int64_t K,
                                                             int64_t M4, uint8_t* __restrict__ q,
                                                             uint8_t* __restrict__ scale_t) {
  const int64_t nb = K / 32;
  const int64_t total = M4 * nb;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t row = i / nb, kb = i % nb;
    uint32_t sbyte = 0;
    if (row < M) {
      float v[32];
      if constexpr (sizeof(T) == 2) {
        const uint4* src = reinterpret_cast<const uint4*>(x + row * K + kb * 32);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const uint4 w = src[c];
          const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            v[c * 8 + 2 * d] = __uint_as_float(u[d] << 16);
            v[c * 8 + 2 * d + 1] = __uint_as_float(u[d] & 0xffff0000u);
          }
        }
      } else {
        const float4* src = reinterpret_cast<const float4*>(x + row * K + kb * 32);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const float4 w = src[c];
          v[4 * c] = w.x;
          v[4 * c + 1] = w.y;
          v[4 * c + 2] = w.z;
          v[4 * c + 3] = w.w;
        }
      }
      float amax = 0.0f;
#pragma unroll
      for (int e = 0; e < 32; ++e) {
        const float a = __builtin_fabsf(v[e]);
        amax = a <= 3.402823466e38f ? __builtin_fmaxf(amax, a) : amax;  // finite values only
      }
      int ex = amax > 0.0f ? __builtin_amdgcn_frexp_expf(amax) - 1 - 8 : -127;
      ex = ex < -127 ? -127 : (ex > 127 ? 127 : ex);
      sbyte = static_cast<uint32_t>(ex + 127);
      uint32_t words[8];
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        float y[4];
#pragma unroll
        for (int b = 0; b < 4; ++b)
          y[b] = __builtin_amdgcn_fmed3f(__builtin_amdgcn_ldexpf(v[4 * w + b], -ex), -448.0f, 448.0f);
        int packed = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
        packed = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], packed, true);
        uint32_t u = static_cast<uint32_t>(packed);
#pragma unroll
        for (int b = 0; b < 4; ++b)
          if (v[4 * w + b] != v[4 * w + b]) u = (u & ~(0xffu << (8 * b))) | (0x7fu << (8 * b));
        words[w] = u;
      }
      uint4* dst = reinterpret_cast<uint4*>(q + row * K + kb * 32);
      dst[0] = uint4{words[0], words[1], words[2], words[3]};
      dst[1] = uint4{words[4], words[5], words[6], words[7]};
    }
    scale_t[((kb / 4) * M4 + row) * 4 + kb % 4] = static_cast<uint8_t>(sbyte);
  }
}

// ---- scaled grouped GEMM ------------------------------------------------------
template <int BM, int BN, int EPI, int NS>
struct XCfg {
  static constexpr int kWN = 4, kThreads = 256;
  static constexpr int kTM = BM / 16, kTN = BN / kWN / 16;
  static constexpr int kABytes = BM * kXK;      // E4M3 codes
  static constexpr int kASBytes = BM * 4;       // A scales: 4 k-blocks per row
  static constexpr int kBBytes = 2 * BN * 32;   // two 64-k records of packed E2M1
  static constexpr int kBSBytes = 2 * BN * 2;   // their scales
  static constexpr int kSlot = kABytes + kASBytes + kBBytes + kBSBytes;
  static constexpr int kAOps = BM * 8 / kThreads;
  static constexpr int kBOps = BN * 4 / kThreads;
  static constexpr int kOps = kAOps + kBOps;  // every wave, per step
  static constexpr int kOps0 = kOps + 2;      // wave 0 also fetches both scale sets
  static constexpr int kBSLanes = BN / 4;     // 16-byte lanes of the B-scale DMA
  static_assert(kAOps >= 1 && BM * 8 % kThreads == 0 && BM <= 64, "A DMA split (one scale lane per row)");
  static_assert(kBOps >= 1 && BN * 4 % kThreads == 0 && kBSLanes <= 64, "B DMA split");
  static_assert(kTM >= 1 && kTN >= 1, "wave tile");
  static_assert(EPI != kEpiSitu || kTN % 2 == 0, "SiTU pairs gate/up sub-tiles");
  static_assert(kSlot % 16 == 0, "slot alignment");
  static_assert((NS - 2) * kOps0 < 64, "vmcnt range");
  static constexpr int kLdsBlocks = 163840 / (NS * kSlot + 64);
  static constexpr int kWavesPerEu = kLdsBlocks < 1 ? 1 : (kLdsBlocks > 8 ? 8 : kLdsBlocks);
};

template <int BN, int TN, int EPI>
__device__ __forceinline__ int xlds_col(int wn, int j) {
  if constexpr (EPI == kEpiSitu) {
    constexpr int half = TN / 2;
    return j < half ? wn * half * 16 + j * 16 : BN / 2 + wn * half * 16 + (j - half) * 16;
  } else {
    return wn * TN * 16 + j * 16;
  }
}

template <int BN, int EPI>
__device__ __forceinline__ int64_t xrhs_col(int64_t nt, int c, int64_t N) {
  if constexpr (EPI == kEpiSitu) {
    const int64_t I = N / 2;
    int64_t j = nt * (BN / 2) + (c < BN / 2 ? c : c - BN / 2);
    j = j < I ? j : I - 1;
    return c < BN / 2 ? j : I + j;
  } else {
    const int64_t n = nt * BN + c;
    return n < N ? n : N - 1;
  }
}

template <int BM, int BN, int EPI, int NS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(XCfg<BM, BN, EPI, NS>::kWavesPerEu)))
void grouped_gemm_mx_kernel(Params p, int64_t n_tiles, int gm) {
  using C = XCfg<BM, BN, EPI, NS>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ TileInfo s_tile;
  __shared__ int64_t s_nt;

  const int tid = threadIdx.x;
  const int lane = tid % 64, wave = tid / 64;
  const int wn = wave;
  if (wave == 0) {
    const int64_t tm = total_m_tiles<BM>(p.group_sizes, p.G, p.M);
    int64_t nt = 0;
    const TileInfo ti = schedule_tile<BM>(p, n_tiles, gm, blockIdx.x, tm, nt);
    if (lane == 0) {
      s_tile = ti;
      s_nt = nt;
    }
  }
  __syncthreads();
  const TileInfo tile = s_tile;
  if (tile.group < 0) return;
  const int64_t nt = s_nt;
  const int64_t K = p.K, N = p.N, M4 = (p.M + 3) / 4 * 4;
  const int64_t g = tile.group;

  floatx4 acc[C::kTM][C::kTN];
#pragma unroll
  for (int i = 0; i < C::kTM; ++i)
#pragma unroll
    for (int j = 0; j < C::kTN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  if (!tile.zero) {
    const uint32_t smem0 = lds_offset(smem);
    const int64_t nk = K / kXK;
    const uint8_t* lhs = reinterpret_cast<const uint8_t*>(p.lhs);

    // A codes: LDS chunk q = tid + 256 v <- row q/8, logical chunk (q%8) ^ swz8(row)
    const uint8_t* a_base = uniform_ptr(lhs + tile.row0 * K);
    uint32_t a_off[C::kAOps];
#pragma unroll
    for (int v = 0; v < C::kAOps; ++v) {
      const int q = tid + C::kThreads * v;
      const int row = q / 8, kc = (q % 8) ^ swz8(row);
      const int rr = row < tile.rows ? row : 0;
      a_off[v] = static_cast<uint32_t>(rr * K + kc * 16);
    }
    // A scales: wave 0 lane i <- the 4 scale bytes of tile row i for this step
    const uint8_t* as_base = uniform_ptr(p.lhs_scale + tile.row0 * 4);
    const uint32_t as_off = static_cast<uint32_t>((lane < tile.rows ? lane : 0) * 4);
    const bool as_active = lane < BM;
    // B: chunk q = tid + 256 u of the slot's B region <- record h = q / (2 BN),
    // column c = (q % 2BN) / 2, chunk q % 2 (tiled records copied as they are)
    const int64_t rec = N * 32;  // one 64-k record of all columns
    const uint8_t* b_base = uniform_ptr(static_cast<const uint8_t*>(p.rhs) + g * (K / 64) * rec);
    uint32_t b_off[C::kBOps];
#pragma unroll
    for (int u = 0; u < C::kBOps; ++u) {
      const int q = tid + C::kThreads * u;
      const int h = q / (2 * BN), rem = q % (2 * BN);
      const int c = rem / 2, ch = rem % 2;
      b_off[u] = static_cast<uint32_t>(h * rec + xrhs_col<BN, EPI>(nt, c, N) * 32 + ch * 16);
    }
    // B scales: wave 0 lane sl <- record h = sl / (BN/8), 8 columns from c0
    const int64_t srec = N * 2;
    const uint8_t* bs_base = uniform_ptr(p.scale + g * (K / 64) * srec);
    uint32_t bs_off = 0;
    const bool bs_active = lane < C::kBSLanes;
    {
      const int sl = lane % C::kBSLanes;
      const int h = sl / (BN / 8), c0 = (sl % (BN / 8)) * 8;
      int64_t n0;
      if constexpr (EPI == kEpiSitu) {
        const int64_t I = N / 2;
        int64_t j0 = nt * (BN / 2) + (c0 % (BN / 2));
        j0 = j0 <= I - 8 ? j0 : I - 8;
        n0 = c0 < BN / 2 ? j0 : I + j0;
      } else {
        n0 = nt * BN + c0;
        n0 = n0 <= N - 8 ? n0 : N - 8;
      }
      bs_off = static_cast<uint32_t>(h * srec + n0 * 2);
    }
    const uint32_t lds_wave = __builtin_amdgcn_readfirstlane(smem0 + wave * 64 * 16);
    const uint32_t lds_slot0 = __builtin_amdgcn_readfirstlane(smem0);

    auto issue = [&](int64_t s, int slot) __attribute__((always_inline)) {
      if (s >= nk) return;
      const uint32_t base = lds_wave + slot * C::kSlot;
#pragma unroll
      for (int v = 0; v < C::kAOps; ++v) dma16s(a_off[v], a_base + s * kXK, base + v * C::kThreads * 16);
#pragma unroll
      for (int u = 0; u < C::kBOps; ++u)
        dma16s(b_off[u], b_base + s * 2 * rec, base + C::kABytes + C::kASBytes + u * C::kThreads * 16);
      if (wave == 0) {
        const uint32_t sb = lds_slot0 + slot * C::kSlot;
        if (as_active) dma4s(as_off, as_base + s * M4 * 4, sb + C::kABytes);
        if (bs_active) dma16s(bs_off, bs_base + s * 2 * srec, sb + C::kABytes + C::kASBytes + C::kBBytes);
      }
    };

    static_for<NS - 1>([&](auto sc) __attribute__((always_inline)) {
      constexpr int s = decltype(sc)::value;
      issue(s, s);
      return true;
    });

    const int r_lane = lane % 16, g_lane = lane / 16;
    int cur = 0;
    for (int64_t kt = 0; kt < nk; ++kt) {
      const int ahead = static_cast<int>(nk - 1 - kt < NS - 2 ? nk - 1 - kt : NS - 2);
      if (wave == 0)
        wait_step<NS, C::kOps0>(ahead);
      else
        wait_step<NS, C::kOps>(ahead);
      barrier();
      issue(kt + NS - 1, cur == 0 ? NS - 1 : cur - 1);
      const uint8_t* as = smem + cur * C::kSlot;
      const uint8_t* asc = as + C::kABytes;
      const uint8_t* bs = asc + C::kASBytes;
      const uint8_t* bsc = bs + C::kBBytes;
      v8i_t af[C::kTM];
      int sa[C::kTM];
#pragma unroll
      for (int i = 0; i < C::kTM; ++i) {
        const int r = i * 16 + r_lane;
        const uint4 lo = *reinterpret_cast<const uint4*>(as + r * kXK + ((g_lane ^ swz8(r)) * 16));
        const uint4 hi = *reinterpret_cast<const uint4*>(as + r * kXK + (((4 + g_lane) ^ swz8(r)) * 16));
        af[i] = v8i_t{static_cast<int>(lo.x), static_cast<int>(lo.y), static_cast<int>(lo.z), static_cast<int>(lo.w),
                      static_cast<int>(hi.x), static_cast<int>(hi.y), static_cast<int>(hi.z), static_cast<int>(hi.w)};
        sa[i] = asc[r * 4 + g_lane];
      }
#pragma unroll
      for (int j = 0; j < C::kTN; ++j) {
        const int c = xlds_col<BN, C::kTN, EPI>(wn, j) + r_lane;
        // logical dwords 4*(g%2) .. +3 of record h = g/2: physical
        // (mx_dword_pos) 2*(g%2), 4 + 2*(g%2), 2*(g%2) + 1, 4 + 2*(g%2) + 1
        const int h = g_lane / 2, hb = (g_lane % 2) * 8;
        const uint8_t* rec0 = bs + (h * BN + c) * 32;
        const uint2 lo = *reinterpret_cast<const uint2*>(rec0 + hb);
        const uint2 hi = *reinterpret_cast<const uint2*>(rec0 + 16 + hb);
        const v8i_t bf = v8i_t{static_cast<int>(lo.x), static_cast<int>(hi.x), static_cast<int>(lo.y),
                               static_cast<int>(hi.y), 0, 0, 0, 0};
        const int sb = bsc[(h * BN + c) * 2 + (g_lane % 2)];
#pragma unroll
        for (int i = 0; i < C::kTM; ++i)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[i], bf, acc[i][j], 0, 4, 0, sa[i], 0, sb);
      }
      cur = cur == NS - 1 ? 0 : cur + 1;
    }
  }

  // Epilogue: lane holds column (lane % 16) and rows 4*(lane/16) + r.
  if constexpr (EPI == kEpiSitu) {
    const int64_t I = N / 2;
    constexpr int half = C::kTN / 2;
    const SituConsts sc = situ_consts(p.beta, p.beta_lin);
#pragma unroll
    for (int i = 0; i < C::kTM; ++i) {
#pragma unroll
      for (int j = 0; j < half; ++j) {
        const int64_t col = nt * (BN / 2) + wn * half * 16 + j * 16 + (lane % 16);
        if (col >= I) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = i * 16 + 4 * (lane / 16) + r;
          if (row >= tile.rows) continue;
          float v = 0.0f;
          if (!tile.zero) {
            float gv = acc[i][j][r], uv = acc[i][j + half][r];
            if (p.round_before_act) {
              round_pair_bf16(gv, uv);
            }
            v = situ_epi(gv, uv, sc);
          }
          static_cast<uint16_t*>(p.out)[(tile.row0 + row) * I + col] = f32_to_bf16(v);
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < C::kTM; ++i) {
#pragma unroll
      for (int j = 0; j < C::kTN; ++j) {
        const int64_t col = nt * BN + wn * C::kTN * 16 + j * 16 + (lane % 16);
        if (col >= N) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = i * 16 + 4 * (lane / 16) + r;
          if (row >= tile.rows) continue;
          store_from_f32(p.out, (tile.row0 + row) * N + col, acc[i][j][r], p.out_dtype);
        }
      }
    }
  }
}

template <int BM, int BN, int EPI, int NS>
int launch_mx(const Params& p, hipStream_t st, const char* name) {
  using C = XCfg<BM, BN, EPI, NS>;
  const int64_t out_cols = EPI == kEpiSitu ? p.N / 2 : p.N;
  const int64_t cols_per_tile = EPI == kEpiSitu ? BN / 2 : BN;
  const int64_t ntiles = ceil_div(out_cols, cols_per_tile);
  const int64_t mtiles = ceil_div(p.M, BM) + p.G + 1;
  if (ntiles == 0 || p.M == 0) return LMOE_OK;
  int gm = p.G == 1 ? 4 : 1;
  int64_t blocks = kXcds * ceil_div(ceil_div(mtiles, gm), kXcds) * gm * ntiles;
  // grouped problems: n-tiles striped over the XCDs (each weight slice read
  // by one XCD), as in the bf16-dequant kernels
  if (p.G > 1 && ntiles % kXcds == 0) {
    gm = 0;
    blocks = mtiles * ntiles;
  }
  LMOE_CHECK_SUPPORTED(blocks < (1ll << 31), "%s: grid too large", name);
  LMOE_CHECK_SUPPORTED(p.N * p.K / 2 * 2 < (1ll << 32) && BM * p.K < (1ll << 32), "%s: group too large", name);
  const size_t lds = static_cast<size_t>(NS) * C::kSlot;
  static const hipError_t attr_rc =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&grouped_gemm_mx_kernel<BM, BN, EPI, NS>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  if (attr_rc != hipSuccess)
    return fail(LMOE_ERR_HIP, "%s: LDS size attribute (%zu bytes): %s", name, lds, hipGetErrorString(attr_rc));
  grouped_gemm_mx_kernel<BM, BN, EPI, NS><<<dim3(static_cast<unsigned>(blocks)), C::kThreads, lds, st>>>(p, ntiles, gm);
  LMOE_CHECK_LAUNCH(name);
  return LMOE_OK;
}

}  // namespace
}  // namespace gemm
}  // namespace lmoe

using namespace lmoe;
using namespace lmoe::gemm;

extern "C" int64_t lmoe_mxfp8_scale_bytes(int64_t M, int64_t K) {
  if (M < 0 || K <= 0 || K % 128 || !extent_ok({M + 3, K})) return -1;
  return (K / 128) * ((M + 3) / 4 * 4) * 4;
}

extern "C" int lmoe_quantize_mxfp8(const void* x, int x_dtype, int64_t M, int64_t K, uint8_t* q, uint8_t* scale_t,
                                   void* stream) {
  const char* name = "quantize_mxfp8";
  LMOE_CHECK_ARG(M >= 0 && K > 0, "%s: bad sizes M=%lld K=%lld", name, (long long)M, (long long)K);
  LMOE_CHECK_ARG(valid_dtype(x_dtype), "%s: bad dtype", name);
  LMOE_CHECK_SUPPORTED(K % 128 == 0, "%s: needs K %% 128 == 0 (K=%lld)", name, (long long)K);
  LMOE_CHECK_SUPPORTED(extent_ok({M + 3, K}), "%s: sizes beyond device memory", name);
  if (M == 0) return LMOE_OK;
  LMOE_CHECK_ARG(x && q && scale_t, "%s: null pointer", name);
  LMOE_CHECK_SUPPORTED(aligned(x, 16) && aligned(q, 16), "%s: x and q must be 16-byte aligned", name);
  const int64_t M4 = (M + 3) / 4 * 4;
  const int64_t total = M4 * (K / 32);
  const int64_t b = ceil_div(total, 256);
  const unsigned grid = static_cast<unsigned>(b < 65536 * 4 ? b : 65536 * 4);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (x_dtype == LMOE_BF16)
    quantize_mxfp8_kernel<uint16_t><<<grid, 256, 0, st>>>(static_cast<const uint16_t*>(x), M, K, M4, q, scale_t);
  else
    quantize_mxfp8_kernel<float><<<grid, 256, 0, st>>>(static_cast<const float*>(x), M, K, M4, q, scale_t);
  LMOE_CHECK_LAUNCH(name);
  return LMOE_OK;
}

extern "C" int lmoe_ragged_dot_mxfp8_mxfp4(const uint8_t* lhs_q, const uint8_t* lhs_scale_t,
                                           const uint8_t* w_packed_t, const uint8_t* w_scale_t,
                                           const int32_t* group_sizes, int64_t M, int64_t K, int64_t N, int64_t G,
                                           int zero_group, int epilogue, float beta, float beta_lin, void* out,
                                           int out_dtype, void* stream) {
  const char* name = "ragged_dot_mxfp8_mxfp4";
  LMOE_CHECK_ARG(M >= 0 && K > 0 && N > 0 && G > 0, "%s: bad sizes", name);
  LMOE_CHECK_SUPPORTED(M < (1ll << 31), "%s: M=%lld rows (the tile scan counts rows in 32 bits)", name, (long long)M);
  LMOE_CHECK_ARG(zero_group >= -1 && zero_group < G, "%s: bad zero_group %d", name, zero_group);
  LMOE_CHECK_ARG(epilogue == LMOE_EPI_NONE || epilogue == LMOE_EPI_SITU, "%s: bad epilogue", name);
  LMOE_CHECK_ARG(valid_dtype(out_dtype), "%s: bad out dtype", name);
  LMOE_CHECK_ARG(epilogue == LMOE_EPI_NONE || out_dtype == LMOE_BF16, "%s: SiTU output is bf16", name);
  LMOE_CHECK_SUPPORTED(K % 128 == 0, "%s: needs K %% 128 == 0 (K=%lld)", name, (long long)K);
  LMOE_CHECK_SUPPORTED(N % (epilogue == LMOE_EPI_SITU ? 16 : 8) == 0 && N >= 8, "%s: N=%lld", name, (long long)N);
  LMOE_CHECK_SUPPORTED(extent_ok({M, K}) && extent_ok({G, K, N}) && extent_ok({M, N}),
                       "%s: sizes beyond device memory", name);
  if (M == 0) return LMOE_OK;
  LMOE_CHECK_ARG(lhs_q && lhs_scale_t && w_packed_t && w_scale_t && group_sizes && out, "%s: null pointer", name);
  LMOE_CHECK_SUPPORTED(aligned(lhs_q, 16) && aligned(w_packed_t, 16) && aligned(w_scale_t, 16) &&
                           aligned(lhs_scale_t, 4),
                       "%s: alignment", name);
  Params p{reinterpret_cast<const uint16_t*>(lhs_q), w_packed_t, w_scale_t, group_sizes, M, K, N, G, zero_group,
           out, out_dtype, beta, beta_lin, 1, lhs_scale_t};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (epilogue == LMOE_EPI_SITU) return launch_mx<64, 128, kEpiSitu, 4>(p, st, name);
  return launch_mx<64, 128, kEpiNone, 4>(p, st, name);
}
