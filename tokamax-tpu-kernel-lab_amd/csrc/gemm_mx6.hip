// MXFP6 activations x MXFP4 weights on gfx950's block-scaled MFMA at the
// FP4/FP6 rate (v_mfma_scale_f32_32x32x64_f8f6f4 with A in FP6 E2M3 and B in
// FP4 E2M1).
//
// The 32x32x64 scaled MFMA issues at the FP4/FP6 rate only when both operands
// are 6 bits or narrower: a probe on the device measured 34.7 cycles per
// instruction per wave for FP6 x FP4 and FP4 x FP4 against 64.7 for FP8 x FP4
// and FP8 x FP8 (the 16x16x128 form of the MXFP8 path runs at the FP8 rate
// for every format).  Activations are therefore quantised once to OCP MX FP6
// E2M3 (3 mantissa bits, as E4M3, with 2 exponent bits under the block scale)
// with one E8M0 scale per 32 elements along K.
//
// Operand lane layouts (random-operand probes on the device, every output
// element reproduced exactly):
//   A (E2M3, 6 dwords used): lane l holds row l%32 and the 32 values
//     k = 32*(l/32) .. +31 of the 64-deep step, value j at bits 6j .. 6j+5;
//   B (E2M1, 4 dwords used): lane l holds column l%32, k = 32*(l/32) .. +31,
//     value j at bits 4j .. 4j+3 (low nibble first);
//   scales: each lane supplies the E8M0 byte of its own 32-value k-block;
//   D: lane l holds column l%32, rows 8*(e/4) + 4*(l/32) + e%4 for e < 16.
//
// Packed activations: (M, K*3/4) bytes, 24 bytes per 32-element block (the
// layout of the A operand, so one lane's values are one contiguous run).
// Scales use the MXFP8 path's k-step-major (K/128, roundup(M, 4), 4) layout.
//
// Pipeline: one block per 128x128 tile, 4 waves as 2 x 2 (64x64 each, 2 x 2
// MFMA sub-tiles), an NS-deep LDS ring filled by global_load_lds with one
// vmcnt wait + s_barrier per 128-deep k step.  Measured at config 4 (K = 7168,
// N = 2048): 72.5 us at M = 4096 (1.66 PFLOP/s) and 130 us at M = 8192;
// 256x128 tiles of 4 x 2 waves 78.5 / 148 us; 256x256 tiles 107 / 115 us
// (2.09 PFLOP/s at M = 8192, too few tiles below).  One tile's K loop takes
// about 0.86 us per 128-deep step even when only 16 tiles run (M = 128), and
// deeper rings (5 or 6 slots, one block per CU; 4 slots at 256x128) do not
// shorten it: the per-block stream of DMA issues and barriers (about 25 GB/s
// per block, as in the bf16 kernels) sets the pace, not the 8 MFMAs per wave
// of a step.  A rows are 96 bytes in LDS with
// their 16-byte chunks rotated by one position for rows 8..15 and 24..31 of
// every 32: the three 8-byte reads that fetch a lane's 24-byte run then fall
// on all 64 banks twice (the minimum for 512 bytes).

#include "dma_util.h"
#include "gemm_tile.h"

namespace lmoe {
namespace gemm {
namespace {

using namespace lmoe::dma;

typedef int v8i_t __attribute__((ext_vector_type(8)));

constexpr int kXK6 = 128;         // K per pipeline step
constexpr int kARow6 = kXK6 * 3 / 4;  // packed A bytes per row per step (96)

// ---- activation quantiser ---------------------------------------------------
// E2M3 code of a value already scaled by the block exponent: magnitude
// clamped to 7.5, rounded to nearest even on the grid (1/8 below 2, 1/4 in
// [2, 4), 1/2 in [4, 7.5]); the code is 8 * binade + the mantissa count, so a
// rounding carry moves into the next binade by itself.  NaN -> +-0.
__device__ __forceinline__ uint32_t e2m3_code(float y) {
  const uint32_t sign = (__float_as_uint(y) >> 31) << 5;
  if (y != y) return sign;
  const float a = __builtin_fminf(__builtin_fabsf(y), 7.5f);
  uint32_t c;
  if (a < 2.0f)
    c = static_cast<uint32_t>(__builtin_rintf(a * 8.0f));
  else if (a < 4.0f)
    c = 8u + static_cast<uint32_t>(__builtin_rintf(a * 4.0f));
  else
    c = 16u + static_cast<uint32_t>(__builtin_rintf(a * 2.0f));
  return c | sign;
}

// One thread per (row, 32-element block): shared exponent floor(log2(max|x|))
// - 2 over the block's finite values (E2M3 emax = 2), clamped to [-127, 127];
// the 32 codes packed into 24 bytes.
template <typename T>
__global__ __launch_bounds__(256) void quantize_mxfp6_kernel(const T* __restrict__ x, int64_t M, int64_t K,
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
      int ex = amax > 0.0f ? __builtin_amdgcn_frexp_expf(amax) - 1 - 2 : -127;
      ex = ex < -127 ? -127 : (ex > 127 ? 127 : ex);
      sbyte = static_cast<uint32_t>(ex + 127);
      // 4 codes -> 3 bytes; 8 groups -> 6 dwords
      uint32_t dw[6];
#pragma unroll
      for (int w = 0; w < 6; ++w) dw[w] = 0u;
#pragma unroll
      for (int e = 0; e < 32; ++e) {
        const uint32_t c = e2m3_code(__builtin_amdgcn_ldexpf(v[e], -ex));
        const int bit = 6 * e;
        dw[bit / 32] |= c << (bit % 32);
        if (bit % 32 > 26) dw[bit / 32 + 1] |= c >> (32 - bit % 32);
      }
      uint2* dst = reinterpret_cast<uint2*>(q + row * (K * 3 / 4) + kb * 24);
      dst[0] = uint2{dw[0], dw[1]};
      dst[1] = uint2{dw[2], dw[3]};
      dst[2] = uint2{dw[4], dw[5]};
    }
    scale_t[((kb / 4) * M4 + row) * 4 + kb % 4] = static_cast<uint8_t>(sbyte);
  }
}

// ---- grouped GEMM ------------------------------------------------------------
template <int BM_, int BN_, int WM, int WN, int NS>
struct X6Cfg {
  static constexpr int BM = BM_, BN = BN_;
  static constexpr int kWM = WM, kWN = WN, kThreads = 64 * WM * WN;
  static constexpr int kTM = BM / kWM / 32, kTN = BN / kWN / 32;  // 32x32 sub-tiles per wave
  static constexpr int kABytes = BM * kARow6;   // packed E2M3 codes
  static constexpr int kASBytes = BM * 4;       // A scales: 4 k-blocks per row
  static constexpr int kBBytes = 2 * BN * 32;   // two 64-k records of packed E2M1
  static constexpr int kBSBytes = 2 * BN * 2;   // their scales
  static constexpr int kSlot = kABytes + kASBytes + kBBytes + kBSBytes;
  static constexpr int kAOps = BM * (kARow6 / 16) / kThreads;  // 16-byte A chunks per thread
  static constexpr int kBOps = BN * 4 / kThreads;
  static constexpr int kASOps = BM / 64;                        // wave 0: one dword lane per row
  static constexpr int kOps = kAOps + kBOps;
  static constexpr int kOps0 = kOps + kASOps + 1;  // wave 0 also fetches both scale sets
  static constexpr int kBSLanes = BN / 4;          // 16-byte lanes of the B-scale DMA
  static_assert(BM * (kARow6 / 16) % kThreads == 0 && BN * 4 % kThreads == 0, "DMA split");
  static_assert(kTM >= 1 && kTN >= 1 && BM % 64 == 0, "wave tile");
  static_assert(kBSLanes <= 64 && kSlot % 16 == 0, "scale DMA / slot alignment");
  static_assert((NS - 2) * kOps0 < 64, "vmcnt range");
  static constexpr int kLdsBlocks = 163840 / (NS * kSlot + 64);
};

// 16-byte chunk rotation of A row r (see the header): rows 8..15 (mod 32) and
// 24..31 are rotated by one of their six chunks.
__device__ __forceinline__ int arot6(int r) { return (r / 8) % 2; }

// Byte of logical A offset o (0..95, 8-aligned runs stay in one chunk) of
// row r in the LDS tile.
__device__ __forceinline__ int aphys6(int r, int o) {
  int c = o / 16 + arot6(r);
  c = c >= 6 ? c - 6 : c;
  return r * kARow6 + c * 16 + o % 16;
}

template <int BM_, int BN_, int WM, int WN, int NS>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(
    X6Cfg<BM_, BN_, WM, WN, NS>::kLdsBlocks * WM * WN / 4 < 1 ? 1 : X6Cfg<BM_, BN_, WM, WN, NS>::kLdsBlocks * WM * WN / 4)))
void grouped_gemm_mx6_kernel(Params p, int64_t n_tiles, int gm) {
  using C = X6Cfg<BM_, BN_, WM, WN, NS>;
  constexpr int BM = C::BM, BN = C::BN;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ TileInfo s_tile;
  __shared__ int64_t s_nt;

  const int tid = threadIdx.x;
  const int lane = tid % 64, wave = tid / 64;
  const int wm = wave / C::kWN, wn = wave % C::kWN;
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
  const int64_t KP = K * 3 / 4;  // packed bytes per activation row
  const int64_t g = tile.group;

  floatx16 acc[C::kTM][C::kTN];
#pragma unroll
  for (int i = 0; i < C::kTM; ++i)
#pragma unroll
    for (int j = 0; j < C::kTN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  if (!tile.zero) {
    const uint32_t smem0 = lds_offset(smem);
    const int64_t nk = K / kXK6;
    const uint8_t* lhs = reinterpret_cast<const uint8_t*>(p.lhs);

    // A: LDS chunk q = tid + 256 v <- row q / 6, physical chunk q % 6 holding
    // logical chunk (q % 6 - rot) mod 6.  Rows past the tile read row 0.
    const uint8_t* a_base = uniform_ptr(lhs + tile.row0 * KP);
    uint32_t a_off[C::kAOps];
#pragma unroll
    for (int v = 0; v < C::kAOps; ++v) {
      const int q = tid + C::kThreads * v;
      const int row = q / 6, pc = q % 6;
      int lc = pc - arot6(row);
      lc = lc < 0 ? lc + 6 : lc;
      const int rr = row < tile.rows ? row : 0;
      a_off[v] = static_cast<uint32_t>(rr * KP + lc * 16);
    }
    // A scales: wave 0 lane l of op u <- the 4 scale bytes of tile row 64u + l
    const uint8_t* as_base = uniform_ptr(p.lhs_scale + tile.row0 * 4);
    uint32_t as_off[C::kASOps];
#pragma unroll
    for (int u = 0; u < C::kASOps; ++u) {
      const int r = 64 * u + lane;
      as_off[u] = static_cast<uint32_t>((r < tile.rows ? r : 0) * 4);
    }
    // B: chunk q = tid + 256 u <- record h = q / (2 BN), column c, chunk q % 2
    const int64_t rec = N * 32;
    const uint8_t* b_base = uniform_ptr(static_cast<const uint8_t*>(p.rhs) + g * (K / 64) * rec);
    uint32_t b_off[C::kBOps];
#pragma unroll
    for (int u = 0; u < C::kBOps; ++u) {
      const int q = tid + C::kThreads * u;
      const int h = q / (2 * BN), rem = q % (2 * BN);
      const int c = rem / 2, ch = rem % 2;
      int64_t n = nt * BN + c;
      n = n < N ? n : N - 1;
      b_off[u] = static_cast<uint32_t>(h * rec + n * 32 + ch * 16);
    }
    // B scales: wave 0 lane sl <- record h = sl / (BN/8), 8 columns from c0
    const int64_t srec = N * 2;
    const uint8_t* bs_base = uniform_ptr(p.scale + g * (K / 64) * srec);
    const bool bs_active = lane < C::kBSLanes;
    uint32_t bs_off;
    {
      const int sl = lane % C::kBSLanes;
      const int h = sl / (BN / 8), c0 = (sl % (BN / 8)) * 8;
      int64_t n0 = nt * BN + c0;
      n0 = n0 <= N - 8 ? n0 : N - 8;
      bs_off = static_cast<uint32_t>(h * srec + n0 * 2);
    }
    const uint32_t lds_wave = __builtin_amdgcn_readfirstlane(smem0 + wave * 64 * 16);
    const uint32_t lds_slot0 = __builtin_amdgcn_readfirstlane(smem0);

    auto issue = [&](int64_t s, int slot) __attribute__((always_inline)) {
      if (s >= nk) return;
      const uint32_t base = lds_wave + slot * C::kSlot;
#pragma unroll
      for (int v = 0; v < C::kAOps; ++v) dma16s(a_off[v], a_base + s * kARow6, base + v * C::kThreads * 16);
#pragma unroll
      for (int u = 0; u < C::kBOps; ++u)
        dma16s(b_off[u], b_base + s * 2 * rec, base + C::kABytes + C::kASBytes + u * C::kThreads * 16);
      if (wave == 0) {
        const uint32_t sb = lds_slot0 + slot * C::kSlot;
#pragma unroll
        for (int u = 0; u < C::kASOps; ++u) dma4s(as_off[u], as_base + s * M4 * 4, sb + C::kABytes + u * 256);
        if (bs_active) dma16s(bs_off, bs_base + s * 2 * srec, sb + C::kABytes + C::kASBytes + C::kBBytes);
      }
    };

    static_for<NS - 1>([&](auto sc) __attribute__((always_inline)) {
      constexpr int s = decltype(sc)::value;
      issue(s, s);
      return true;
    });

    const int r_lane = lane % 32, g_lane = lane / 32;
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
#pragma unroll
      for (int s = 0; s < 2; ++s) {  // the two 64-deep MFMA steps
        v8i_t af[C::kTM];
        int sa[C::kTM];
#pragma unroll
        for (int i = 0; i < C::kTM; ++i) {
          const int r = wm * (BM / C::kWM) + i * 32 + r_lane;
          const int o = s * 48 + g_lane * 24;
          const uint2 d0 = *reinterpret_cast<const uint2*>(as + aphys6(r, o));
          const uint2 d1 = *reinterpret_cast<const uint2*>(as + aphys6(r, o + 8));
          const uint2 d2 = *reinterpret_cast<const uint2*>(as + aphys6(r, o + 16));
          af[i] = v8i_t{static_cast<int>(d0.x), static_cast<int>(d0.y), static_cast<int>(d1.x),
                        static_cast<int>(d1.y), static_cast<int>(d2.x), static_cast<int>(d2.y), 0, 0};
          sa[i] = asc[r * 4 + 2 * s + g_lane];
        }
#pragma unroll
        for (int j = 0; j < C::kTN; ++j) {
          const int c = wn * (BN / C::kWN) + j * 32 + r_lane;
          // logical dwords 4g .. 4g+3 of record s: physical (mx_dword_pos)
          // 2g, 4 + 2g, 2g + 1, 4 + 2g + 1
          const uint8_t* rec0 = bs + (s * BN + c) * 32;
          const uint2 lo = *reinterpret_cast<const uint2*>(rec0 + g_lane * 8);
          const uint2 hi = *reinterpret_cast<const uint2*>(rec0 + 16 + g_lane * 8);
          const v8i_t bf = v8i_t{static_cast<int>(lo.x), static_cast<int>(hi.x), static_cast<int>(lo.y),
                                 static_cast<int>(hi.y), 0, 0, 0, 0};
          const int sb = bsc[(s * BN + c) * 2 + g_lane];
#pragma unroll
          for (int i = 0; i < C::kTM; ++i)
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[i], bf, acc[i][j], 2, 4, 0, sa[i], 0, sb);
        }
      }
      cur = cur == NS - 1 ? 0 : cur + 1;
    }
  }

  // Epilogue: lane holds column (lane % 32) of each sub-tile and rows
  // 8*(e/4) + 4*(lane/32) + e%4.  Zero tiles (padding bucket, tail rows)
  // store zeros.
#pragma unroll
  for (int i = 0; i < C::kTM; ++i) {
#pragma unroll
    for (int j = 0; j < C::kTN; ++j) {
      const int64_t col = nt * BN + wn * (BN / C::kWN) + j * 32 + (lane % 32);
      if (col >= N) continue;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = wm * (BM / C::kWM) + i * 32 + 8 * (e / 4) + 4 * (lane / 32) + e % 4;
        if (row >= tile.rows) continue;
        store_from_f32(p.out, (tile.row0 + row) * N + col, acc[i][j][e], p.out_dtype);
      }
    }
  }
}

template <int BM_, int BN_, int WM, int WN, int NS>
int launch_mx6(const Params& p, hipStream_t st, const char* name) {
  using C = X6Cfg<BM_, BN_, WM, WN, NS>;
  const int64_t ntiles = ceil_div(p.N, C::BN);
  const int64_t mtiles = ceil_div(p.M, C::BM) + p.G + 1;
  if (ntiles == 0 || p.M == 0) return LMOE_OK;
  int gm = p.G == 1 ? 4 : 1;
  if (p.G == 1) {
    // one group: keep every XCD busy with at least one m-tile group
    const int64_t real_m = ceil_div(p.M, C::BM);
    while (gm > 1 && ceil_div(real_m, gm) < kXcds) gm /= 2;
  }
  int64_t blocks = kXcds * ceil_div(ceil_div(mtiles, gm), kXcds) * gm * ntiles;
  if (ntiles % kXcds == 0) {
    gm = 0;  // n-tiles striped over the XCDs
    blocks = mtiles * ntiles;
  }
  LMOE_CHECK_SUPPORTED(blocks < (1ll << 31), "%s: grid too large", name);
  LMOE_CHECK_SUPPORTED(p.N * p.K / 2 < (1ll << 32) && C::BM * p.K < (1ll << 32), "%s: group too large", name);
  const size_t lds = static_cast<size_t>(NS) * C::kSlot;
  static const hipError_t attr_rc = hipFuncSetAttribute(reinterpret_cast<const void*>(&grouped_gemm_mx6_kernel<BM_, BN_, WM, WN, NS>),
                                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                                        static_cast<int>(lds));
  if (attr_rc != hipSuccess)
    return fail(LMOE_ERR_HIP, "%s: LDS size attribute (%zu bytes): %s", name, lds, hipGetErrorString(attr_rc));
  grouped_gemm_mx6_kernel<BM_, BN_, WM, WN, NS><<<dim3(static_cast<unsigned>(blocks)), C::kThreads, lds, st>>>(p, ntiles, gm);
  LMOE_CHECK_LAUNCH(name);
  return LMOE_OK;
}

// Tile shape: 128x128 tiles of 2x2 waves with a 3-deep ring (swept against
// 256x128 with 2- and 3-deep rings and 256x256 with a 2-deep ring; 256x256
// is faster only from M = 8192 on).
int run_mx6(const Params& p, hipStream_t st, const char* name) {
  return launch_mx6<128, 128, 2, 2, 3>(p, st, name);
}

}  // namespace
}  // namespace gemm
}  // namespace lmoe

using namespace lmoe;
using namespace lmoe::gemm;

extern "C" int lmoe_quantize_mxfp6(const void* x, int x_dtype, int64_t M, int64_t K, uint8_t* q, uint8_t* scale_t,
                                   void* stream) {
  const char* name = "quantize_mxfp6";
  LMOE_CHECK_ARG(M >= 0 && K > 0, "%s: bad sizes M=%lld K=%lld", name, (long long)M, (long long)K);
  LMOE_CHECK_ARG(valid_dtype(x_dtype), "%s: bad dtype", name);
  LMOE_CHECK_SUPPORTED(K % 128 == 0, "%s: needs K %% 128 == 0 (K=%lld)", name, (long long)K);
  LMOE_CHECK_SUPPORTED(extent_ok({M + 3, K}), "%s: sizes beyond device memory", name);
  if (M == 0) return LMOE_OK;
  LMOE_CHECK_ARG(x && q && scale_t, "%s: null pointer", name);
  LMOE_CHECK_SUPPORTED(aligned(x, 16) && aligned(q, 8), "%s: x 16-byte and q 8-byte alignment", name);
  const int64_t M4 = (M + 3) / 4 * 4;
  const int64_t total = M4 * (K / 32);
  const int64_t b = ceil_div(total, 256);
  const unsigned grid = static_cast<unsigned>(b < 65536 * 4 ? b : 65536 * 4);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (x_dtype == LMOE_BF16)
    quantize_mxfp6_kernel<uint16_t><<<grid, 256, 0, st>>>(static_cast<const uint16_t*>(x), M, K, M4, q, scale_t);
  else
    quantize_mxfp6_kernel<float><<<grid, 256, 0, st>>>(static_cast<const float*>(x), M, K, M4, q, scale_t);
  LMOE_CHECK_LAUNCH(name);
  return LMOE_OK;
}

extern "C" int lmoe_ragged_dot_mxfp6_mxfp4(const uint8_t* lhs_q, const uint8_t* lhs_scale_t,
                                           const uint8_t* w_packed_t, const uint8_t* w_scale_t,
                                           const int32_t* group_sizes, int64_t M, int64_t K, int64_t N, int64_t G,
                                           int zero_group, void* out, int out_dtype, void* stream) {
  const char* name = "ragged_dot_mxfp6_mxfp4";
  LMOE_CHECK_ARG(M >= 0 && K > 0 && N > 0 && G > 0, "%s: bad sizes", name);
  LMOE_CHECK_SUPPORTED(M < (1ll << 31), "%s: M=%lld rows (the tile scan counts rows in 32 bits)", name, (long long)M);
  LMOE_CHECK_ARG(zero_group >= -1 && zero_group < G, "%s: bad zero_group %d", name, zero_group);
  LMOE_CHECK_ARG(valid_dtype(out_dtype), "%s: bad out dtype", name);
  LMOE_CHECK_SUPPORTED(K % 128 == 0, "%s: needs K %% 128 == 0 (K=%lld)", name, (long long)K);
  LMOE_CHECK_SUPPORTED(N % 8 == 0, "%s: N=%lld", name, (long long)N);
  LMOE_CHECK_SUPPORTED(extent_ok({M, K}) && extent_ok({G, K, N}) && extent_ok({M, N}),
                       "%s: sizes beyond device memory", name);
  if (M == 0) return LMOE_OK;
  LMOE_CHECK_ARG(lhs_q && lhs_scale_t && w_packed_t && w_scale_t && group_sizes && out, "%s: null pointer", name);
  LMOE_CHECK_SUPPORTED(aligned(lhs_q, 16) && aligned(w_packed_t, 16) && aligned(w_scale_t, 16) &&
                           aligned(lhs_scale_t, 4),
                       "%s: alignment", name);
  Params p{reinterpret_cast<const uint16_t*>(lhs_q), w_packed_t, w_scale_t, group_sizes, M, K, N, G, zero_group,
           out, out_dtype, 0.f, 0.f, 0, lhs_scale_t};
  return run_mx6(p, static_cast<hipStream_t>(stream), name);
}
