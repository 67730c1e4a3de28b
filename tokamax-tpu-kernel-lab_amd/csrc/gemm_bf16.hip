// Grouped GEMM on bf16 MFMA (v_mfma_f32_16x16x32_bf16), fp32 accumulation.
//
// Entry points: lmoe_ragged_dot (tokamax.ragged_dot, rd.py:358-369),
// lmoe_ragged_dot_gateup_situ (fused gate/up + SiTU-GLU, rd.py:644-723 with
// the epilogue convention of gk.py:114-125) and the LDS-dequant mode of
// lmoe_ragged_dot_mxfp4 (odq.py:94-99 semantics on the checkpoint layout).
//
// Block = 256 threads = WM x WN wavefronts; each wave owns a
// (BM/WM) x (BN/WN) sub-tile made of 16x16 MFMA tiles.  One K step stages a
// BM x 64 A tile and a BN x 64 B^T tile in LDS; the next step's global loads
// are issued into registers before the current step's MFMAs (register double
// buffering), so HBM latency overlaps the math.
#include "gemm_tile.h"

namespace lmoe {
namespace gemm {
namespace {

template <int BM, int BN, int WM, int WN, int LAYOUT, int EPI>
struct Cfg {
  static constexpr int kWTM = BM / WM;
  static constexpr int kWTN = BN / WN;
  static constexpr int kTM = kWTM / 16;
  static constexpr int kTN = kWTN / 16;
  static constexpr int kAVec = BM * kBK / 8 / kThreads;  // 16-byte A loads per thread
  // B staging units per thread
  static constexpr int kBUnits = LAYOUT == kGKN   ? (kBK / 4) * (BN / 8)
                                 : LAYOUT == kGNK ? BN * (kBK / 8)
                                                  : BN * (kBK / 32);
  static constexpr int kBPer = (kBUnits + kThreads - 1) / kThreads;
  static_assert(WM * WN * 64 == kThreads, "4 waves");
  static_assert(kWTM % 16 == 0 && kWTN % 16 == 0, "16x16 MFMA tiles");
  static_assert(BM * kBK / 8 % kThreads == 0, "A tile split");
  static_assert(EPI != kEpiSitu || kTN % 2 == 0, "SiTU pairs gate/up sub-tiles");
};

// LDS column of the wave's j-th 16-wide sub-tile.  For SiTU the first half of
// a wave's sub-tiles are gate columns and the second half the matching up
// columns, so one lane holds gate and up of the same output element.
template <int BN, int WN, int TN, int EPI>
__device__ __forceinline__ int lds_col(int wn, int j) {
  if constexpr (EPI == kEpiSitu) {
    constexpr int half = TN / 2;
    return j < half ? wn * half * 16 + j * 16 : BN / 2 + wn * half * 16 + (j - half) * 16;
  } else {
    return wn * TN * 16 + j * 16;
  }
}

// Global rhs column for LDS column c of n-tile nt.
template <int BN, int EPI>
__device__ __forceinline__ int64_t rhs_col(int64_t nt, int c, int64_t N, bool* ok) {
  if constexpr (EPI == kEpiSitu) {
    const int64_t I = N / 2;
    const int64_t j = nt * (BN / 2) + (c < BN / 2 ? c : c - BN / 2);
    *ok = j < I;
    return c < BN / 2 ? j : I + j;
  } else {
    const int64_t n = nt * BN + c;
    *ok = n < N;
    return n;
  }
}

template <int BM, int BN, int WM, int WN, int LAYOUT, int EPI>
__global__ __launch_bounds__(kThreads) void grouped_gemm_kernel(Params p) {
  using C = Cfg<BM, BN, WM, WN, LAYOUT, EPI>;
  __shared__ __attribute__((aligned(16))) uint16_t As[BM * kLdsRow];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * kLdsRow];
  __shared__ TileInfo s_tile;

  const int tid = threadIdx.x;
  const int lane = tid % 64, wave = tid / 64;
  const int wm = wave / WN, wn = wave % WN;
  if (wave == 0) {
    TileInfo ti = locate_tile<BM>(p.group_sizes, p.G, p.M, p.zero_group, blockIdx.y);
    if (lane == 0) s_tile = ti;
  }
  __syncthreads();
  const TileInfo tile = s_tile;
  if (tile.group < 0) return;
  const int64_t nt = blockIdx.x;
  const int64_t K = p.K, N = p.N;
  const int64_t g = tile.group;

  floatx4 acc[C::kTM][C::kTN];
#pragma unroll
  for (int i = 0; i < C::kTM; ++i)
#pragma unroll
    for (int j = 0; j < C::kTN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  if (!tile.zero) {
    uint4 ra[C::kAVec];
    uint4 rb[C::kBPer][LAYOUT == kGKN ? 4 : (LAYOUT == kGNK ? 1 : 1)];
    uint32_t rs[C::kBPer];  // MXFP4 scale bytes
    (void)rs;

    auto load_tiles = [&](int64_t k0) {
      // A: BM rows x 64 k, 8 bf16 per load
#pragma unroll
      for (int v = 0; v < C::kAVec; ++v) {
        const int idx = tid + v * kThreads;
        const int r = idx / (kBK / 8), kv = idx % (kBK / 8);
        const int64_t k = k0 + kv * 8;
        uint4 val = uint4{0, 0, 0, 0};
        if (r < tile.rows && k < K)
          val = *reinterpret_cast<const uint4*>(p.lhs + (tile.row0 + r) * K + k);
        ra[v] = val;
      }
#pragma unroll
      for (int u = 0; u < C::kBPer; ++u) {
        const int idx = tid + u * kThreads;
        if (idx >= C::kBUnits) continue;
        if constexpr (LAYOUT == kGKN) {
          const int kb = idx / (BN / 8), nb = idx % (BN / 8);
          bool ok;
          const int64_t n = rhs_col<BN, EPI>(nt, nb * 8, N, &ok);
          const uint16_t* base = static_cast<const uint16_t*>(p.rhs) + g * K * N + n;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int64_t k = k0 + kb * 4 + q;
            rb[u][q] = (ok && k < K) ? *reinterpret_cast<const uint4*>(base + k * N) : uint4{0, 0, 0, 0};
          }
        } else if constexpr (LAYOUT == kGNK) {
          const int c = idx / (kBK / 8), kv = idx % (kBK / 8);
          bool ok;
          const int64_t n = rhs_col<BN, EPI>(nt, c, N, &ok);
          const int64_t k = k0 + kv * 8;
          rb[u][0] = (ok && k < K) ? *reinterpret_cast<const uint4*>(
                                         static_cast<const uint16_t*>(p.rhs) + (g * N + n) * K + k)
                                   : uint4{0, 0, 0, 0};
        } else {
          const int c = idx / (kBK / 32), h = idx % (kBK / 32);
          bool ok;
          const int64_t n = rhs_col<BN, EPI>(nt, c, N, &ok);
          const int64_t k = k0 + h * 32;
          const bool in = ok && k < K;
          rb[u][0] = in ? *reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(p.rhs) +
                                                          (g * N + n) * (K / 2) + k / 2)
                        : uint4{0, 0, 0, 0};
          rs[u] = in ? p.scale[(g * N + n) * (K / 32) + k / 32] : 127u;
        }
      }
    };

    auto store_tiles = [&]() {
#pragma unroll
      for (int v = 0; v < C::kAVec; ++v) {
        const int idx = tid + v * kThreads;
        const int r = idx / (kBK / 8), kv = idx % (kBK / 8);
        *reinterpret_cast<uint4*>(&As[r * kLdsRow + kv * 8]) = ra[v];
      }
#pragma unroll
      for (int u = 0; u < C::kBPer; ++u) {
        const int idx = tid + u * kThreads;
        if (idx >= C::kBUnits) continue;
        if constexpr (LAYOUT == kGKN) {
          const int kb = idx / (BN / 8), nb = idx % (BN / 8);
          const uint32_t w0[4] = {rb[u][0].x, rb[u][0].y, rb[u][0].z, rb[u][0].w};
          const uint32_t w1[4] = {rb[u][1].x, rb[u][1].y, rb[u][1].z, rb[u][1].w};
          const uint32_t w2[4] = {rb[u][2].x, rb[u][2].y, rb[u][2].z, rb[u][2].w};
          const uint32_t w3[4] = {rb[u][3].x, rb[u][3].y, rb[u][3].z, rb[u][3].w};
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            uint2 lo, hi;  // columns 2d and 2d+1, k = 4kb..4kb+3
            lo.x = (w0[d] & 0xffffu) | (w1[d] << 16);
            lo.y = (w2[d] & 0xffffu) | (w3[d] << 16);
            hi.x = (w0[d] >> 16) | (w1[d] & 0xffff0000u);
            hi.y = (w2[d] >> 16) | (w3[d] & 0xffff0000u);
            *reinterpret_cast<uint2*>(&Bs[(nb * 8 + 2 * d) * kLdsRow + kb * 4]) = lo;
            *reinterpret_cast<uint2*>(&Bs[(nb * 8 + 2 * d + 1) * kLdsRow + kb * 4]) = hi;
          }
        } else if constexpr (LAYOUT == kGNK) {
          const int c = idx / (kBK / 8), kv = idx % (kBK / 8);
          *reinterpret_cast<uint4*>(&Bs[c * kLdsRow + kv * 8]) = rb[u][0];
        } else {
          const int c = idx / (kBK / 32), h = idx % (kBK / 32);
          uint32_t o[16];
          dequant32(rb[u][0], rs[u], o);
          uint4* dst = reinterpret_cast<uint4*>(&Bs[c * kLdsRow + h * 32]);
#pragma unroll
          for (int q = 0; q < 4; ++q) dst[q] = uint4{o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]};
        }
      }
    };

    const int64_t nk = (K + kBK - 1) / kBK;
    load_tiles(0);
    for (int64_t kt = 0; kt < nk; ++kt) {
      __syncthreads();
      store_tiles();
      __syncthreads();
      if (kt + 1 < nk) load_tiles((kt + 1) * kBK);
#pragma unroll
      for (int ks = 0; ks < kBK / 32; ++ks) {
        bf16x8_t af[C::kTM], bfr[C::kTN];
        const int kofs = ks * 32 + (lane / 16) * 8;
#pragma unroll
        for (int i = 0; i < C::kTM; ++i) {
          const int r = wm * C::kWTM + i * 16 + (lane % 16);
          af[i] = *reinterpret_cast<const bf16x8_t*>(&As[r * kLdsRow + kofs]);
        }
#pragma unroll
        for (int j = 0; j < C::kTN; ++j) {
          const int c = lds_col<BN, WN, C::kTN, EPI>(wn, j) + (lane % 16);
          bfr[j] = *reinterpret_cast<const bf16x8_t*>(&Bs[c * kLdsRow + kofs]);
        }
#pragma unroll
        for (int i = 0; i < C::kTM; ++i)
#pragma unroll
          for (int j = 0; j < C::kTN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
      }
    }
  }

  // Epilogue: lane holds column (lane % 16) and rows 4*(lane/16) + r of each
  // 16x16 tile.
  if constexpr (EPI == kEpiSitu) {
    const int64_t I = N / 2;
    constexpr int half = C::kTN / 2;
#pragma unroll
    for (int i = 0; i < C::kTM; ++i) {
#pragma unroll
      for (int j = 0; j < half; ++j) {
        const int64_t col = nt * (BN / 2) + wn * half * 16 + j * 16 + (lane % 16);
        if (col >= I) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = wm * C::kWTM + i * 16 + 4 * (lane / 16) + r;
          if (row >= tile.rows) continue;
          float gv = acc[i][j][r], uv = acc[i][j + half][r];
          if (p.round_before_act) {
            gv = round_bf16(gv);
            uv = round_bf16(uv);
          }
          const float v = tile.zero ? 0.0f : situ(gv, uv, p.beta, p.beta_lin);
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
          const int row = wm * C::kWTM + i * 16 + 4 * (lane / 16) + r;
          if (row >= tile.rows) continue;
          store_from_f32(p.out, (tile.row0 + row) * N + col, acc[i][j][r], p.out_dtype);
        }
      }
    }
  }
}

template <int BM, int BN, int WM, int WN, int LAYOUT, int EPI>
int launch(const Params& p, hipStream_t st, const char* name) {
  const int64_t out_cols = EPI == kEpiSitu ? p.N / 2 : p.N;
  const int64_t cols_per_tile = EPI == kEpiSitu ? BN / 2 : BN;
  const int64_t ntiles = ceil_div(out_cols, cols_per_tile);
  const int64_t mtiles = ceil_div(p.M, BM) + p.G + 1;
  if (ntiles == 0 || mtiles == 0 || p.M == 0) return LMOE_OK;
  LMOE_CHECK_SUPPORTED(ntiles < (1ll << 31) && mtiles < 65536, "%s: grid too large", name);
  dim3 grid(static_cast<unsigned>(ntiles), static_cast<unsigned>(mtiles));
  grouped_gemm_kernel<BM, BN, WM, WN, LAYOUT, EPI><<<grid, kThreads, 0, st>>>(p);
  LMOE_CHECK_LAUNCH(name);
  return LMOE_OK;
}

// Tile shape by average rows per group: small groups (the local-shard expert
// FFN, ~37-73 rows) use BM = 64 so fewer MFMA cycles go to padding rows.
template <int LAYOUT, int EPI>
int dispatch_shape(const Params& p, hipStream_t st, const char* name) {
  const int64_t avg = p.G > 0 ? p.M / p.G : p.M;
  if (avg <= 96) return launch<64, 128, 2, 2, LAYOUT, EPI>(p, st, name);
  return launch<128, 128, 2, 2, LAYOUT, EPI>(p, st, name);
}

}  // namespace

int run_bf16(const Params& p, int layout, int epi, hipStream_t st, const char* name) {
  if (layout == kGKN && epi == kEpiNone) return dispatch_shape<kGKN, kEpiNone>(p, st, name);
  if (layout == kGKN && epi == kEpiSitu) return dispatch_shape<kGKN, kEpiSitu>(p, st, name);
  if (layout == kGNK && epi == kEpiNone) return dispatch_shape<kGNK, kEpiNone>(p, st, name);
  if (layout == kGNK && epi == kEpiSitu) return dispatch_shape<kGNK, kEpiSitu>(p, st, name);
  if (layout == kMXFP4 && epi == kEpiNone) return dispatch_shape<kMXFP4, kEpiNone>(p, st, name);
  if (layout == kMXFP4 && epi == kEpiSitu) return dispatch_shape<kMXFP4, kEpiSitu>(p, st, name);
  return fail(LMOE_ERR_UNSUPPORTED, "%s: layout %d epilogue %d", name, layout, epi);
}

}  // namespace gemm
}  // namespace lmoe
