// Grouped GEMM on bf16 MFMA (v_mfma_f32_16x16x32_bf16), fp32 accumulation.
//
// Entry points: lmoe_ragged_dot (tokamax.ragged_dot, rd.py:358-369),
// lmoe_ragged_dot_gateup_situ (fused gate/up + SiTU-GLU, rd.py:644-723 with
// the epilogue convention of gk.py:114-125), the LDS-dequant mode of
// lmoe_ragged_dot_mxfp4 (odq.py:94-99 semantics on the checkpoint layout) and
// lmoe_ragged_dot_fp8_scaled (fp8 E4M3 weights with f32 block scales,
// rd.py:2789-2811 / rd.py:2836-2953: each weight is bf16(f32(code) * scale)
// when its tile is written to LDS, then the bf16 MFMA).
//
// Block = 256 threads = WM x WN wavefronts; each wave owns a
// (BM/WM) x (BN/WN) sub-tile of 16x16 MFMA tiles.  K advances 64 at a time
// through two LDS buffers: while the MFMAs consume buffer k%2, the global
// loads of step k+1 are in flight in registers and are then written (for
// MXFP4: dequantised) into the other buffer, so there is one barrier per step.
//
// Work mapping: the grid is 1-D.  Workgroups are dispatched round-robin over
// the 8 XCDs, so block b runs on XCD b % 8; each XCD is given a contiguous
// range of the (m-tile, n-tile) work list, walked in groups of GM m-tiles
// (n-tile outer, m-tile inner).  Blocks that run together on one XCD then share
// A rows (and, with GM > 1, B columns) in that XCD's L2.
#include <utility>

#include "gemm_tile.h"

namespace lmoe {
namespace gemm {
namespace {


// Calls f(integral_constant<int, 0>) ... f(integral_constant<int, N-1>) in
// order while f returns true, so register-ring indices are compile-time.
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (void)(f(std::integral_constant<int, I>{}) && ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <int BM, int BN, int WM, int WN, int LAYOUT, int EPI, int S>
struct Cfg {
  static constexpr int kStages = S;  // global->register pipeline depth
  static constexpr int kWTM = BM / WM;
  static constexpr int kWTN = BN / WN;
  static constexpr int kTM = kWTM / 16;
  static constexpr int kTN = kWTN / 16;
  static constexpr int kAVec = BM * kBK / 8 / kThreads;  // 16-byte A loads per thread
  // B staging unit: GKN / FP8GKN 4 k-rows x 8 columns (transposed on the LDS
  // store), GNK 8 k values of one column, MXFP4 32 k values of one column
  static constexpr int kBUnits = (LAYOUT == kGKN || LAYOUT == kFP8GKN) ? (kBK / 4) * (BN / 8)
                                 : LAYOUT == kGNK                    ? BN * (kBK / 8)
                                                                     : BN * (kBK / 32);
  static constexpr int kBPer = kBUnits / kThreads;
  static constexpr int kBRegs = (LAYOUT == kGKN || LAYOUT == kFP8GKN) ? 4 : 1;
  static constexpr int kBScales = LAYOUT == kFP8GKN ? 2 : 1;  // float4s of f32 scales per unit
  static_assert(WM * WN * 64 == kThreads, "4 waves");
  static_assert(kWTM % 16 == 0 && kWTN % 16 == 0, "16x16 MFMA tiles");
  static_assert(BM * kBK / 8 % kThreads == 0, "A tile split");
  static_assert(EPI != kEpiSitu || kTN % 2 == 0, "SiTU pairs gate/up sub-tiles");
  // every thread stages the same number of B units: no guard around the loads
  // (a load under divergent control flow makes the compiler wait for all
  // outstanding loads at the join, which serialises the prefetch ring)
  static_assert(kBUnits % kThreads == 0, "B tile split");
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

template <int BM, int BN, int WM, int WN, int LAYOUT, int EPI, int S>
__global__ __launch_bounds__(kThreads) void grouped_gemm_kernel(Params p, int64_t n_tiles, int gm) {
  using C = Cfg<BM, BN, WM, WN, LAYOUT, EPI, S>;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * kLdsRow];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * kLdsRow];
  __shared__ TileInfo s_tile;
  __shared__ int64_t s_nt;

  const int tid = threadIdx.x;
  const int lane = tid % 64, wave = tid / 64;
  const int wm = wave / WN, wn = wave % WN;
  if (wave == 0) {
    // Groups of gm m-tiles go round-robin over the XCDs; an XCD walks its
    // groups in order, each group n-tile outer / m-tile inner.
    const int64_t tm = total_m_tiles<BM>(p.group_sizes, p.G, p.M);
    const int64_t b = blockIdx.x;
    const int64_t xcd = b % kXcds, slot = b / kXcds;
    const int64_t span = static_cast<int64_t>(gm) * n_tiles;
    const int64_t m_base = ((slot / span) * kXcds + xcd) * gm;
    const int64_t r = slot % span;
    TileInfo ti{-1, 0, 0, false};
    int64_t nt = 0;
    if (m_base < tm) {
      const int64_t gm_eff = tm - m_base < gm ? tm - m_base : gm;
      if (r < gm_eff * n_tiles) {
        nt = r / gm_eff;
        ti = locate_tile<BM>(p.group_sizes, p.G, p.M, p.zero_group, m_base + r % gm_eff);
      }
    }
    if (lane == 0) {
      s_tile = ti;
      s_nt = nt;
    }
  }
  __syncthreads();
  const TileInfo tile = s_tile;
  if (tile.group < 0) return;
  const int64_t nt = s_nt;
  const int64_t K = p.K, N = p.N;
  const int64_t g = tile.group;

  floatx4 acc[C::kTM][C::kTN];
#pragma unroll
  for (int i = 0; i < C::kTM; ++i)
#pragma unroll
    for (int j = 0; j < C::kTN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  if (!tile.zero) {
    // Ring of S register stages: the loads of step k+S are issued while step k
    // is computed, so S steps of A and B are in flight per thread.  Loads are
    // branch-free: out-of-range rows / columns / k read a clamped in-bounds
    // address and a mask bit zeroes them when the stage is written to LDS, so
    // the compiler never has to wait for a load at a control-flow join.
    uint4 ra_s[S][C::kAVec];
    uint4 rb_s[S][C::kBPer][C::kBRegs];
    uint32_t rs_s[S][C::kBPer];  // MXFP4 scale bytes
    float4 rf_s[S][C::kBPer][C::kBScales];  // FP8GKN: the unit's 8 column scales
    uint32_t mk_s[S];            // bit v: A vector v valid; bit 16+u: B unit u valid

    const int64_t k_last8 = K - 8;  // K % 8 == 0 (K % 64 == 0 for MXFP4)
    auto load_tiles = [&](int64_t k0, uint4 (&ra)[C::kAVec], uint4 (&rb)[C::kBPer][C::kBRegs],
                          uint32_t (&rs)[C::kBPer], float4 (&rf)[C::kBPer][C::kBScales],
                          uint32_t& mk) __attribute__((always_inline)) {
      uint32_t m = 0;
#pragma unroll
      for (int v = 0; v < C::kAVec; ++v) {
        const int idx = tid + v * kThreads;
        const int r = idx / (kBK / 8), kv = idx % (kBK / 8);
        const int64_t k = k0 + kv * 8;
        const bool in = r < tile.rows && k < K;
        m |= static_cast<uint32_t>(in) << v;
        const int64_t rr = r < tile.rows ? r : 0;
        const int64_t kk = k < K ? k : k_last8;
        ra[v] = *reinterpret_cast<const uint4*>(p.lhs + (tile.row0 + rr) * K + kk);
      }
#pragma unroll
      for (int u = 0; u < C::kBPer; ++u) {
        const int idx = tid + u * kThreads;
        if constexpr (LAYOUT == kGKN) {
          const int kb = idx / (BN / 8), nb = idx % (BN / 8);
          bool ok;
          int64_t n = rhs_col<BN, EPI>(nt, nb * 8, N, &ok);
          n = ok ? n : 0;
          const uint16_t* base = static_cast<const uint16_t*>(p.rhs) + g * K * N + n;
          const int64_t kq = k0 + kb * 4;
          m |= static_cast<uint32_t>(ok && kq < K) << (16 + u);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int64_t k = kq + q < K ? kq + q : K - 1;
            rb[u][q] = *reinterpret_cast<const uint4*>(base + k * N);
          }
        } else if constexpr (LAYOUT == kFP8GKN) {
          const int kb = idx / (BN / 8), nb = idx % (BN / 8);
          bool ok;
          int64_t n = rhs_col<BN, EPI>(nt, nb * 8, N, &ok);
          n = ok ? n : 0;
          const uint8_t* base = static_cast<const uint8_t*>(p.rhs) + g * K * N + n;
          const int64_t kq = k0 + kb * 4;
          m |= static_cast<uint32_t>(ok && kq < K) << (16 + u);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int64_t k = kq + q < K ? kq + q : K - 1;
            const uint2 v = *reinterpret_cast<const uint2*>(base + k * N);
            rb[u][q] = uint4{v.x, v.y, 0u, 0u};
          }
          // the 4 rows lie in one scale block (scale_block % 4 == 0)
          const int64_t kc = kq < K ? kq : K - 1;
          const float* sp = p.scale_f32 + (g * (K / p.scale_block) + kc / p.scale_block) * N + n;
          rf[u][0] = *reinterpret_cast<const float4*>(sp);
          rf[u][1] = *reinterpret_cast<const float4*>(sp + 4);
        } else if constexpr (LAYOUT == kGNK) {
          const int c = idx / (kBK / 8), kv = idx % (kBK / 8);
          bool ok;
          int64_t n = rhs_col<BN, EPI>(nt, c, N, &ok);
          const int64_t k = k0 + kv * 8;
          m |= static_cast<uint32_t>(ok && k < K) << (16 + u);
          n = ok ? n : 0;
          const int64_t kk = k < K ? k : k_last8;
          rb[u][0] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.rhs) + (g * N + n) * K + kk);
        } else {
          const int c = idx / (kBK / 32), h = idx % (kBK / 32);
          bool ok;
          int64_t n = rhs_col<BN, EPI>(nt, c, N, &ok);
          const int64_t k = k0 + h * 32;
          m |= static_cast<uint32_t>(ok && k < K) << (16 + u);
          n = ok ? n : 0;
          const int64_t kk = k < K ? k : K - 32;
          rb[u][0] = *reinterpret_cast<const uint4*>(static_cast<const uint8_t*>(p.rhs) +
                                                     (g * N + n) * (K / 2) + kk / 2);
          rs[u] = p.scale[(g * N + n) * (K / 32) + kk / 32];
        }
      }
      mk = m;
    };

    // v & mask, componentwise (a ternary on uint4 aggregates is lowered to a
    // pointer select through scratch memory).
    auto masked = [](const uint4& v, uint32_t m) __attribute__((always_inline)) {
      return uint4{v.x & m, v.y & m, v.z & m, v.w & m};
    };

    auto store_tiles = [&](int buf, const uint4 (&ra)[C::kAVec], const uint4 (&rb)[C::kBPer][C::kBRegs],
                           const uint32_t (&rs)[C::kBPer], const float4 (&rf)[C::kBPer][C::kBScales],
                           uint32_t mk) __attribute__((always_inline)) {
      uint16_t* as = As[buf];
      uint16_t* bs = Bs[buf];
#pragma unroll
      for (int v = 0; v < C::kAVec; ++v) {
        const int idx = tid + v * kThreads;
        const int r = idx / (kBK / 8), kv = idx % (kBK / 8);
        *reinterpret_cast<uint4*>(&as[r * kLdsRow + kv * 8]) = masked(ra[v], 0u - ((mk >> v) & 1u));
      }
#pragma unroll
      for (int u = 0; u < C::kBPer; ++u) {
        const int idx = tid + u * kThreads;
        const uint32_t okm = 0u - ((mk >> (16 + u)) & 1u);
        if constexpr (LAYOUT == kGKN) {
          const int kb = idx / (BN / 8), nb = idx % (BN / 8);
          const uint4 v0 = masked(rb[u][0], okm), v1 = masked(rb[u][1], okm);
          const uint4 v2 = masked(rb[u][2], okm), v3 = masked(rb[u][3], okm);
          const uint32_t w0[4] = {v0.x, v0.y, v0.z, v0.w};
          const uint32_t w1[4] = {v1.x, v1.y, v1.z, v1.w};
          const uint32_t w2[4] = {v2.x, v2.y, v2.z, v2.w};
          const uint32_t w3[4] = {v3.x, v3.y, v3.z, v3.w};
          // (K % 8 == 0, so a 4-row block is entirely inside or outside K)
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            uint2 lo, hi;  // columns 2d and 2d+1, k = 4kb..4kb+3
            lo.x = (w0[d] & 0xffffu) | (w1[d] << 16);
            lo.y = (w2[d] & 0xffffu) | (w3[d] << 16);
            hi.x = (w0[d] >> 16) | (w1[d] & 0xffff0000u);
            hi.y = (w2[d] >> 16) | (w3[d] & 0xffff0000u);
            *reinterpret_cast<uint2*>(&bs[(nb * 8 + 2 * d) * kLdsRow + kb * 4]) = lo;
            *reinterpret_cast<uint2*>(&bs[(nb * 8 + 2 * d + 1) * kLdsRow + kb * 4]) = hi;
          }
        } else if constexpr (LAYOUT == kFP8GKN) {
          const int kb = idx / (BN / 8), nb = idx % (BN / 8);
          // row q holds k = 4kb + q, columns 0..3 in .x and 4..7 in .y; a
          // masked unit becomes zero codes under a zero scale
          const uint32_t lo[4] = {rb[u][0].x & okm, rb[u][1].x & okm, rb[u][2].x & okm, rb[u][3].x & okm};
          const uint32_t hi[4] = {rb[u][0].y & okm, rb[u][1].y & okm, rb[u][2].y & okm, rb[u][3].y & okm};
          const float sc[8] = {rf[u][0].x, rf[u][0].y, rf[u][0].z, rf[u][0].w,
                               rf[u][1].x, rf[u][1].y, rf[u][1].z, rf[u][1].w};
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            const uint32_t* w = c < 4 ? lo : hi;
            const int sh = 8 * (c % 4);
            // the column's four codes, k = 4kb .. 4kb+3 in bytes 0..3
            const uint32_t col = ((w[0] >> sh) & 0xffu) | (((w[1] >> sh) & 0xffu) << 8) |
                                 (((w[2] >> sh) & 0xffu) << 16) | (((w[3] >> sh) & 0xffu) << 24);
            const float s = okm ? sc[c] : 0.0f;
            const floatx2_t f01 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(col), false);
            const floatx2_t f23 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(col), true);
            uint2 o;
            o.x = static_cast<uint32_t>(f32_to_bf16(__fmul_rn(f01[0], s))) |
                  (static_cast<uint32_t>(f32_to_bf16(__fmul_rn(f01[1], s))) << 16);
            o.y = static_cast<uint32_t>(f32_to_bf16(__fmul_rn(f23[0], s))) |
                  (static_cast<uint32_t>(f32_to_bf16(__fmul_rn(f23[1], s))) << 16);
            *reinterpret_cast<uint2*>(&bs[(nb * 8 + c) * kLdsRow + kb * 4]) = o;
          }
        } else if constexpr (LAYOUT == kGNK) {
          const int c = idx / (kBK / 8), kv = idx % (kBK / 8);
          *reinterpret_cast<uint4*>(&bs[c * kLdsRow + kv * 8]) = masked(rb[u][0], okm);
        } else {
          const int c = idx / (kBK / 32), h = idx % (kBK / 32);
          uint32_t o[16];
          // a masked unit dequantises zero bytes with scale 2^0
          dequant32(masked(rb[u][0], okm), (rs[u] & okm) | (127u & ~okm), o);
          uint4* dst = reinterpret_cast<uint4*>(&bs[c * kLdsRow + h * 32]);
#pragma unroll
          for (int q = 0; q < 4; ++q) dst[q] = uint4{o[4 * q], o[4 * q + 1], o[4 * q + 2], o[4 * q + 3]};
        }
      }
    };

    auto compute = [&](int buf) __attribute__((always_inline)) {
      const uint16_t* as = As[buf];
      const uint16_t* bs = Bs[buf];
#pragma unroll
      for (int ks = 0; ks < kBK / 32; ++ks) {
        bf16x8_t af[C::kTM], bfr[C::kTN];
        const int kofs = ks * 32 + (lane / 16) * 8;
#pragma unroll
        for (int i = 0; i < C::kTM; ++i) {
          const int r = wm * C::kWTM + i * 16 + (lane % 16);
          af[i] = *reinterpret_cast<const bf16x8_t*>(&as[r * kLdsRow + kofs]);
        }
#pragma unroll
        for (int j = 0; j < C::kTN; ++j) {
          const int c = lds_col<BN, WN, C::kTN, EPI>(wn, j) + (lane % 16);
          bfr[j] = *reinterpret_cast<const bf16x8_t*>(&bs[c * kLdsRow + kofs]);
        }
#pragma unroll
        for (int i = 0; i < C::kTM; ++i)
#pragma unroll
          for (int j = 0; j < C::kTN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
      }
    };

    const int64_t nk = (K + kBK - 1) / kBK;
    static_for<S>([&](auto st_c) __attribute__((always_inline)) {
      constexpr int st = decltype(st_c)::value;
      if (st < nk) load_tiles(st * kBK, ra_s[st], rb_s[st], rs_s[st], rf_s[st], mk_s[st]);
      return true;
    });
    store_tiles(0, ra_s[0], rb_s[0], rs_s[0], rf_s[0], mk_s[0]);
    __syncthreads();
    for (int64_t kt0 = 0; kt0 < nk; kt0 += S) {
      static_for<S>([&](auto st_c) __attribute__((always_inline)) {
        constexpr int st = decltype(st_c)::value;
        constexpr int nxt = (st + 1) % S;
        const int64_t kt = kt0 + st;
        if (kt >= nk) return false;
        // slot st held step kt, already in LDS: refill it with step kt + S
        if (kt + S < nk) load_tiles((kt + S) * kBK, ra_s[st], rb_s[st], rs_s[st], rf_s[st], mk_s[st]);
        compute(static_cast<int>(kt & 1));
        if (kt + 1 < nk)
          store_tiles(static_cast<int>((kt + 1) & 1), ra_s[nxt], rb_s[nxt], rs_s[nxt], rf_s[nxt], mk_s[nxt]);
        __syncthreads();
        return true;
      });
    }
  }

  // Epilogue: lane holds column (lane % 16) and rows 4*(lane/16) + r of each
  // 16x16 tile.
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
          const int row = wm * C::kWTM + i * 16 + 4 * (lane / 16) + r;
          if (row >= tile.rows) continue;
          float gv = acc[i][j][r], uv = acc[i][j + half][r];
          if (p.round_before_act) round_pair_bf16(gv, uv);
          const float v = tile.zero ? 0.0f : situ_epi(gv, uv, sc);
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

template <int BM, int BN, int WM, int WN, int LAYOUT, int EPI, int S>
int launch(const Params& p, hipStream_t st, const char* name) {
  const int64_t out_cols = EPI == kEpiSitu ? p.N / 2 : p.N;
  const int64_t cols_per_tile = EPI == kEpiSitu ? BN / 2 : BN;
  const int64_t ntiles = ceil_div(out_cols, cols_per_tile);
  const int64_t mtiles = ceil_div(p.M, BM) + p.G + 1;  // upper bound on m-tiles
  if (ntiles == 0 || p.M == 0) return LMOE_OK;
  // Dense problems (one group) group 4 m-tiles per walk so B columns are
  // reused from L2; grouped problems walk each m-tile's n-tiles in turn.
  const int gm = p.G == 1 ? 4 : 1;
  const int64_t groups_per_xcd = ceil_div(ceil_div(mtiles, gm), kXcds);
  const int64_t blocks = kXcds * groups_per_xcd * gm * ntiles;
  LMOE_CHECK_SUPPORTED(blocks < (1ll << 31), "%s: grid too large", name);
  grouped_gemm_kernel<BM, BN, WM, WN, LAYOUT, EPI, S>
      <<<dim3(static_cast<unsigned>(blocks)), kThreads, 0, st>>>(p, ntiles, gm);
  LMOE_CHECK_LAUNCH(name);
  return LMOE_OK;
}

// Tile shape: BM = 64 measured best for every grouped and dense shape of the
// BASELINE configs (two 4-wave blocks per CU; BM = 128 halves occupancy, BM =
// 32 re-reads weights too often).
template <int LAYOUT, int EPI>
int dispatch_shape(const Params& p, hipStream_t st, const char* name) {
  return launch<64, 128, 2, 2, LAYOUT, EPI, 2>(p, st, name);
}

}  // namespace

int run_dma(const Params& p, int layout, int epi, hipStream_t st, const char* name);

// bf16 weights with K % 64 == 0 go to the DMA kernel (faster on every
// BASELINE shape); the register-staged kernel above takes the rest.
int run_bf16(const Params& p, int layout, int epi, hipStream_t st, const char* name) {
  if ((layout == kGNK || layout == kGKN) && p.K % 64 == 0) return run_dma(p, layout, epi, st, name);
  if (layout == kGKN && epi == kEpiNone) return dispatch_shape<kGKN, kEpiNone>(p, st, name);
  if (layout == kGKN && epi == kEpiSitu) return dispatch_shape<kGKN, kEpiSitu>(p, st, name);
  if (layout == kGNK && epi == kEpiNone) return dispatch_shape<kGNK, kEpiNone>(p, st, name);
  if (layout == kGNK && epi == kEpiSitu) return dispatch_shape<kGNK, kEpiSitu>(p, st, name);
  if (layout == kMXFP4 && epi == kEpiNone) return dispatch_shape<kMXFP4, kEpiNone>(p, st, name);
  if (layout == kMXFP4 && epi == kEpiSitu) return dispatch_shape<kMXFP4, kEpiSitu>(p, st, name);
  if (layout == kFP8GKN && epi == kEpiNone) return dispatch_shape<kFP8GKN, kEpiNone>(p, st, name);
  if (layout == kFP8GKN && epi == kEpiSitu) return dispatch_shape<kFP8GKN, kEpiSitu>(p, st, name);
  return fail(LMOE_ERR_UNSUPPORTED, "%s: layout %d epilogue %d", name, layout, epi);
}

}  // namespace gemm
}  // namespace lmoe
