// Grouped GEMM, generation 3: operand tiles move HBM -> LDS by gfx950's
// direct-to-LDS DMA (global_load_lds_dwordx4), never through VGPRs.
//
// Why: the expert FFN is HBM-bound with tiny per-step math (a 64-row x 64-k
// step is ~0.1 us of MFMA work, an HBM round trip ~1-2 us), so each block must
// keep several K steps of loads in flight.  A register ring costs VGPRs and
// occupancy; here an NS-deep LDS ring holds the in-flight steps and VGPRs only
// hold accumulators and MFMA fragments.
//
// Pipeline (one s_barrier per K step):
//   prologue: issue DMA for steps 0 .. NS-2
//   step kt:  s_waitcnt vmcnt(<DMA ops of the NS-2 younger steps>)
//             s_barrier            -- step kt landed for all waves, and every
//                                     wave finished step kt-1's math
//             issue DMA for step kt+NS-1 into the slot of step kt-1
//             MFMAs on slot kt % NS
// The DMA is issued from inline asm, so the compiler neither sees the LDS
// writes nor inserts its conservative vmcnt(0) before LDS reads; all vector
// memory operations inside the K loop are these DMAs, so the wait counts are
// exact.  Steps past the end re-load a valid address (data unused) so every
// step issues the same number of operations.
//
// LDS rows are 128 bytes (64 bf16) with 16-byte chunks XOR-swizzled by
// (row & 7), which makes the MFMA fragment reads (16 rows x 16 bytes at one
// logical chunk) bank-conflict free.  MXFP4 weights stay packed in LDS (32
// bytes per row and step, chunks swizzled by bit 3 of the row) and each MFMA
// B fragment is expanded in registers with v_cvt_scalef32_pk_bf16_fp4.
//
// Layouts: A (M, K) bf16 row-major; B either bf16 (G, N, K) ("GNK") or MXFP4
// packed (G, N, K/2) with scales re-tiled once to (G, K/64, N, 2)
// (lmoe_mxfp4_tile_scales).  K % 64 == 0.
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <utility>

#include "gemm_tile.h"

namespace lmoe {
namespace gemm {
namespace {

constexpr int kXcds = 8;
constexpr int kSK = 64;  // K per pipeline step

template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (void)(f(std::integral_constant<int, I>{}) && ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)p));
}

// One 16-byte DMA per active lane: LDS[base + 16 * lane] = *g.  `base` must be
// wave-uniform.  M0 is written immediately before use (one wait state).
__device__ __forceinline__ void dma16(const void* g, uint32_t base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(g), "s"(base)
               : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// Wait until at most N of this wave's vector memory operations are in flight
// and all its LDS reads have returned, then barrier.  The LDS-read wait keeps a
// slot's last fragment reads ahead of the DMA that the next step issues into it.
template <int N>
__device__ __forceinline__ void wait_and_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

enum DmaLayout { kDGNK = 0, kDMX = 1 };

// 4 waves side by side along N (each wave: all BM rows x BN/4 columns), so
// every weight fragment is expanded by exactly one wave.
template <int BM, int BN, int LAYOUT, int EPI, int NS>
struct DCfg {
  static constexpr int kWM = 1, kWN = 4;
  static constexpr int kWTM = BM / kWM, kWTN = BN / kWN;
  static constexpr int kTM = kWTM / 16, kTN = kWTN / 16;
  static constexpr int kABytes = BM * 128;                       // A slot
  static constexpr int kBBytes = LAYOUT == kDGNK ? BN * 128 : BN * 32;  // B slot
  static constexpr int kSBytes = LAYOUT == kDMX ? BN * 2 : 0;    // scale slot
  static constexpr int kSlot = kABytes + kBBytes + ((kSBytes + 15) / 16) * 16;
  // DMA instructions per wave per step
  static constexpr int kAOps = BM * 8 / 256;                     // 16-byte chunks / 256 lanes
  static constexpr int kBOps = LAYOUT == kDGNK ? BN * 8 / 256 : BN * 2 / 256;
  static constexpr int kSOps = LAYOUT == kDMX ? 1 : 0;           // BN/32 lanes x 16 B per wave
  static constexpr int kSLanes = BN / 32;
  static constexpr int kOps = kAOps + kBOps + kSOps;
  static_assert(BM * 8 % 256 == 0 && (LAYOUT == kDGNK ? BN * 8 : BN * 2) % 256 == 0, "DMA split");
  static_assert(LAYOUT != kDMX || (BN % 32 == 0 && BN <= 2048), "scale DMA: 4 waves x BN/32 lanes x 16 B");
  static_assert((NS - 2) * kOps < 64, "vmcnt range");
  static_assert(EPI != kEpiSitu || kTN % 2 == 0, "SiTU pairs gate/up sub-tiles");
  // blocks per CU the LDS ring allows (160 KB per CU); the register budget is
  // capped so that the same number of waves fits on each SIMD
  static constexpr int kLdsBlocks = 163840 / (NS * kSlot + 64);
  static constexpr int kWavesPerEu = kLdsBlocks < 1 ? 1 : (kLdsBlocks > 8 ? 8 : kLdsBlocks);
};

template <int BN, int TN, int EPI>
__device__ __forceinline__ int dlds_col(int wn, int j) {
  if constexpr (EPI == kEpiSitu) {
    constexpr int half = TN / 2;
    return j < half ? wn * half * 16 + j * 16 : BN / 2 + wn * half * 16 + (j - half) * 16;
  } else {
    return wn * TN * 16 + j * 16;
  }
}

// Global rhs column for LDS column c of n-tile nt (clamped into [0, N)).
template <int BN, int EPI>
__device__ __forceinline__ int64_t drhs_col(int64_t nt, int c, int64_t N) {
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

template <int BM, int BN, int LAYOUT, int EPI, int NS>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(DCfg<BM, BN, LAYOUT, EPI, NS>::kWavesPerEu)))
void grouped_gemm_dma_kernel(Params p, int64_t n_tiles, int gm) {
  using C = DCfg<BM, BN, LAYOUT, EPI, NS>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ TileInfo s_tile;
  __shared__ int64_t s_nt;

  const int tid = threadIdx.x;
  const int lane = tid % 64, wave = tid / 64;
  const int wm = wave / C::kWN, wn = wave % C::kWN;
  if (wave == 0) {
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
    const uint32_t smem0 = lds_offset(smem);
    const int64_t nk = K / kSK;

    // Per-thread DMA sources for step 0; step s adds s * (bytes per step).
    // A: LDS chunk position q = tid + 256 * v of the slot <- row q/8, logical
    // chunk (q%8) ^ (row&7).  Rows past the tile read row 0 of the tile.
    const uint8_t* a_src[C::kAOps];
#pragma unroll
    for (int v = 0; v < C::kAOps; ++v) {
      const int q = tid + 256 * v;
      const int row = q / 8, kc = (q % 8) ^ (row & 7);
      const int64_t rr = row < tile.rows ? row : 0;
      a_src[v] = reinterpret_cast<const uint8_t*>(p.lhs + (tile.row0 + rr) * K) + kc * 16;
    }
    const uint8_t* b_src[C::kBOps];
#pragma unroll
    for (int u = 0; u < C::kBOps; ++u) {
      const int q = tid + 256 * u;
      if constexpr (LAYOUT == kDGNK) {
        const int c = q / 8, kc = (q % 8) ^ (c & 7);
        const int64_t n = drhs_col<BN, EPI>(nt, c, N);
        b_src[u] = reinterpret_cast<const uint8_t*>(static_cast<const uint16_t*>(p.rhs) + (g * N + n) * K) +
                   kc * 16;
      } else {
        const int c = q / 2, ch = (q % 2) ^ ((c >> 3) & 1);
        const int64_t n = drhs_col<BN, EPI>(nt, c, N);
        b_src[u] = static_cast<const uint8_t*>(p.rhs) + (g * N + n) * (K / 2) + ch * 16;
      }
    }
    // Scales (tiled (G, K/64, N, 2)): wave w's lanes 0..3 fetch 16 bytes =
    // 8 columns' two scale bytes; wave w covers columns [32w, 32w + 32).
    const uint8_t* s_src = nullptr;
    bool s_active = false;
    if constexpr (LAYOUT == kDMX) {
      const int sl = lane % C::kSLanes;
      s_active = lane < C::kSLanes;
      const int c0 = wave * (BN / 4) + sl * 8;  // 8 consecutive LDS columns
      // LDS columns c0..c0+7 are 8 consecutive global columns (BN/2 is a
      // multiple of 8); a run past the matrix edge reads the last in-bounds
      // run instead (its values are never stored).  N % 16 == 0 for SiTU and
      // N % 8 == 0 otherwise keep runs 16-byte aligned.
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
      s_src = p.scale + (g * (K / 64) * N + n0) * 2;
    }
    const int64_t a_step = kSK * 2, b_step = LAYOUT == kDGNK ? kSK * 2 : kSK / 2;
    const int64_t s_step = N * 2;

    auto issue = [&](int64_t step, int slot) __attribute__((always_inline)) {
      const int64_t s = step < nk ? step : nk - 1;  // past the end: reload (unused)
      const uint32_t base = smem0 + slot * C::kSlot;
#pragma unroll
      for (int v = 0; v < C::kAOps; ++v)
        dma16(a_src[v] + s * a_step, __builtin_amdgcn_readfirstlane(base + (wave * 64 + v * 256) * 16));
#pragma unroll
      for (int u = 0; u < C::kBOps; ++u)
        dma16(b_src[u] + s * b_step,
              __builtin_amdgcn_readfirstlane(base + C::kABytes + (wave * 64 + u * 256) * 16));
      if constexpr (LAYOUT == kDMX) {
        // lanes 0..BN/32-1 only: one operation per wave either way
        const uint32_t sbase = __builtin_amdgcn_readfirstlane(base + C::kABytes + C::kBBytes + wave * (BN / 2));
        if (s_active) dma16(s_src + s * s_step, sbase);
      }
    };

    static_for<NS - 1>([&](auto sc) __attribute__((always_inline)) {
      constexpr int s = decltype(sc)::value;
      issue(s, s);
      return true;
    });

    // MFMAs of one pipeline step.  `s2[j]` holds the two scale bytes (k
    // halves) of this lane's column in B fragment j; kEdge selects the exact
    // per-byte conversion for scale bytes outside 3..252, taken only when some
    // lane of the wave has one (a wave-uniform branch).
    auto compute = [&](int slot, const uint32_t(&s2)[C::kTN], auto edge_tag) __attribute__((always_inline)) {
      constexpr bool kEdge = decltype(edge_tag)::value;
      const uint8_t* as = smem + slot * C::kSlot;
      const uint8_t* bs = as + C::kABytes;
#pragma unroll
      for (int ks = 0; ks < kSK / 32; ++ks) {
        const int kc = ks * 4 + (lane / 16);  // logical 16-byte chunk of this lane
        bf16x8_t af[C::kTM], bfr[C::kTN];
#pragma unroll
        for (int i = 0; i < C::kTM; ++i) {
          const int r = wm * C::kWTM + i * 16 + (lane % 16);
          af[i] = *reinterpret_cast<const bf16x8_t*>(as + r * 128 + ((kc ^ (r & 7)) * 16));
        }
#pragma unroll
        for (int j = 0; j < C::kTN; ++j) {
          const int c = dlds_col<BN, C::kTN, EPI>(wn, j) + (lane % 16);
          if constexpr (LAYOUT == kDGNK) {
            bfr[j] = *reinterpret_cast<const bf16x8_t*>(bs + c * 128 + ((kc ^ (c & 7)) * 16));
          } else {
            const uint32_t w =
                *reinterpret_cast<const uint32_t*>(bs + c * 32 + ((ks ^ ((c >> 3) & 1)) * 16) + (lane / 16) * 4);
            const uint32_t sb = (s2[j] >> (8 * ks)) & 0xffu;
            uint32_t o[4];
            if constexpr (!kEdge) {
              const float sc = __uint_as_float(sb << 23);
              o[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 0));
              o[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 1));
              o[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 2));
              o[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 3));
            } else {
#pragma unroll
              for (int b = 0; b < 4; ++b) o[b] = dequant_byte((w >> (8 * b)) & 0xffu, sb);
            }
            bfr[j] = __builtin_bit_cast(bf16x8_t, uint4{o[0], o[1], o[2], o[3]});
          }
        }
#pragma unroll
        for (int i = 0; i < C::kTM; ++i)
#pragma unroll
          for (int j = 0; j < C::kTN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
      }
    };

    for (int64_t kt0 = 0; kt0 < nk; kt0 += NS) {
      static_for<NS>([&](auto sc) __attribute__((always_inline)) {
        constexpr int st = decltype(sc)::value;
        const int64_t kt = kt0 + st;
        if (kt >= nk) return false;
        wait_and_barrier<(NS - 2) * C::kOps>();
        issue(kt + NS - 1, (st + NS - 1) % NS);
        uint32_t s2[C::kTN];
        if constexpr (LAYOUT == kDMX) {
          const uint8_t* ss = smem + st * C::kSlot + C::kABytes + C::kBBytes;
          bool edge = false;
#pragma unroll
          for (int j = 0; j < C::kTN; ++j) {
            const int c = dlds_col<BN, C::kTN, EPI>(wn, j) + (lane % 16);
            s2[j] = *reinterpret_cast<const uint16_t*>(ss + c * 2);
            edge |= !hw_scale_ok(s2[j] & 0xffu) || !hw_scale_ok(s2[j] >> 8);
          }
          if (__builtin_amdgcn_ballot_w64(edge) != 0)
            compute(st, s2, std::true_type{});
          else
            compute(st, s2, std::false_type{});
        } else {
#pragma unroll
          for (int j = 0; j < C::kTN; ++j) s2[j] = 0;
          compute(st, s2, std::false_type{});
        }
        return true;
      });
    }
    wait_vmcnt<0>();  // drain the dummy tail loads before the block can exit
  }

  // Epilogue: lane holds column (lane % 16) and rows 4*(lane/16) + r.
  if (EPI == kEpiSitu && tile.zero) {
    // padding bucket: zeros, no activation math (SiTU(0, 0) == 0)
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
          if (row < tile.rows) static_cast<uint16_t*>(p.out)[(tile.row0 + row) * I + col] = 0;
        }
      }
    }
  } else if constexpr (EPI == kEpiSitu) {
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
          const float v = situ_fast(gv, uv, p.beta, p.beta_lin);
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

template <int BM, int BN, int LAYOUT, int EPI, int NS>
int launch_dma(const Params& p, hipStream_t st, const char* name) {
  using C = DCfg<BM, BN, LAYOUT, EPI, NS>;
  const int64_t out_cols = EPI == kEpiSitu ? p.N / 2 : p.N;
  const int64_t cols_per_tile = EPI == kEpiSitu ? BN / 2 : BN;
  const int64_t ntiles = ceil_div(out_cols, cols_per_tile);
  const int64_t mtiles = ceil_div(p.M, BM) + p.G + 1;
  if (ntiles == 0 || p.M == 0) return LMOE_OK;
  const int gm = p.G == 1 ? 4 : 1;
  const int64_t groups_per_xcd = ceil_div(ceil_div(mtiles, gm), kXcds);
  const int64_t blocks = kXcds * groups_per_xcd * gm * ntiles;
  LMOE_CHECK_SUPPORTED(blocks < (1ll << 31), "%s: grid too large", name);
  const size_t lds = static_cast<size_t>(NS) * C::kSlot;
  static const hipError_t attr_rc =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&grouped_gemm_dma_kernel<BM, BN, LAYOUT, EPI, NS>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  if (attr_rc != hipSuccess)
    return fail(LMOE_ERR_HIP, "%s: LDS size attribute (%zu bytes): %s", name, lds, hipGetErrorString(attr_rc));
  grouped_gemm_dma_kernel<BM, BN, LAYOUT, EPI, NS>
      <<<dim3(static_cast<unsigned>(blocks)), kThreads, lds, st>>>(p, ntiles, gm);
  LMOE_CHECK_LAUNCH(name);
  return LMOE_OK;
}

// Re-tile E8M0 scales (G, N, K/32) -> (G, K/64, N, 2).
__global__ __launch_bounds__(256) void tile_scales_kernel(const uint8_t* __restrict__ in, int64_t G,
                                                          int64_t N, int64_t K, uint8_t* __restrict__ out) {
  const int64_t kb64 = K / 64;
  const int64_t total = G * kb64 * N;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = i % N, s = (i / N) % kb64, g = i / (N * kb64);
    const uint8_t* src = in + (g * N + n) * (K / 32) + 2 * s;
    out[2 * i] = src[0];
    out[2 * i + 1] = src[1];
  }
}

// Tile shape / ring depth of the MXFP4 kernel: LMOE_DMA_CFG = "BMxBNxNS"
// picks one of the instantiated variants (tuning sweeps); default 64x128x4.
int mx_variant() {
  static const int v = [] {
    const char* e = std::getenv("LMOE_DMA_CFG");
    if (!e) return 0;
    const char* names[] = {"64x128x4", "64x128x6", "64x256x4", "64x256x6", "128x128x4", "128x256x3"};
    for (int i = 0; i < 6; ++i)
      if (std::strcmp(e, names[i]) == 0) return i;
    return 0;
  }();
  return v;
}

template <int EPI>
int run_mx(const Params& p, hipStream_t st, const char* name) {
  switch (mx_variant()) {
    case 1: return launch_dma<64, 128, kDMX, EPI, 6>(p, st, name);
    case 2: return launch_dma<64, 256, kDMX, EPI, 4>(p, st, name);
    case 3: return launch_dma<64, 256, kDMX, EPI, 6>(p, st, name);
    case 4: return launch_dma<128, 128, kDMX, EPI, 4>(p, st, name);
    case 5: return launch_dma<128, 256, kDMX, EPI, 3>(p, st, name);
    default: return launch_dma<64, 128, kDMX, EPI, 4>(p, st, name);
  }
}

}  // namespace

int run_dma(const Params& p, int layout, int epi, hipStream_t st, const char* name) {
  constexpr int BM = 64, BN = 128;
  if (layout == kGNK && epi == kEpiNone) return launch_dma<BM, BN, kDGNK, kEpiNone, 3>(p, st, name);
  if (layout == kGNK && epi == kEpiSitu) return launch_dma<BM, BN, kDGNK, kEpiSitu, 3>(p, st, name);
  if (layout == kMXFP4 && epi == kEpiNone) return run_mx<kEpiNone>(p, st, name);
  if (layout == kMXFP4 && epi == kEpiSitu) return run_mx<kEpiSitu>(p, st, name);
  return fail(LMOE_ERR_UNSUPPORTED, "%s: DMA path layout %d epilogue %d", name, layout, epi);
}

int tile_scales(const uint8_t* in, int64_t G, int64_t N, int64_t K, uint8_t* out, hipStream_t st) {
  const int64_t total = G * (K / 64) * N;
  if (total == 0) return LMOE_OK;
  const int64_t b = ceil_div(total, 256);
  tile_scales_kernel<<<static_cast<unsigned>(b < 65536 ? b : 65536), 256, 0, st>>>(in, G, N, K, out);
  LMOE_CHECK_LAUNCH("mxfp4_tile_scales");
  return LMOE_OK;
}

}  // namespace gemm
}  // namespace lmoe
