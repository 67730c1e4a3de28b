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
// re-tiled once by lmoe_mxfp4_tile into k-step-major order: packed
// (G, K/64, N, 32) and scales (G, K/64, N, 2), so that one step's weights for
// a run of columns are one contiguous stretch of memory.  K % 64 == 0.
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <utility>

#include "dma_util.h"
#include "gemm_tile.h"

namespace lmoe {
namespace gemm {
namespace {

using namespace lmoe::dma;

constexpr int kSK = 64;  // K per pipeline step

enum DmaLayout { kDGNK = 0, kDMX = 1 };

// WM x WN waves; wave (wm, wn) owns rows [wm*BM/WM, ...) and columns
// [wn*BN/WN, ...) of the tile.  With WM == 1 every weight fragment is expanded
// by exactly one wave.
template <int BM, int BN, int LAYOUT, int EPI, int NS, int WM = 1, int WN = 4>
struct DCfg {
  static constexpr int kWM = WM, kWN = WN;
  static constexpr int kWaves = WM * WN, kThreads = 64 * WM * WN;
  static constexpr int kWTM = BM / kWM, kWTN = BN / kWN;
  static constexpr int kTM = kWTM / 16, kTN = kWTN / 16;
  static constexpr int kABytes = BM * 128;                       // A slot
  static constexpr int kBBytes = LAYOUT == kDGNK ? BN * 128 : BN * 32;  // B slot
  static constexpr int kSBytes = LAYOUT == kDMX ? BN * 2 : 0;    // scale slot
  static constexpr int kSlot = kABytes + kBBytes + ((kSBytes + 15) / 16) * 16;
  // DMA instructions per wave per step
  static constexpr int kAOps = BM * 8 / kThreads;  // 16-byte chunks per thread
  static constexpr int kBOps = LAYOUT == kDGNK ? BN * 8 / kThreads : BN * 2 / kThreads;
  // scales: BN columns x 2 bytes per step, fetched by wave 0 alone (kSLanes
  // lanes x 16 B) -- one instruction instead of one per wave
  static constexpr int kSOps = LAYOUT == kDMX ? 1 : 0;
  static constexpr int kSLanes = BN / 8;
  static constexpr int kOps = kAOps + kBOps;       // per step, every wave
  static constexpr int kOps0 = kAOps + kBOps + kSOps;  // per step, wave 0
  static_assert(kAOps >= 1 && BM * 8 % kThreads == 0, "A DMA split");
  static_assert(kBOps >= 1 && (LAYOUT == kDGNK ? BN * 8 : BN * 2) % kThreads == 0, "B DMA split");
  static_assert(LAYOUT != kDMX || (BN % 8 == 0 && kSLanes <= 64), "scale DMA split");
  static_assert(kTM >= 1 && kTN >= 1 && kWTM % 16 == 0 && kWTN % 16 == 0, "wave tile");
  static_assert((NS - 2) * kOps0 < 64, "vmcnt range");
  static_assert(EPI != kEpiSitu || kTN % 2 == 0, "SiTU pairs gate/up sub-tiles");
  // blocks per CU the LDS ring allows (160 KB per CU); the register budget is
  // capped so that the same number of waves fits on each SIMD
  static constexpr int kLdsBlocks = 163840 / (NS * kSlot + 64);
  static constexpr int kWavesPerEuRaw = kLdsBlocks * kWaves / 4;
  static constexpr int kWavesPerEu = kWavesPerEuRaw < 1 ? 1 : (kWavesPerEuRaw > 8 ? 8 : kWavesPerEuRaw);
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

template <int BM, int BN, int LAYOUT, int EPI, int NS, int WM, int WN>
__global__ __launch_bounds__((DCfg<BM, BN, LAYOUT, EPI, NS, WM, WN>::kThreads))
__attribute__((amdgpu_waves_per_eu(DCfg<BM, BN, LAYOUT, EPI, NS, WM, WN>::kWavesPerEu)))
void grouped_gemm_dma_kernel(Params p, int64_t n_tiles, int gm, int64_t n_virtual) {
  using C = DCfg<BM, BN, LAYOUT, EPI, NS, WM, WN>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ TileInfo s_tile;
  __shared__ int64_t s_nt;

  const int64_t tm = threadIdx.x < 64 ? total_m_tiles<BM>(p.group_sizes, p.G, p.M) : 0;  // used by wave 0
  // Persistent blocks: block b takes virtual tiles b, b + gridDim.x, ... (the
  // grid is a multiple of the XCD count, so a virtual tile keeps its XCD).
  for (int64_t vb = blockIdx.x; vb < n_virtual; vb += gridDim.x) {
  // The thread index is re-read per tile through an opaque move so that no
  // per-lane address math is hoisted out of the tile loop: those values would
  // stay live across every tile and push the kernel past its register budget.
  int tid;
  asm volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"(static_cast<int>(threadIdx.x)));
  const int lane = tid % 64, wave = tid / 64;
  const int wm = wave / C::kWN, wn = wave % C::kWN;
  __syncthreads();  // the previous tile's LDS slots and s_tile are no longer read
  if (wave == 0) {
    int64_t nt = 0;
    const TileInfo ti = schedule_tile<BM>(p, n_tiles, gm, vb, tm, nt);
    if (lane == 0) {
      s_tile = ti;
      s_nt = nt;
    }
  }
  __syncthreads();
  const TileInfo tile = s_tile;
  if (tile.group < 0) continue;
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

    // DMA addressing: a wave-uniform (SGPR) base per operand that advances by
    // one k step per step, plus a loop-invariant 32-bit per-lane offset.
    // A: LDS chunk position q = tid + kThreads * v of the slot <- row q/8,
    // logical chunk (q%8) ^ (row&7).  Rows past the tile read row 0 of the tile.
    const uint8_t* a_base = uniform_ptr(p.lhs + tile.row0 * K);
    uint32_t a_off[C::kAOps];
#pragma unroll
    for (int v = 0; v < C::kAOps; ++v) {
      const int q = tid + C::kThreads * v;
      const int row = q / 8, kc = (q % 8) ^ (row & 7);
      const int rr = row < tile.rows ? row : 0;
      a_off[v] = static_cast<uint32_t>(rr * K * 2 + kc * 16);
    }
    // GNK: row n of group g at (g*N + n) * 2K bytes; MXFP4 (k-step-major):
    // column n of step s of group g at ((g*K/64 + s)*N + n) * 32 bytes
    const int64_t b_row = LAYOUT == kDGNK ? K * 2 : 32;
    const uint8_t* b_base = uniform_ptr(static_cast<const uint8_t*>(p.rhs) + g * N * (LAYOUT == kDGNK ? K * 2 : K / 2));
    uint32_t b_off[C::kBOps];
#pragma unroll
    for (int u = 0; u < C::kBOps; ++u) {
      const int q = tid + C::kThreads * u;
      if constexpr (LAYOUT == kDGNK) {
        const int c = q / 8, kc = (q % 8) ^ (c & 7);
        b_off[u] = static_cast<uint32_t>(drhs_col<BN, EPI>(nt, c, N) * b_row + kc * 16);
      } else {
        const int c = q / 2, ch = (q % 2) ^ ((c >> 3) & 1);
        b_off[u] = static_cast<uint32_t>(drhs_col<BN, EPI>(nt, c, N) * b_row + ch * 16);
      }
    }
    // Scales (tiled (G, K/64, N, 2)): lanes 0..kSLanes-1 of wave 0 each fetch
    // 16 bytes = 8 LDS columns' two scale bytes.
    const uint8_t* s_base = nullptr;
    uint32_t s_off = 0;
    bool s_active = false;
    if constexpr (LAYOUT == kDMX) {
      const int sl = lane % C::kSLanes;
      s_active = lane < C::kSLanes;
      const int c0 = sl * 8;  // 8 consecutive LDS columns
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
      s_base = uniform_ptr(p.scale + g * (K / 64) * N * 2);
      s_off = static_cast<uint32_t>(n0 * 2);
    }
    const int64_t b_step = LAYOUT == kDGNK ? kSK * 2 : N * 32;
    const int64_t s_step = N * 2;
    // LDS destination of this wave's chunk 0 (M0 must be wave-uniform)
    const uint32_t lds_wave = __builtin_amdgcn_readfirstlane(smem0 + wave * 64 * 16);

    // DMA of step `step` into ring slot `slot`; nothing past the last step.
    auto issue = [&](int64_t step, int slot) __attribute__((always_inline)) {
      if (step >= nk) return;
      const int64_t s = step;
      const uint32_t base = lds_wave + slot * C::kSlot;
#pragma unroll
      for (int v = 0; v < C::kAOps; ++v) dma16s(a_off[v], a_base + s * (kSK * 2), base + v * C::kThreads * 16);
#pragma unroll
      for (int u = 0; u < C::kBOps; ++u)
        dma16s(b_off[u], b_base + s * b_step, base + C::kABytes + u * C::kThreads * 16);
      if constexpr (LAYOUT == kDMX) {
        if (wave == 0) {
          const uint32_t sbase = base + C::kABytes + C::kBBytes;  // wave 0: base is the slot start
          if (s_active) dma16s(s_off, s_base + s * s_step, sbase);
        }
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
        bf16x8_t af[C::kTM];
#pragma unroll
        for (int i = 0; i < C::kTM; ++i) {
          const int r = wm * C::kWTM + i * 16 + (lane % 16);
          af[i] = *reinterpret_cast<const bf16x8_t*>(as + r * 128 + ((kc ^ (r & 7)) * 16));
        }
        // B fragments one at a time: read, expand, feed the column of MFMAs
#pragma unroll
        for (int j = 0; j < C::kTN; ++j) {
          const int c = dlds_col<BN, C::kTN, EPI>(wn, j) + (lane % 16);
          bf16x8_t bfr;
          if constexpr (LAYOUT == kDGNK) {
            bfr = *reinterpret_cast<const bf16x8_t*>(bs + c * 128 + ((kc ^ (c & 7)) * 16));
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
            bfr = __builtin_bit_cast(bf16x8_t, uint4{o[0], o[1], o[2], o[3]});
          }
#pragma unroll
          for (int i = 0; i < C::kTM; ++i)
            // weight fragment first: the accumulator holds the transposed
            // sub-tile (a lane owns one row and four adjacent columns)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfr, af[i], acc[i][j], 0, 0, 0);
        }
      }
    };

    // One pipeline step per iteration; the slot index is a run-time value so
    // the accumulators keep one register assignment across steps.
    int cur = 0;  // slot of step kt
    for (int64_t kt = 0; kt < nk; ++kt) {
      const int ahead = static_cast<int>(nk - 1 - kt < NS - 2 ? nk - 1 - kt : NS - 2);
      if (wave == 0)
        wait_step<NS, C::kOps0>(ahead);
      else
        wait_step<NS, C::kOps>(ahead);
      barrier();
      issue(kt + NS - 1, cur == 0 ? NS - 1 : cur - 1);
      uint32_t s2[C::kTN];
      if constexpr (LAYOUT == kDMX) {
        const uint8_t* ss = smem + cur * C::kSlot + C::kABytes + C::kBBytes;
        bool edge = false;
#pragma unroll
        for (int j = 0; j < C::kTN; ++j) {
          const int c = dlds_col<BN, C::kTN, EPI>(wn, j) + (lane % 16);
          s2[j] = *reinterpret_cast<const uint16_t*>(ss + c * 2);
          edge |= !hw_scale_ok(s2[j] & 0xffu) || !hw_scale_ok(s2[j] >> 8);
        }
        if (__builtin_amdgcn_ballot_w64(edge) != 0)
          compute(cur, s2, std::true_type{});
        else
          compute(cur, s2, std::false_type{});
      } else {
#pragma unroll
        for (int j = 0; j < C::kTN; ++j) s2[j] = 0;
        compute(cur, s2, std::false_type{});
      }
      cur = cur == NS - 1 ? 0 : cur + 1;
    }
    // every DMA of this tile has been waited for by the last step
  }

  // Epilogue.  A lane holds output row (lane % 16) of row sub-tile i and the
  // four adjacent columns 4*(lane/16) .. +3 of column sub-tile j: one 8-byte
  // (bf16) or 16-byte (f32) store per sub-tile.  Column counts are multiples
  // of 8 (checked on the host), so a group of four is in or out as a whole.
  const int r_in = lane % 16, c_in = 4 * (lane / 16);
  if constexpr (EPI == kEpiSitu) {
    const int64_t I = N / 2;
    constexpr int half = C::kTN / 2;
    const SituConsts sc = situ_consts(p.beta, p.beta_lin);
#pragma unroll
    for (int i = 0; i < C::kTM; ++i) {
      const int row = wm * C::kWTM + i * 16 + r_in;
      if (row >= tile.rows) continue;
      uint16_t* orow = static_cast<uint16_t*>(p.out) + (tile.row0 + row) * I;
#pragma unroll
      for (int j = 0; j < half; ++j) {
        const int64_t col = nt * (BN / 2) + wn * half * 16 + j * 16 + c_in;
        if (col >= I) continue;
        uint2 packed{0u, 0u};  // padding bucket: zeros (SiTU(0, 0) == 0)
        if (!tile.zero) {
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float gv = acc[i][j][r], uv = acc[i][j + half][r];
            if (p.round_before_act) {
              gv = static_cast<float>(static_cast<__bf16>(gv));
              uv = static_cast<float>(static_cast<__bf16>(uv));
            }
            v[r] = situ_epi(gv, uv, sc);
          }
          packed = uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        }
        *reinterpret_cast<uint2*>(orow + col) = packed;
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < C::kTM; ++i) {
      const int row = wm * C::kWTM + i * 16 + r_in;
      if (row >= tile.rows) continue;
      const int64_t obase = (tile.row0 + row) * N;
#pragma unroll
      for (int j = 0; j < C::kTN; ++j) {
        const int64_t col = nt * BN + wn * C::kTN * 16 + j * 16 + c_in;
        if (col >= N) continue;
        const floatx4 a = acc[i][j];
        if (p.out_dtype == LMOE_F32) {
          *reinterpret_cast<float4*>(static_cast<float*>(p.out) + obase + col) = float4{a[0], a[1], a[2], a[3]};
        } else {
          *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.out) + obase + col) =
              uint2{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3])};
        }
      }
    }
  }
  }  // persistent tile loop
}

// Compute units of the current device (cached per device).
int cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cache[dev] = v;
  }
  return cache[dev];
}

// LMOE_PERSIST=1 launches only as many blocks as fit on the device at once,
// each looping over tiles; the default launches one block per tile (measured
// equal or faster on the expert shapes, where the hardware's block refill
// overlaps one block's epilogue with its neighbours' main loops).
bool persistent_blocks() {
  static const bool v = [] {
    const char* e = std::getenv("LMOE_PERSIST");
    return e && std::strcmp(e, "1") == 0;
  }();
  return v;
}

// LMOE_XCD_MAP=mtile keeps m-tile groups per XCD for grouped problems (A/B
// timing); the default stripes n-tiles over the XCDs when they divide evenly.
bool xcd_stripe_n() {
  static const bool v = [] {
    const char* e = std::getenv("LMOE_XCD_MAP");
    return !(e && std::strcmp(e, "mtile") == 0);
  }();
  return v;
}

template <int BM, int BN, int LAYOUT, int EPI, int NS, int WM = 1, int WN = 4>
int launch_dma(const Params& p, hipStream_t st, const char* name) {
  using C = DCfg<BM, BN, LAYOUT, EPI, NS, WM, WN>;
  const int64_t out_cols = EPI == kEpiSitu ? p.N / 2 : p.N;
  const int64_t cols_per_tile = EPI == kEpiSitu ? BN / 2 : BN;
  const int64_t ntiles = ceil_div(out_cols, cols_per_tile);
  const int64_t mtiles = ceil_div(p.M, BM) + p.G + 1;
  if (ntiles == 0 || p.M == 0) return LMOE_OK;
  int gm = p.G == 1 ? 4 : 1;
  int64_t blocks = kXcds * ceil_div(ceil_div(mtiles, gm), kXcds) * gm * ntiles;
  if (p.G > 1 && ntiles % kXcds == 0 && xcd_stripe_n()) {
    gm = 0;  // n-tiles striped over the XCDs
    blocks = mtiles * ntiles;
  }
  LMOE_CHECK_SUPPORTED(blocks < (1ll << 31), "%s: grid too large", name);
  // per-lane DMA offsets are 32-bit: one group's weights and one tile's rows
  const int64_t w_bytes = p.N * (LAYOUT == kDGNK ? p.K * 2 : p.K / 2);
  LMOE_CHECK_SUPPORTED(w_bytes < (1ll << 32) && BM * p.K * 2 < (1ll << 32), "%s: group too large for the DMA path",
                       name);
  const size_t lds = static_cast<size_t>(NS) * C::kSlot;
  static const hipError_t attr_rc =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&grouped_gemm_dma_kernel<BM, BN, LAYOUT, EPI, NS, WM, WN>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  if (attr_rc != hipSuccess)
    return fail(LMOE_ERR_HIP, "%s: LDS size attribute (%zu bytes): %s", name, lds, hipGetErrorString(attr_rc));
  int64_t grid = blocks;
  if (persistent_blocks()) {
    const int64_t resident = kXcds * ((static_cast<int64_t>(cu_count()) * C::kLdsBlocks) / kXcds);
    if (resident >= kXcds && resident < grid) grid = resident;
  }
  grouped_gemm_dma_kernel<BM, BN, LAYOUT, EPI, NS, WM, WN>
      <<<dim3(static_cast<unsigned>(grid)), C::kThreads, lds, st>>>(p, ntiles, gm, blocks);
  LMOE_CHECK_LAUNCH(name);
  return LMOE_OK;
}

// Re-tile MXFP4 weights to k-step-major order: packed (G, N, K/2) ->
// (G, K/64, N, 32) and E8M0 scales (G, N, K/32) -> (G, K/64, N, 2).  One
// thread per (group, step, column): two 16-byte copies and one 2-byte copy.
__global__ __launch_bounds__(256) void tile_mxfp4_kernel(const uint8_t* __restrict__ packed,
                                                         const uint8_t* __restrict__ scale, int64_t G, int64_t N,
                                                         int64_t K, uint8_t* __restrict__ packed_out,
                                                         uint8_t* __restrict__ scale_out) {
  const int64_t kb64 = K / 64;
  const int64_t total = G * kb64 * N;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t n = i % N, s = (i / N) % kb64, g = i / (N * kb64);
    const uint4* src = reinterpret_cast<const uint4*>(packed + (g * N + n) * (K / 2) + 32 * s);
    uint4* dst = reinterpret_cast<uint4*>(packed_out + 32 * i);
    dst[0] = src[0];
    dst[1] = src[1];
    const uint8_t* ss = scale + (g * N + n) * (K / 32) + 2 * s;
    scale_out[2 * i] = ss[0];
    scale_out[2 * i + 1] = ss[1];
  }
}

// Tile shape / ring depth of the MXFP4 kernel: LMOE_DMA_CFG = "BMxBNxNS"
// picks one of the instantiated variants (tuning sweeps).  Defaults, from
// sweeps on the LatentMoE expert shapes: 64x256x4 with the fused SiTU
// epilogue (gate/up: each activation tile feeds 128 gate + 128 up columns),
// 64x128x4 without (down projection: more blocks in flight).
int mx_variant() {
  static const int v = [] {
    const char* e = std::getenv("LMOE_DMA_CFG");
    if (!e) return -1;
    const char* names[] = {"64x128x4", "64x128x6", "64x256x4", "64x256x3", "64x128x3", "32x128x4", "32x256x4",
                           "64x256x5"};
    for (int i = 0; i < 8; ++i)
      if (std::strcmp(e, names[i]) == 0) return i;
    return -1;
  }();
  return v;
}

template <int EPI>
int run_mx(const Params& p, hipStream_t st, const char* name) {
  int v = mx_variant();
  if (v < 0) v = EPI == kEpiSitu ? 2 : 0;
  switch (v) {
    case 1: return launch_dma<64, 128, kDMX, EPI, 6>(p, st, name);
    case 2: return launch_dma<64, 256, kDMX, EPI, 4>(p, st, name);
    case 3: return launch_dma<64, 256, kDMX, EPI, 3>(p, st, name);
    case 4: return launch_dma<64, 128, kDMX, EPI, 3>(p, st, name);
    case 5: return launch_dma<32, 128, kDMX, EPI, 4>(p, st, name);
    case 6: return launch_dma<32, 256, kDMX, EPI, 4>(p, st, name);
    case 7: return launch_dma<64, 256, kDMX, EPI, 5>(p, st, name);
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

int tile_mxfp4(const uint8_t* packed, const uint8_t* scale, int64_t G, int64_t N, int64_t K, uint8_t* packed_out,
               uint8_t* scale_out, hipStream_t st) {
  const int64_t total = G * (K / 64) * N;
  if (total == 0) return LMOE_OK;
  const int64_t b = ceil_div(total, 256);
  tile_mxfp4_kernel<<<static_cast<unsigned>(b < 65536 ? b : 65536), 256, 0, st>>>(packed, scale, G, N, K,
                                                                                  packed_out, scale_out);
  LMOE_CHECK_LAUNCH("mxfp4_tile");
  return LMOE_OK;
}

}  // namespace gemm
}  // namespace lmoe
