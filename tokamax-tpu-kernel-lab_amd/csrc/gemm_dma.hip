// Grouped GEMM, generation 3: operand tiles move HBM -> LDS by gfx950's
// direct-to-LDS DMA (global_load_lds_dwordx4), never through VGPRs.
//
// Why: the expert FFN is HBM-bound with tiny per-step math (a 64-row x 64-k
// step is ~0.1 us of MFMA work, an HBM round trip ~1-2 us), so each block must
// keep several K steps of loads in flight.  A register ring costs VGPRs and
// occupancy; here an NS-deep LDS ring holds the in-flight steps and VGPRs only
// hold accumulators and MFMA fragments.
//
// Pipeline (one s_barrier per K step, NS-slot LDS ring):
//   prologue: issue DMA for steps 0 .. NS-1; wait for step 0, barrier, read
//             step 0's operand fragments into registers
//   step k:   s_waitcnt vmcnt(<DMA ops of the younger steps>) lgkmcnt(0)
//             s_barrier            -- step k+1 landed for all waves, and every
//                                     wave holds step k's fragments
//             issue DMA for step k+NS into slot k % NS
//             read step k+1's fragments (LDS -> registers)
//             conversions + MFMAs of step k from registers
// The DMA is issued from inline asm, so the compiler neither sees the LDS
// writes nor inserts its conservative vmcnt(0) before LDS reads; all vector
// memory operations inside the K loop are these DMAs, so the wait counts are
// exact.  No DMA is issued past the last step.
//
// LDS rows are 128 bytes (64 bf16) with 16-byte chunks XOR-swizzled by
// swz8(row), which makes the MFMA fragment reads (16 rows x 16 bytes at one
// logical chunk per 16-lane group) bank-conflict free.  MXFP4 weights stay
// packed in LDS (the 32-byte tiled records, copied as they are) and each MFMA
// B fragment is expanded in registers with v_cvt_scalef32_pk_bf16_fp4.
//
// Layouts: A (M, K) bf16 row-major; B either bf16 (G, N, K) ("GNK") or MXFP4
// re-tiled once by lmoe_mxfp4_tile into k-step-major order: packed
// (G, K/64, N, 32) and scales (G, K/64, N, 2), so that one step's weights for
// a run of columns are one contiguous stretch of memory.  K % 64 == 0.
#include <atomic>
#include <mutex>
#include <type_traits>
#include <utility>

#include "dma_util.h"
#include "gemm_tile.h"

namespace lmoe {
namespace gemm {
namespace {

using namespace lmoe::dma;

constexpr int kSK = 64;  // K per pipeline step

// kDGKN: bf16 weights in the reference's (G, K, N) layout.  A k step's B
// tile is 64 k-rows of BN columns, DMA'd as it lies (16-byte chunks of a row
// XOR-swizzled by swzk(row)), and each MFMA B fragment (8 consecutive k of
// one column) is read with two gfx950 transposing LDS reads
// (ds_read_b64_tr_b16): within each 16-lane group, lane c supplies the
// address of the 4-column run (k0 + c/4, n0 + 4 (c%4)) and lane i receives
// column n0 + i at rows k0 .. k0+3.
enum DmaLayout { kDGNK = 0, kDMX = 1, kDGKN = 2 };

// 16-byte chunk swizzle of the kDGKN B tile: the 8 k-rows one transposing
// read touches (k0..k0+3, k0+8..k0+11) x 4 chunks land on 32 distinct chunk
// positions mod 256 bytes, so the read runs at the full LDS rate.
__device__ __forceinline__ int swzk(int row) { return 4 * (row % 4); }

// WM x WN waves; wave (wm, wn) owns rows [wm*BM/WM, ...) and columns
// [wn*BN/WN, ...) of the tile.  With WM == 1 every weight fragment is expanded
// by exactly one wave.  MF is the MFMA tile edge: 32 (v_mfma_f32_32x32x16_bf16,
// the one a single wave issues at the full matrix rate) or 16
// (v_mfma_f32_16x16x32_bf16, which one wave issues at half rate).
template <int BM, int BN, int LAYOUT, int EPI, int NS, int WM = 1, int WN = 4, int MF = 32>
struct DCfg {
  static constexpr int kWM = WM, kWN = WN, kMF = MF;
  static constexpr int kWaves = WM * WN, kThreads = 64 * WM * WN;
  static constexpr int kWTM = BM / kWM, kWTN = BN / kWN;
  static constexpr int kTM = kWTM / MF, kTN = kWTN / MF;
  static constexpr int kKS = kSK / (MF == 32 ? 16 : 32);  // MFMA k sub-steps per pipeline step
  static constexpr int kAccN = MF == 32 ? 16 : 4;         // accumulator floats per lane per sub-tile
  using Acc = std::conditional_t<MF == 32, floatx16, floatx4>;
  static constexpr int kABytes = BM * 128;                       // A slot
  static constexpr int kBBytes = LAYOUT != kDMX ? BN * 128 : BN * 32;  // B slot
  static constexpr int kSBytes = LAYOUT == kDMX ? BN * 2 : 0;    // scale slot
  static constexpr int kSlot = kABytes + kBBytes + ((kSBytes + 15) / 16) * 16;
  // DMA instructions per wave per step
  static constexpr int kAOps = BM * 8 / kThreads;  // 16-byte chunks per thread
  static constexpr int kBOps = LAYOUT != kDMX ? BN * 8 / kThreads : BN * 2 / kThreads;
  // scales: BN columns x 2 bytes per step, fetched by wave 0 alone (kSLanes
  // lanes x 16 B) -- one instruction instead of one per wave
  static constexpr int kSOps = LAYOUT == kDMX ? 1 : 0;
  static constexpr int kSLanes = BN / 8;
  static constexpr int kOps = kAOps + kBOps;       // per step, every wave
  static constexpr int kOps0 = kAOps + kBOps + kSOps;  // per step, wave 0
  static_assert(kAOps >= 1 && BM * 8 % kThreads == 0, "A DMA split");
  static_assert(kBOps >= 1 && (LAYOUT != kDMX ? BN * 8 : BN * 2) % kThreads == 0, "B DMA split");
  static_assert(LAYOUT != kDGKN || (MF == 32 && BN % 128 == 0), "(G, K, N) tiles: 32x32 MFMAs, BN % 128 == 0");
  static_assert(LAYOUT != kDMX || (BN % 8 == 0 && kSLanes <= 64), "scale DMA split");
  static_assert(MF == 16 || MF == 32, "MFMA shape");
  static_assert(kTM >= 1 && kTN >= 1 && kWTM % MF == 0 && kWTN % MF == 0, "wave tile");
  static_assert((NS - 1) * kOps0 < 64, "vmcnt range");
  static_assert(EPI != kEpiSitu || kTN % 2 == 0, "SiTU pairs gate/up sub-tiles");
  // blocks per CU the LDS ring allows (160 KB per CU); the register budget is
  // capped so that the same number of waves fits on each SIMD
  static constexpr int kLdsBlocks = 163840 / (NS * kSlot + 64);
  static constexpr int kWavesPerEuRaw = kLdsBlocks * kWaves / 4;
  // at most 3 waves per SIMD
  static constexpr int kWavesCap = 3;
  static constexpr int kWavesPerEu =
      kWavesPerEuRaw < 1 ? 1 : (kWavesPerEuRaw > kWavesCap ? kWavesCap : kWavesPerEuRaw);
};

// First LDS column of column sub-tile j of wave wn.  With the SiTU epilogue
// the first half of a wave's sub-tiles are gate columns and the second half
// the matching up columns (LDS columns BN/2 ...), so a lane holds both.
template <int BN, int TN, int EPI, int MF>
__device__ __forceinline__ int dlds_col(int wn, int j) {
  if constexpr (EPI == kEpiSitu) {
    constexpr int half = TN / 2;
    return j < half ? wn * half * MF + j * MF : BN / 2 + wn * half * MF + (j - half) * MF;
  } else {
    return wn * TN * MF + j * MF;
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

// First global column of the run of 8 LDS columns c .. c+7 (c % 8 == 0) of
// n-tile nt: runs past the matrix edge read the last in-bounds run instead
// (their values are never stored).  N % 8 == 0 (I % 8 == 0 with SiTU).
template <int BN, int EPI>
__device__ __forceinline__ int64_t drhs_col8(int64_t nt, int c, int64_t N) {
  if constexpr (EPI == kEpiSitu) {
    const int64_t I = N / 2;
    int64_t j = nt * (BN / 2) + (c < BN / 2 ? c : c - BN / 2);
    j = j <= I - 8 ? j : I - 8;
    return c < BN / 2 ? j : I + j;
  } else {
    const int64_t n = nt * BN + c;
    return n <= N - 8 ? n : N - 8;
  }
}

typedef short lds_v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) lds_v4i16 lds_v4i16_as3;

// Transposing LDS read (ds_read_b64_tr_b16) at a byte offset into dynamic LDS.
__device__ __forceinline__ uint2 lds_read_tr16(const uint8_t* base, int byte) {
  const lds_v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4i16_as3*)((__attribute__((address_space(3))) uint8_t*)base + byte));
  return __builtin_bit_cast(uint2, v);
}

template <int BM, int BN, int LAYOUT, int EPI, int NS, int WM, int WN, int MF>
__global__ __launch_bounds__((DCfg<BM, BN, LAYOUT, EPI, NS, WM, WN, MF>::kThreads))
__attribute__((amdgpu_waves_per_eu(DCfg<BM, BN, LAYOUT, EPI, NS, WM, WN, MF>::kWavesPerEu)))
void grouped_gemm_dma_kernel(Params p, int64_t n_tiles, int gm, int64_t n_virtual) {
  using C = DCfg<BM, BN, LAYOUT, EPI, NS, WM, WN, MF>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ TileInfo s_tile;
  __shared__ int64_t s_nt;

  // total m-tiles, used by wave 0 to map virtual tiles when m-tiles are
  // spread over the XCDs by group or range (gm != 0); with n-tiles striped
  // (gm == 0) locate_tile itself returns "no work" past the last tile
  const int64_t tm = (gm != 0 && threadIdx.x < 64) ? total_m_tiles<BM>(p.group_sizes, p.G, p.M) : INT64_MAX;
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
  // split-K: virtual block vb is K range ks of the tile of virtual block tvb
  // (n_virtual is k_split times the tile grid, a multiple of the XCD count,
  // so both keep the same XCD)
  const int64_t nv_tile = n_virtual / p.k_split;
  const int64_t ks = vb / nv_tile, tvb = vb - ks * nv_tile;
  __syncthreads();  // the previous tile's LDS slots and s_tile are no longer read
  if (wave == 0) {
    int64_t nt = 0;
    const TileInfo ti = schedule_tile<BM>(p, n_tiles, gm, tvb, tm, nt);
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

  typename C::Acc acc[C::kTM][C::kTN];
#pragma unroll
  for (int i = 0; i < C::kTM; ++i)
#pragma unroll
    for (int j = 0; j < C::kTN; ++j)
#pragma unroll
      for (int e = 0; e < C::kAccN; ++e) acc[i][j][e] = 0.f;

  if (!tile.zero) {
    const uint32_t smem0 = lds_offset(smem);
    // this block's K steps: [k0, k0 + nk) (all of them without split-K; the
    // host keeps every range non-empty)
    const int64_t nk_all = K / kSK, per = (nk_all + p.k_split - 1) / p.k_split;
    const int64_t k0 = ks * per;
    const int64_t nk = nk_all - k0 < per ? nk_all - k0 : per;

    // DMA addressing: a wave-uniform (SGPR) base per operand that advances by
    // one k step per step, plus a loop-invariant 32-bit per-lane offset.
    // A: LDS chunk position q = tid + kThreads * v of the slot <- row q/8,
    // logical chunk (q%8) ^ swz8(row).  Rows past the tile read row 0 of the tile.
    const uint8_t* a_base = uniform_ptr(p.lhs + tile.row0 * K + k0 * kSK);
    uint32_t a_off[C::kAOps];
#pragma unroll
    for (int v = 0; v < C::kAOps; ++v) {
      const int q = tid + C::kThreads * v;
      const int row = q / 8, kc = (q % 8) ^ swz8(row);
      const int rr = row < tile.rows ? row : 0;
      a_off[v] = static_cast<uint32_t>(rr * K * 2 + kc * 16);
    }
    // GNK: row n of group g at (g*N + n) * 2K bytes; GKN: row k of group g at
    // (g*K + k) * 2N bytes; MXFP4 (k-step-major): column n of step s of group
    // g at ((g*K/64 + s)*N + n) * 32 bytes
    const int64_t b_row = LAYOUT == kDGNK ? K * 2 : 32;
    const int64_t b_step = LAYOUT == kDGNK ? kSK * 2 : LAYOUT == kDGKN ? kSK * N * 2 : N * 32;
    const int64_t s_step = N * 2;
    const uint8_t* b_base =
        uniform_ptr(static_cast<const uint8_t*>(p.rhs) + g * N * (LAYOUT != kDMX ? K * 2 : K / 2) + k0 * b_step);
    uint32_t b_off[C::kBOps];
#pragma unroll
    for (int u = 0; u < C::kBOps; ++u) {
      const int q = tid + C::kThreads * u;
      if constexpr (LAYOUT == kDGNK) {
        const int c = q / 8, kc = (q % 8) ^ swz8(c);
        b_off[u] = static_cast<uint32_t>(drhs_col<BN, EPI>(nt, c, N) * b_row + kc * 16);
      } else if constexpr (LAYOUT == kDGKN) {
        // LDS chunk q: k-row q / (BN/8), position q % (BN/8) <- logical chunk
        // position ^ swzk(row), i.e. LDS columns 8 ch .. 8 ch + 7
        const int row = q / (BN / 8), ch = (q % (BN / 8)) ^ swzk(row);
        b_off[u] = static_cast<uint32_t>(row * N * 2 + drhs_col8<BN, EPI>(nt, ch * 8, N) * 2);
      } else {
        const int c = q / 2, ch = q % 2;
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
      s_base = uniform_ptr(p.scale + g * (K / 64) * N * 2 + k0 * s_step);
      s_off = static_cast<uint32_t>(n0 * 2);
    }
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

    // The ring has NS slots; the prologue fills NS-1 of them (steps
    // 0 .. NS-2).  Each K step lands, refills the slot of the previous step
    // (step k+NS-1) and reads + computes its own fragments.
    static_for<NS - 1>([&](auto sc) __attribute__((always_inline)) {
      constexpr int s = decltype(sc)::value;
      issue(s, s);
      return true;
    });

    // MF-row sub-tiles of this wave past the tile's valid rows are skipped
    // (no MFMAs), so the last tile of a group costs what its rows need.
    // Wave-uniform (scalar) value.
    const int tm_eff = __builtin_amdgcn_readfirstlane((tile.rows - wm * C::kWTM + MF - 1) / MF);

    // MFMA of one sub-tile; the weight fragment goes first, so the
    // accumulator holds the transposed sub-tile (a lane owns one activation
    // row and runs of four adjacent output columns).
    auto mfma = [](const bf16x8_t& w, const bf16x8_t& x, const typename C::Acc& c) __attribute__((always_inline)) {
      if constexpr (MF == 32)
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(w, x, c, 0, 0, 0);
      else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(w, x, c, 0, 0, 0);
    };
    // Fragment coordinates.  An MF x 16*64/MF (k) operand fragment: lane l
    // holds row / column (l % MF) and the 8 consecutive k values of 16-byte
    // chunk kc = kk * (64 / MF) + l / MF of the 128-byte LDS row.
    const int f_rc = lane % MF, f_kc = lane / MF;

    // Operand fragments of one step.  GNK: bf16 weight fragments; MXFP4: the
    // packed dwords (a lane's 8 k values of sub-step kk are logical dword
    // kk * (64 / MF) + l / MF of the column's 32-byte record, at
    // mx_dword_pos; with MF == 32 the four are one 16-byte chunk) and the two
    // scale bytes.
    struct Frags {
      bf16x8_t af[C::kKS][C::kTM];
      bf16x8_t bf[LAYOUT != kDMX ? C::kKS : 1][C::kTN];
      uint32_t bw[C::kKS][C::kTN];
      uint32_t s2[C::kTN];
    };
    auto read_frags = [&](int slot, Frags& f) __attribute__((always_inline)) {
      const uint8_t* as = smem + slot * C::kSlot;
      const uint8_t* bs = as + C::kABytes;
      if constexpr (LAYOUT == kDMX) {
        const uint8_t* ss = bs + C::kBBytes;
#pragma unroll
        for (int j = 0; j < C::kTN; ++j) {
          const int c = dlds_col<BN, C::kTN, EPI, MF>(wn, j) + f_rc;
          f.s2[j] = *reinterpret_cast<const uint16_t*>(ss + c * 2);
        }
      }
#pragma unroll
      for (int kk = 0; kk < C::kKS; ++kk) {
        const int kc = kk * (64 / MF) + f_kc;
#pragma unroll
        for (int j = 0; j < C::kTN; ++j) {
          const int c = dlds_col<BN, C::kTN, EPI, MF>(wn, j) + f_rc;
          if constexpr (LAYOUT == kDMX) {
            if constexpr (MF == 32) {
              if (kk == 0) {
                const uint4 w = *reinterpret_cast<const uint4*>(bs + c * 32 + f_kc * 16);
                f.bw[0][j] = w.x;
                f.bw[1][j] = w.y;
                f.bw[2][j] = w.z;
                f.bw[3][j] = w.w;
              }
            } else {
              f.bw[kk][j] = *reinterpret_cast<const uint32_t*>(bs + c * 32 + mx_dword_pos(kc) * 4);
            }
          } else if constexpr (LAYOUT == kDGKN) {
            // this lane supplies the address of the run (k-row kc*8 + 4r +
            // l16/4, columns n0 + 4 (l16%4) ..) and receives column n0 + l16,
            // k-rows kc*8 + 4r .. +3; n0 = the sub-tile's first column + 16
            // for lanes 16..31 and 48..63
            const int l16 = lane % 16;
            const int col = dlds_col<BN, C::kTN, EPI, MF>(wn, j) + 16 * ((lane / 16) % 2) + 4 * (l16 % 4);
            uint2 h[2];
#pragma unroll
            for (int r = 0; r < 2; ++r) {
              const int row = kc * 8 + 4 * r + l16 / 4;
              h[r] = lds_read_tr16(bs, row * (BN * 2) + (((col / 8) ^ swzk(row)) * 16) + (col % 8) * 2);
            }
            f.bf[kk][j] = __builtin_bit_cast(bf16x8_t, uint4{h[0].x, h[0].y, h[1].x, h[1].y});
          } else {
            f.bf[kk][j] = *reinterpret_cast<const bf16x8_t*>(bs + c * 128 + ((kc ^ swz8(c)) * 16));
          }
        }
        // read even for skipped sub-tiles: unconditional reads keep the
        // compiler's lgkmcnt accounting exact
#pragma unroll
        for (int i = 0; i < C::kTM; ++i) {
          const int r = wm * C::kWTM + i * MF + f_rc;
          f.af[kk][i] = *reinterpret_cast<const bf16x8_t*>(as + r * 128 + ((kc ^ swz8(r)) * 16));
        }
      }
    };
    // Conversions and MFMAs of one step.  All weight fragments of the step are
    // converted first (straight-line code); the exact per-byte conversion for
    // scale bytes outside 3..252 then rewrites them behind one wave-uniform
    // branch, taken when some lane of the wave holds such a byte, and the
    // MFMAs follow.  kFull: every sub-tile holds valid rows; otherwise the
    // MFMAs of sub-tiles past the valid rows are skipped (wave-uniform).
    auto compute = [&](const Frags& f, auto full_tag) __attribute__((always_inline)) {
      auto mfmas = [&](auto full_tag, auto get_b) __attribute__((always_inline)) {
        constexpr bool kFull = decltype(full_tag)::value;
#pragma unroll
        for (int kk = 0; kk < C::kKS; ++kk)
#pragma unroll
          for (int j = 0; j < C::kTN; ++j) {
            const bf16x8_t bfr = get_b(kk, j);
#pragma unroll
            for (int i = 0; i < C::kTM; ++i) {
              if (!kFull && i >= tm_eff) break;
              acc[i][j] = mfma(bfr, f.af[kk][i], acc[i][j]);
            }
          }
      };
      if constexpr (LAYOUT == kDMX) {
        bool edge_lane = false;
#pragma unroll
        for (int j = 0; j < C::kTN; ++j) edge_lane |= !hw_scale_ok(f.s2[j] & 0xffu) || !hw_scale_ok(f.s2[j] >> 8);
        const bool edge = __builtin_amdgcn_ballot_w64(edge_lane) != 0;
        uint32_t bq[C::kKS][C::kTN][4];
#pragma unroll
        for (int kk = 0; kk < C::kKS; ++kk)
#pragma unroll
          for (int j = 0; j < C::kTN; ++j) {
            const uint32_t w = f.bw[kk][j];
            const uint32_t sb = (f.s2[j] >> (8 * (kk / (C::kKS / 2)))) & 0xffu;  // 32-k scale block of sub-step kk
            const float sc = __uint_as_float(sb << 23);
            bq[kk][j][0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 0));
            bq[kk][j][1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 1));
            bq[kk][j][2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 2));
            bq[kk][j][3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 3));
          }
        if (__builtin_expect(edge, false)) {
#pragma unroll
          for (int kk = 0; kk < C::kKS; ++kk)
#pragma unroll
            for (int j = 0; j < C::kTN; ++j) {
              const uint32_t w = f.bw[kk][j];
              const uint32_t sb = (f.s2[j] >> (8 * (kk / (C::kKS / 2)))) & 0xffu;
#pragma unroll
              for (int b = 0; b < 4; ++b) bq[kk][j][b] = dequant_byte((w >> (8 * b)) & 0xffu, sb);
            }
        }
        auto get_b = [&](int kk, int j) __attribute__((always_inline)) {
          return __builtin_bit_cast(bf16x8_t, uint4{bq[kk][j][0], bq[kk][j][1], bq[kk][j][2], bq[kk][j][3]});
        };
        mfmas(full_tag, get_b);
      } else {
        auto get_b = [&](int kk, int j) __attribute__((always_inline)) { return f.bf[kk][j]; };
        mfmas(full_tag, get_b);
      }
    };
    // Wait for step k's DMA with `ahead` younger steps still allowed in
    // flight, then barrier.
    auto land = [&](int64_t k) __attribute__((always_inline)) {
      // youngest step whose DMA has been issued: the prologue issues 0 ..
      // NS-2 and step j issues j+NS-1 after its land
      const int64_t youngest = k + NS - 2;
      const int64_t last = nk - 1 < youngest ? nk - 1 : youngest;
      const int ahead = static_cast<int>(last - k);
      if (wave == 0)
        wait_step<NS + 1, C::kOps0>(ahead);
      else
        wait_step<NS + 1, C::kOps>(ahead);
      barrier();
    };
    // The K loop, instantiated once for tiles whose sub-tiles all hold valid
    // rows and once for the last, partial tile of a group (one wave-uniform
    // test per tile instead of one per MFMA).
    auto k_loop = [&](auto full_tag) __attribute__((always_inline)) {
      // land step k, refill the slot of step k-1, read and compute step k
      int cur = 0;  // slot of step k
      for (int64_t kt = 0; kt < nk; ++kt) {
        land(kt);
        issue(kt + NS - 1, cur == 0 ? NS - 1 : cur - 1);
        Frags f;
        read_frags(cur, f);
        compute(f, full_tag);
        cur = cur == NS - 1 ? 0 : cur + 1;
      }
    };
    if (tm_eff >= C::kTM)
      k_loop(std::true_type{});
    else
      k_loop(std::false_type{});
    // every DMA of this tile has been waited for by the last step
  }
  // the caller never reads the zero group's rows or those past the groups
  // (block-uniform)
  if (tile.zero && p.skip_zero_rows) continue;

  // Epilogue.  A lane holds output row (lane % MF) of row sub-tile i and, for
  // each q < MF / 8 (q < 1 for MF == 16), the four adjacent columns
  // q*8 + 4*(lane/MF) .. +3 (MF == 32) or 4*(lane/16) .. +3 (MF == 16) of
  // column sub-tile j, accumulator elements 4q .. 4q+3.  Column counts are
  // multiples of 8 (checked on the host), so a run of four is in or out as a
  // whole.
  //
  // bf16 output (always with SiTU) is staged through LDS: each lane writes
  // its 8-byte runs into a row-major copy of the output tile (rows padded by
  // 16 bytes, which spreads the 32 rows of one write over all banks), then the
  // block writes whole rows with consecutive 16-byte stores.  Written
  // directly, every store instruction would touch 32 rows with 16 bytes each,
  // which costs the address unit one cycle per row and HBM a 32-byte write
  // per 16 bytes.  f32 output (16-byte runs) is stored directly.
  constexpr int kRuns = MF == 32 ? 4 : 1;
  constexpr int kOutCols = EPI == kEpiSitu ? BN / 2 : BN;  // output columns of a tile
  constexpr int kOutTN = EPI == kEpiSitu ? C::kTN / 2 : C::kTN;  // output sub-tiles of a wave
  constexpr int kStageRow = kOutCols * 2 + 16;              // bytes per staged row
  constexpr bool kCanStage = BM * kStageRow <= NS * C::kSlot;
  const int r_in = lane % MF;
  auto c_run = [&](int q) { return MF == 32 ? q * 8 + 4 * (lane / 32) : 4 * (lane / 16); };
  const int64_t n_out = EPI == kEpiSitu ? N / 2 : N;
  const int64_t col0 = nt * kOutCols;  // first output column of the tile
  // split-K: this range's f32 partial plane
  void* const out_base = p.k_split > 1 ? static_cast<void*>(static_cast<float*>(p.out) + ks * p.split_stride) : p.out;
  // bf16 values of run q of output sub-tile j of row sub-tile i
  auto bf16_run = [&](int i, int j, int q) __attribute__((always_inline)) {
    float v[4];
    if constexpr (EPI == kEpiSitu) {
      const SituConsts sc = situ_consts(p.beta, p.beta_lin);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float gv = acc[i][j][q * 4 + r], uv = acc[i][j + kOutTN][q * 4 + r];
        if (p.round_before_act) {
          round_pair_bf16(gv, uv);
        }
        v[r] = situ_epi(gv, uv, sc);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = acc[i][j][q * 4 + r];
    }
    return uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  };
  if (kCanStage && (EPI == kEpiSitu || p.out_dtype != LMOE_F32)) {
    __syncthreads();  // every wave is done with the K loop's LDS slots
    if (!tile.zero) {
#pragma unroll
      for (int i = 0; i < C::kTM; ++i) {
        // rows past the tile are staged too (never stored)
        uint8_t* srow = smem + (wm * C::kWTM + i * MF + r_in) * kStageRow;
#pragma unroll
        for (int j = 0; j < kOutTN; ++j)
#pragma unroll
          for (int q = 0; q < kRuns; ++q)
            *reinterpret_cast<uint2*>(srow + (wn * kOutTN * MF + j * MF + c_run(q)) * 2) = bf16_run(i, j, q);
      }
    }
    __syncthreads();
    constexpr int kChunks = kOutCols / 8;  // 16-byte chunks per output row
    static_assert(BM * kChunks % C::kThreads == 0, "staged store split");
    uint16_t* out = static_cast<uint16_t*>(out_base);
#pragma unroll
    for (int v = 0; v < BM * kChunks / C::kThreads; ++v) {
      const int idx = tid + C::kThreads * v;
      const int row = idx / kChunks, ch = idx % kChunks;
      if (row >= tile.rows || col0 + ch * 8 >= n_out) continue;
      // padding bucket: zeros (SiTU(0, 0) == 0)
      const uint4 val = tile.zero ? uint4{0u, 0u, 0u, 0u}
                                  : *reinterpret_cast<const uint4*>(smem + row * kStageRow + ch * 16);
      *reinterpret_cast<uint4*>(out + (tile.row0 + row) * n_out + col0 + ch * 8) = val;
    }
  } else {
#pragma unroll
    for (int i = 0; i < C::kTM; ++i) {
      const int row = wm * C::kWTM + i * MF + r_in;
      if (row >= tile.rows) continue;
      const int64_t obase = (tile.row0 + row) * n_out;
#pragma unroll
      for (int j = 0; j < kOutTN; ++j)
#pragma unroll
        for (int q = 0; q < kRuns; ++q) {
          const int64_t col = col0 + wn * kOutTN * MF + j * MF + c_run(q);
          if (col >= n_out) continue;
          if (EPI != kEpiSitu && p.out_dtype == LMOE_F32) {
            *reinterpret_cast<float4*>(static_cast<float*>(out_base) + obase + col) =
                float4{acc[i][j][q * 4], acc[i][j][q * 4 + 1], acc[i][j][q * 4 + 2], acc[i][j][q * 4 + 3]};
          } else {
            *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out_base) + obase + col) =
                tile.zero ? uint2{0u, 0u} : bf16_run(i, j, q);
          }
        }
    }
  }
  }  // persistent tile loop
}

// ---------------------------------------------------------------------------
// Streamed persistent variant (MXFP4 weights, bf16 output).
//
// Each block builds the tile table in LDS once and then loops over its tiles
// (virtual tiles blockIdx.x, + gridDim.x, ...).  Every wave looks its tiles up
// itself, and the DMA ring runs as one stream across tiles: during the last
// NS-1 K steps of a tile the refills fetch the first NS-1 steps of the next
// tile, so the next tile's operands land while this one finishes its MFMAs
// and its epilogue.  The epilogue stages the output through the ring slot of
// the tile's last K step (free once every wave has read that step) in rounds
// of kStageRows rows; the other slots keep receiving the next tile's steps.
//
// Wait accounting: at step k of a tile, the vector memory operations issued
// after step k's DMA are (a) the later DMA steps already issued, NS-2 of them
// or fewer near the end of a tile with nothing to prefetch, and, in a tile
// whose first NS-1 steps were prefetched, for k <= NS-2, (b) the previous
// tile's epilogue stores, issued after those prefetched steps.  Every lane
// issues the same number of stores per round (out-of-range rows and columns
// store a valid neighbour's value again), so (b) is a wave-uniform count.
// Vector memory operations complete in issue order (one vmcnt counter), so
// s_waitcnt vmcnt(a + b) waits for exactly step k.
// ---------------------------------------------------------------------------
template <int BM, int BN, int EPI, int NS, int MF>
struct SCfg {
  using C = DCfg<BM, BN, kDMX, EPI, NS, 1, 4, MF>;
  static constexpr int kOutCols = EPI == kEpiSitu ? BN / 2 : BN;  // bf16 output columns of a tile
  static constexpr int kChunks = kOutCols / 8;                     // 16-byte chunks per output row
  // staged rows: 8 bytes of padding put row r's dword 0 in bank 2r (mod 64),
  // so the 32 rows of one half-wave's 8-byte writes hit every bank once
  static constexpr int kStageRow = kOutCols * 2 + 8;
  static constexpr int kStageRows0 = (C::kSlot / kStageRow) / MF * MF;
  static constexpr int kStageRows = kStageRows0 < BM ? kStageRows0 : BM;
  static constexpr int kRounds = BM / kStageRows;
  static constexpr int kStoresPerRound = kStageRows * kChunks / C::kThreads;  // per wave
  static_assert(kStageRows >= MF && BM % kStageRows == 0, "staging rounds");
  static_assert(kStageRows * kChunks % C::kThreads == 0, "staged store split");
  static_assert((NS - 2) * C::kOps0 + kRounds * kStoresPerRound < 64, "vmcnt range");
  // gathered rows: the lhs row (< 65536) of every row of the block's tiles,
  // loaded into LDS once at the start (at most kIdxTiles tiles per block);
  // small enough to keep three blocks per CU
  static constexpr int kIdxTiles = 8;
  static constexpr int kIdxBytes = kIdxTiles * BM * 2;
};

// s_waitcnt vmcnt(a * OPS + r * SPR) lgkmcnt(0) for runtime a in [0, NS-2]
// and r in [0, R] (wave-uniform).
template <int NS, int OPS, int SPR, int R>
__device__ __forceinline__ void wait_stream(int a, int r) {
  static_for<NS - 1>([&](auto ac) __attribute__((always_inline)) {
    constexpr int A = decltype(ac)::value;
    if (a == A) {
      static_for<R + 1>([&](auto rc) __attribute__((always_inline)) {
        constexpr int Rr = decltype(rc)::value;
        if (r == Rr) wait_vm_lgkm<A * OPS + Rr * SPR>();
        return true;
      });
    }
    return true;
  });
}

__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory"); }

template <int BM, int BN, int EPI, int NS, int MF>
__global__ __launch_bounds__((DCfg<BM, BN, kDMX, EPI, NS, 1, 4, MF>::kThreads))
__attribute__((amdgpu_waves_per_eu(DCfg<BM, BN, kDMX, EPI, NS, 1, 4, MF>::kWavesPerEu)))
void grouped_gemm_stream_kernel(Params p, int64_t n_tiles, int gm, int64_t n_virtual) {
  using S = SCfg<BM, BN, EPI, NS, MF>;
  using C = typename S::C;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ uint32_t s_wsum[2 * C::kWaves];
  const int G = static_cast<int>(p.G);
  uint32_t* tt = reinterpret_cast<uint32_t*>(smem + NS * C::kSlot);
  uint32_t* tr = tt + (G + 1);
  build_tile_table<BM, C::kThreads>(p.group_sizes, G, static_cast<uint32_t>(p.M), tt, tr, s_wsum);
  const int64_t K = p.K, N = p.N;
  const int64_t nk = K / kSK;
  const int64_t n_out = EPI == kEpiSitu ? N / 2 : N;
  const int64_t rows_tail = p.M - static_cast<int64_t>(tr[G]);
  const int64_t tm = static_cast<int64_t>(tt[G]) + (rows_tail + BM - 1) / BM;

  // wave-uniform tile lookup (lane from the per-tile opaque thread index, so
  // that no lane-dependent LDS address is hoisted out of the tile loop and
  // held across the K loop)
  // m-tiles before a trailing zero group (the padding bucket): the real work
  const int64_t tm_work = p.zero_group == G - 1 ? static_cast<int64_t>(tt[G - 1]) : tm;
  uint16_t* s_idx = reinterpret_cast<uint16_t*>(tr + (G + 1));  // gathered rows: kIdxTiles x BM
  auto sched = [&](int64_t vb, int64_t& nt, int lane) __attribute__((always_inline)) {
    TileInfo t = schedule_tile_with(n_tiles, gm, vb, tm, nt, [&](int64_t mt) {
      return locate_tile_lds<BM>(tt, tr, G, p.M, p.zero_group, mt, lane);
    }, tm_work);
    t.group = __builtin_amdgcn_readfirstlane(t.group);
    t.rows = __builtin_amdgcn_readfirstlane(t.rows);
    t.zero = __builtin_amdgcn_readfirstlane(static_cast<int>(t.zero)) != 0;
    t.row0 = static_cast<int64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(t.row0))) |
             (static_cast<int64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(t.row0 >> 32))) << 32);
    nt = static_cast<int64_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(nt)));
    return t;
  };

  // DMA addressing of one tile: wave-uniform bases, 32-bit per-lane offsets
  // (the same layout as grouped_gemm_dma_kernel).
  struct Addr {
    const uint8_t* a_base;
    const uint8_t* b_base;
    const uint8_t* s_base;
    uint32_t a_off[C::kAOps];
    uint32_t b_off[C::kBOps];
    uint32_t s_off;
  };
  auto make_addr = [&](const TileInfo& t, int64_t nt, int tid, int ordinal) __attribute__((always_inline)) {
    Addr d;
    const bool gathered = p.a_index != nullptr;
    d.a_base = uniform_ptr(gathered ? p.lhs : p.lhs + t.row0 * K);
#pragma unroll
    for (int v = 0; v < C::kAOps; ++v) {
      const int q = tid + C::kThreads * v;
      const int row = q / 8, kc = (q % 8) ^ swz8(row);
      const int rr = gathered ? static_cast<int>(s_idx[ordinal * BM + row]) : (row < t.rows ? row : 0);
      d.a_off[v] = static_cast<uint32_t>(rr * K * 2 + kc * 16);
    }
    d.b_base = uniform_ptr(static_cast<const uint8_t*>(p.rhs) + t.group * N * (K / 2));
#pragma unroll
    for (int u = 0; u < C::kBOps; ++u) {
      const int q = tid + C::kThreads * u;
      d.b_off[u] = static_cast<uint32_t>(drhs_col<BN, EPI>(nt, q / 2, N) * 32 + (q % 2) * 16);
    }
    const int c0 = (tid % 64 % C::kSLanes) * 8;
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
    d.s_base = uniform_ptr(p.scale + t.group * (K / 64) * N * 2);
    d.s_off = static_cast<uint32_t>(n0 * 2);
    return d;
  };

  if (p.a_index != nullptr) {
    // Gathered rows: wave w looks up the block's tiles w, w + kWaves, ... and
    // stores the lhs row of each tile row (rows past the tile's valid rows
    // repeat its first row; indices clamped into [0, a_rows)).  Done before
    // any DMA is issued, so the loads' waits hold up nothing.
    const int wave = static_cast<int>(threadIdx.x) / 64, lane = static_cast<int>(threadIdx.x) % 64;
    const int64_t n_my = blockIdx.x < n_virtual ? (n_virtual - blockIdx.x + gridDim.x - 1) / gridDim.x : 0;
    for (int64_t i = wave; i < n_my && i < S::kIdxTiles; i += C::kWaves) {
      int64_t nti = 0;
      const TileInfo ti = sched(blockIdx.x + i * gridDim.x, nti, lane);
      if (ti.group < 0 || ti.zero) continue;
      for (int r = lane; r < BM; r += 64) {
        int32_t src = p.a_index[ti.row0 + (r < ti.rows ? r : 0)];
        src = src < 0 ? 0 : (src >= p.a_rows ? static_cast<int32_t>(p.a_rows - 1) : src);
        s_idx[i * BM + r] = static_cast<uint16_t>(src);
      }
    }
    __syncthreads();
  }
  int64_t vb = blockIdx.x;
  int64_t nt = 0;
  int ord = 0;  // ordinal of cur among this block's virtual tiles
  TileInfo cur = vb < n_virtual ? sched(vb, nt, static_cast<int>(threadIdx.x % 64)) : TileInfo{-1, 0, 0, false};
  bool cur_pf = false;  // cur's first NS-1 steps were issued during the previous tile
  int prev_rounds = 0;  // store rounds of the previous tile's epilogue
  int slot0 = 0;        // ring slot of cur's step 0
  while (vb < n_virtual) {
    int tid;
    asm volatile("v_mov_b32 %0, %1" : "=v"(tid) : "v"(static_cast<int>(threadIdx.x)));
    const int lane = tid % 64, wave = tid / 64;
    const int wn = wave;  // WM == 1

    const int64_t vb_n = vb + gridDim.x;
    int64_t nt_n = 0;
    const TileInfo nxt = vb_n < n_virtual ? sched(vb_n, nt_n, lane) : TileInfo{-1, 0, 0, false};
    const bool pf = cur.group >= 0 && !cur.zero && nxt.group >= 0 && !nxt.zero && nk >= NS - 1;
    const int rounds = cur.group < 0 || cur.zero ? 0 : (cur.rows + S::kStageRows - 1) / S::kStageRows;

    typename C::Acc acc[C::kTM][C::kTN];
#pragma unroll
    for (int i = 0; i < C::kTM; ++i)
#pragma unroll
      for (int j = 0; j < C::kTN; ++j)
#pragma unroll
        for (int e = 0; e < C::kAccN; ++e) acc[i][j][e] = 0.f;

    const int r_in = lane % MF;
    auto c_run = [&](int q) { return MF == 32 ? q * 8 + 4 * (lane / 32) : 4 * (lane / 16); };
    constexpr int kRuns = MF == 32 ? 4 : 1;
    constexpr int kOutTN = EPI == kEpiSitu ? C::kTN / 2 : C::kTN;
    const int64_t col0 = nt * S::kOutCols;
    uint16_t* out = static_cast<uint16_t*>(p.out);

    if (cur.group < 0) {
      // no work (virtual tiles past the last m-tile)
    } else if (!cur.zero) {
      const Addr ca = make_addr(cur, nt, tid, ord);
      const uint32_t lds_wave = __builtin_amdgcn_readfirstlane(lds_offset(smem) + wave * 64 * 16);
      auto issue = [&](const Addr& d, int64_t step, int slot) __attribute__((always_inline)) {
        const uint32_t base = lds_wave + slot * C::kSlot;
#pragma unroll
        for (int v = 0; v < C::kAOps; ++v) dma16s(d.a_off[v], d.a_base + step * (kSK * 2), base + v * C::kThreads * 16);
#pragma unroll
        for (int u = 0; u < C::kBOps; ++u)
          dma16s(d.b_off[u], d.b_base + step * (N * 32), base + C::kABytes + u * C::kThreads * 16);
        if (wave == 0) {
          const uint32_t sbase = base + C::kABytes + C::kBBytes;
          if (lane < C::kSLanes) dma16s(d.s_off, d.s_base + step * (N * 2), sbase);
        }
      };
      if (!cur_pf) {
        for (int64_t s = 0; s < NS - 1 && s < nk; ++s) issue(ca, s, static_cast<int>((slot0 + s) % NS));
      }
      const int tm_eff = __builtin_amdgcn_readfirstlane((cur.rows + MF - 1) / MF);
      auto mfma = [](const bf16x8_t& w, const bf16x8_t& x, const typename C::Acc& c) __attribute__((always_inline)) {
        if constexpr (MF == 32)
          return __builtin_amdgcn_mfma_f32_32x32x16_bf16(w, x, c, 0, 0, 0);
        else
          return __builtin_amdgcn_mfma_f32_16x16x32_bf16(w, x, c, 0, 0, 0);
      };
      const int f_rc = lane % MF, f_kc = lane / MF;
      struct Frags {
        bf16x8_t af[C::kKS][C::kTM];
        uint32_t bw[C::kKS][C::kTN];
        uint32_t s2[C::kTN];
      };
      // MF == 32: the lane's LDS byte offsets inside a ring slot, computed once
      // per tile and held in registers for the K loop (the opaque moves keep
      // the compiler from recomputing them every step): one per A k sub-step
      // (row sub-tile i adds i * MF rows: swz8 depends on the low four row
      // bits only), one for the weights and one for the scales (column
      // sub-tile j adds a constant column offset).  A step then adds the
      // slot base to these six registers and reads with immediate offsets.
      uint32_t fo_a[C::kKS], fo_b = 0, fo_s = 0;
      if constexpr (MF == 32) {
#pragma unroll
        for (int kk = 0; kk < C::kKS; ++kk) {
          const int kc = kk * 2 + f_kc;
          fo_a[kk] = opaque_u32(static_cast<uint32_t>(f_rc * 128 + ((kc ^ swz8(f_rc)) * 16)));
        }
        const int c0 = dlds_col<BN, C::kTN, EPI, MF>(wn, 0) + f_rc;
        fo_b = opaque_u32(static_cast<uint32_t>(C::kABytes + c0 * 32 + f_kc * 16));
        fo_s = opaque_u32(static_cast<uint32_t>(C::kABytes + C::kBBytes + c0 * 2));
      }
      auto read_frags = [&](int slot, Frags& f) __attribute__((always_inline)) {
        if constexpr (MF == 32) {
          const uint32_t sb = lds_offset(smem) + static_cast<uint32_t>(slot * C::kSlot);
          const uint32_t pa0 = sb + fo_a[0], pb = sb + fo_b, ps = sb + fo_s;
#pragma unroll
          for (int j = 0; j < C::kTN; ++j) {
            const int dc = dlds_col<BN, C::kTN, EPI, MF>(0, j) - dlds_col<BN, C::kTN, EPI, MF>(0, 0);
            f.s2[j] = lds_load<uint16_t>(ps + dc * 2);
            typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
            const u32x4_t w = lds_load<u32x4_t>(pb + dc * 32);
            f.bw[0][j] = w[0];
            f.bw[1][j] = w[1];
            f.bw[2][j] = w[2];
            f.bw[3][j] = w[3];
          }
#pragma unroll
          for (int kk = 0; kk < C::kKS; ++kk) {
            const uint32_t pa = kk == 0 ? pa0 : sb + fo_a[kk];
#pragma unroll
            for (int i = 0; i < C::kTM; ++i) f.af[kk][i] = lds_load<bf16x8_t>(pa + i * MF * 128);
          }
          return;
        }
        const uint8_t* as = smem + slot * C::kSlot;
        const uint8_t* bs = as + C::kABytes;
        const uint8_t* ss = bs + C::kBBytes;
#pragma unroll
        for (int j = 0; j < C::kTN; ++j) {
          const int c = dlds_col<BN, C::kTN, EPI, MF>(wn, j) + f_rc;
          f.s2[j] = *reinterpret_cast<const uint16_t*>(ss + c * 2);
        }
#pragma unroll
        for (int kk = 0; kk < C::kKS; ++kk) {
          const int kc = kk * (64 / MF) + f_kc;
#pragma unroll
          for (int j = 0; j < C::kTN; ++j) {
            const int c = dlds_col<BN, C::kTN, EPI, MF>(wn, j) + f_rc;
            if constexpr (MF == 32) {
              if (kk == 0) {
                const uint4 w = *reinterpret_cast<const uint4*>(bs + c * 32 + f_kc * 16);
                f.bw[0][j] = w.x;
                f.bw[1][j] = w.y;
                f.bw[2][j] = w.z;
                f.bw[3][j] = w.w;
              }
            } else {
              f.bw[kk][j] = *reinterpret_cast<const uint32_t*>(bs + c * 32 + mx_dword_pos(kc) * 4);
            }
          }
#pragma unroll
          for (int i = 0; i < C::kTM; ++i) {
            const int r = i * MF + f_rc;
            f.af[kk][i] = *reinterpret_cast<const bf16x8_t*>(as + r * 128 + ((kc ^ swz8(r)) * 16));
          }
        }
      };
      // Conversions and MFMAs of one step: every weight fragment converted
      // with v_cvt_scalef32_pk_bf16_fp4, rewritten by the exact per-byte
      // conversion behind one wave-uniform branch when some lane holds a
      // scale byte outside 3..252, then the MFMAs.
      uint64_t edge_seen = 0;  // lanes that met a scale byte outside 3..252 in this tile
      auto compute = [&](const Frags& f, auto full_tag) __attribute__((always_inline)) {
        constexpr bool kFull = decltype(full_tag)::value;
        bool edge_lane = false;
#pragma unroll
        for (int j = 0; j < C::kTN; ++j) edge_lane |= !hw_scale_ok(f.s2[j] & 0xffu) || !hw_scale_ok(f.s2[j] >> 8);
        const uint64_t edge_mask = __builtin_amdgcn_ballot_w64(edge_lane);
        // MF == 32: no branch inside the step, so the conversions and the
        // MFMAs stay one basic block; a wave that met an edge scale byte
        // recomputes its tile exactly after the K loop (exact_tile below).
        // MF == 16: the exact conversion replaces the step's values here.
        const bool edge = MF == 32 ? false : edge_mask != 0;
        if constexpr (MF == 32) edge_seen |= edge_mask;
        uint32_t bq[C::kKS][C::kTN][4];
#pragma unroll
        for (int kk = 0; kk < C::kKS; ++kk)
#pragma unroll
          for (int j = 0; j < C::kTN; ++j) {
            const uint32_t w = f.bw[kk][j];
            const uint32_t sb = (f.s2[j] >> (8 * (kk / (C::kKS / 2)))) & 0xffu;  // 32-k scale block of sub-step kk
            const float sc = __uint_as_float(sb << 23);
            bq[kk][j][0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 0));
            bq[kk][j][1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 1));
            bq[kk][j][2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 2));
            bq[kk][j][3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 3));
          }
        if (__builtin_expect(edge, false)) {
#pragma unroll
          for (int kk = 0; kk < C::kKS; ++kk)
#pragma unroll
            for (int j = 0; j < C::kTN; ++j) {
              const uint32_t w = f.bw[kk][j];
              const uint32_t sb = (f.s2[j] >> (8 * (kk / (C::kKS / 2)))) & 0xffu;
#pragma unroll
              for (int b = 0; b < 4; ++b) bq[kk][j][b] = dequant_byte((w >> (8 * b)) & 0xffu, sb);
            }
        }
#pragma unroll
        for (int kk = 0; kk < C::kKS; ++kk)
#pragma unroll
          for (int j = 0; j < C::kTN; ++j) {
            const bf16x8_t bfr =
                __builtin_bit_cast(bf16x8_t, uint4{bq[kk][j][0], bq[kk][j][1], bq[kk][j][2], bq[kk][j][3]});
#pragma unroll
            for (int i = 0; i < C::kTM; ++i) {
              if (!kFull && i >= tm_eff) break;
              acc[i][j] = mfma(bfr, f.af[kk][i], acc[i][j]);
            }
          }
      };
      auto k_loop = [&](auto full_tag) __attribute__((always_inline)) {
        // 32-bit wave-uniform loop state, so the loop control, slot rotation
        // and DMA bases stay on the scalar unit
        int slot = __builtin_amdgcn_readfirstlane(slot0);  // slot of step kt
        const int nk32 = static_cast<int>(nk);
        for (int kt = 0; kt < nk32; ++kt) {
          // wait for step kt: (a) later DMA steps issued, (b) prefetched
          // tiles' first steps are older than the previous epilogue's stores
          const int left = nk32 - 1 - kt;
          const int a = pf || left >= NS - 2 ? NS - 2 : left;
          const int b = (cur_pf && kt <= NS - 2) ? prev_rounds : 0;
          if (__builtin_expect(a == NS - 2 && b == 0, 1)) {  // steady state: one test
            if (wave == 0)
              wait_vm_lgkm<(NS - 2) * C::kOps0>();
            else
              wait_vm_lgkm<(NS - 2) * C::kOps>();
          } else if (wave == 0) {
            wait_stream<NS, C::kOps0, S::kStoresPerRound, S::kRounds>(a, b);
          } else {
            wait_stream<NS, C::kOps, S::kStoresPerRound, S::kRounds>(a, b);
          }
          barrier();
          // the step's DMA issue, fragment reads, conversions and MFMAs at a
          // raised wave priority, so the SIMD's arbiter favours the wave that
          // has just passed its barrier over the waves still waiting or in
          // their epilogue (gate/up 131.7 -> 128.8 us, A/B on two boxes; the
          // priority through the MFMAs is what counts)
          __builtin_amdgcn_s_setprio(1);
          // refill the slot of step kt-1: this tile's step kt+NS-1, or the
          // next tile's step kt+NS-1-nk
          const int wslot = __builtin_amdgcn_readfirstlane(slot == 0 ? NS - 1 : slot - 1);
          const int s = kt + NS - 1;
          if (s < nk32)
            issue(ca, s, wslot);
          else if (pf)
            issue(make_addr(nxt, nt_n, tid, ord + 1), s - nk32, wslot);
          Frags f;
          read_frags(slot, f);
          compute(f, full_tag);
          __builtin_amdgcn_s_setprio(0);
          slot = slot == NS - 1 ? 0 : slot + 1;
        }
      };
      if (tm_eff >= C::kTM)
        k_loop(std::true_type{});
      else
        k_loop(std::false_type{});

      // exact_tile: a wave whose columns met a scale byte outside 3..252 in
      // this tile (the hardware conversion is exact only inside that range;
      // such bytes mean weights below 2^-124 or above 2^125) recomputes its
      // accumulators from global memory with the exact per-byte conversion,
      // the fragments read exactly as the K loop reads them from LDS.  It
      // touches neither the LDS ring nor the DMA stream; waiting for its loads
      // (vmcnt(0)) only waits longer than the stream's own counts require.
      if constexpr (MF == 32) {
        if (__builtin_expect(edge_seen != 0, 0)) {
          const bool gathered = p.a_index != nullptr;
          const uint16_t* arow[C::kTM];
#pragma unroll
          for (int i = 0; i < C::kTM; ++i) {
            const int row = i * MF + f_rc;
            arow[i] = gathered ? p.lhs + static_cast<int64_t>(s_idx[ord * BM + row]) * K
                               : p.lhs + (cur.row0 + (row < cur.rows ? row : 0)) * K;
          }
          const uint8_t* wg = static_cast<const uint8_t*>(p.rhs) + cur.group * N * (K / 2);
          const uint8_t* sg = p.scale + cur.group * (K / 64) * N * 2;
          int64_t gcol[C::kTN];
#pragma unroll
          for (int j = 0; j < C::kTN; ++j) gcol[j] = drhs_col<BN, EPI>(nt, dlds_col<BN, C::kTN, EPI, MF>(wn, j) + f_rc, N);
#pragma unroll
          for (int i = 0; i < C::kTM; ++i)
#pragma unroll
            for (int j = 0; j < C::kTN; ++j)
#pragma unroll
              for (int e = 0; e < C::kAccN; ++e) acc[i][j][e] = 0.f;
          for (int64_t kt = 0; kt < nk; ++kt) {
            uint4 w[C::kTN];
            uint32_t s2[C::kTN];
#pragma unroll
            for (int j = 0; j < C::kTN; ++j) {
              w[j] = *reinterpret_cast<const uint4*>(wg + kt * (N * 32) + gcol[j] * 32 + f_kc * 16);
              s2[j] = *reinterpret_cast<const uint16_t*>(sg + kt * (N * 2) + gcol[j] * 2);
            }
#pragma unroll
            for (int kk = 0; kk < C::kKS; ++kk) {
              const int kc = kk * 2 + f_kc;
#pragma unroll
              for (int j = 0; j < C::kTN; ++j) {
                const uint32_t wd = kk == 0 ? w[j].x : kk == 1 ? w[j].y : kk == 2 ? w[j].z : w[j].w;
                const uint32_t sb = (s2[j] >> (8 * (kk / (C::kKS / 2)))) & 0xffu;
                uint32_t q[4];
#pragma unroll
                for (int b = 0; b < 4; ++b) q[b] = dequant_byte((wd >> (8 * b)) & 0xffu, sb);
                const bf16x8_t bfr = __builtin_bit_cast(bf16x8_t, uint4{q[0], q[1], q[2], q[3]});
#pragma unroll
                for (int i = 0; i < C::kTM; ++i) {
                  if (i >= tm_eff) break;
                  const bf16x8_t af = *reinterpret_cast<const bf16x8_t*>(arow[i] + kt * kSK + kc * 8);
                  acc[i][j] = mfma(bfr, af, acc[i][j]);
                }
              }
            }
          }
        }
      }

      // Epilogue: stage in the slot of the last step, round by round.
      const int stage_slot = static_cast<int>((slot0 + nk - 1) % NS);
      uint8_t* stg = smem + stage_slot * C::kSlot;
      const int last_ch = static_cast<int>((n_out - col0 < S::kOutCols ? n_out - col0 : S::kOutCols) / 8) - 1;
      const SituConsts sc = situ_consts(p.beta, p.beta_lin);
      static_for<S::kRounds>([&](auto rc) __attribute__((always_inline)) {
        constexpr int R = decltype(rc)::value;
        if (R > 0 && R >= rounds) return false;  // a tile has >= 1 row: round 0 always runs
        lds_barrier();  // the slot's previous readers are done
#pragma unroll
        for (int i = 0; i < C::kTM; ++i) {
          if (i * MF / S::kStageRows != R) continue;
          uint8_t* srow = stg + (i * MF + r_in - R * S::kStageRows) * S::kStageRow;
#pragma unroll
          for (int j = 0; j < kOutTN; ++j)
#pragma unroll
            for (int q = 0; q < kRuns; ++q) {
              float v[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                if constexpr (EPI == kEpiSitu) {
                  float gv = acc[i][j][q * 4 + e], uv = acc[i][j + kOutTN][q * 4 + e];
                  if (p.round_before_act) {
                    round_pair_bf16(gv, uv);
                  }
                  v[e] = situ_epi(gv, uv, sc);
                } else {
                  v[e] = acc[i][j][q * 4 + e];
                }
              }
              *reinterpret_cast<uint2*>(srow + (wn * kOutTN * MF + j * MF + c_run(q)) * 2) =
                  uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            }
        }
        lds_barrier();
#pragma unroll
        for (int v = 0; v < S::kStoresPerRound; ++v) {
          const int idx = tid + C::kThreads * v;
          int row = R * S::kStageRows + idx / S::kChunks, ch = idx % S::kChunks;
          // out-of-range rows / columns store a valid neighbour again, so
          // every lane issues the same number of stores
          row = row < cur.rows ? row : cur.rows - 1;
          ch = ch <= last_ch ? ch : last_ch;
          const uint4 val =
              *reinterpret_cast<const uint4*>(stg + (row - R * S::kStageRows) * S::kStageRow + ch * 16);
          *reinterpret_cast<uint4*>(out + (cur.row0 + row) * n_out + col0 + ch * 8) = val;
        }
        return true;
      });
      slot0 = static_cast<int>((slot0 + nk) % NS);
    } else if (p.skip_zero_rows) {
      // the caller never reads the zero group's rows or those past the
      // groups: nothing to store
    } else {
      // padding bucket / tail rows: zeros, stored directly (the zero comes
      // from an opaque move, so it is not a constant held across the K loop)
      uint32_t z;
      asm volatile("v_mov_b32 %0, 0" : "=v"(z));
      constexpr int kZeroOps = BM * S::kChunks / C::kThreads;
#pragma unroll
      for (int v = 0; v < kZeroOps; ++v) {
        const int idx = tid + C::kThreads * v;
        const int row = idx / S::kChunks, ch = idx % S::kChunks;
        if (row < cur.rows && col0 + ch * 8 < n_out)
          *reinterpret_cast<uint4*>(out + (cur.row0 + row) * n_out + col0 + ch * 8) = uint4{z, z, z, z};
      }
    }
    cur = nxt;
    nt = nt_n;
    vb = vb_n;
    ++ord;
    cur_pf = pf;
    prev_rounds = rounds;
  }
}

// Compute units of the current device (cached per device; threads that race
// on the first query store the same value).
int cu_count() {
  static std::atomic<int> cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

template <int BM, int BN, int LAYOUT, int EPI, int NS, int WM = 1, int WN = 4, int MF = 32>
int launch_dma(const Params& p, hipStream_t st, const char* name) {
  if constexpr (EPI == kEpiSitu && (BN / WN / MF) % 2 != 0) {
    return fail(LMOE_ERR_UNSUPPORTED, "%s: SiTU tile %dx%d with %dx%d MFMAs has no gate/up pairing", name, BM, BN, MF,
                MF);
  } else {
  using C = DCfg<BM, BN, LAYOUT, EPI, NS, WM, WN, MF>;
  const int64_t out_cols = EPI == kEpiSitu ? p.N / 2 : p.N;
  const int64_t cols_per_tile = EPI == kEpiSitu ? BN / 2 : BN;
  const int64_t ntiles = ceil_div(out_cols, cols_per_tile);
  const int64_t mtiles = ceil_div(p.M, BM) + p.G + 1;
  if (ntiles == 0 || p.M == 0) return LMOE_OK;
  int gm = p.G == 1 ? 4 : 1;
  if (p.G == 1) {
    // dense: groups of gm m-tiles go round-robin over the XCDs; keep every
    // XCD busy (at least one group each) with tall tiles
    const int64_t real_m = ceil_div(p.M, BM);
    while (gm > 1 && ceil_div(real_m, gm) < kXcds) gm /= 2;
  }
  int64_t blocks = kXcds * ceil_div(ceil_div(mtiles, gm), kXcds) * gm * ntiles;
  if ((p.G > 1 || p.k_split > 1) && ntiles % kXcds == 0) {
    // n-tiles striped over the XCDs (split-K too: with few m-tiles the
    // m-tile groups would leave most XCDs without work); measured against
    // round-robin m-tiles and per-XCD m-tile ranges, which were slower
    gm = 0;
    blocks = mtiles * ntiles;
  }
  blocks *= p.k_split;  // one virtual block per (tile, K range)
  LMOE_CHECK_SUPPORTED(blocks < (1ll << 31), "%s: grid too large", name);
  // per-lane DMA offsets are 32-bit: one group's weights and one tile's rows
  const int64_t w_bytes = p.N * (LAYOUT != kDMX ? p.K * 2 : p.K / 2);
  LMOE_CHECK_SUPPORTED(w_bytes < (1ll << 32) && BM * p.K * 2 < (1ll << 32), "%s: group too large for the DMA path",
                       name);
  const size_t lds = static_cast<size_t>(NS) * C::kSlot;
  static const hipError_t attr_rc =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&grouped_gemm_dma_kernel<BM, BN, LAYOUT, EPI, NS, WM, WN, MF>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  if (attr_rc != hipSuccess)
    return fail(LMOE_ERR_HIP, "%s: LDS size attribute (%zu bytes): %s", name, lds, hipGetErrorString(attr_rc));
  // one block per tile (measured equal to or faster than a persistent grid on
  // the expert shapes: the hardware's block refill overlaps one block's
  // epilogue with its neighbours' main loops)
  grouped_gemm_dma_kernel<BM, BN, LAYOUT, EPI, NS, WM, WN, MF>
      <<<dim3(static_cast<unsigned>(blocks)), C::kThreads, lds, st>>>(p, ntiles, gm, blocks);
  LMOE_CHECK_LAUNCH(name);
  return LMOE_OK;
  }
}

// The streamed persistent kernel: bf16 output, and the LDS tile table
// (8 (G + 1) bytes) must leave room for the blocks per CU that the ring alone
// allows.  Returns 1 when it ran (or failed: *rc set), 0 when it does not
// apply.
template <int BM, int BN, int EPI, int NS, int MF>
int try_stream(const Params& p, hipStream_t st, const char* name, int* rc) {
  using S = SCfg<BM, BN, EPI, NS, MF>;
  using C = typename S::C;
  if (p.G < 1 || p.M == 0) return 0;
  if (EPI != kEpiSitu && p.out_dtype != LMOE_BF16) return 0;
  const int64_t ring = static_cast<int64_t>(NS) * C::kSlot;
  const int64_t lds = ring + ((8 * (p.G + 1) + 15) / 16) * 16 + (p.a_index ? S::kIdxBytes : 0);
  const int64_t per_cu = 163840 / (lds + 64);
  if (per_cu < 1 || per_cu < C::kLdsBlocks) return 0;
  const int64_t out_cols = EPI == kEpiSitu ? p.N / 2 : p.N;
  const int64_t ntiles = ceil_div(out_cols, S::kOutCols);
  const int64_t mtiles = ceil_div(p.M, BM) + p.G + 1;
  int gm = p.G == 1 ? 4 : 1;
  int64_t blocks = kXcds * ceil_div(ceil_div(mtiles, gm), kXcds) * gm * ntiles;
  // grouped problems: n-tiles striped over the XCDs (each weight slice read
  // by one XCD; measured fastest at config 5, 137.8 us for the gate/up).  A
  // balanced contiguous m-tile range per XCD (gm < 0) moved 21% less HBM
  // traffic (297 against 377 MB for the gate/up) but measured 4% slower.
  if (p.G > 1 && ntiles % kXcds == 0) {
    gm = 0;
    blocks = mtiles * ntiles;
  }
  *rc = LMOE_OK;
  if (blocks >= (1ll << 31)) {
    *rc = fail(LMOE_ERR_UNSUPPORTED, "%s: grid too large", name);
    return 1;
  }
  const int64_t w_bytes = p.N * (p.K / 2);
  if (!(w_bytes < (1ll << 32) && BM * p.K * 2 < (1ll << 32))) {
    *rc = fail(LMOE_ERR_UNSUPPORTED, "%s: group too large for the DMA path", name);
    return 1;
  }
  // raise the kernel's dynamic LDS limit when a larger table needs it; the
  // raise and its record happen under one lock, so the limit only grows and a
  // thread that needs less never lowers it under one that needs more
  static std::mutex lds_mu;
  static std::atomic<int64_t> lds_set{0};
  if (lds > lds_set.load(std::memory_order_acquire)) {
    std::lock_guard<std::mutex> lock(lds_mu);
    if (lds > lds_set.load(std::memory_order_relaxed)) {
      const hipError_t attr_rc =
          hipFuncSetAttribute(reinterpret_cast<const void*>(&grouped_gemm_stream_kernel<BM, BN, EPI, NS, MF>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
      if (attr_rc != hipSuccess) {
        *rc = fail(LMOE_ERR_HIP, "%s: LDS size attribute (%lld bytes): %s", name, (long long)lds,
                   hipGetErrorString(attr_rc));
        return 1;
      }
      lds_set.store(lds, std::memory_order_release);
    }
  }
  const int64_t resident = kXcds * ((static_cast<int64_t>(cu_count()) * C::kLdsBlocks) / kXcds);
  const int64_t grid = resident >= kXcds && resident < blocks ? resident : blocks;
  if (p.a_index && ceil_div(blocks, grid) > S::kIdxTiles) {
    *rc = fail(LMOE_ERR_UNSUPPORTED, "%s: gathered rows need <= %d tiles per block (%lld)", name, S::kIdxTiles,
               (long long)ceil_div(blocks, grid));
    return 1;
  }
  grouped_gemm_stream_kernel<BM, BN, EPI, NS, MF>
      <<<dim3(static_cast<unsigned>(grid)), C::kThreads, static_cast<size_t>(lds), st>>>(p, ntiles, gm, blocks);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) *rc = fail(LMOE_ERR_HIP, "%s: launch failed: %s", name, hipGetErrorString(e));
  return 1;
}

// Re-tile MXFP4 weights to k-step-major order: packed (G, N, K/2) ->
// (G, K/64, N, 32) with each 32-byte record's dwords in mx_dword_pos order,
// and E8M0 scales (G, N, K/32) -> (G, K/64, N, 2).  One thread per (group,
// step, column): two 16-byte copies and one 2-byte copy.
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
    const uint4 a = src[0], b = src[1];  // logical dwords 0..3, 4..7
    dst[0] = uint4{a.x, a.z, b.x, b.z};  // 0, 2, 4, 6
    dst[1] = uint4{a.y, a.w, b.y, b.w};  // 1, 3, 5, 7
    const uint8_t* ss = scale + (g * N + n) * (K / 32) + 2 * s;
    scale_out[2 * i] = ss[0];
    scale_out[2 * i + 1] = ss[1];
  }
}

// Tile shapes of the MXFP4 kernel, from sweeps on the LatentMoE expert shapes
// (64x128 / 64x256 / 128x128 / 128x256 / 32x128 / 32x256 tiles, ring depths
// 2-6, 16x16x32 against 32x32x16 MFMAs, fragments read one step ahead): the
// streamed kernel with 64x256 tiles and a 3-deep ring (3 blocks per CU) where
// it applies, else the one-block-per-tile kernel with 64x256 tiles, ring depth
// 3 for the fused gate/up and 4 for the down projection.
template <int EPI>
int run_mx(const Params& p, hipStream_t st, const char* name) {
  int rc = LMOE_OK;
  if (try_stream<64, 256, EPI, 3, 32>(p, st, name, &rc)) return rc;
  // gathered rows: the streamed kernel only
  if (p.a_index) return fail(LMOE_ERR_UNSUPPORTED, "%s: gathered rows need the streamed 64x256 kernel", name);
  if constexpr (EPI == kEpiSitu)
    return launch_dma<64, 256, kDMX, EPI, 3, 1, 4, 32>(p, st, name);
  else
    return launch_dma<64, 256, kDMX, EPI, 4, 1, 4, 32>(p, st, name);
}

// Tile shapes of the bf16 (GNK) kernel, the sweep winners on the LatentMoE
// dense projections and bf16 expert shapes: 128x128 tiles of 2x2 waves for a
// short K (the 1024-deep up-projection as one group), else 64x128 tiles of
// 1x4 waves on 16x16x32 MFMAs.
template <int EPI>
int run_gnk(const Params& p, hipStream_t st, const char* name) {
  if constexpr (EPI == kEpiNone) {
    if (p.K <= 1024 && p.G == 1) return launch_dma<128, 128, kDGNK, EPI, 2, 2, 2, 32>(p, st, name);
  }
  return launch_dma<64, 128, kDGNK, EPI, 3, 1, 4, 16>(p, st, name);
}

// Split-K reduction: out = epilogue(plane 0 + plane 1 + ... + plane S-1),
// the planes added in that order in f32.  The SiTU epilogue pairs columns j
// and N/2 + j of the summed planes as the fused kernels do (both rounded to
// bf16 first).  One thread per run of four output columns.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ ws, int64_t S, int64_t stride,
                                                            int64_t M, int64_t N, int epi, float beta, float beta_lin,
                                                            int out_dtype, void* __restrict__ out) {
  const int64_t n_out = epi == kEpiSitu ? N / 2 : N;
  const int64_t runs = n_out / 4;
  const int64_t total = M * runs;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t r = i / runs, c = (i - r * runs) * 4;
    if (epi == kEpiSitu) {
      const float* pg = ws + r * N + c;
      float4 g = *reinterpret_cast<const float4*>(pg);
      float4 u = *reinterpret_cast<const float4*>(pg + N / 2);
      for (int64_t sp = 1; sp < S; ++sp) {
        const float4 dg = *reinterpret_cast<const float4*>(pg + sp * stride);
        const float4 du = *reinterpret_cast<const float4*>(pg + sp * stride + N / 2);
        g.x += dg.x; g.y += dg.y; g.z += dg.z; g.w += dg.w;
        u.x += du.x; u.y += du.y; u.z += du.z; u.w += du.w;
      }
      const SituConsts sc = situ_consts(beta, beta_lin);
      const float gv[4] = {g.x, g.y, g.z, g.w}, uv[4] = {u.x, u.y, u.z, u.w};
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float a = gv[e], b = uv[e];
        round_pair_bf16(a, b);
        v[e] = situ_epi(a, b, sc);
      }
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + r * n_out + c) =
          uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    } else {
      const float* pa = ws + r * N + c;
      float4 a = *reinterpret_cast<const float4*>(pa);
      for (int64_t sp = 1; sp < S; ++sp) {
        const float4 d = *reinterpret_cast<const float4*>(pa + sp * stride);
        a.x += d.x; a.y += d.y; a.z += d.z; a.w += d.w;
      }
      if (out_dtype == LMOE_F32)
        *reinterpret_cast<float4*>(static_cast<float*>(out) + r * n_out + c) = a;
      else
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + r * n_out + c) =
            uint2{pack_bf16x2(a.x, a.y), pack_bf16x2(a.z, a.w)};
    }
  }
}

// The bf16 (G, K, N) kernel: 128x256 tiles of 2x4 waves, 32x32 MFMAs
// (config 2, the reference-layout ragged_dot: 71.8 us, the speed of the
// prepared (G, N, K) layout; 64x128 tiles 77.2 us; 128x128 and 64x256 tiles
// slower; transpose + (G, N, K) kernel 118.2 us).
template <int EPI>
int run_gkn(const Params& p, hipStream_t st, const char* name) {
  return launch_dma<128, 256, kDGKN, EPI, 2, 2, 4, 32>(p, st, name);
}

}  // namespace

// Split-K: the DMA kernel (64x128 tiles, 64x256 for M > kSplitWideM)
// computes k_split K ranges of every tile as f32 partial planes in `ws`
// (k_split * M * N floats), then
// splitk_reduce_kernel sums them in order and applies the epilogue.  For a
// few long-K tiles (one group, M <= ~1024) the tile grid alone leaves most of
// the chip idle and each tile's K loop is latency-bound.
constexpr int64_t kSplitWideM = 256;

int run_dma_splitk(const Params& p, int layout, int epi, int64_t k_split, float* ws, hipStream_t st,
                   const char* name) {
  Params q = p;
  q.k_split = k_split;
  q.split_stride = p.M * p.N;
  q.out = ws;
  q.out_dtype = LMOE_F32;
  q.skip_zero_rows = 0;
  int rc;
  // MXFP4: 64 x 128 tiles for a few m-tiles (M <= 256), 64 x 256 above, where
  // half as many n-tiles re-read each activation row (config 4, M = 1024 in
  // 4 ranges: 45.5 us against 48.7 with 64 x 128 tiles in 2 ranges)
  if (layout == kMXFP4 && p.M > kSplitWideM)
    rc = launch_dma<64, 256, kDMX, kEpiNone, 4, 1, 4, 32>(q, st, name);
  else if (layout == kMXFP4)
    rc = launch_dma<64, 128, kDMX, kEpiNone, 4, 1, 4, 32>(q, st, name);
  else if (layout == kGNK)
    rc = launch_dma<64, 128, kDGNK, kEpiNone, 3, 1, 4, 16>(q, st, name);
  else
    rc = fail(LMOE_ERR_UNSUPPORTED, "%s: split-K layout %d", name, layout);
  if (rc != LMOE_OK) return rc;
  const int64_t n_out = epi == kEpiSitu ? p.N / 2 : p.N;
  const int64_t total = p.M * (n_out / 4);
  if (total == 0) return LMOE_OK;
  const int64_t b = ceil_div(total, 256);
  splitk_reduce_kernel<<<static_cast<unsigned>(b < 65536 ? b : 65536), 256, 0, st>>>(
      ws, k_split, q.split_stride, p.M, p.N, epi, p.beta, p.beta_lin, p.out_dtype, p.out);
  LMOE_CHECK_LAUNCH(name);
  return LMOE_OK;
}

int run_dma(const Params& p, int layout, int epi, hipStream_t st, const char* name) {
  if (layout == kGKN && epi == kEpiNone) return run_gkn<kEpiNone>(p, st, name);
  if (layout == kGKN && epi == kEpiSitu) return run_gkn<kEpiSitu>(p, st, name);
  if (layout == kGNK && epi == kEpiNone) return run_gnk<kEpiNone>(p, st, name);
  if (layout == kGNK && epi == kEpiSitu) return run_gnk<kEpiSitu>(p, st, name);
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
