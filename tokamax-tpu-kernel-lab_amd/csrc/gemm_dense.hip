// Dense bf16 GEMM for the layer's plain projections (gfx950):
//   out (M, N) = x (M, K) @ w^T, w stored (N, K) (k-contiguous), f32
//   accumulation, out f32 or bf16.
// The projections it serves: the router logits + down-projection of the
// hidden states (ref.py:620 and ref.py:634-655, one GEMM over the
// concatenated weights, f32 out) and the latent -> hidden up-projection
// (ref.py:430, bf16 out).
//
// Shapes at BASELINE config 5: 4096 x 7168 -> 1920 and 4096 x 1024 -> 7168,
// both MFMA-bound.  A 256 x 128 tile gives 16 x 15 = 240 tiles for the first
// (one round on 256 CUs) and 896 for the second.
//
// Block = 4 waves in a 2 x 2 grid; wave (wm, wn) computes rows
// [128 wm, +128) x columns [64 wn, +64) of the tile as 4 x 2 sub-tiles of
// v_mfma_f32_32x32x16_bf16, the weight fragment as the first operand (the
// accumulator is the transposed sub-tile: a lane owns one output row and runs
// of four adjacent columns).
//
// Pipeline: K advances 64 per step through an NS-slot LDS ring filled by
// direct-to-LDS DMA (global_load_lds_dwordx4, 16-byte chunks of 128-byte rows,
// chunk c of row r stored at position c ^ swz8(r), so fragment reads are
// bank-conflict free).  Each 64-deep step is four 16-deep sub-steps; the 8
// MFMAs of a sub-step run from registers while the next sub-step's 6 operand
// fragments are read from LDS (two fragment sets of 24 VGPRs, so the 128
// accumulators stay in architectural VGPRs).  Before the first read of step
// k+1: wait for its DMA (s_waitcnt vmcnt) and this wave's LDS reads, then
// s_barrier, after which every wave holds step k's last fragments, so the
// slot of step k refills with the DMA of step k+NS.
// The DMA is issued from inline asm, so every vector memory operation inside
// the K loop is one of these and the wait counts are exact.
//
// Tile order: tile t = mt * n_tiles + nt; XCD x (block b runs on XCD b % 8)
// takes the contiguous range of tiles [x T / 8, (x + 1) T / 8), so an XCD
// works on a few m-panels and reads each of their A rows from its own L2.

#include "dma_util.h"
#include "gemm_tile.h"

namespace lmoe {
namespace gemm {
namespace {

using namespace lmoe::dma;

// KG wave groups of 2 x 2 waves split every 64-deep step's four 16-deep
// sub-steps between them (group g takes sub-steps [g * 4 / KG, +4 / KG)); the
// groups' accumulators are added through LDS after the K loop.  KG = 2 puts
// two waves on each SIMD: twice the waves issuing the DMA (one wave moves
// about 20 GB/s through global_load_lds, so four waves cannot feed a
// 256 x 128 tile at the MFMA rate) and a second wave to issue MFMAs while the
// first waits, with the same per-wave fragment traffic.
template <int BM, int BN, int NS, int KG>
struct DenseCfg {
  static constexpr int kThreads = 256 * KG, kWaves = 4 * KG, kWM = 2, kWN = 2;
  static constexpr int kWTM = BM / kWM, kWTN = BN / kWN;  // wave tile
  static constexpr int kTM = kWTM / 32, kTN = kWTN / 32;  // 32x32 sub-tiles per wave
  static constexpr int kKS = 4 / KG;                      // 16-deep MFMA sub-steps per wave per 64-deep step
  static constexpr int kABytes = BM * 128, kBBytes = BN * 128;
  static constexpr int kSlot = kABytes + kBBytes;
  static constexpr int kAOps = BM * 8 / kThreads, kBOps = BN * 8 / kThreads;  // DMA per thread per step
  static constexpr int kOps = kAOps + kBOps;
  static constexpr int kRedBytes = (KG - 1) * 4 * kTM * kTN * 16 * 64 * 4;  // group 1's accumulators
  static_assert(BM % 64 == 0 && BN % 64 == 0, "tile");
  static_assert(KG == 1 || KG == 2, "wave groups");
  static_assert(kAOps * kThreads == BM * 8 && kBOps * kThreads == BN * 8, "DMA split");
  static_assert((NS - 1) * kOps < 64, "vmcnt range");
  static_assert(NS * kSlot <= 163840 && kRedBytes <= NS * kSlot, "LDS ring");
};

template <int BM, int BN, int NS, int KG, bool F32>
__global__ __launch_bounds__(256 * KG) __attribute__((amdgpu_waves_per_eu(KG, KG)))
void dense_gemm_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, int M, int N, int K,
                       int n_tiles, int tiles, int per_xcd, void* __restrict__ out) {
  using C = DenseCfg<BM, BN, NS, KG>;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int b = blockIdx.x;
  const int t = (b % kXcds) * per_xcd + b / kXcds;
  if (b / kXcds >= per_xcd || t >= tiles) return;
  const int mt = t / n_tiles, nt = t % n_tiles;
  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int kg = wave / 4, wq = wave % 4;  // wave group, wave within the group
  const int wm = wq / C::kWN, wn = wq % C::kWN;
  const int kb = kg * C::kKS;  // this group's first sub-step
  const int nk = K / 64;

  // DMA addressing: SGPR bases advanced by one step (128 bytes) per step,
  // loop-invariant 32-bit per-lane offsets.  Rows past M / N read the last
  // valid row (never stored).
  const uint8_t* a_base = uniform_ptr(x + static_cast<int64_t>(mt) * BM * K);
  const uint8_t* b_base = uniform_ptr(w + static_cast<int64_t>(nt) * BN * K);
  const int a_rows = M - mt * BM < BM ? M - mt * BM : BM;
  const int b_rows = N - nt * BN < BN ? N - nt * BN : BN;
  uint32_t a_off[C::kAOps], b_off[C::kBOps];
#pragma unroll
  for (int v = 0; v < C::kAOps; ++v) {
    const int q = tid + C::kThreads * v;
    const int row = q / 8, kc = (q % 8) ^ swz8(row);
    a_off[v] = static_cast<uint32_t>((row < a_rows ? row : a_rows - 1) * K * 2 + kc * 16);
  }
#pragma unroll
  for (int u = 0; u < C::kBOps; ++u) {
    const int q = tid + C::kThreads * u;
    const int row = q / 8, kc = (q % 8) ^ swz8(row);
    b_off[u] = static_cast<uint32_t>((row < b_rows ? row : b_rows - 1) * K * 2 + kc * 16);
  }
  const uint32_t lds_wave = __builtin_amdgcn_readfirstlane(lds_offset(smem) + wave * 64 * 16);
  auto issue = [&](int step, int slot) __attribute__((always_inline)) {
    const uint32_t base = lds_wave + slot * C::kSlot;
#pragma unroll
    for (int v = 0; v < C::kAOps; ++v) dma16s(a_off[v], a_base + step * 128, base + v * C::kThreads * 16);
#pragma unroll
    for (int u = 0; u < C::kBOps; ++u) dma16s(b_off[u], b_base + step * 128, base + C::kABytes + u * C::kThreads * 16);
  };

  // fragment coordinates: lane holds row / column (lane % 32), k chunk
  // kk * 2 + lane / 32 of the 128-byte row
  const int f_rc = lane % 32, f_kc = lane / 32;
  // operand fragments of one 16-deep sub-step
  struct Frag {
    bf16x8_t a[C::kTM];
    bf16x8_t b[C::kTN];
  };
  auto read_frag = [&](int slot, int kk, Frag& f) __attribute__((always_inline)) {
    const uint8_t* as = smem + slot * C::kSlot;
    const uint8_t* bs = as + C::kABytes;
    const int kc = kk * 2 + f_kc;
#pragma unroll
    for (int j = 0; j < C::kTN; ++j) {
      const int c = wn * C::kWTN + j * 32 + f_rc;
      f.b[j] = *reinterpret_cast<const bf16x8_t*>(bs + c * 128 + ((kc ^ swz8(c)) * 16));
    }
#pragma unroll
    for (int i = 0; i < C::kTM; ++i) {
      const int r = wm * C::kWTM + i * 32 + f_rc;
      f.a[i] = *reinterpret_cast<const bf16x8_t*>(as + r * 128 + ((kc ^ swz8(r)) * 16));
    }
  };

  floatx16 acc[C::kTM][C::kTN];
#pragma unroll
  for (int i = 0; i < C::kTM; ++i)
#pragma unroll
    for (int j = 0; j < C::kTN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  auto compute = [&](const Frag& f) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < C::kTM; ++i)
#pragma unroll
      for (int j = 0; j < C::kTN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.b[j], f.a[i], acc[i][j], 0, 0, 0);
  };
  // wait until a step has landed when `younger` (0 .. NS-1) later steps were
  // issued after it (anything else waits for every DMA), then barrier
  auto land = [&](int younger) __attribute__((always_inline)) {
    if (younger < 0 || younger >= NS) wait_vm_lgkm<0>();
    static_for<NS>([&](auto yc) __attribute__((always_inline)) {
      constexpr int Y = decltype(yc)::value;
      if (younger == Y) wait_vm_lgkm<Y * C::kOps>();
      return true;
    });
    barrier();
  };

  // prologue: steps 0 .. NS-1 in flight, sub-step (0, 0)'s fragments in
  // registers
  static_for<NS>([&](auto sc) __attribute__((always_inline)) {
    constexpr int s = decltype(sc)::value;
    if (s < nk) issue(s, s);
    return true;
  });
  Frag fa, fb;
  land((nk - 1 < NS - 1 ? nk - 1 : NS - 1));
  read_frag(0, kb, fa);
  // Sub-step (k, kk) computes from registers while the next sub-step's
  // fragments are read.  Before the read of (k+1, 0): step k+1 lands and the
  // barrier also makes every wave's reads of step k complete, so slot k % NS
  // refills with step k + NS.  Four sub-steps per step alternate fa / fb, so
  // each step starts from fa.
  for (int k = 0; k < nk; ++k) {
    const int slot = k % NS;
    read_frag(slot, kb + 1, fb);
    compute(fa);
    if constexpr (C::kKS == 4) {
      read_frag(slot, kb + 2, fa);
      compute(fb);
      read_frag(slot, kb + 3, fb);
      compute(fa);
    }
    if (k + 1 < nk) {
      // steps issued after k+1: k+2 .. min(k+NS-1, nk-1)
      const int last = nk - 1 < k + NS - 1 ? nk - 1 : k + NS - 1;
      land(last - (k + 1));
      if (k + NS < nk) issue(k + NS, slot);
      read_frag((k + 1) % NS, kb, fa);
    }
    compute(fb);
  }

  if constexpr (KG == 2) {
    // group 1 hands its accumulators to group 0 through the (drained) ring:
    // lane-contiguous float4 runs, conflict-free both ways
    float4* red = reinterpret_cast<float4*>(smem);
    auto red_at = [&](int i, int j, int q) __attribute__((always_inline)) {
      return ((wq * C::kTM * C::kTN + i * C::kTN + j) * 4 + q) * 64 + lane;
    };
    __syncthreads();  // every wave's last fragment reads of the ring are done
    if (kg == 1) {
#pragma unroll
      for (int i = 0; i < C::kTM; ++i)
#pragma unroll
        for (int j = 0; j < C::kTN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            red[red_at(i, j, q)] = float4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                          acc[i][j][4 * q + 3]};
    }
    __syncthreads();
    if (kg == 1) return;
#pragma unroll
    for (int i = 0; i < C::kTM; ++i)
#pragma unroll
      for (int j = 0; j < C::kTN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float4 v = red[red_at(i, j, q)];
          acc[i][j][4 * q] += v.x;
          acc[i][j][4 * q + 1] += v.y;
          acc[i][j][4 * q + 2] += v.z;
          acc[i][j][4 * q + 3] += v.w;
        }
  }

  // epilogue: lane holds output row (lane % 32) of sub-tile i and, for
  // q = 0..3, columns 8q + 4 (lane / 32) .. +3 of sub-tile j
#pragma unroll
  for (int i = 0; i < C::kTM; ++i) {
    const int row = wm * C::kWTM + i * 32 + f_rc;
    if (row >= a_rows) continue;
    const int64_t obase = (static_cast<int64_t>(mt) * BM + row) * N;
#pragma unroll
    for (int j = 0; j < C::kTN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = wn * C::kWTN + j * 32 + q * 8 + 4 * f_kc;
        if (col >= b_rows) continue;
        const int64_t o = obase + static_cast<int64_t>(nt) * BN + col;
        if constexpr (F32) {
          *reinterpret_cast<float4*>(static_cast<float*>(out) + o) =
              float4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
        } else {
          *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + o) =
              uint2{pack_bf16x2(acc[i][j][4 * q], acc[i][j][4 * q + 1]),
                    pack_bf16x2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3])};
        }
      }
  }
}

template <int BM, int BN, int NS, int KG, bool F32>
int launch_dense(const uint16_t* x, const uint16_t* w, int64_t M, int64_t N, int64_t K, void* out, hipStream_t st) {
  using C = DenseCfg<BM, BN, NS, KG>;
  const int64_t n_tiles = ceil_div(N, BN), tiles = ceil_div(M, BM) * n_tiles;
  const int64_t per_xcd = ceil_div(tiles, kXcds);
  const size_t lds = static_cast<size_t>(NS) * C::kSlot;
  static const hipError_t attr_rc = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&dense_gemm_kernel<BM, BN, NS, KG, F32>),
      hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
  if (attr_rc != hipSuccess)
    return fail(LMOE_ERR_HIP, "dense_gemm: LDS size attribute: %s", hipGetErrorString(attr_rc));
  dense_gemm_kernel<BM, BN, NS, KG, F32><<<dim3(static_cast<unsigned>(kXcds * per_xcd)), C::kThreads, lds, st>>>(
      x, w, static_cast<int>(M), static_cast<int>(N), static_cast<int>(K), static_cast<int>(n_tiles),
      static_cast<int>(tiles), static_cast<int>(per_xcd), out);
  LMOE_CHECK_LAUNCH("dense_gemm");
  return LMOE_OK;
}

}  // namespace
}  // namespace gemm
}  // namespace lmoe

extern "C" int lmoe_dense(const void* x, const void* w_nk, int64_t M, int64_t K, int64_t N, void* out, int out_dtype,
                          void* stream) {
  using namespace lmoe;
  using namespace lmoe::gemm;
  LMOE_CHECK_ARG(M >= 0 && K > 0 && N > 0, "dense: bad sizes M=%lld K=%lld N=%lld", (long long)M, (long long)K,
                 (long long)N);
  LMOE_CHECK_ARG(valid_dtype(out_dtype), "dense: bad out dtype %d", out_dtype);
  if (M == 0) return LMOE_OK;
  LMOE_CHECK_ARG(x && w_nk && out, "dense: null pointer");
  LMOE_CHECK_SUPPORTED(K % 64 == 0 && N % 8 == 0, "dense: needs K %% 64 == 0 and N %% 8 == 0 (K=%lld N=%lld)",
                       (long long)K, (long long)N);
  LMOE_CHECK_SUPPORTED(aligned(x, 16) && aligned(w_nk, 16) && aligned(out, 16), "dense: 16-byte aligned buffers");
  // per-lane DMA offsets are 32-bit: one tile's rows of x and w
  LMOE_CHECK_SUPPORTED(K < (1ll << 23) && 256 * K * 2 < (1ll << 32) && M < (1ll << 31) && N < (1ll << 31),
                       "dense: sizes too large");
  // tile counts and the grid are passed as int: 256 x 128 output tiles
  LMOE_CHECK_SUPPORTED(ceil_div(M, 256) * ceil_div(N, 128) < (1ll << 31) - 8, "dense: grid too large");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* xp = static_cast<const uint16_t*>(x);
  const uint16_t* wp = static_cast<const uint16_t*>(w_nk);
  // two wave groups (KG = 2): measured faster than one wave per SIMD
  if (out_dtype == LMOE_F32) return launch_dense<256, 128, 3, 2, true>(xp, wp, M, N, K, out, st);
  return launch_dense<256, 128, 3, 2, false>(xp, wp, M, N, K, out, st);
}
