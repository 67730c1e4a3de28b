// Grouped (ragged) GEMM tile machinery for gfx950: bf16 MFMA 16x16x32, LDS
// tiles kept K-contiguous, per-group tile scheduling computed on the device.
//
// A block owns one BM x BN output tile of one group.  blockIdx.y enumerates
// the m-tiles of all groups back to back (group g has ceil(n_g / BM) of them),
// followed by "tail" tiles that zero rows past sum(group_sizes); each block
// finds its group with a wavefront prefix scan over group_sizes, so no host
// synchronisation or schedule buffer is needed.  blockIdx.x is the n-tile.
//
// Weight tiles reach LDS in one of three ways (the only part that differs
// between layouts):
//   GKN   rhs[g][k][n] (n contiguous, the reference's x @ W layout): each
//         thread loads a 4(k) x 8(n) block with four 16-byte loads and writes
//         it transposed as eight 8-byte LDS stores, so LDS holds B^T.
//   GNK   rhs[g][n][k] (k contiguous): straight 16-byte copies.
//   MXFP4 packed[g][n][k/2] + scale[g][n][k/32]: each thread expands 16 packed
//         bytes (one 32-element scale block) to 32 bf16 in registers.
// The MFMA loop then reads 16-byte A and B fragments from LDS.
#pragma once

#include "lmoe_common.h"

namespace lmoe {
namespace gemm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx2_t __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int kBK = 64;
constexpr int kPad = 8;             // bf16 elements of padding per LDS row
constexpr int kLdsRow = kBK + kPad;  // LDS row stride (elements)

// kFP8GKN: (G, K, N) OCP E4M3 codes with f32 scales (G, K/scale_block, N),
// each weight used as bf16(f32(code) * scale).
enum BLayout { kGKN = 0, kGNK = 1, kMXFP4 = 2, kFP8GKN = 3 };
enum Epilogue { kEpiNone = 0, kEpiSitu = 1 };

struct Params {
  const uint16_t* lhs;     // (M, K) bf16 (MXFP8 path: E4M3 codes, read as bytes)
  const void* rhs;         // layout-dependent
  const uint8_t* scale;    // MXFP4 scales (G, N, K/32)
  const int32_t* group_sizes;
  int64_t M, K, N, G;      // N = full rhs width (2I for SiTU)
  int zero_group;
  void* out;               // (M, N) or (M, N/2) for SiTU
  int out_dtype;
  float beta, beta_lin;
  int round_before_act;
  const uint8_t* lhs_scale = nullptr;  // MXFP8 path: E8M0 (K/128, roundup(M, 4), 4)
  int skip_zero_rows = 0;              // zero_group rows may be left unwritten
  const float* scale_f32 = nullptr;    // kFP8GKN: (G, K/scale_block, N) f32
  int64_t scale_block = 0;             // kFP8GKN: rows of K per scale
  // split-K (DMA kernel, no epilogue): the K steps of every tile are dealt
  // into k_split contiguous ranges; range r writes its f32 partial sums to
  // plane r of out, split_stride elements apart
  int64_t k_split = 1;
  int64_t split_stride = 0;
  // gathered rows (streamed MXFP4 kernel only): row r of the grouped problem
  // is row a_index[r] of lhs, an (a_rows, K) array; nullptr: row r of lhs
  const int32_t* a_index = nullptr;
  int64_t a_rows = 0;
};

struct TileInfo {
  int group;     // -1: no work
  int64_t row0;  // first output row
  int rows;      // valid rows in this tile
  bool zero;     // write zeros without computing
};

// Total m-tiles of the problem: every group's ceil(n_g / BM) tiles plus the
// tail tiles that zero rows [sum(group_sizes), M).  Executed by one wave.
template <int BM>
__device__ int64_t total_m_tiles(const int32_t* __restrict__ gs, int64_t G, int64_t M) {
  const int lane = threadIdx.x % 64;
  int64_t tiles = 0, rows = 0;
  for (int64_t g = lane; g < G; g += 64) {
    int64_t n = gs[g];
    n = n < 0 ? 0 : n;
    tiles += (n + BM - 1) / BM;
    rows += n;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    tiles += __shfl_xor(tiles, off, 64);
    rows += __shfl_xor(rows, off, 64);
  }
  const int64_t tail = rows < M ? M - rows : 0;
  return tiles + (tail + BM - 1) / BM;
}

// Find (group, first row, rows) of m-tile `mt`.  Executed by wave 0.  Lane l
// holds groups l, l + 64, ...: the group sizes of up to kPre chunks of 64 are
// loaded before any is scanned, so their latencies overlap; group counts are
// clipped to [0, M] and the running sums saturate at M (row counts) and at
// 2^31 - 1 (tile counts), so 32-bit scans are exact where it matters.
template <int BM>
__device__ TileInfo locate_tile(const int32_t* __restrict__ gs, int64_t G, int64_t M, int zero_group,
                                int64_t mt) {
  constexpr int kPre = 4;
  constexpr uint32_t kTileCap = 0x7fffffffu;
  const int lane = threadIdx.x % 64;
  const uint32_t m32 = static_cast<uint32_t>(M);  // M < 2^31 (checked on the host)
  uint32_t cum_tiles = 0, cum_rows = 0;
  TileInfo info{-1, 0, 0, false};
  for (int64_t g0 = 0; g0 < G; g0 += 64 * kPre) {
    uint32_t n_pre[kPre];
#pragma unroll
    for (int c = 0; c < kPre; ++c) {
      const int64_t g = g0 + 64 * c + lane;
      const int32_t v = g < G ? gs[g] : 0;
      n_pre[c] = v < 0 ? 0u : (static_cast<uint32_t>(v) < m32 ? static_cast<uint32_t>(v) : m32);
    }
#pragma unroll
    for (int c = 0; c < kPre; ++c) {
      if (g0 + 64 * c >= G) break;
      const int64_t g = g0 + 64 * c + lane;
      const uint32_t n = n_pre[c];
      const uint32_t tiles = (n + BM - 1) / BM;
      const uint32_t incl_t = wave_scan_sat(tiles, kTileCap), incl_r = wave_scan_sat(n, m32);
      // exclusive prefixes: the previous lane's inclusive ones (wave_shr:1);
      // a saturated prefix stays >= M, so such groups get no rows
      const uint32_t prev_t = __builtin_amdgcn_update_dpp(0u, incl_t, 0x138, 0xf, 0xf, false);
      const uint32_t prev_r = __builtin_amdgcn_update_dpp(0u, incl_r, 0x138, 0xf, 0xf, false);
      const int64_t excl_t = sat_add(cum_tiles, prev_t, kTileCap);
      const int64_t excl_r = sat_add(cum_rows, prev_r, m32);
      if (g < G && mt >= excl_t && mt < excl_t + tiles) {
        const int64_t local = mt - excl_t;
        info.group = static_cast<int>(g);
        info.row0 = excl_r + local * BM;
        const int64_t left = static_cast<int64_t>(n) - local * BM;
        info.rows = static_cast<int>(left < BM ? left : BM);
        info.zero = (g == zero_group);
      }
      cum_tiles = sat_add(cum_tiles, __builtin_amdgcn_readlane(incl_t, 63), kTileCap);
      cum_rows = sat_add(cum_rows, __builtin_amdgcn_readlane(incl_r, 63), m32);
    }
  }
  // broadcast the (single) hit
  const uint64_t hit = __ballot(info.group >= 0);
  if (hit) {
    const int src = __ffsll(static_cast<long long>(hit)) - 1;
    info.group = __shfl(info.group, src, 64);
    info.row0 = __shfl(info.row0, src, 64);
    info.rows = __shfl(info.rows, src, 64);
    info.zero = __shfl(static_cast<int>(info.zero), src, 64) != 0;
  } else {
    // tail tiles: zero rows [sum(group_sizes), M)
    const int64_t q = mt - cum_tiles;
    const int64_t r0 = cum_rows + q * BM;
    if (q >= 0 && r0 < M) {
      info.group = 0;
      info.row0 = r0;
      const int64_t left = M - r0;
      info.rows = static_cast<int>(left < BM ? left : BM);
      info.zero = true;
    }
  }
  // never touch rows >= M (group sizes summing past M are clipped)
  if (info.group >= 0) {
    if (info.row0 >= M) {
      info.group = -1;
    } else if (info.row0 + info.rows > M) {
      info.rows = static_cast<int>(M - info.row0);
    }
  }
  return info;
}

// 16-byte chunk swizzle of 128-byte LDS rows: logical chunk kc of row r sits
// at physical chunk kc ^ swz8(r).  MFMA fragment reads fetch one chunk from
// each of 16 consecutive rows per 16-lane group; with 64 four-byte banks the
// rows r and r + 8 must then land in different chunks too, which plain
// (r & 7) does not give (a 2-way conflict on every fragment read).
__device__ __forceinline__ int swz8(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// Tiled MXFP4 record: the 32 bytes (64 k) of one column and k step hold the
// eight 4-byte groups of 8 k values in the order 0, 2, 4, 6, 1, 3, 5, 7, so
// a lane of a 32x32x16 MFMA fragment (k groups g, g+2, g+4, g+6 of its
// column) reads its whole k step as one contiguous 16-byte chunk.  Physical
// dword of logical dword d:
__device__ __forceinline__ int mx_dword_pos(int d) { return (d & 1) * 4 + (d >> 1); }

constexpr int kXcds = 8;  // MI355X: 8 XCDs; consecutive blocks go to consecutive XCDs

// Virtual tile vb -> (m-tile, n-tile) with an XCD-aware order; executed by
// wave 0 (tm = total_m_tiles).  gm == 0: n-tiles striped over the XCDs (each
// weight column slice is read by one XCD only, and the m-tiles of a group,
// which share it, follow each other there so its later reads hit that XCD's
// L2); gm > 0: groups of gm m-tiles round-robin over the XCDs with all n-tiles
// of a group on one XCD (the A rows are read by one XCD only); gm < 0: XCD x
// takes the contiguous m-tile range [x * ceil(tm/8), (x+1) * ceil(tm/8)), each
// m-tile with all its n-tiles in a row, so both the A rows and (but for the
// groups that straddle a range boundary) a group's weights are read by one
// XCD only.
//
// gm < 0: XCD x takes the contiguous m-tile range [x per, (x + 1) per),
// per = ceil(tm_work / 8), of the first tm_work m-tiles (the groups before a
// trailing zero group, so the ranges hold equal real work), each m-tile's
// n-tiles in turn; the m-tiles from tm_work on (zero group, tail rows) follow,
// dealt round-robin.  An XCD then reads an expert's weights and a tile's
// activation rows from its own L2.  No launch selects gm < 0 today (it moved
// 21% less HBM traffic for the config-5 gate/up but measured 4% slower than
// gm == 0); the branch stays because the measured kernels were compiled with
// it, and taking it out changes their code.
template <class Locate>
__host__ __device__ __forceinline__ TileInfo schedule_tile_with(int64_t n_tiles, int gm, int64_t vb, int64_t tm, int64_t& nt,
                                                       Locate&& locate, int64_t tm_work = -1) {
  // grids and tile counts are < 2^31 (checked on the host): 32-bit index math
  const uint32_t v32 = static_cast<uint32_t>(vb), nt32 = static_cast<uint32_t>(n_tiles);
  const uint32_t xcd = v32 % kXcds, slot = v32 / kXcds;
  TileInfo ti{-1, 0, 0, false};
  nt = 0;
  if (gm == 0) {
    const uint32_t per = nt32 / kXcds;
    const uint32_t mt = slot / per;
    nt = xcd + kXcds * (slot % per);
    if (mt < tm) ti = locate(mt);
  } else if (gm < 0) {
    const int64_t work = tm_work < 0 || tm_work > tm ? tm : tm_work;
    const uint32_t per = static_cast<uint32_t>((work + kXcds - 1) / kXcds);
    const uint32_t ml = slot / nt32;
    nt = slot % nt32;
    const int64_t mt = ml < per ? static_cast<int64_t>(xcd) * per + ml
                                : work + static_cast<int64_t>(ml - per) * kXcds + xcd;
    if (ml < per ? mt < work : mt < tm) ti = locate(mt);
  } else {
    const uint32_t span = static_cast<uint32_t>(gm) * nt32;
    const int64_t m_base = (static_cast<int64_t>(slot / span) * kXcds + xcd) * gm;
    const uint32_t r = slot % span;
    if (m_base < tm) {
      const uint32_t gm_eff = static_cast<uint32_t>(tm - m_base < gm ? tm - m_base : gm);
      if (r < gm_eff * nt32) {
        nt = r / gm_eff;
        ti = locate(m_base + r % gm_eff);
      }
    }
  }
  return ti;
}

template <int BM>
__device__ TileInfo schedule_tile(const Params& p, int64_t n_tiles, int gm, int64_t vb, int64_t tm, int64_t& nt) {
  return schedule_tile_with(n_tiles, gm, vb, tm, nt, [&](int64_t mt) {
    return locate_tile<BM>(p.group_sizes, p.G, p.M, p.zero_group, mt);
  });
}

// Tile table in LDS, built once per block by the streamed (persistent)
// kernels: tt[g] = exclusive prefix of the m-tile counts ceil(n_g / BM)
// (saturating at 2^31 - 1) and tr[g] = exclusive prefix of the row counts
// (saturating at M), g = 0 .. G, with n_g = group_sizes[g] clipped to
// [0, M].  The same clipping and saturation as locate_tile, so both give the
// same tiles.  Runs on all threads of the block (THREADS, a multiple of 64);
// `wsum` holds THREADS / 64 scratch words.  Ends with the table visible to
// every wave.
template <int BM, int THREADS>
__device__ __forceinline__ void build_tile_table(const int32_t* __restrict__ gs, int G, uint32_t m32, uint32_t* tt, uint32_t* tr,
                                 uint32_t* wsum) {
  constexpr uint32_t kTileCap = 0x7fffffffu;
  constexpr int kWaves = THREADS / 64;
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  uint32_t carry_t = 0, carry_r = 0;
  for (int g0 = 0; g0 < G; g0 += THREADS) {
    const int g = g0 + static_cast<int>(threadIdx.x);
    const int32_t v = g < G ? gs[g] : 0;
    const uint32_t n = v < 0 ? 0u : (static_cast<uint32_t>(v) < m32 ? static_cast<uint32_t>(v) : m32);
    const uint32_t tiles = (n + BM - 1) / BM;
    const uint32_t it = wave_scan_sat(tiles, kTileCap), ir = wave_scan_sat(n, m32);
    // wave totals -> exclusive wave offsets (two words per wave)
    if (lane == 63) {
      wsum[2 * wave] = it;
      wsum[2 * wave + 1] = ir;
    }
    __syncthreads();
    uint32_t off_t = carry_t, off_r = carry_r, tot_t = carry_t, tot_r = carry_r;
    for (int w = 0; w < kWaves; ++w) {
      if (w < wave) {
        off_t = sat_add(off_t, wsum[2 * w], kTileCap);
        off_r = sat_add(off_r, wsum[2 * w + 1], m32);
      }
      tot_t = sat_add(tot_t, wsum[2 * w], kTileCap);
      tot_r = sat_add(tot_r, wsum[2 * w + 1], m32);
    }
    if (g < G) {
      // exclusive = offset + inclusive - own (the own term never saturated
      // alone: recompute from the previous lane's inclusive value)
      const uint32_t pt = __builtin_amdgcn_update_dpp(0u, it, 0x138, 0xf, 0xf, false);  // wave_shr:1
      const uint32_t pr = __builtin_amdgcn_update_dpp(0u, ir, 0x138, 0xf, 0xf, false);
      tt[g] = sat_add(off_t, lane == 0 ? 0u : pt, kTileCap);
      tr[g] = sat_add(off_r, lane == 0 ? 0u : pr, m32);
    }
    carry_t = tot_t;
    carry_r = tot_r;
    __syncthreads();  // wsum is reused by the next chunk
  }
  if (threadIdx.x == 0) {
    tt[G] = carry_t;
    tr[G] = carry_r;
  }
  __syncthreads();
}

// locate_tile from the LDS tile table; executed by every wave for itself
// (wave-uniform result; `lane` = this thread's lane).
template <int BM>
__device__ __forceinline__ TileInfo locate_tile_lds(const uint32_t* tt, const uint32_t* tr, int G, int64_t M,
                                                    int zero_group, int64_t mt, int lane) {
  TileInfo info{-1, 0, 0, false};
  int hit_g = -1;
  for (int g0 = 0; g0 < G; g0 += 64) {
    const int g = g0 + lane;
    const bool hit = g < G && static_cast<int64_t>(tt[g]) <= mt && mt < static_cast<int64_t>(tt[g + 1]);
    const uint64_t b = __ballot(hit);
    if (b) {
      hit_g = g0 + __ffsll(static_cast<long long>(b)) - 1;
      break;
    }
  }
  if (hit_g >= 0) {
    const int64_t local = mt - tt[hit_g];
    const int64_t n_eff = static_cast<int64_t>(tr[hit_g + 1]) - tr[hit_g];  // rows left before M
    const int64_t left = n_eff - local * BM;
    if (left > 0) {
      info.group = hit_g;
      info.row0 = tr[hit_g] + local * BM;
      info.rows = static_cast<int>(left < BM ? left : BM);
      info.zero = hit_g == zero_group;
    }
  } else {
    // tail tiles: zero rows [sum(group_sizes), M)
    const int64_t q = mt - tt[G];
    const int64_t r0 = tr[G] + q * BM;
    if (q >= 0 && r0 < M) {
      info.group = 0;
      info.row0 = r0;
      const int64_t left = M - r0;
      info.rows = static_cast<int>(left < BM ? left : BM);
      info.zero = true;
    }
  }
  return info;
}

__device__ __forceinline__ float situ(float g, float u, float beta, float beta_lin) {
  // ref.py:305-310: beta*tanh(g/beta)*sigmoid(g) * beta_lin*tanh(u/beta_lin)
  const float sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-g)));
  const float sg = __fmul_rn(__fmul_rn(beta, tanhf(__fdiv_rn(g, beta))), sig);
  const float bu = __fmul_rn(beta_lin, tanhf(__fdiv_rn(u, beta_lin)));
  return __fmul_rn(sg, bu);
}

// Two f32 -> packed bf16 pair (round to nearest even, hardware conversion).
typedef __bf16 bf16x2_pack_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const bf16x2_pack_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

// SiTU-GLU for the fused epilogue (ref.py:305-310):
//   beta*tanh(g/beta)*sigmoid(g) * beta_lin*tanh(u/beta_lin)
// with three hardware exp2, two reciprocals and no branches:
// tanh(x) = (a - 1) / (a + 1) with a = e^(2x) and sigmoid(g) = 1 / (1 + e^-g),
//   SiTU = beta*beta_lin * (a - 1)(c - 1) / ((a + 1)(c + 1)) / (1 + e),
//   a = 2^(2 log2(e) g / beta), c = 2^(2 log2(e) u / beta_lin), e = 2^(-log2(e) g).
// The tanh exponents are clamped to [-26, 26] (|x| <= 9: tanh(9) = 1 - 3e-8,
// saturated in f32), so the tanh quotient cannot overflow.  For beta != 4 the
// sigmoid keeps its own reciprocal and goes to 0 where e^-g overflows
// (g < -88).  For beta == 4 the sigmoid is built from the same clamped
// exponential a = e^(g/2) (below), so below g = -36.04 (a = 2^-26) it stays at
// 2^-52 instead of decaying as e^g: the result there is at most
// beta*beta_lin*2^-52 in magnitude instead of about 0, far below the bf16
// rounding of any output of ordinary size.  Near g = 0 (u = 0) a - 1 (c - 1)
// cancels: the absolute error of the result stays below beta*beta_lin*2^-23,
// far below the bf16 rounding of results of ordinary size.  Hardware exp2 / reciprocal: a few f32 ulp.  A NaN gate or
// up value gives NaN.  Every GEMM epilogue uses this one function, so the
// kernels agree bit for bit on equal accumulators.
struct SituConsts {
  float kg, ku;  // 2*log2(e)/beta, 2*log2(e)/beta_lin
  float bbl;     // beta*beta_lin
  bool beta4;    // beta == 4 (the model's value): one exponential serves tanh(g/4) and sigmoid(g)
};
__device__ __forceinline__ SituConsts situ_consts(float beta, float beta_lin) {
  constexpr float kL2e = 1.44269504088896341f;
  return SituConsts{2.0f * kL2e / beta, 2.0f * kL2e / beta_lin, beta * beta_lin, beta == 4.0f};
}
// SiTU-GLU of one (gate, up) pair: beta tanh(g/beta) sigmoid(g) * beta_lin
// tanh(u/beta_lin), with tanh(x) = (e^2x - 1)/(e^2x + 1) and the exponentials
// clamped to 2^+-26 (tanh is +-1 to f32 precision there).  With beta == 4,
// a = e^(g/2) gives tanh(g/4) = (a-1)/(a+1) and sigmoid(g) = a^2/(1+a^2), so
// the pair costs two exponentials and one reciprocal (numerator and
// denominator stay below 2^104; with a clamped at 2^-26, sigmoid(g) bottoms
// out at 2^-52 for g < -36.04); otherwise sigmoid takes its own exponential
// and reciprocal.  NaN in either input gives NaN.  Every fused kernel uses
// this one function, so they agree bit for bit.
__device__ __forceinline__ float situ_epi(float g, float u, const SituConsts& c) {
  const float a = __builtin_amdgcn_exp2f(__builtin_amdgcn_fmed3f(g * c.kg, -26.0f, 26.0f));
  const float b = __builtin_amdgcn_exp2f(__builtin_amdgcn_fmed3f(u * c.ku, -26.0f, 26.0f));
  float r;
  if (c.beta4) {
    const float a2 = a * a;
    r = c.bbl * ((a - 1.0f) * a2 * (b - 1.0f)) * __builtin_amdgcn_rcpf((a + 1.0f) * (1.0f + a2) * (b + 1.0f));
  } else {
    const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
    const float q = (a - 1.0f) * (b - 1.0f) * __builtin_amdgcn_rcpf((a + 1.0f) * (b + 1.0f));
    r = c.bbl * q * __builtin_amdgcn_rcpf(1.0f + e);
  }
  return __builtin_isunordered(g, u) ? __builtin_nanf("") : r;
}

// gate / up accumulators rounded to bf16 (nearest even) with one packed
// conversion (the epilogue convention of gk.py:114-125).
__device__ __forceinline__ void round_pair_bf16(float& g, float& u) {
  const bf16x2_pack_t v = {static_cast<__bf16>(g), static_cast<__bf16>(u)};
  const uint32_t p = __builtin_bit_cast(uint32_t, v);
  g = __uint_as_float(p << 16);
  u = __uint_as_float(p & 0xffff0000u);
}

// E2M1 nibble with E8M0 scale byte s -> bf16 bits, exact (value has <= 2
// significant bits, so the f32 product truncates to bf16 without rounding).
__device__ __forceinline__ uint32_t fp4_to_bf16_bits(uint32_t nib, float scale) {
  const uint32_t e = (nib >> 1) & 3u, m = nib & 1u;
  uint32_t bits;
  if (e == 0)
    bits = m ? 0x3f000000u : 0u;  // 0.5 or 0
  else
    bits = ((e + 126u) << 23) | (m << 22);  // 2^(e-1) * (1 + m/2)
  float v = __uint_as_float(bits) * scale;
  uint32_t r = __float_as_uint(v) >> 16;
  return r | ((nib & 8u) << 12);  // sign (also for zero: -0.0)
}

__device__ __forceinline__ float e8m0_to_float(uint32_t s) {
  if (s == 0) return __uint_as_float(0x00400000u);  // 2^-127 (denormal)
  if (s == 255) return __uint_as_float(0x7f800000u);  // 2^128 overflows to inf
  return __uint_as_float(s << 23);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// 16 packed bytes (32 e2m1 values, low nibble first) -> 32 bf16 (as 16 u32).
// Scale bytes 3..252 use gfx950's v_cvt_scalef32_pk_bf16_fp4 (two values per
// instruction, exact: every product is a normal bf16 with <= 2 significant
// bits); the edge bytes, whose products can be denormal (0..2) or overflow
// (253..255), take the bit-level path.
__device__ __forceinline__ bool hw_scale_ok(uint32_t s) { return s - 3u <= 249u; }

__device__ __forceinline__ void dequant32(const uint4 p, uint32_t scale_byte, uint32_t* o) {
  const uint32_t w[4] = {p.x, p.y, p.z, p.w};
  if (hw_scale_ok(scale_byte)) {
    const float sc = __uint_as_float(scale_byte << 23);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      bf16x2_t r0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], sc, 0);
      bf16x2_t r1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], sc, 1);
      bf16x2_t r2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], sc, 2);
      bf16x2_t r3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[d], sc, 3);
      o[d * 4 + 0] = __builtin_bit_cast(uint32_t, r0);
      o[d * 4 + 1] = __builtin_bit_cast(uint32_t, r1);
      o[d * 4 + 2] = __builtin_bit_cast(uint32_t, r2);
      o[d * 4 + 3] = __builtin_bit_cast(uint32_t, r3);
    }
    return;
  }
  const float sc = e8m0_to_float(scale_byte);
#pragma unroll
  for (int d = 0; d < 4; ++d) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t byte = (w[d] >> (8 * b)) & 0xffu;
      const uint32_t lo = fp4_to_bf16_bits(byte & 15u, sc);
      const uint32_t hi = fp4_to_bf16_bits(byte >> 4, sc);
      o[d * 4 + b] = lo | (hi << 16);
    }
  }
}

// Same conversion for one packed byte (two values) -> one u32 of two bf16.
__device__ __forceinline__ uint32_t dequant_byte(uint32_t byte, uint32_t scale_byte) {
  if (hw_scale_ok(scale_byte)) {
    const float sc = __uint_as_float(scale_byte << 23);
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(byte, sc, 0));
  }
  const float sc = e8m0_to_float(scale_byte);
  return fp4_to_bf16_bits(byte & 15u, sc) | (fp4_to_bf16_bits(byte >> 4, sc) << 16);
}

}  // namespace gemm
}  // namespace lmoe
