// Skinny-M grouped MXFP4 GEMM for the decode regime: the ragged_dot of the
// local-shard expert FFN when each group holds a handful of rows
// (rd.py:553-577 sweeps num_tokens 1..128 through the same ragged_dot; at
// T=1, k=16 about three local experts receive one row each), and the config-4
// MXFP4 matmul at small M.  Math: lhs @ deq(W_g)^T as in odq.py:65-172.
//
// Here the weight read is the whole cost (a few rows per 2 MB expert) and
// the time is set by memory latency, so the kernel is built to put each
// weight byte in flight once, early, from as many waves as possible:
//   * work item = (hit group, 16 output columns); the block's waves (4, or 8
//     when there are few items) split the item's K axis and reduce their
//     accumulators in LDS in a fixed wave order -- deterministic, no atomics,
//     no workspace;
//   * the hit groups (nonzero rows, not the padding group) are compacted in
//     LDS first, so padding and empty experts cost no work, and the grid is
//     the number of blocks resident at once, each walking items with a grid
//     stride;
//   * a wave issues the loads of up to four k-step pairs (weights and the
//     activations of every row chunk) before their MFMAs;
//   * weights come from the k-step-major tiled layout (lmoe_mxfp4_tile): the
//     16 columns x 2 k-steps a wave reads per load are two contiguous 512 B
//     runs, expanded in registers with v_cvt_scalef32_pk_bf16_fp4 and fed to
//     v_mfma_f32_16x16x32_bf16 as the A operand (rows of the MFMA = weight
//     columns), the activations as the B operand, so each lane ends with four
//     consecutive output columns of one row (8-byte stores).
// A group's rows are taken 16, 32 or 64 at a time (template NC, from the
// caller's bound on group rows); larger groups take further passes over the
// same weights (correct for any group size, fast for small ones).
#include "lmoe_common.h"
#include "gemm_tile.h"

#include <algorithm>
#include <atomic>

namespace lmoe {
namespace gemm {
namespace {

constexpr int kSkMaxChunks = 4;    // 16-row chunks per pass: 1, 2 or 4 (template NC)
constexpr int kSkMaxGroups = 1024;

struct SkinnyParams {
  const uint16_t* x;     // (M, K) bf16, rows sorted by group
  const uint8_t* w;      // (G, K/64, N, 32) tiled e2m1 pairs
  const uint8_t* s;      // (G, K/64, N, 2) tiled E8M0 scales
  const int32_t* gs;     // (G,)
  int64_t M, K, N, G;
  int zero_group;
  int skip_zero_rows;
  float beta, beta_lin;
  uint16_t* out;         // (M, N) bf16, or (M, N/2) with the SiTU epilogue
  int n_ct;              // 16-column output tiles
  // Fused dispatch (skinny_mx_kernel<..., true>): every block sorts the
  // top-k slots in LDS as the one-launch dispatch does, block 0 writes the
  // dispatch metadata, and x is the (T, >= K) bf16 token rows (row stride
  // x_ld) read through the sorted order; then M = m_padded, G = L + 1 and
  // zero_group = L.
  const int32_t* d_idx = nullptr;  // (T*k,) global expert ids
  const uint8_t* d_w_in = nullptr; // (T*k,) combine weights, d_wsize bytes each
  int d_wsize = 0;
  int64_t d_n = 0, d_k = 1, x_ld = 0;
  int d_start = 0, d_L = 0;
  int32_t* d_group_sizes = nullptr;  // (L + 1,)
  uint8_t* d_valid = nullptr;        // (m_padded,)
  int32_t* d_counts = nullptr;       // (L,)
  int32_t* d_tok = nullptr;          // (m_padded,)
  uint8_t* d_w_out = nullptr;        // (m_padded,) d_wsize bytes each
  int32_t* d_slot_pos = nullptr;     // (T*k,) or null
};

constexpr int kSkDispSlots = 1024;  // T*k of the fused dispatch
constexpr int kSkDispRows = 2048;   // its m_padded

// One packed dword (8 e2m1 values, low nibble first) with its scale byte ->
// 8 bf16, exactly as dequant32 does it.
__device__ __forceinline__ bf16x8_t dq8(uint32_t w, uint32_t sb) {
  uint4 o;
  if (hw_scale_ok(sb)) {
    const float sc = __uint_as_float(sb << 23);
    o.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 0));
    o.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 1));
    o.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 2));
    o.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 3));
  } else {
    const float sc = e8m0_to_float(sb);
    uint32_t r[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t byte = (w >> (8 * b)) & 0xffu;
      r[b] = fp4_to_bf16_bits(byte & 15u, sc) | (fp4_to_bf16_bits(byte >> 4, sc) << 16);
    }
    o = uint4{r[0], r[1], r[2], r[3]};
  }
  return __builtin_bit_cast(bf16x8_t, o);
}

__device__ __forceinline__ uint32_t word(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

template <int EPI>
__device__ __forceinline__ void store_out(const SkinnyParams& p, int64_t row, int64_t col, int64_t nout,
                                          const floatx4 (&v)[EPI == kEpiSitu ? 2 : 1]) {
  float o[4];
  if constexpr (EPI == kEpiSitu) {
    const SituConsts sc = situ_consts(p.beta, p.beta_lin);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // the reference rounds both GEMM outputs to bf16 before the activation
      float g = v[0][e], u = v[1][e];
      round_pair_bf16(g, u);
      o[e] = situ_epi(g, u, sc);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = v[0][e];
  }
  *reinterpret_cast<uint2*>(p.out + row * nout + col) = uint2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
}

template <int EPI, int NC, int WAVES, bool DISP = false>
__global__ __launch_bounds__(WAVES * 64) void skinny_mx_kernel(SkinnyParams p) {
  constexpr int kThreads = WAVES * 64;
  constexpr int GPT = kSkMaxGroups / kThreads;       // groups per thread in the table scan
  constexpr int NB = EPI == kEpiSitu ? 2 : 1;        // gate and up tiles
  // k-step pairs in flight per wave (fewer with two weight tiles: registers)
  constexpr int D = (NC == 1 ? 4 : NC == 2 ? 2 : 1) / (NB == 2 && NC < 4 ? 2 : 1);
  __shared__ int32_t s_hit_g[kSkMaxGroups];
  __shared__ int32_t s_hit_n[kSkMaxGroups];
  __shared__ int64_t s_hit_r0[kSkMaxGroups];
  __shared__ uint64_t s_wsum[WAVES];
  __shared__ int64_t s_misc[4];  // zero-group first row, zero-group rows, sum of rows (<= M), hit groups
  __shared__ floatx4 s_red[WAVES - 1][NB][64];

  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int64_t M = p.M, K = p.K, N = p.N, G = p.G;
  const int64_t nout = N / NB;

  // ---- fused dispatch: the sort of dispatch_small_kernel (stable expert-major
  // order, tail truncation at m_padded = M, padding bucket L), in LDS
  constexpr int kDS = DISP ? kSkDispSlots : 1, kDR = DISP ? kSkDispRows : 1, kDG = DISP ? kSkMaxGroups : 1;
  __shared__ uint16_t s_key[kDS];
  __shared__ int32_t s_row_slot[kDR];
  __shared__ int32_t s_dcnt[kDG], s_doff[kDG], s_dgs[kDG];
  __shared__ int32_t s_dtotal;
  if constexpr (DISP) {
    const int Ld = p.d_L;
    const int64_t ns = p.d_n;
    for (int e = t; e <= Ld; e += kThreads) {
      s_dcnt[e] = 0;
      s_dgs[e] = 0;  // the rank pass's per-expert run
    }
    for (int64_t r = t; r < M; r += kThreads) s_row_slot[r] = -1;
    __syncthreads();
    for (int64_t s = t; s < ns; s += kThreads) {
      const int g = p.d_idx[s];
      const int key = (g >= p.d_start && g < p.d_start + Ld) ? g - p.d_start : Ld;
      s_key[s] = static_cast<uint16_t>(key);
      if (key < Ld) atomicAdd(&s_dcnt[key], 1);
    }
    __syncthreads();
    if (wv == 0) {  // exclusive offsets of the L experts, each lane a run of keys
      const int per = (Ld + 63) / 64;
      const int e0 = lane * per, e1 = e0 + per < Ld ? e0 + per : Ld;
      int sum = 0;
      for (int e = e0; e < e1; ++e) sum += s_dcnt[e];
      int incl = sum;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(incl, d, 64);
        if (lane >= d) incl += o;
      }
      int run = incl - sum;
      for (int e = e0; e < e1; ++e) {
        s_doff[e] = run;
        run += s_dcnt[e];
      }
      if (lane == 63) s_dtotal = incl;
    }
    __syncthreads();
    if (wv == 0) {  // stable ranks: wave 0 walks the slots in order, 64 at a time
      int kb = 1;
      while ((1 << kb) <= Ld) ++kb;
      const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
      for (int64_t c = 0; c < ns; c += 64) {
        const int64_t s = c + lane;
        const int key = s < ns ? s_key[s] : Ld;
        uint64_t m = __ballot(s < ns && key < Ld);
        for (int b = 0; b < kb; ++b) {
          const uint64_t bal = __ballot((key >> b) & 1);
          m &= ((key >> b) & 1) ? bal : ~bal;
        }
        if (s < ns && key < Ld) {
          const int base = s_dgs[key];
          const int pos = s_doff[key] + base + __popcll(m & below);
          const bool kept = pos < M;
          if (kept) s_row_slot[pos] = static_cast<int32_t>(s);
          if (blockIdx.x == 0 && p.d_slot_pos) p.d_slot_pos[s] = kept ? pos : -1;
          if ((m & below) == 0) s_dgs[key] = base + __popcll(m);  // the group's lowest lane
        } else if (s < ns && blockIdx.x == 0 && p.d_slot_pos) {
          p.d_slot_pos[s] = -1;
        }
      }
    }
    __syncthreads();
    const int64_t nkept = s_dtotal < M ? s_dtotal : M;
    for (int e = t; e < Ld; e += kThreads) {
      const int64_t room = M - s_doff[e];
      s_dgs[e] = static_cast<int32_t>(room <= 0 ? 0 : (room < s_dcnt[e] ? room : s_dcnt[e]));
    }
    if (t == 0) s_dgs[Ld] = static_cast<int32_t>(M - nkept);
    __syncthreads();
    if (blockIdx.x == 0) {  // the dispatch's metadata, as lmoe_dispatch_local_small writes it
      for (int e = t; e <= Ld; e += kThreads) {
        p.d_group_sizes[e] = s_dgs[e];
        if (e < Ld) p.d_counts[e] = s_dgs[e];
      }
      for (int64_t r = t; r < M; r += kThreads) {
        const int32_t s = s_row_slot[r];
        p.d_valid[r] = s >= 0 ? 1 : 0;
        p.d_tok[r] = s >= 0 ? static_cast<int32_t>(s / p.d_k) : -1;
        if (p.d_wsize == 4)
          reinterpret_cast<uint32_t*>(p.d_w_out)[r] = s >= 0 ? reinterpret_cast<const uint32_t*>(p.d_w_in)[s] : 0u;
        else
          reinterpret_cast<uint16_t*>(p.d_w_out)[r] = s >= 0 ? reinterpret_cast<const uint16_t*>(p.d_w_in)[s] : 0;
      }
    }
  }

  // ---- hit-group table: exclusive scan of (rows << 16 | hit) over <= 1024 groups
  if (t == 0) {
    s_misc[0] = 0;
    s_misc[1] = 0;
  }
  int64_t sz[GPT];
  uint64_t v = 0;
#pragma unroll
  for (int i = 0; i < GPT; ++i) {
    const int64_t g = GPT * t + i;
    int32_t n = 0;
    if constexpr (DISP)
      n = g < G ? s_dgs[g] : 0;
    else
      n = g < G ? p.gs[g] : 0;
    sz[i] = n > 0 ? n : 0;
    v += (static_cast<uint64_t>(sz[i]) << 16) + ((sz[i] > 0 && g != p.zero_group) ? 1u : 0u);
  }
  uint64_t incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const uint64_t o = __shfl_up(incl, d, 64);
    if (lane >= d) incl += o;
  }
  if (lane == 63) s_wsum[wv] = incl;
  __syncthreads();
  uint64_t excl = incl - v;
  for (int w = 0; w < wv; ++w) excl += s_wsum[w];
  {
    int64_t r = static_cast<int64_t>(excl >> 16);
    int h = static_cast<int>(excl & 0xffffu);
#pragma unroll
    for (int i = 0; i < GPT; ++i) {
      const int64_t g = GPT * t + i;
      if (g < G) {
        const int64_t n = sz[i];
        const int64_t rows = std::max<int64_t>(0, std::min<int64_t>(n, M - r));  // rows past M are dropped
        if (n > 0 && g != p.zero_group) {
          s_hit_g[h] = static_cast<int32_t>(g);
          s_hit_r0[h] = r;
          s_hit_n[h] = static_cast<int32_t>(rows);
          ++h;
        }
        if (g == p.zero_group) {
          s_misc[0] = r;
          s_misc[1] = rows;
        }
        r += n;
      }
    }
    if (t == kThreads - 1) {
      s_misc[2] = std::min<int64_t>(r, M);
      s_misc[3] = h;
    }
  }
  __syncthreads();

  // ---- zero rows: the padding group and rows past sum(group_sizes)
  if (!p.skip_zero_rows) {
    const int64_t z0 = s_misc[0], zn = s_misc[1], S = s_misc[2];
    const int64_t per_row = nout / 8;
    const int64_t total = (zn + (M - S)) * per_row;
    for (int64_t c = static_cast<int64_t>(blockIdx.x) * kThreads + t; c < total;
         c += static_cast<int64_t>(gridDim.x) * kThreads) {
      const int64_t rr = c / per_row, cc = c % per_row;
      const int64_t row = rr < zn ? z0 + rr : S + (rr - zn);
      reinterpret_cast<uint4*>(p.out + row * nout)[cc] = uint4{0u, 0u, 0u, 0u};
    }
  }

  // ---- items: (hit group, 16-column tile), K split over the block's waves
  const int64_t nhit = s_misc[3];
  const int nct = p.n_ct;
  const int64_t items = nhit * nct;
  const int64_t K64 = K / 64;
  const int P = static_cast<int>(K / 128);  // k-step pairs
  const int q = lane >> 4, ks_off = q >> 1, hh = q & 1, l16 = lane & 15;

  for (int64_t it = blockIdx.x; it < items; it += gridDim.x) {
    const int ct = static_cast<int>(it % nct);
    const int64_t hi = it / nct;
    const int64_t g = s_hit_g[hi], r0 = s_hit_r0[hi];
    const int rows = s_hit_n[hi];
    const int64_t colw = static_cast<int64_t>(ct) * 16 + l16;  // this lane's weight column (gate half)
    const uint8_t* wb = p.w + g * K64 * N * 32 + hh * 16;
    const uint8_t* sb = p.s + g * K64 * N * 2;
    auto ldw = [&](int pr, uint4 (&w)[NB], uint32_t (&sc)[NB]) {
      const int64_t kst = 2 * static_cast<int64_t>(pr) + ks_off;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int64_t col = colw + nb * nout;
        w[nb] = *reinterpret_cast<const uint4*>(wb + (kst * N + col) * 32);
        sc[nb] = *reinterpret_cast<const uint16_t*>(sb + (kst * N + col) * 2);
      }
    };
    const int64_t oc = static_cast<int64_t>(ct) * 16 + 4 * q;  // this lane's first output column

    for (int rb = 0; rb < rows; rb += 16 * NC) {
      const int nrc = std::min(NC, (rows - rb + 15) / 16);
      auto ldx = [&](int pr, int rc, uint4 (&x)[4]) {
        const int lr = rb + rc * 16 + l16;
        int64_t xrow = -1;  // this lane's activation row
        if (lr < rows) {
          if constexpr (DISP) {
            const int32_t sl = s_row_slot[r0 + lr];
            xrow = sl >= 0 ? static_cast<int64_t>(sl / p.d_k) * p.x_ld : -1;
          } else {
            xrow = (r0 + lr) * K;
          }
        }
        if (xrow >= 0) {
          const uint16_t* xp = p.x + xrow + (2 * static_cast<int64_t>(pr) + ks_off) * 64 + hh * 8;
#pragma unroll
          for (int s = 0; s < 4; ++s) x[s] = *reinterpret_cast<const uint4*>(xp + 16 * s);
        } else {
#pragma unroll
          for (int s = 0; s < 4; ++s) x[s] = uint4{0u, 0u, 0u, 0u};
        }
      };

      floatx4 acc[NC][NB];
#pragma unroll
      for (int rc = 0; rc < NC; ++rc)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[rc][nb] = floatx4{0.f, 0.f, 0.f, 0.f};

      // this wave's k-step pairs wv, wv + WAVES, ...: D of them in flight at
      // once (weights and every row chunk's activations), then their MFMAs
      for (int j0 = wv; j0 < P; j0 += WAVES * D) {
        uint4 w[D][NB], x[D][NC][4];
        uint32_t sc[D][NB];
#pragma unroll
        for (int d = 0; d < D; ++d) {
          const int pr = j0 + WAVES * d;
          if (pr < P) {
            ldw(pr, w[d], sc[d]);
#pragma unroll
            for (int rc = 0; rc < NC; ++rc)
              if (rc < nrc) ldx(pr, rc, x[d][rc]);
          }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
          if (j0 + WAVES * d < P) {
            bf16x8_t a[NB][4];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
              for (int s = 0; s < 4; ++s)
                a[nb][s] = dq8(word(w[d][nb], s), s < 2 ? (sc[d][nb] & 0xffu) : (sc[d][nb] >> 8));
#pragma unroll
            for (int rc = 0; rc < NC; ++rc) {
              if (rc < nrc) {
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                  const bf16x8_t bx = __builtin_bit_cast(bf16x8_t, x[d][rc][s]);
#pragma unroll
                  for (int nb = 0; nb < NB; ++nb)
                    acc[rc][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[nb][s], bx, acc[rc][nb], 0, 0, 0);
                }
              }
            }
          }
        }
      }

      // block reduction in wave order 0, 1, ..., WAVES-1, then the epilogue
#pragma unroll
      for (int rc = 0; rc < NC; ++rc) {
        if (rc < nrc) {
          __syncthreads();
          if (wv > 0) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) s_red[wv - 1][nb][lane] = acc[rc][nb];
          }
          __syncthreads();
          if (wv == 0) {
            floatx4 sum[NB];
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
              sum[nb] = acc[rc][nb];
#pragma unroll
              for (int w = 0; w < WAVES - 1; ++w) sum[nb] += s_red[w][nb][lane];
            }
            const int lr = rb + rc * 16 + l16;
            if (lr < rows) store_out<EPI>(p, r0 + lr, oc, nout, sum);
          }
        }
      }
    }
  }
}

// Dense x (M, K) @ W^T with bf16 W stored (N, K), for a few rows (the dense
// projections of a decode step, M = T): the same work split as above with one
// group -- item = 16 output columns, K over the block's waves, LDS reduction
// in wave order -- and the weights loaded straight into the MFMA A operand:
// within a 128-deep k-step pair lane (column c, q) holds k = 32q .. 32q+31 of
// column c (64 contiguous bytes), the activations the same k of its row.
template <int NC, int WAVES, bool OUT_F32>
__global__ __launch_bounds__(WAVES * 64) void skinny_dense_kernel(const uint16_t* __restrict__ x,
                                                                   const uint16_t* __restrict__ w, int64_t M,
                                                                   int64_t K, int64_t N, void* __restrict__ out) {
  constexpr int D = NC == 1 ? 4 : NC == 2 ? 2 : 1;  // k-step pairs in flight per wave
  __shared__ floatx4 s_red[WAVES - 1][64];
  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int q = lane >> 4, l16 = lane & 15;
  const int P = static_cast<int>(K / 128);
  const int64_t nct = N / 16;
  for (int64_t ct = blockIdx.x; ct < nct; ct += gridDim.x) {
    const uint16_t* wr = w + (ct * 16 + l16) * K + 32 * q;
    for (int64_t rb = 0; rb < M; rb += 16 * NC) {
      const int nrc = static_cast<int>(std::min<int64_t>(NC, (M - rb + 15) / 16));
      floatx4 acc[NC];
#pragma unroll
      for (int rc = 0; rc < NC; ++rc) acc[rc] = floatx4{0.f, 0.f, 0.f, 0.f};
      for (int j0 = wv; j0 < P; j0 += WAVES * D) {
        uint4 a[D][4], b[D][NC][4];
#pragma unroll
        for (int d = 0; d < D; ++d) {
          const int pr = j0 + WAVES * d;
          if (pr < P) {
#pragma unroll
            for (int s = 0; s < 4; ++s) a[d][s] = *reinterpret_cast<const uint4*>(wr + 128 * static_cast<int64_t>(pr) + 8 * s);
#pragma unroll
            for (int rc = 0; rc < NC; ++rc) {
              if (rc < nrc) {
                const int64_t row = rb + rc * 16 + l16;
                const uint16_t* xr = x + row * K + 128 * static_cast<int64_t>(pr) + 32 * q;
#pragma unroll
                for (int s = 0; s < 4; ++s)
                  b[d][rc][s] = row < M ? *reinterpret_cast<const uint4*>(xr + 8 * s) : uint4{0u, 0u, 0u, 0u};
              }
            }
          }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
          if (j0 + WAVES * d < P) {
#pragma unroll
            for (int rc = 0; rc < NC; ++rc) {
              if (rc < nrc) {
#pragma unroll
                for (int s = 0; s < 4; ++s)
                  acc[rc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a[d][s]),
                                                                    __builtin_bit_cast(bf16x8_t, b[d][rc][s]), acc[rc],
                                                                    0, 0, 0);
              }
            }
          }
        }
      }
#pragma unroll
      for (int rc = 0; rc < NC; ++rc) {
        if (rc < nrc) {
          __syncthreads();
          if (wv > 0) s_red[wv - 1][lane] = acc[rc];
          __syncthreads();
          if (wv == 0) {
            floatx4 sum = acc[rc];
#pragma unroll
            for (int v = 0; v < WAVES - 1; ++v) sum += s_red[v][lane];
            const int64_t row = rb + rc * 16 + l16;
            if (row < M) {
              const int64_t o = row * N + ct * 16 + 4 * q;
              if constexpr (OUT_F32)
                *reinterpret_cast<floatx4*>(static_cast<float*>(out) + o) = sum;
              else
                *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + o) =
                    uint2{pack_bf16x2(sum[0], sum[1]), pack_bf16x2(sum[2], sum[3])};
            }
          }
        }
      }
    }
  }
}

template <int NC, int WAVES, bool F32>
void launch_dense(const uint16_t* x, const uint16_t* w, int64_t M, int64_t K, int64_t N, void* out, hipStream_t st) {
  static std::atomic<unsigned> cached{0};
  unsigned res = cached.load(std::memory_order_relaxed);
  if (res == 0) {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, skinny_dense_kernel<NC, WAVES, F32>, WAVES * 64, 0) !=
            hipSuccess ||
        cus <= 0 || per_cu <= 0) {
      cus = 256;
      per_cu = 1;
    }
    res = static_cast<unsigned>(cus * per_cu);
    cached.store(res, std::memory_order_relaxed);
  }
  const unsigned grid = static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(N / 16, res)));
  skinny_dense_kernel<NC, WAVES, F32><<<grid, WAVES * 64, 0, st>>>(x, w, M, K, N, out);
}

template <int WAVES, bool F32>
void dense_nc(int nc, const uint16_t* x, const uint16_t* w, int64_t M, int64_t K, int64_t N, void* out,
              hipStream_t st) {
  switch (nc) {
    case 1: launch_dense<1, WAVES, F32>(x, w, M, K, N, out, st); break;
    case 2: launch_dense<2, WAVES, F32>(x, w, M, K, N, out, st); break;
    default: launch_dense<4, WAVES, F32>(x, w, M, K, N, out, st); break;
  }
}

// Rows per pass: the smallest of 16, 32, 64 covering the largest group
// (bounded by M and by the caller's hint); larger groups take more passes.
int skinny_chunks(int64_t M, int64_t max_group_rows) {
  const int64_t bound = max_group_rows > 0 ? std::min(M, max_group_rows) : M;
  int nc = 1;
  while (nc < kSkMaxChunks && 16 * nc < bound) nc *= 2;
  return nc;
}

// Blocks of one instance resident at once on the device: the grid size (each
// block walks items with a grid stride, so no block sits idle past the first
// wave of blocks).
template <int EPI, int NC, int WAVES, bool DISP = false>
unsigned resident_blocks() {
  static std::atomic<unsigned> cached{0};
  unsigned v = cached.load(std::memory_order_relaxed);
  if (v == 0) {
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, skinny_mx_kernel<EPI, NC, WAVES, DISP>, WAVES * 64, 0) !=
            hipSuccess ||
        cus <= 0 || per_cu <= 0) {
      cus = 256;
      per_cu = 1;
    }
    v = static_cast<unsigned>(cus * per_cu);
    cached.store(v, std::memory_order_relaxed);
  }
  return v;
}

template <int EPI, int NC, int WAVES, bool DISP = false>
void launch_one(const SkinnyParams& p, int64_t upper, hipStream_t st) {
  const unsigned grid =
      static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(upper, resident_blocks<EPI, NC, WAVES, DISP>())));
  skinny_mx_kernel<EPI, NC, WAVES, DISP><<<grid, WAVES * 64, 0, st>>>(p);
}

template <int EPI, int WAVES, bool DISP = false>
void launch_nc(const SkinnyParams& p, int nc, int64_t upper, hipStream_t st) {
  switch (nc) {
    case 1: launch_one<EPI, 1, WAVES, DISP>(p, upper, st); break;
    case 2: launch_one<EPI, 2, WAVES, DISP>(p, upper, st); break;
    default: launch_one<EPI, 4, WAVES, DISP>(p, upper, st); break;
  }
}

}  // namespace
}  // namespace gemm
}  // namespace lmoe

using namespace lmoe;
using namespace lmoe::gemm;

extern "C" int lmoe_ragged_dot_mxfp4_skinny(const void* lhs, const uint8_t* w_tiled, const uint8_t* s_tiled,
                                            const int32_t* group_sizes, int64_t M, int64_t K, int64_t N, int64_t G,
                                            int zero_group, int flags, int epilogue, float beta, float beta_lin,
                                            int64_t max_group_rows, void* out, void* stream) {
  const char* name = "ragged_dot_mxfp4_skinny";
  LMOE_CHECK_ARG(M >= 0 && K > 0 && N > 0 && G > 0, "%s: bad sizes M=%lld K=%lld N=%lld G=%lld", name,
                 (long long)M, (long long)K, (long long)N, (long long)G);
  LMOE_CHECK_ARG(zero_group >= -1 && zero_group < G, "%s: bad zero_group %d", name, zero_group);
  LMOE_CHECK_ARG(epilogue == LMOE_EPI_NONE || epilogue == LMOE_EPI_SITU, "%s: bad epilogue", name);
  LMOE_CHECK_ARG((flags & ~LMOE_MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS) == 0, "%s: unknown flags 0x%x", name, flags);
  const int epi = epilogue == LMOE_EPI_SITU ? kEpiSitu : kEpiNone;
  LMOE_CHECK_SUPPORTED(K % 128 == 0, "%s: needs K %% 128 == 0 (K=%lld)", name, (long long)K);
  LMOE_CHECK_SUPPORTED(N % (epi == kEpiSitu ? 32 : 16) == 0, "%s: needs 16-column output tiles (N=%lld)", name,
                       (long long)N);
  LMOE_CHECK_SUPPORTED(G <= kSkMaxGroups, "%s: at most %d groups (G=%lld)", name, kSkMaxGroups, (long long)G);
  LMOE_CHECK_SUPPORTED(M < (1ll << 31) && K < (1ll << 31) && N < (1ll << 31) && extent_ok({M, K}) &&
                           extent_ok({G, K, N}) && extent_ok({M, N}),
                       "%s: sizes beyond device memory (M=%lld K=%lld N=%lld)", name, (long long)M, (long long)K,
                       (long long)N);
  if (M == 0) return LMOE_OK;
  LMOE_CHECK_ARG(lhs && w_tiled && s_tiled && group_sizes && out, "%s: null pointer", name);
  LMOE_CHECK_SUPPORTED(aligned(lhs, 16) && aligned(w_tiled, 16) && aligned(out, 16) && aligned(s_tiled, 2),
                       "%s: lhs, weights and out must be 16-byte aligned", name);
  const int nc = skinny_chunks(M, max_group_rows);
  const int64_t nout = epi == kEpiSitu ? N / 2 : N;
  const int64_t nct = nout / 16;
  SkinnyParams p{static_cast<const uint16_t*>(lhs), w_tiled, s_tiled, group_sizes, M, K, N, G, zero_group,
                 (flags & LMOE_MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS) != 0, beta, beta_lin, static_cast<uint16_t*>(out),
                 static_cast<int>(nct)};
  // at most min(G, M) groups have rows: with fewer items than one per CU,
  // eight waves per item (more of the K axis in flight), else four
  const int64_t items_bound = std::min<int64_t>(G, M) * nct;
  const int64_t upper = std::max(items_bound, ceil_div(M * nout / 8, 256));
  const bool wide = items_bound < 256;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (epi == kEpiSitu) {
    if (wide)
      launch_nc<kEpiSitu, 8>(p, nc, upper, st);
    else
      launch_nc<kEpiSitu, 4>(p, nc, upper, st);
  } else {
    if (wide)
      launch_nc<kEpiNone, 8>(p, nc, upper, st);
    else
      launch_nc<kEpiNone, 4>(p, nc, upper, st);
  }
  LMOE_CHECK_LAUNCH(name);
  return LMOE_OK;
}

extern "C" int lmoe_dispatch_mxfp4_skinny(const int32_t* topk_idx, const void* topk_w, int w_dtype, const void* x,
                                          int64_t x_ld, int64_t T, int64_t k, int64_t local_start, int64_t L,
                                          int64_t m_padded, const uint8_t* w_tiled, const uint8_t* s_tiled, int64_t K,
                                          int64_t N, int epilogue, float beta, float beta_lin, int flags,
                                          int32_t* group_sizes, uint8_t* valid, int32_t* per_expert_counts,
                                          int32_t* padded_token_idx, void* padded_w, int32_t* slot_pos, void* out,
                                          void* stream) {
  const char* name = "dispatch_mxfp4_skinny";
  LMOE_CHECK_ARG(T >= 0 && k > 0 && L > 0 && m_padded >= 0 && local_start >= 0 && K > 0 && N > 0 && x_ld >= K,
                 "%s: bad sizes T=%lld k=%lld L=%lld m_padded=%lld K=%lld N=%lld x_ld=%lld", name, (long long)T,
                 (long long)k, (long long)L, (long long)m_padded, (long long)K, (long long)N, (long long)x_ld);
  LMOE_CHECK_ARG(w_dtype == LMOE_BF16 || w_dtype == LMOE_F32, "%s: combine weights must be bf16 or f32", name);
  LMOE_CHECK_ARG(epilogue == LMOE_EPI_NONE || epilogue == LMOE_EPI_SITU, "%s: bad epilogue", name);
  LMOE_CHECK_ARG((flags & ~LMOE_MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS) == 0, "%s: unknown flags 0x%x", name, flags);
  const int epi = epilogue == LMOE_EPI_SITU ? kEpiSitu : kEpiNone;
  LMOE_CHECK_SUPPORTED(T <= kSkDispSlots && k <= kSkDispSlots && T * k <= kSkDispSlots && m_padded <= kSkDispRows &&
                           L + 1 <= kSkMaxGroups,
                       "%s: at most %d slots, %d rows and %d experts (T=%lld k=%lld m_padded=%lld L=%lld)", name,
                       kSkDispSlots, kSkDispRows, kSkMaxGroups - 1, (long long)T, (long long)k, (long long)m_padded,
                       (long long)L);
  LMOE_CHECK_SUPPORTED(local_start < (1ll << 31) - L && K < (1ll << 31) && N < (1ll << 31) && extent_ok({T, x_ld}) &&
                           extent_ok({L + 1, K, N}) && extent_ok({m_padded, N}),
                       "%s: sizes beyond device memory (local_start=%lld K=%lld N=%lld x_ld=%lld)", name,
                       (long long)local_start, (long long)K, (long long)N, (long long)x_ld);
  LMOE_CHECK_SUPPORTED(K % 128 == 0 && x_ld % 8 == 0, "%s: needs K %% 128 == 0 and 16-byte rows (K=%lld x_ld=%lld)",
                       name, (long long)K, (long long)x_ld);
  LMOE_CHECK_SUPPORTED(N % (epi == kEpiSitu ? 32 : 16) == 0, "%s: needs 16-column output tiles (N=%lld)", name,
                       (long long)N);
  LMOE_CHECK_ARG(group_sizes && valid && per_expert_counts && padded_token_idx && padded_w && w_tiled && s_tiled &&
                     (T == 0 || (topk_idx && topk_w && x)) && (out || m_padded == 0),
                 "%s: null pointer", name);
  LMOE_CHECK_SUPPORTED((T == 0 || aligned(x, 16)) && aligned(w_tiled, 16) && aligned(out, 16) && aligned(s_tiled, 2),
                       "%s: x, weights and out must be 16-byte aligned", name);
  const int64_t G = L + 1;
  const int nc = skinny_chunks(m_padded, T);
  const int64_t nout = epi == kEpiSitu ? N / 2 : N;
  const int64_t nct = nout / 16;
  SkinnyParams p{static_cast<const uint16_t*>(x), w_tiled, s_tiled, group_sizes, m_padded, K, N, G,
                 static_cast<int>(L), (flags & LMOE_MXFP4_FLAG_SKIP_ZERO_GROUP_ROWS) != 0, beta, beta_lin,
                 static_cast<uint16_t*>(out), static_cast<int>(nct)};
  p.d_idx = topk_idx;
  p.d_w_in = static_cast<const uint8_t*>(topk_w);
  p.d_wsize = dtype_size(w_dtype);
  p.d_n = T * k;
  p.d_k = k;
  p.x_ld = x_ld;
  p.d_start = static_cast<int>(local_start);
  p.d_L = static_cast<int>(L);
  p.d_group_sizes = group_sizes;
  p.d_valid = valid;
  p.d_counts = per_expert_counts;
  p.d_tok = padded_token_idx;
  p.d_w_out = static_cast<uint8_t*>(padded_w);
  p.d_slot_pos = slot_pos;
  const int64_t items_bound = std::min<int64_t>(G, std::max<int64_t>(m_padded, 1)) * nct;
  const int64_t upper = std::max(items_bound, ceil_div(m_padded * nout / 8, 256));
  const bool wide = items_bound < 256;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (epi == kEpiSitu) {
    if (wide)
      launch_nc<kEpiSitu, 8, true>(p, nc, upper, st);
    else
      launch_nc<kEpiSitu, 4, true>(p, nc, upper, st);
  } else {
    if (wide)
      launch_nc<kEpiNone, 8, true>(p, nc, upper, st);
    else
      launch_nc<kEpiNone, 4, true>(p, nc, upper, st);
  }
  LMOE_CHECK_LAUNCH(name);
  return LMOE_OK;
}

extern "C" int lmoe_dense_skinny(const void* x, const void* w_nk, int64_t M, int64_t K, int64_t N, void* out,
                                 int out_dtype, void* stream) {
  const char* name = "dense_skinny";
  LMOE_CHECK_ARG(M >= 0 && K > 0 && N > 0, "%s: bad sizes M=%lld K=%lld N=%lld", name, (long long)M, (long long)K,
                 (long long)N);
  LMOE_CHECK_ARG(out_dtype == LMOE_BF16 || out_dtype == LMOE_F32, "%s: bad out dtype", name);
  LMOE_CHECK_SUPPORTED(K % 128 == 0 && N % 16 == 0, "%s: needs K %% 128 == 0 and N %% 16 == 0 (K=%lld N=%lld)",
                       name, (long long)K, (long long)N);
  LMOE_CHECK_SUPPORTED(M < (1ll << 31) && K < (1ll << 31) && N < (1ll << 31) && extent_ok({M, K}) &&
                           extent_ok({N, K}) && extent_ok({M, N}),
                       "%s: sizes beyond device memory (M=%lld K=%lld N=%lld)", name, (long long)M, (long long)K,
                       (long long)N);
  if (M == 0) return LMOE_OK;
  LMOE_CHECK_ARG(x && w_nk && out, "%s: null pointer", name);
  LMOE_CHECK_SUPPORTED(aligned(x, 16) && aligned(w_nk, 16) && aligned(out, 16), "%s: 16-byte alignment", name);
  const int nc = skinny_chunks(M, 0);
  const auto* xp = static_cast<const uint16_t*>(x);
  const auto* wp = static_cast<const uint16_t*>(w_nk);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // fewer 16-column items than CUs: eight waves per item, else four
  const bool wide = N / 16 < 256;
  if (out_dtype == LMOE_F32) {
    if (wide)
      dense_nc<8, true>(nc, xp, wp, M, K, N, out, st);
    else
      dense_nc<4, true>(nc, xp, wp, M, K, N, out, st);
  } else {
    if (wide)
      dense_nc<8, false>(nc, xp, wp, M, K, N, out, st);
    else
      dense_nc<4, false>(nc, xp, wp, M, K, N, out, st);
  }
  LMOE_CHECK_LAUNCH(name);
  return LMOE_OK;
}
