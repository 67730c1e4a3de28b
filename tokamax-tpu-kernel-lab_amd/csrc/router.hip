// Router top-k (reference _router_gate, ref.py:601-631, and latent_moe_forward
// step 1, ref.py:347-361): one 64-wide wavefront per token.
//
// Each lane owns the experts e = c*64 + lane (c < EPL), so the logits row is read
// with fully coalesced loads.  The order is "descending score + bias, ties to
// the lower expert id" -- jax.lax.top_k's order.
//
// Exact scores are the gate functions of gate_math.h (binary64 evaluation with
// a fixed operation sequence, one rounding to f32), so the host-side checker
// can reproduce them bit for bit; the softmax denominator is summed in
// binary64 in a fixed order (each lane over its experts c = 0, 1, ..., then an
// xor butterfly over lane distances 32, 16, ..., 1).  The renormalisation sum
// of the k chosen weights runs in f32 in top-k order.
//
// Candidate path (sigmoid gate, k <= 64, no full score output): every score
// is first computed with the hardware exp / reciprocal (a few f32 ulp), which
// only serves to find a threshold: the k-th largest of the 64 lane maxima
// (radix select over ballots) is <= the k-th largest approximate key, so
// every exact top-k element lies within the approximation error of it or
// above.  Elements above threshold - 2^-18 (|threshold| + 1) -- a margin far
// above twice that error -- are compacted to LDS (usually barely more than
// k), their exact scores recomputed with the same correctly rounded
// operations as the full path, and each of the at most 64 candidates ranked
// on (key, -expert) by counting the larger keys, broadcast from LDS (one
// dependent step instead of a 21-stage sort network).  The result is
// identical to the full path's.  More than 64 candidates (massive ties) fall
// back to the full path.
//
// Full path: exact scores for all experts, then k rounds of a wavefront
// arg-max: a wave maximum of the order-preserving float bits of every lane's
// best remaining candidate, then a wave minimum of the expert ids holding that
// value.  Both reductions are DPP row shifts / broadcasts; only the winning
// lane rescans its EPL candidates.
#include <cmath>

#include "gate_math.h"
#include "lmoe_common.h"

namespace lmoe {
namespace {

constexpr int kWave = 64;
constexpr int kWavesPerBlock = 4;

__device__ __forceinline__ uint32_t ordered_bits(float f) {
  if (f == 0.0f) f = 0.0f;  // -0 and +0 compare equal: canonicalise
  uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Sum over the wave by an xor butterfly (distances 32, 16, ..., 1); every
// lane ends with the same bits (each step adds the same two values).
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = __dadd_rn(v, __shfl_xor(v, off, kWave));
  return v;
}

__device__ __forceinline__ float from_ordered(uint32_t u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

// Largest v with #{lanes : x >= v} >= k (the k-th largest x), by radix
// select from the top bit: one ballot per bit.
__device__ __forceinline__ uint32_t wave_kth_largest(uint32_t x, int k) {
  uint32_t prefix = 0;
#pragma unroll
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = prefix | (1u << bit);
    if (__popcll(__ballot(x >= cand)) >= k) prefix = cand;
  }
  return prefix;
}

// CAST: the same wave also rounds the token's projection row xsrc[t, :lat]
// (f32, row stride xld) to bf16 into xout[t, :] (lat <= kCastCols, lat % 4
// == 0): its loads go out with the logits loads and its stores come last, so
// the latency-bound selection hides them.
constexpr int kCastCols = 4 * 4 * kWave;

template <int EPL, bool CAST>
__global__ __launch_bounds__(256) void router_topk_kernel(
    const float* __restrict__ logits, int64_t ld, const float* __restrict__ bias, int T, int E, int k, int act,
    int renorm, float scale, int wdtype, int32_t* __restrict__ idx_out, void* __restrict__ w_out,
    float* __restrict__ scores_out, const float* __restrict__ xsrc, int64_t xld, int lat,
    uint16_t* __restrict__ xout) {
  const int lane = threadIdx.x % kWave;
  const int t = blockIdx.x * kWavesPerBlock + threadIdx.x / kWave;
  if (t >= T) return;
  const float* row = logits + static_cast<int64_t>(t) * ld;

  float s[EPL];
  uint32_t key[EPL];
#pragma unroll
  for (int c = 0; c < EPL; ++c) {
    const int e = c * kWave + lane;
    s[c] = e < E ? row[e] : -INFINITY;
  }
  float4 xv[CAST ? 4 : 1];
  if constexpr (CAST) {
    const float* xr = xsrc + static_cast<int64_t>(t) * xld;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int col = c * 4 * kWave + 4 * lane;
      if (col < lat) xv[c] = *reinterpret_cast<const float4*>(xr + col);
    }
  }
  auto emit_x = [&]() __attribute__((always_inline)) {
    if constexpr (CAST) {
      typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
      uint16_t* xo = xout + static_cast<int64_t>(t) * lat;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int col = c * 4 * kWave + 4 * lane;
        if (col < lat) {
          const bf16x2_v a = {static_cast<__bf16>(xv[c].x), static_cast<__bf16>(xv[c].y)};
          const bf16x2_v b = {static_cast<__bf16>(xv[c].z), static_cast<__bf16>(xv[c].w)};
          *reinterpret_cast<uint2*>(xo + col) = uint2{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b)};
        }
      }
    }
  };
  if (act == LMOE_ACT_SIGMOID && scores_out == nullptr && k <= kWave) {
    __shared__ float s_logit[kWavesPerBlock][kWave];
    __shared__ int32_t s_expert[kWavesPerBlock][kWave];
    __shared__ __attribute__((aligned(16))) uint64_t s_key[kWavesPerBlock][kWave];
    __shared__ __attribute__((aligned(16))) float s_w[kWavesPerBlock][kWave];
    const int wv = threadIdx.x / kWave;
    // the bias loads go out with the logits loads (one memory round trip)
    float bv[EPL];
#pragma unroll
    for (int c = 0; c < EPL; ++c) {
      const int e = c * kWave + lane;
      bv[c] = bias ? bias[e < E ? e : 0] : 0.0f;
    }
    // approximate selection keys and their lane maximum
    float ap[EPL];
    uint32_t lmax = 0;
#pragma unroll
    for (int c = 0; c < EPL; ++c) {
      const int e = c * kWave + lane;
      const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(s[c] * -1.44269504088896341f));
      ap[c] = sg + bv[c];
      if (e < E) lmax = max(lmax, ordered_bits(ap[c]));
    }
    const float th = from_ordered(wave_kth_largest(lmax, k));
    const float thr = th - 0x1p-18f * (__builtin_fabsf(th) + 1.0f);
    uint32_t n = 0;
#pragma unroll
    for (int c = 0; c < EPL; ++c) n += (c * kWave + lane < E && ap[c] >= thr) ? 1u : 0u;
    const uint32_t incl = wave_scan_sat(n, 0xffffffffu);
    const uint32_t total = __builtin_amdgcn_readlane(incl, 63);
    if (total >= static_cast<uint32_t>(k) && total <= static_cast<uint32_t>(kWave)) {
      uint32_t pos = incl - n;
#pragma unroll
      for (int c = 0; c < EPL; ++c) {
        const int e = c * kWave + lane;
        if (e < E && ap[c] >= thr) {
          s_logit[wv][pos] = s[c];
          s_expert[wv][pos] = e;
          ++pos;
        }
      }
      __builtin_amdgcn_wave_barrier();
      asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
      uint64_t ck = 0;  // below every real key
      float cs = 0.0f;
      if (static_cast<uint32_t>(lane) < total) {
        const float lg = s_logit[wv][lane];
        const int e = s_expert[wv][lane];
        cs = gate_sigmoid(lg);
        const float sel = bias ? __fadd_rn(cs, bias[e]) : __fadd_rn(cs, 0.0f);
        ck = (static_cast<uint64_t>(ordered_bits(sel)) << 32) | (0xffffffffu - static_cast<uint32_t>(e));
      }
      // rank of each candidate = number of larger keys (keys are distinct:
      // the expert id is in the low word); the candidates broadcast from LDS
      s_key[wv][lane] = ck;
      __builtin_amdgcn_wave_barrier();
      asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
      uint32_t rank = 0;
      const int n_cand = static_cast<int>(total);
      int j = 0;
      for (; j + 1 < n_cand; j += 2) {
        const ulonglong2 kk = *reinterpret_cast<const ulonglong2*>(&s_key[wv][j]);
        rank += (kk.x > ck ? 1u : 0u) + (kk.y > ck ? 1u : 0u);
      }
      if (j < n_cand) rank += s_key[wv][j] > ck ? 1u : 0u;
      // renormalisation sum in top-k order (sequential f32 adds)
      const bool top = static_cast<uint32_t>(lane) < total && rank < static_cast<uint32_t>(k);
      if (top) s_w[wv][rank] = cs;
      __builtin_amdgcn_wave_barrier();
      asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
      float sum = 0.0f;
      int q = 0;
      for (; q + 3 < k; q += 4) {
        const float4 v = *reinterpret_cast<const float4*>(&s_w[wv][q]);
        sum = __fadd_rn(__fadd_rn(__fadd_rn(__fadd_rn(sum, v.x), v.y), v.z), v.w);
      }
      for (; q < k; ++q) sum = __fadd_rn(sum, s_w[wv][q]);
      if (top) {
        float w = cs;
        if (renorm && k > 1) w = __fdiv_rn(w, __fadd_rn(sum, 1e-20f));
        w = __fmul_rn(w, scale);
        const int64_t o = static_cast<int64_t>(t) * k + rank;
        idx_out[o] = static_cast<int32_t>(0xffffffffu - static_cast<uint32_t>(ck));
        store_from_f32(w_out, o, w, wdtype);
      }
      emit_x();
      return;
    }
  }
  if (act == LMOE_ACT_SOFTMAX) {
    float m = -INFINITY;
#pragma unroll
    for (int c = 0; c < EPL; ++c) m = fmaxf(m, s[c]);
    m = wave_max_f32(m);
    double ex[EPL];
    double sum = 0.0;
#pragma unroll
    for (int c = 0; c < EPL; ++c) {
      const int e = c * kWave + lane;
      ex[c] = e < E ? gate_exp64(static_cast<double>(__fsub_rn(s[c], m))) : 0.0;
      sum = __dadd_rn(sum, ex[c]);
    }
    sum = wave_sum_f64(sum);
#pragma unroll
    for (int c = 0; c < EPL; ++c) s[c] = __double2float_rn(__ddiv_rn(ex[c], sum));
  } else {
#pragma unroll
    for (int c = 0; c < EPL; ++c) s[c] = gate_sigmoid(s[c]);
  }
  uint64_t taken = 0;
#pragma unroll
  for (int c = 0; c < EPL; ++c) {
    const int e = c * kWave + lane;
    if (e < E) {
      if (scores_out) scores_out[static_cast<int64_t>(t) * E + e] = s[c];
      const float sel = bias ? __fadd_rn(s[c], bias[e]) : __fadd_rn(s[c], 0.0f);
      key[c] = ordered_bits(sel);
    } else {
      key[c] = 0;
      taken |= 1ull << c;
    }
  }

  // this lane's best remaining candidate: largest key, ties to the lower c
  uint32_t best_key = 0;
  int best_c = -1;
  auto local_best = [&]() {
    best_key = 0;
    best_c = -1;
#pragma unroll
    for (int c = 0; c < EPL; ++c) {
      if (!((taken >> c) & 1ull) && (best_c < 0 || key[c] > best_key)) {
        best_key = key[c];
        best_c = c;
      }
    }
  };

  local_best();
  int my_idx = 0;
  float my_w = 0.0f;
  float sum = 0.0f;
  for (int j = 0; j < k; ++j) {
    const uint32_t m = wave_max_u32(best_c >= 0 ? best_key : 0u);
    const uint32_t cand = (best_c >= 0 && best_key == m) ? static_cast<uint32_t>(best_c * kWave + lane) : 0xffffffffu;
    const uint32_t e = wave_min_u32(cand);  // k <= E, so some lane holds a candidate
    const int wl = static_cast<int>(e % kWave);
    const int wc = static_cast<int>(e / kWave);
    float v = 0.0f;
#pragma unroll
    for (int c = 0; c < EPL; ++c) v = (c == wc) ? s[c] : v;
    const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), wl));
    if (lane == wl) {
      taken |= 1ull << wc;
      local_best();
    }
    if (lane == j) {
      my_idx = static_cast<int>(e);
      my_w = w;
    }
    sum = __fadd_rn(sum, w);
  }
  if (lane < k) {
    float w = my_w;
    if (renorm && k > 1) w = __fdiv_rn(w, __fadd_rn(sum, 1e-20f));
    w = __fmul_rn(w, scale);
    const int64_t o = static_cast<int64_t>(t) * k + lane;
    idx_out[o] = my_idx;
    store_from_f32(w_out, o, w, wdtype);
  }
  emit_x();
}

template <int EPL>
void launch_router(const float* logits, int64_t ld, const float* bias, int T, int E, int k, int act, int renorm,
                   float scale, int wdtype, int32_t* idx, void* w, float* scores, hipStream_t st,
                   const float* xsrc = nullptr, int64_t xld = 0, int lat = 0, uint16_t* xout = nullptr) {
  dim3 grid(static_cast<unsigned>(ceil_div(T, kWavesPerBlock)));
  if (xout)
    router_topk_kernel<EPL, true><<<grid, 256, 0, st>>>(logits, ld, bias, T, E, k, act, renorm, scale, wdtype,
                                                         idx, w, scores, xsrc, xld, lat, xout);
  else
    router_topk_kernel<EPL, false><<<grid, 256, 0, st>>>(logits, ld, bias, T, E, k, act, renorm, scale, wdtype,
                                                          idx, w, scores, nullptr, 0, 0, nullptr);
}

}  // namespace
}  // namespace lmoe

namespace {
int router_impl(const float* logits, int64_t ld, const float* bias, int64_t T, int64_t E, int64_t k, int act,
                int renorm, float scale, int weight_dtype, int32_t* topk_idx, void* topk_w, float* scores_out,
                const float* x_src, int64_t x_ld, int64_t lat, uint16_t* x_out, void* stream) {
  using namespace lmoe;
  LMOE_CHECK_ARG(T >= 0 && E > 0 && k > 0, "router_topk: bad sizes T=%lld E=%lld k=%lld",
                 (long long)T, (long long)E, (long long)k);
  LMOE_CHECK_ARG(ld >= E, "router_topk: row stride %lld < E=%lld", (long long)ld, (long long)E);
  LMOE_CHECK_ARG(k <= E, "router_topk: k=%lld > E=%lld", (long long)k, (long long)E);
  LMOE_CHECK_SUPPORTED(k <= 64, "router_topk: k=%lld > 64", (long long)k);
  LMOE_CHECK_SUPPORTED(E <= 4096, "router_topk: E=%lld > 4096", (long long)E);
  LMOE_CHECK_ARG(act == LMOE_ACT_SIGMOID || act == LMOE_ACT_SOFTMAX, "router_topk: bad act %d", act);
  LMOE_CHECK_ARG(valid_dtype(weight_dtype), "router_topk: bad weight dtype %d", weight_dtype);
  LMOE_CHECK_ARG(T <= (1ll << 30), "router_topk: T too large");
  LMOE_CHECK_SUPPORTED(extent_ok({T, ld}) && extent_ok({T, x_ld}), "router_topk: sizes beyond device memory");
  if (T == 0) return LMOE_OK;
  LMOE_CHECK_ARG(logits && topk_idx && topk_w, "router_topk: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int epl = static_cast<int>(ceil_div(E, 64));
  const int Ti = static_cast<int>(T), Ei = static_cast<int>(E), ki = static_cast<int>(k);
#define LMOE_ROUTER_CASE(N)                                                                   \
  if (epl <= N) {                                                                             \
    launch_router<N>(logits, ld, bias, Ti, Ei, ki, act, renorm, scale, weight_dtype, topk_idx, \
                     topk_w, scores_out, st, x_src, x_ld, static_cast<int>(lat), x_out);      \
    LMOE_CHECK_LAUNCH("router_topk");                                                         \
    return LMOE_OK;                                                                           \
  }
  LMOE_ROUTER_CASE(1)
  LMOE_ROUTER_CASE(2)
  LMOE_ROUTER_CASE(4)
  LMOE_ROUTER_CASE(8)
  LMOE_ROUTER_CASE(16)
  LMOE_ROUTER_CASE(32)
  LMOE_ROUTER_CASE(64)
#undef LMOE_ROUTER_CASE
  return fail(LMOE_ERR_UNSUPPORTED, "router_topk: E=%lld", (long long)E);
}
}  // namespace

extern "C" int lmoe_router_topk_ld(const float* logits, int64_t ld, const float* bias, int64_t T, int64_t E,
                                   int64_t k, int act, int renorm, float scale, int weight_dtype,
                                   int32_t* topk_idx, void* topk_w, float* scores_out, void* stream) {
  return router_impl(logits, ld, bias, T, E, k, act, renorm, scale, weight_dtype, topk_idx, topk_w, scores_out,
                     nullptr, 0, 0, nullptr, stream);
}

extern "C" int lmoe_router_topk_proj(const float* logits, int64_t ld, const float* bias, int64_t T, int64_t E,
                                     int64_t k, int act, int renorm, float scale, int weight_dtype,
                                     int32_t* topk_idx, void* topk_w, const float* x_src, int64_t x_ld,
                                     int64_t lat, uint16_t* x_out, void* stream) {
  using namespace lmoe;
  LMOE_CHECK_ARG(lat > 0 && x_ld >= lat, "router_topk_proj: bad latent sizes lat=%lld x_ld=%lld", (long long)lat,
                 (long long)x_ld);
  LMOE_CHECK_SUPPORTED(lat <= kCastCols && lat % 4 == 0 && x_ld % 4 == 0,
                       "router_topk_proj: lat=%lld (<= %d, lat %% 4 == 0)", (long long)lat, kCastCols);
  LMOE_CHECK_ARG(T == 0 || (x_src && x_out), "router_topk_proj: null pointer");
  LMOE_CHECK_SUPPORTED(aligned(x_src, 16) && aligned(x_out, 8), "router_topk_proj: x_src 16-, x_out 8-byte aligned");
  return router_impl(logits, ld, bias, T, E, k, act, renorm, scale, weight_dtype, topk_idx, topk_w, nullptr, x_src,
                     x_ld, lat, x_out, stream);
}

extern "C" int lmoe_router_topk(const float* logits, const float* bias, int64_t T, int64_t E, int64_t k, int act,
                                int renorm, float scale, int weight_dtype, int32_t* topk_idx, void* topk_w,
                                float* scores_out, void* stream) {
  return lmoe_router_topk_ld(logits, E, bias, T, E, k, act, renorm, scale, weight_dtype, topk_idx, topk_w,
                             scores_out, stream);
}
