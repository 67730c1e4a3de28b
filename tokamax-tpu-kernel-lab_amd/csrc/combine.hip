// Weighted top-k combine (reference _combine_shard_contribution,
// ref.py:1113-1141, and the unsharded combine of latent_moe_forward,
// ref.py:413-416).
//
// Atomic-free and deterministic: one 64-wide wavefront owns one token and
// accumulates that token's contributing rows itself, in ascending row order,
// which is the order the reference's scatter-add applies its updates.  The
// rows of a token come either from the dispatch's slot_pos (k slots per token,
// sorted in-wave) or, for arbitrary padded_token_idx, from a stable counting
// sort by token (csort.h).
#include "csort.h"

namespace lmoe {
namespace {

constexpr int kWave = 64;
constexpr int kTokensPerBlock = 4;
constexpr int kMaxRowsInLds = 256;

// The LDS staging arrays are private to one wavefront, so only wave-level
// ordering is needed (waves of a block work on different tokens and may run
// different trip counts, so a block barrier would be wrong here).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Accumulation state for VEC consecutive output elements of one lane.
template <int VEC>
struct Acc {
  float v[VEC];
};

template <int VEC>
__device__ __forceinline__ void load_vec(const void* p, int64_t i, int dtype, float* out) {
  if (dtype == LMOE_BF16) {
    const uint16_t* q = static_cast<const uint16_t*>(p) + i;
    if constexpr (VEC == 8) {
      const uint4 raw = *reinterpret_cast<const uint4*>(q);
      const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        out[2 * j] = __uint_as_float(w[j] << 16);
        out[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
      }
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) out[j] = bf16_to_f32(q[j]);
    }
  } else {
    const float* q = static_cast<const float*>(p) + i;
#pragma unroll
    for (int j = 0; j < VEC; ++j) out[j] = q[j];
  }
}

// VEC elements of either dtype kept as raw 32-bit words (bf16: the first
// VEC/2 words), to be converted later: a load issued early without holding
// VEC floats.
template <int VEC>
struct RawVec {
  uint32_t w[VEC];
};

template <int VEC>
__device__ __forceinline__ RawVec<VEC> load_raw(const void* p, int64_t i, int dtype) {
  RawVec<VEC> r{};
  if (dtype == LMOE_BF16) {
    const uint16_t* q = static_cast<const uint16_t*>(p) + i;
    if constexpr (VEC == 8) {
      const uint4 v = *reinterpret_cast<const uint4*>(q);
      r.w[0] = v.x, r.w[1] = v.y, r.w[2] = v.z, r.w[3] = v.w;
    } else {
#pragma unroll
      for (int j = 0; j < VEC / 2; ++j) r.w[j] = static_cast<uint32_t>(q[2 * j]) | (static_cast<uint32_t>(q[2 * j + 1]) << 16);
    }
  } else {
    const float* q = static_cast<const float*>(p) + i;
#pragma unroll
    for (int j = 0; j < VEC; ++j) r.w[j] = __float_as_uint(q[j]);
  }
  return r;
}

template <int VEC>
__device__ __forceinline__ void unpack_raw(const RawVec<VEC>& r, int dtype, float* out) {
  if (dtype == LMOE_BF16) {
#pragma unroll
    for (int j = 0; j < VEC / 2; ++j) {
      out[2 * j] = __uint_as_float(r.w[j] << 16);
      out[2 * j + 1] = __uint_as_float(r.w[j] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int j = 0; j < VEC; ++j) out[j] = __uint_as_float(r.w[j]);
  }
}

template <int VEC>
__device__ __forceinline__ void store_vec(void* p, int64_t i, int dtype, const float* v) {
  if (dtype == LMOE_BF16) {
    uint16_t* q = static_cast<uint16_t*>(p) + i;
    if constexpr (VEC == 8) {
      uint4 raw;
      raw.x = f32_to_bf16(v[0]) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
      raw.y = f32_to_bf16(v[2]) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
      raw.z = f32_to_bf16(v[4]) | (static_cast<uint32_t>(f32_to_bf16(v[5])) << 16);
      raw.w = f32_to_bf16(v[6]) | (static_cast<uint32_t>(f32_to_bf16(v[7])) << 16);
      *reinterpret_cast<uint4*>(q) = raw;
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j) q[j] = f32_to_bf16(v[j]);
    }
  } else {
    float* q = static_cast<float*>(p) + i;
#pragma unroll
    for (int j = 0; j < VEC; ++j) q[j] = v[j];
  }
}

// Adds the rows rows[0..n) (ascending) with weights wts[] into routed_out[t]
// with the scatter-add rounding: product in promoted(shard, w) dtype, cast to
// out dtype, each add rounded to out dtype.  Rows are loaded kBatch at a time
// before any is added, so their memory latencies overlap; the adds keep the
// ascending order.
template <int VEC>
__device__ __forceinline__ void accumulate_token(const void* shard, int sdt, const int32_t* rows, const float* wts,
                                                 int n, int64_t lat, void* out, int odt, int64_t t, int prod_dt,
                                                 int lane) {
  constexpr int kBatch = VEC == 8 ? 8 : 4;
  for (int64_t c0 = static_cast<int64_t>(lane) * VEC; c0 < lat; c0 += kWave * VEC) {
    float acc[VEC];
    load_vec<VEC>(out, t * lat + c0, odt, acc);
    for (int r0 = 0; r0 < n; r0 += kBatch) {
      // unconditional loads (a batch past n re-reads row n-1) keep the loads
      // of a batch together ahead of the adds
      float x[kBatch][VEC];
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        const int r = r0 + b < n ? r0 + b : n - 1;
        load_vec<VEC>(shard, static_cast<int64_t>(rows[r]) * lat + c0, sdt, x[b]);
      }
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        if (r0 + b >= n) break;
        const float w = wts[r0 + b];
#pragma unroll
        for (int j = 0; j < VEC; ++j) {
          float v = round_to(__fmul_rn(x[b][j], w), prod_dt);
          v = round_to(v, odt);
          acc[j] = round_to(__fadd_rn(acc[j], v), odt);
        }
      }
    }
    store_vec<VEC>(out, t * lat + c0, odt, acc);
  }
}

// SDT / ODT >= 0 fix the shard / output dtypes at compile time (the layer's
// bf16 case), which keeps the batched row loads free of dtype branches; -1
// reads them from the arguments.
template <int VEC, int SDT = -1, int ODT = -1>
__global__ __launch_bounds__(256) void combine_slots_kernel(
    const void* __restrict__ shard, int sdt_arg, const int32_t* __restrict__ slot_pos,
    const void* __restrict__ w, int wdt, int T, int k, int64_t lat, int mode, void* __restrict__ out,
    int odt_arg) {
  const int sdt = SDT >= 0 ? SDT : sdt_arg, odt = ODT >= 0 ? ODT : odt_arg;
  __shared__ int32_t rows_s[kTokensPerBlock][kWave];
  __shared__ float wts_s[kTokensPerBlock][kWave];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int t = blockIdx.x * kTokensPerBlock + wave;
  if (t >= T) return;
  int p = -1;
  if (lane < k) p = slot_pos[static_cast<int64_t>(t) * k + lane];
  if (mode == LMOE_COMBINE_SLOT_SUM) {
    // f32 weighted sum over slots j = 0..k-1, one cast at the end (ref.py:413-416).
    float wj = lane < k ? load_as_f32(w, static_cast<int64_t>(t) * k + lane, wdt) : 0.0f;
    rows_s[wave][lane] = p;
    wts_s[wave][lane] = wj;
    wave_sync();
    for (int64_t c0 = static_cast<int64_t>(lane) * VEC; c0 < lat; c0 += kWave * VEC) {
      float acc[VEC];
#pragma unroll
      for (int j = 0; j < VEC; ++j) acc[j] = 0.0f;
      constexpr int kBatch = VEC == 8 ? 8 : 4;  // row loads in flight before the adds
      for (int j0 = 0; j0 < k; j0 += kBatch) {
        float x[kBatch][VEC];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
          // unconditional loads (dropped slots re-read row 0) keep the batch's
          // loads together ahead of the adds
          const int row = j0 + b < k ? rows_s[wave][j0 + b] : -1;
          load_vec<VEC>(shard, static_cast<int64_t>(row >= 0 ? row : 0) * lat + c0, sdt, x[b]);
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
          const int row = j0 + b < k ? rows_s[wave][j0 + b] : -1;
          if (row < 0) continue;
          const float wv = wts_s[wave][j0 + b];
#pragma unroll
          for (int q = 0; q < VEC; ++q) acc[q] = __fadd_rn(acc[q], __fmul_rn(x[b][q], wv));
        }
      }
      store_vec<VEC>(out, static_cast<int64_t>(t) * lat + c0, odt, acc);
    }
    return;
  }
  // Scatter-add mode: order this token's kept rows ascending (k <= 64).
  const bool valid = lane < k && p >= 0;
  int rank = 0;
  for (int j = 0; j < k; ++j) {
    const int pj = __shfl(p, j, kWave);
    rank += (pj >= 0 && pj < p) ? 1 : 0;
  }
  const int n = __popcll(__ballot(valid));
  if (valid) {
    rows_s[wave][rank] = p;
    wts_s[wave][rank] = load_as_f32(w, p, wdt);
  }
  wave_sync();
  const int prod_dt = (sdt == LMOE_F32 || wdt == LMOE_F32) ? LMOE_F32 : LMOE_BF16;
  accumulate_token<VEC>(shard, sdt, rows_s[wave], wts_s[wave], n, lat, out, odt, t, prod_dt, lane);
}

// ---- generic scatter-add over an arbitrary padded_token_idx --------------------

struct TokenKey {
  const int32_t* idx;
  int T;
  __device__ __forceinline__ int operator()(int64_t s) const {
    const int t = idx[s];
    return (t >= 0 && t < T) ? t : T;
  }
};

struct OrderSink {
  int32_t* order;
  __device__ __forceinline__ uint32_t load(int64_t) const { return 0u; }
  __device__ __forceinline__ void operator()(int64_t s, int key, int pos, bool real, uint32_t) const {
    if (real) order[pos] = static_cast<int32_t>(s);
  }
};

template <int VEC>
__global__ __launch_bounds__(256) void combine_csr_kernel(
    const void* __restrict__ shard, int sdt, const int32_t* __restrict__ order,
    const int32_t* __restrict__ offsets, const void* __restrict__ w, int wdt, int T, int64_t lat,
    void* __restrict__ out, int odt) {
  __shared__ int32_t rows_s[kTokensPerBlock][kMaxRowsInLds];
  __shared__ float wts_s[kTokensPerBlock][kMaxRowsInLds];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int t = blockIdx.x * kTokensPerBlock + wave;
  if (t >= T) return;
  const int prod_dt = (sdt == LMOE_F32 || wdt == LMOE_F32) ? LMOE_F32 : LMOE_BF16;
  const int b = offsets[t], e = offsets[t + 1];
  // Rows are consumed in batches that fit the LDS staging area; the running
  // sum lives in routed_out between batches, so the add order is unchanged.
  for (int q0 = b; q0 < e; q0 += kMaxRowsInLds) {
    const int n = (e - q0) < kMaxRowsInLds ? (e - q0) : kMaxRowsInLds;
    for (int i = lane; i < n; i += kWave) {
      const int row = order[q0 + i];
      rows_s[wave][i] = row;
      wts_s[wave][i] = load_as_f32(w, row, wdt);
    }
    wave_sync();
    accumulate_token<VEC>(shard, sdt, rows_s[wave], wts_s[wave], n, lat, out, odt, t, prod_dt, lane);
    wave_sync();
  }
}

// Combine into a zero-initialised routed row followed by the RMSNorm of
// that row (ref.py:413-416 / 1113-1141, then ref.py:286-293 / 427): the wave
// that builds token t's row keeps it in registers (R passes of VEC elements
// per lane, lat <= 64 * VEC * R) and normalises it, so the routed row need not
// be written (routed_out may be NULL) or read back.  Same per-element
// rounding sequence as lmoe_combine_slots on a zeroed output followed by
// lmoe_rms_norm, and the same element-to-lane split as lmoe_rms_norm (VEC 8
// for bf16, 4 for f32), so the sum of squares runs in the same order and the
// result is bit-identical to the two-kernel path.
template <int VEC, int R, int SDT = -1, int ODT = -1>
__global__ __launch_bounds__(256) void combine_norm_kernel(
    const void* __restrict__ shard, int sdt_arg, const int32_t* __restrict__ slot_pos,
    const void* __restrict__ w, int wdt, int T, int k, int64_t lat, int mode, const void* __restrict__ norm_scale,
    float eps, void* __restrict__ routed_out, void* __restrict__ normed_out, int odt_arg) {
  const int sdt = SDT >= 0 ? SDT : sdt_arg, odt = ODT >= 0 ? ODT : odt_arg;
  __shared__ int32_t rows_s[kTokensPerBlock][kWave];
  __shared__ float wts_s[kTokensPerBlock][kWave];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int t = blockIdx.x * kTokensPerBlock + wave;
  if (t >= T) return;
  // the norm scale does not depend on the routing: its loads go out first
  RawVec<VEC> sc_raw[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t c0 = static_cast<int64_t>(r) * kWave * VEC + static_cast<int64_t>(lane) * VEC;
    if (c0 < lat) sc_raw[r] = load_raw<VEC>(norm_scale, c0, odt);
  }
  int p = -1;
  if (lane < k) p = slot_pos[static_cast<int64_t>(t) * k + lane];
  const bool slot_sum = mode == LMOE_COMBINE_SLOT_SUM;
  int n;
  if (slot_sum) {
    rows_s[wave][lane] = p;
    wts_s[wave][lane] = lane < k ? load_as_f32(w, static_cast<int64_t>(t) * k + lane, wdt) : 0.0f;
    n = k;
  } else {
    // ascending row order: rank = number of this token's kept rows below p,
    // counted against the k slots broadcast from LDS (the weight load is in
    // flight meanwhile)
    const bool valid = lane < k && p >= 0;
    const float wp = valid ? load_as_f32(w, p, wdt) : 0.0f;
    rows_s[wave][lane] = p;
    wave_sync();
    int rank = 0;
    for (int j = 0; j < k; ++j) {
      const int pj = rows_s[wave][j];
      rank += (pj >= 0 && pj < p) ? 1 : 0;
    }
    n = __popcll(__ballot(valid));
    wave_sync();
    if (valid) {
      rows_s[wave][rank] = p;
      wts_s[wave][rank] = wp;
    }
  }
  wave_sync();
  const int prod_dt = (sdt == LMOE_F32 || wdt == LMOE_F32) ? LMOE_F32 : LMOE_BF16;
  constexpr int kBatch = VEC == 8 ? 8 : 4;
  float v[R][VEC];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t c0 = static_cast<int64_t>(r) * kWave * VEC + static_cast<int64_t>(lane) * VEC;
#pragma unroll
    for (int q = 0; q < VEC; ++q) v[r][q] = 0.0f;
    if (c0 >= lat) continue;
    for (int r0 = 0; r0 < n; r0 += kBatch) {
      float x[kBatch][VEC];
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        // unconditional loads (past the end / dropped slots re-read a valid
        // row) keep a batch's loads together ahead of its adds
        int row = rows_s[wave][r0 + b < n ? r0 + b : n - 1];
        row = row >= 0 ? row : 0;
        load_vec<VEC>(shard, static_cast<int64_t>(row) * lat + c0, sdt, x[b]);
      }
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        if (r0 + b >= n) break;
        const float wv = wts_s[wave][r0 + b];
        if (slot_sum) {
          if (rows_s[wave][r0 + b] < 0) continue;
#pragma unroll
          for (int q = 0; q < VEC; ++q) v[r][q] = __fadd_rn(v[r][q], __fmul_rn(x[b][q], wv));
        } else {
#pragma unroll
          for (int q = 0; q < VEC; ++q) {
            float a = round_to(__fmul_rn(x[b][q], wv), prod_dt);
            a = round_to(a, odt);
            v[r][q] = round_to(__fadd_rn(v[r][q], a), odt);
          }
        }
      }
    }
    if (slot_sum) {
#pragma unroll
      for (int q = 0; q < VEC; ++q) v[r][q] = round_to(v[r][q], odt);
    }
    if (routed_out) store_vec<VEC>(routed_out, static_cast<int64_t>(t) * lat + c0, odt, v[r]);
  }
  // RMSNorm of the routed row: the per-lane order of lmoe_rms_norm
  float ss = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (static_cast<int64_t>(r) * kWave * VEC + static_cast<int64_t>(lane) * VEC >= lat) continue;
#pragma unroll
    for (int q = 0; q < VEC; ++q) ss = __fadd_rn(ss, __fmul_rn(v[r][q], v[r][q]));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss = __fadd_rn(ss, __shfl_xor(ss, off, kWave));
  const float var = __fdiv_rn(ss, static_cast<float>(lat));
  const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(var, eps)));
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int64_t c0 = static_cast<int64_t>(r) * kWave * VEC + static_cast<int64_t>(lane) * VEC;
    if (c0 >= lat) continue;
    float sc[VEC], o[VEC];
    unpack_raw<VEC>(sc_raw[r], odt, sc);
#pragma unroll
    for (int q = 0; q < VEC; ++q) o[q] = __fmul_rn(round_to(__fmul_rn(v[r][q], inv), odt), sc[q]);
    store_vec<VEC>(normed_out, static_cast<int64_t>(t) * lat + c0, odt, o);
  }
}

// Many bins (tokens): large chunks keep the scanned (token, chunk) array small.
constexpr int kCombineChunk = 1024;

int64_t combine_ws_bytes(int64_t m, int64_t T) {
  const int64_t chunks = csort::num_chunks<kCombineChunk>(m > 0 ? m : 1);
  return (2 * chunks * T + (T + 1) + m + 64) * static_cast<int64_t>(sizeof(int32_t));
}

bool vec8_ok(const void* a, const void* b, int64_t lat, int adt, int bdt) {
  return lat % 8 == 0 && aligned(a, adt == LMOE_BF16 ? 16 : 32) && aligned(b, bdt == LMOE_BF16 ? 16 : 32);
}

}  // namespace
}  // namespace lmoe

extern "C" int64_t lmoe_combine_workspace_size(int64_t m, int64_t T) {
  if (m < 0 || T < 0 || m >= (1ll << 31) || T >= (1ll << 31)) return -1;
  return lmoe::combine_ws_bytes(m, T);
}

extern "C" int lmoe_combine_slots(const void* shard_out, int shard_dtype, const int32_t* slot_pos,
                                  const void* w, int w_dtype, int64_t T, int64_t k, int64_t lat,
                                  int mode, void* routed_out, int out_dtype, void* stream) {
  using namespace lmoe;
  LMOE_CHECK_ARG(T >= 0 && k > 0 && lat > 0, "combine_slots: bad sizes");
  LMOE_CHECK_SUPPORTED(k <= 64, "combine_slots: k=%lld > 64", (long long)k);
  LMOE_CHECK_ARG(valid_dtype(shard_dtype) && valid_dtype(w_dtype) && valid_dtype(out_dtype),
                 "combine_slots: bad dtype");
  LMOE_CHECK_ARG(mode == LMOE_COMBINE_SCATTER_ADD || mode == LMOE_COMBINE_SLOT_SUM,
                 "combine_slots: bad mode %d", mode);
  LMOE_CHECK_SUPPORTED(T < (1ll << 31), "combine_slots: T too large");
  LMOE_CHECK_SUPPORTED(extent_ok({T, lat}), "combine_slots: sizes beyond device memory");
  if (T == 0) return LMOE_OK;
  LMOE_CHECK_ARG(shard_out && slot_pos && w && routed_out, "combine_slots: null pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned blocks = static_cast<unsigned>(ceil_div(T, kTokensPerBlock));
  if (vec8_ok(shard_out, routed_out, lat, shard_dtype, out_dtype) && shard_dtype == LMOE_BF16 &&
      out_dtype == LMOE_BF16)
    combine_slots_kernel<8, LMOE_BF16, LMOE_BF16><<<blocks, 256, 0, st>>>(
        shard_out, shard_dtype, slot_pos, w, w_dtype, (int)T, (int)k, lat, mode, routed_out, out_dtype);
  else if (vec8_ok(shard_out, routed_out, lat, shard_dtype, out_dtype))
    combine_slots_kernel<8><<<blocks, 256, 0, st>>>(shard_out, shard_dtype, slot_pos, w, w_dtype,
                                                   (int)T, (int)k, lat, mode, routed_out, out_dtype);
  else
    combine_slots_kernel<1><<<blocks, 256, 0, st>>>(shard_out, shard_dtype, slot_pos, w, w_dtype,
                                                   (int)T, (int)k, lat, mode, routed_out, out_dtype);
  LMOE_CHECK_LAUNCH("combine_slots");
  return LMOE_OK;
}

extern "C" int lmoe_combine_scatter_add(const void* shard_out, int shard_dtype,
                                        const int32_t* padded_token_idx, const void* padded_w,
                                        int w_dtype, int64_t m, int64_t lat, int64_t T,
                                        void* routed_out, int out_dtype, void* workspace,
                                        int64_t workspace_size, void* stream) {
  using namespace lmoe;
  LMOE_CHECK_ARG(m >= 0 && lat > 0 && T >= 0, "combine_scatter_add: bad sizes");
  LMOE_CHECK_ARG(valid_dtype(shard_dtype) && valid_dtype(w_dtype) && valid_dtype(out_dtype),
                 "combine_scatter_add: bad dtype");
  LMOE_CHECK_SUPPORTED(T + 1 <= 16384, "combine_scatter_add: T=%lld exceeds the LDS histogram",
                       (long long)T);
  LMOE_CHECK_SUPPORTED(m < (1ll << 31), "combine_scatter_add: m too large");
  LMOE_CHECK_SUPPORTED(extent_ok({m, lat}) && extent_ok({T, lat}), "combine_scatter_add: sizes beyond device memory");
  if (T == 0 || m == 0) return LMOE_OK;
  LMOE_CHECK_ARG(shard_out && padded_token_idx && padded_w && routed_out, "combine_scatter_add: null pointer");
  const int64_t need = combine_ws_bytes(m, T);
  if (!workspace || workspace_size < need)
    return fail(LMOE_ERR_WORKSPACE, "combine_scatter_add: workspace %lld < %lld",
                (long long)workspace_size, (long long)need);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t chunks = csort::num_chunks<kCombineChunk>(m);
  int32_t* ws = static_cast<int32_t*>(workspace);
  int32_t* hist = ws;
  int32_t* base = hist + chunks * T;
  int32_t* offsets = base + chunks * T;
  int32_t* order = offsets + (T + 1);
  int32_t* num_kept = order + m;
  const int Ti = static_cast<int>(T);
  TokenKey key{padded_token_idx, Ti};
  csort::hist_kernel<kCombineChunk><<<dim3(static_cast<unsigned>(chunks)), 256, (T + 1) * sizeof(int32_t), st>>>(
      key, m, Ti, chunks, hist);
  LMOE_CHECK_LAUNCH("combine_hist");
  if (csort::launch_scan(hist, chunks, Ti, (1ll << 40), base, nullptr, offsets, num_kept, st) != hipSuccess)
    return fail(LMOE_ERR_HIP, "combine_scan: LDS attribute");
  LMOE_CHECK_LAUNCH("combine_scan");
  csort::place_kernel<kCombineChunk><<<dim3(static_cast<unsigned>(chunks)), 64, T * sizeof(int32_t), st>>>(
      key, m, Ti, csort::key_bits_for(Ti), chunks, base, OrderSink{order});
  LMOE_CHECK_LAUNCH("combine_place");
  const unsigned blocks = static_cast<unsigned>(ceil_div(T, kTokensPerBlock));
  if (vec8_ok(shard_out, routed_out, lat, shard_dtype, out_dtype))
    combine_csr_kernel<8><<<blocks, 256, 0, st>>>(shard_out, shard_dtype, order, offsets, padded_w,
                                                 w_dtype, Ti, lat, routed_out, out_dtype);
  else
    combine_csr_kernel<1><<<blocks, 256, 0, st>>>(shard_out, shard_dtype, order, offsets, padded_w,
                                                 w_dtype, Ti, lat, routed_out, out_dtype);
  LMOE_CHECK_LAUNCH("combine_csr");
  return LMOE_OK;
}

extern "C" int lmoe_combine_slots_rms_norm(const void* shard_out, int shard_dtype, const int32_t* slot_pos,
                                           const void* w, int w_dtype, int64_t T, int64_t k, int64_t lat, int mode,
                                           const void* norm_scale, float eps, void* routed_out, void* normed_out,
                                           int dtype, void* stream) {
  using namespace lmoe;
  LMOE_CHECK_ARG(T >= 0 && k > 0 && lat > 0, "combine_rms_norm: bad sizes");
  LMOE_CHECK_SUPPORTED(k <= 64, "combine_rms_norm: k=%lld > 64", (long long)k);
  LMOE_CHECK_ARG(valid_dtype(shard_dtype) && valid_dtype(w_dtype) && valid_dtype(dtype),
                 "combine_rms_norm: bad dtype");
  LMOE_CHECK_ARG(mode == LMOE_COMBINE_SCATTER_ADD || mode == LMOE_COMBINE_SLOT_SUM,
                 "combine_rms_norm: bad mode %d", mode);
  LMOE_CHECK_SUPPORTED(T < (1ll << 31), "combine_rms_norm: T too large");
  LMOE_CHECK_SUPPORTED(lat % 8 == 0 && lat <= 2048, "combine_rms_norm: lat=%lld (needs a multiple of 8, <= 2048)",
                       (long long)lat);
  if (T == 0) return LMOE_OK;
  LMOE_CHECK_ARG(shard_out && slot_pos && w && norm_scale && normed_out, "combine_rms_norm: null pointer");
  const size_t oa = dtype == LMOE_BF16 ? 16 : 32;
  LMOE_CHECK_SUPPORTED(aligned(shard_out, shard_dtype == LMOE_BF16 ? 16 : 32) && aligned(normed_out, oa) &&
                           aligned(norm_scale, oa) && (!routed_out || aligned(routed_out, oa)),
                       "combine_rms_norm: buffers must be 16-byte (bf16) / 32-byte (f32) aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned blocks = static_cast<unsigned>(ceil_div(T, kTokensPerBlock));
  const bool bf = shard_dtype == LMOE_BF16 && dtype == LMOE_BF16;
  // lmoe_rms_norm's split: 8 elements per lane and pass for bf16, 4 for f32
  const int vec = dtype == LMOE_BF16 ? 8 : 4;
  const int passes = static_cast<int>(ceil_div(lat, 64 * vec));
#define LMOE_CN_CASE(V, R)                                                                                    \
  if (vec == V && passes == R) {                                                                             \
    if (V == 8 && bf)                                                                                        \
      combine_norm_kernel<V, R, LMOE_BF16, LMOE_BF16><<<blocks, 256, 0, st>>>(                               \
          shard_out, shard_dtype, slot_pos, w, w_dtype, (int)T, (int)k, lat, mode, norm_scale, eps, routed_out, \
          normed_out, dtype);                                                                                \
    else                                                                                                     \
      combine_norm_kernel<V, R><<<blocks, 256, 0, st>>>(shard_out, shard_dtype, slot_pos, w, w_dtype, (int)T,  \
                                                        (int)k, lat, mode, norm_scale, eps, routed_out,        \
                                                        normed_out, dtype);                                  \
  }
  LMOE_CN_CASE(8, 1)
  LMOE_CN_CASE(8, 2)
  LMOE_CN_CASE(8, 3)
  LMOE_CN_CASE(8, 4)
  LMOE_CN_CASE(4, 1)
  LMOE_CN_CASE(4, 2)
  LMOE_CN_CASE(4, 3)
  LMOE_CN_CASE(4, 4)
  LMOE_CN_CASE(4, 5)
  LMOE_CN_CASE(4, 6)
  LMOE_CN_CASE(4, 7)
  LMOE_CN_CASE(4, 8)
#undef LMOE_CN_CASE
  LMOE_CHECK_LAUNCH("combine_rms_norm");
  return LMOE_OK;
}
