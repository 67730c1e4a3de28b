// Local-shard dispatch in one launch, for decode-sized batches (T*k slots up
// to kSmallSlots): the same outputs as lmoe_dispatch_local (ref.py:754-877,
// stable expert-major order, tail truncation at m_padded, padding bucket),
// with the activations read from a row-strided bf16 or f32 array and written
// as bf16 (the f32 -> bf16 rounding of the projection output fused in).
//
// A decode step's dispatch is a few hundred slots: four launches of the
// counting sort (histogram, scan, place, gather) plus the cast cost about
// 20 us of launch latency for under a microsecond of work.  Here every block
// rebuilds the whole (small) sort in LDS -- histogram by LDS atomics, one-wave
// scan of the expert offsets, stable ranks by one wave walking the slots 64 at
// a time (lanes with the same key found with one ballot per key bit) -- then
// block 0 writes the per-slot and per-row metadata and all blocks gather
// their share of the rows.
#include "lmoe_common.h"
#include "gemm_tile.h"

namespace lmoe {
namespace {

constexpr int kSmallSlots = 8192;    // T*k
constexpr int kSmallRows = 8192;     // m_padded
constexpr int kSmallKeys = 1024;     // L + 1
constexpr int kSmallThreads = 256;

struct SmallDispatch {
  const int32_t* idx;     // (T*k,) global expert ids
  const uint8_t* w;       // (T*k,) combine weights, wsize bytes each
  int wsize;
  const void* x;          // (T, >= lat) row stride x_ld, bf16 or f32
  int x_f32;
  int64_t x_ld;
  int64_t n, k, lat;
  int start, L;
  int64_t m_padded;
  uint16_t* sorted;       // (m_padded, lat) bf16
  int32_t* group_sizes;   // (L + 1,)
  uint8_t* valid;         // (m_padded,)
  int32_t* counts;        // (L,)
  int32_t* tok;           // (m_padded,)
  uint8_t* w_out;         // (m_padded,) wsize bytes each
  int32_t* slot_pos;      // (T*k,) or null
  int skip_padding_rows;
};

__global__ __launch_bounds__(kSmallThreads) void dispatch_small_kernel(SmallDispatch p) {
  __shared__ uint16_t s_key[kSmallSlots];
  __shared__ int32_t s_row_slot[kSmallRows];
  __shared__ int32_t s_cnt[kSmallKeys];
  __shared__ int32_t s_off[kSmallKeys];
  __shared__ int32_t s_run[kSmallKeys];
  __shared__ int32_t s_total;

  const int t = threadIdx.x, lane = t & 63, wv = t >> 6;
  const int L = p.L;
  const int64_t n = p.n, mp = p.m_padded;

  for (int e = t; e <= L; e += kSmallThreads) {
    s_cnt[e] = 0;
    s_run[e] = 0;
  }
  for (int64_t r = t; r < mp; r += kSmallThreads) s_row_slot[r] = -1;
  __syncthreads();
  // keys and expert counts
  for (int64_t s = t; s < n; s += kSmallThreads) {
    const int g = p.idx[s];
    const int key = (g >= p.start && g < p.start + L) ? g - p.start : L;
    s_key[s] = static_cast<uint16_t>(key);
    if (key < L) atomicAdd(&s_cnt[key], 1);
  }
  __syncthreads();
  // exclusive offsets of the L experts (wave 0: each lane a run of keys)
  if (wv == 0) {
    const int per = (L + 63) / 64;
    const int e0 = lane * per, e1 = e0 + per < L ? e0 + per : L;
    int sum = 0;
    for (int e = e0; e < e1; ++e) sum += s_cnt[e];
    int incl = sum;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(incl, d, 64);
      if (lane >= d) incl += o;
    }
    int run = incl - sum;
    for (int e = e0; e < e1; ++e) {
      s_off[e] = run;
      run += s_cnt[e];
    }
    if (lane == 63) s_total = incl;
  }
  __syncthreads();
  // stable ranks: wave 0 walks the slots in order, 64 at a time
  int kb = 1;
  while ((1 << kb) <= L) ++kb;  // bits of a key in [0, L]
  if (wv == 0) {
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int64_t c = 0; c < n; c += 64) {
      const int64_t s = c + lane;
      const int key = s < n ? s_key[s] : L;
      uint64_t m = __ballot(s < n && key < L);
      for (int b = 0; b < kb; ++b) {
        const uint64_t bal = __ballot((key >> b) & 1);
        m &= ((key >> b) & 1) ? bal : ~bal;
      }
      if (s < n && key < L) {
        const int base = s_run[key];
        const int pos = s_off[key] + base + __popcll(m & below);
        const bool kept = pos < mp;
        if (kept) s_row_slot[pos] = static_cast<int32_t>(s);
        if (blockIdx.x == 0 && p.slot_pos) p.slot_pos[s] = kept ? pos : -1;
        if ((m & below) == 0) s_run[key] = base + __popcll(m);  // the group's lowest lane
      } else if (s < n && blockIdx.x == 0 && p.slot_pos) {
        p.slot_pos[s] = -1;
      }
    }
  }
  __syncthreads();
  const int64_t nk = s_total < mp ? s_total : mp;

  // per-row and per-expert metadata (block 0)
  if (blockIdx.x == 0) {
    for (int e = t; e < L; e += kSmallThreads) {
      const int64_t room = mp - s_off[e];
      const int32_t c = static_cast<int32_t>(room <= 0 ? 0 : (room < s_cnt[e] ? room : s_cnt[e]));
      p.group_sizes[e] = c;
      p.counts[e] = c;
    }
    if (t == 0) p.group_sizes[L] = static_cast<int32_t>(mp - nk);
    for (int64_t r = t; r < mp; r += kSmallThreads) {
      const int32_t s = s_row_slot[r];
      p.valid[r] = s >= 0 ? 1 : 0;
      p.tok[r] = s >= 0 ? static_cast<int32_t>(s / p.k) : -1;
      if (p.wsize == 4)
        reinterpret_cast<uint32_t*>(p.w_out)[r] = s >= 0 ? reinterpret_cast<const uint32_t*>(p.w)[s] : 0u;
      else
        reinterpret_cast<uint16_t*>(p.w_out)[r] = s >= 0 ? reinterpret_cast<const uint16_t*>(p.w)[s] : 0;
    }
  }

  // rows: 8 values (16 output bytes) per thread step, grid-strided
  const int64_t vecs = p.lat / 8;
  const int64_t rows = p.skip_padding_rows ? nk : mp;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kSmallThreads + t; i < rows * vecs;
       i += static_cast<int64_t>(gridDim.x) * kSmallThreads) {
    const int64_t r = i / vecs, v = i % vecs;
    const int32_t s = s_row_slot[r];
    uint4 o{0u, 0u, 0u, 0u};
    if (s >= 0) {
      const int64_t src = (s / p.k) * p.x_ld + v * 8;
      if (p.x_f32) {
        const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p.x) + src);
        const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p.x) + src + 4);
        o = uint4{gemm::pack_bf16x2(a.x, a.y), gemm::pack_bf16x2(a.z, a.w), gemm::pack_bf16x2(b.x, b.y),
                  gemm::pack_bf16x2(b.z, b.w)};
      } else {
        o = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.x) + src);
      }
    }
    reinterpret_cast<uint4*>(p.sorted + r * p.lat)[v] = o;
  }
}

}  // namespace
}  // namespace lmoe

extern "C" int lmoe_dispatch_local_small(const int32_t* topk_idx, const void* topk_w, int w_dtype, const void* x,
                                         int x_dtype, int64_t x_ld, int64_t T, int64_t k, int64_t lat,
                                         int64_t local_start, int64_t L, int64_t m_padded, uint16_t* sorted_tokens,
                                         int32_t* group_sizes, uint8_t* valid, int32_t* per_expert_counts,
                                         int32_t* padded_token_idx, void* padded_w, int32_t* slot_pos, int flags,
                                         void* stream) {
  using namespace lmoe;
  const char* name = "dispatch_local_small";
  LMOE_CHECK_ARG(T >= 0 && k > 0 && lat > 0 && L > 0 && m_padded >= 0 && local_start >= 0 && x_ld >= lat,
                 "%s: bad sizes T=%lld k=%lld lat=%lld L=%lld m_padded=%lld x_ld=%lld", name, (long long)T,
                 (long long)k, (long long)lat, (long long)L, (long long)m_padded, (long long)x_ld);
  LMOE_CHECK_ARG(valid_dtype(w_dtype) && valid_dtype(x_dtype), "%s: bad dtype", name);
  LMOE_CHECK_ARG((flags & ~LMOE_DISPATCH_FLAG_SKIP_PADDING_ROWS) == 0, "%s: unknown flags 0x%x", name, flags);
  LMOE_CHECK_SUPPORTED(T <= kSmallSlots && k <= kSmallSlots && T * k <= kSmallSlots && m_padded <= kSmallRows &&
                           L + 1 <= kSmallKeys,
                       "%s: at most %d slots, %d rows and %d experts (T=%lld k=%lld m_padded=%lld L=%lld)", name,
                       kSmallSlots, kSmallRows, kSmallKeys - 1, (long long)T, (long long)k, (long long)m_padded,
                       (long long)L);
  LMOE_CHECK_SUPPORTED(local_start < (1ll << 31) - L && extent_ok({T, x_ld}) && extent_ok({m_padded, lat}),
                       "%s: sizes beyond device memory (local_start=%lld lat=%lld x_ld=%lld)", name,
                       (long long)local_start, (long long)lat, (long long)x_ld);
  LMOE_CHECK_SUPPORTED(lat % 8 == 0 && x_ld % (x_dtype == LMOE_F32 ? 4 : 8) == 0,
                       "%s: lat %% 8 == 0 and 16-byte aligned rows (lat=%lld x_ld=%lld)", name, (long long)lat,
                       (long long)x_ld);
  LMOE_CHECK_ARG(group_sizes && valid && per_expert_counts && padded_token_idx && padded_w &&
                     (T == 0 || (topk_idx && topk_w && x)) && (sorted_tokens || m_padded == 0),
                 "%s: null pointer", name);
  LMOE_CHECK_SUPPORTED(aligned(sorted_tokens, 16) && (T == 0 || aligned(x, 16)), "%s: 16-byte alignment", name);
  SmallDispatch p{topk_idx, static_cast<const uint8_t*>(topk_w), dtype_size(w_dtype), x, x_dtype == LMOE_F32, x_ld,
                  T * k, k, lat, static_cast<int>(local_start), static_cast<int>(L), m_padded, sorted_tokens,
                  group_sizes, valid, per_expert_counts, padded_token_idx, static_cast<uint8_t*>(padded_w),
                  slot_pos, (flags & LMOE_DISPATCH_FLAG_SKIP_PADDING_ROWS) != 0};
  // about 32 KB of rows per block, at most 64 blocks (each rebuilds the sort)
  const int64_t bytes = m_padded * lat * 2;
  const int64_t b = ceil_div(bytes > 0 ? bytes : 1, 32 << 10);
  const unsigned grid = static_cast<unsigned>(b < 64 ? b : 64);
  dispatch_small_kernel<<<grid, kSmallThreads, 0, static_cast<hipStream_t>(stream)>>>(p);
  LMOE_CHECK_LAUNCH(name);
  return LMOE_OK;
}
