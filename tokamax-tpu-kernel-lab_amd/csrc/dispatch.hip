// Local-shard dispatch (reference filter_and_pad_to_shard_jittable,
// ref.py:754-877, bit-identical to the eager filter_and_pad_to_shard,
// ref.py:658-751).
//
// Slot s = t*k + j carries key = local expert id if the global id is in
// [local_start, local_start + L), else the sentinel L.  A stable counting
// sort (csort.h) gives each in-shard slot its row in expert-major order; rows
// >= m_padded are dropped (tail truncation), and rows past the kept count are
// the padding bucket.  Then one gather pass copies x rows into sorted_tokens
// and fills the padding rows (zero row, token -1, weight 0, valid 0).
#include <mutex>

#include "csort.h"
#include "gemm_tile.h"

namespace lmoe {
namespace {

struct DispatchKey {
  const int32_t* idx;
  int start;
  int L;
  __device__ __forceinline__ int operator()(int64_t s) const {
    const int g = idx[s];
    return (g >= start && g < start + L) ? g - start : L;
  }
};

struct DispatchSink {
  int k;
  const uint8_t* w;
  int wsize;
  int32_t* tok_out;
  uint8_t* w_out;
  int32_t* slot_pos;
  int64_t limit;  // m_padded
  // metadata written by the place kernel (LMOE_DISPATCH_FLAG_NO_ROWS, no
  // gather launch after it): valid, the padding rows' token (-1) and weight
  // (0), per_expert_counts and the padding bucket's size group_sizes[L]
  uint8_t* valid = nullptr;
  int32_t* per_expert = nullptr;
  int32_t* pad_group = nullptr;
  __device__ __forceinline__ void bin_kept(int b, int32_t kept) const {
    if (per_expert) per_expert[b] = kept;
  }
  __device__ __forceinline__ void positions(int64_t nk, int block, int blocks) const {
    if (!valid) return;
    if (block == 0 && threadIdx.x == 0) *pad_group = static_cast<int32_t>(limit - nk);
    const int64_t per = (limit + blocks - 1) / blocks;
    const int64_t p0 = static_cast<int64_t>(block) * per, p1 = p0 + per < limit ? p0 + per : limit;
    for (int64_t p = p0 + threadIdx.x; p < p1; p += blockDim.x) {
      valid[p] = p < nk ? 1 : 0;
      if (p >= nk) {
        tok_out[p] = -1;
        if (wsize == 4)
          reinterpret_cast<uint32_t*>(w_out)[p] = 0u;
        else
          reinterpret_cast<uint16_t*>(w_out)[p] = 0;
      }
    }
  }
  // the slot's combine weight bits, read before the ranks are known
  __device__ __forceinline__ uint32_t load(int64_t s) const {
    return wsize == 4 ? reinterpret_cast<const uint32_t*>(w)[s] : reinterpret_cast<const uint16_t*>(w)[s];
  }
  __device__ __forceinline__ void operator()(int64_t s, int key, int pos, bool real, uint32_t wbits) const {
    const bool kept = real && pos < limit;
    if (kept) {
      tok_out[pos] = static_cast<int32_t>(s / k);
      if (wsize == 4)
        reinterpret_cast<uint32_t*>(w_out)[pos] = wbits;
      else
        reinterpret_cast<uint16_t*>(w_out)[pos] = static_cast<uint16_t>(wbits);
    }
    if (slot_pos) slot_pos[s] = kept ? pos : -1;
  }
};

constexpr int kGatherRows = 16;

template <typename VT>
__global__ __launch_bounds__(256) void gather_kernel(
    const VT* __restrict__ x, int64_t row_vecs, const int32_t* __restrict__ num_kept_p,
    int64_t m_padded, VT* __restrict__ out, uint8_t* __restrict__ valid, int32_t* __restrict__ tok,
    uint8_t* __restrict__ w_out, int wsize, int32_t* __restrict__ group_sizes,
    int32_t* __restrict__ per_expert, int L) {
  const int nk = *num_kept_p;
  if (blockIdx.x == 0) {
    for (int i = threadIdx.x; i < L; i += blockDim.x) per_expert[i] = group_sizes[i];
    if (threadIdx.x == 0) group_sizes[L] = static_cast<int32_t>(m_padded - nk);
  }
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kGatherRows;
  const int64_t r1 = r0 + kGatherRows < m_padded ? r0 + kGatherRows : m_padded;
  for (int64_t p = r0 + threadIdx.x; p < r1; p += blockDim.x) {
    valid[p] = p < nk ? 1 : 0;
    if (p >= nk) {
      tok[p] = -1;
      if (wsize == 4)
        reinterpret_cast<uint32_t*>(w_out)[p] = 0;
      else
        reinterpret_cast<uint16_t*>(w_out)[p] = 0;
    }
  }
  const int64_t total = (r1 - r0) * row_vecs;
  for (int64_t i = threadIdx.x; i < total; i += blockDim.x) {
    const int64_t p = r0 + i / row_vecs;
    const int64_t v = i % row_vecs;
    VT val{};
    if (p < nk) {
      const int32_t t = tok[p];
      val = x[static_cast<int64_t>(t) * row_vecs + v];
    }
    out[p * row_vecs + v] = val;
  }
}

// The gather for a row-strided bf16 or f32 x written as bf16 (f32 rounded to
// nearest even), optionally leaving the padding rows of out unwritten; the
// metadata of every row as gather_kernel writes it.
template <bool F32>
__global__ __launch_bounds__(256) void gather_rows_kernel(
    const void* __restrict__ x, int64_t x_ld, int64_t lat, const int32_t* __restrict__ num_kept_p,
    int64_t m_padded, uint16_t* __restrict__ out, int skip_padding, uint8_t* __restrict__ valid,
    int32_t* __restrict__ tok, uint8_t* __restrict__ w_out, int wsize, int32_t* __restrict__ group_sizes,
    int32_t* __restrict__ per_expert, int L) {
  const int nk = *num_kept_p;
  if (blockIdx.x == 0) {
    for (int i = threadIdx.x; i < L; i += blockDim.x) per_expert[i] = group_sizes[i];
    if (threadIdx.x == 0) group_sizes[L] = static_cast<int32_t>(m_padded - nk);
  }
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kGatherRows;
  const int64_t r1 = r0 + kGatherRows < m_padded ? r0 + kGatherRows : m_padded;
  for (int64_t p = r0 + threadIdx.x; p < r1; p += blockDim.x) {
    valid[p] = p < nk ? 1 : 0;
    if (p >= nk) {
      tok[p] = -1;
      if (wsize == 4)
        reinterpret_cast<uint32_t*>(w_out)[p] = 0;
      else
        reinterpret_cast<uint16_t*>(w_out)[p] = 0;
    }
  }
  const int64_t vecs = lat / 8;
  const int64_t re = skip_padding ? (r1 < nk ? r1 : (r0 > nk ? r0 : nk)) : r1;
  for (int64_t i = threadIdx.x; i < (re - r0) * vecs; i += blockDim.x) {
    const int64_t p = r0 + i / vecs, v = i % vecs;
    uint4 o{0u, 0u, 0u, 0u};
    if (p < nk) {
      const int64_t src = static_cast<int64_t>(tok[p]) * x_ld + v * 8;
      if constexpr (F32) {
        const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(x) + src);
        const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(x) + src + 4);
        o = uint4{gemm::pack_bf16x2(a.x, a.y), gemm::pack_bf16x2(a.z, a.w), gemm::pack_bf16x2(b.x, b.y),
                  gemm::pack_bf16x2(b.z, b.w)};
      } else {
        o = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + src);
      }
    }
    reinterpret_cast<uint4*>(out + p * lat)[v] = o;
  }
}

// The gather's metadata without the rows (LMOE_DISPATCH_FLAG_NO_ROWS): a
// small grid striding over the rows, since there is no row data to spread.
__global__ __launch_bounds__(256) void dispatch_meta_kernel(const int32_t* __restrict__ num_kept_p, int64_t m_padded,
                                                            uint8_t* __restrict__ valid, int32_t* __restrict__ tok,
                                                            uint8_t* __restrict__ w_out, int wsize,
                                                            int32_t* __restrict__ group_sizes,
                                                            int32_t* __restrict__ per_expert, int L) {
  const int nk = *num_kept_p;
  if (blockIdx.x == 0) {
    for (int i = threadIdx.x; i < L; i += blockDim.x) per_expert[i] = group_sizes[i];
    if (threadIdx.x == 0) group_sizes[L] = static_cast<int32_t>(m_padded - nk);
  }
  for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < m_padded;
       p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    valid[p] = p < nk ? 1 : 0;
    if (p >= nk) {
      tok[p] = -1;
      if (wsize == 4)
        reinterpret_cast<uint32_t*>(w_out)[p] = 0;
      else
        reinterpret_cast<uint16_t*>(w_out)[p] = 0;
    }
  }
}

// Few bins (local experts): small chunks, many place waves (and a scanned
// (expert, chunk) array that stays within a few thousand entries).
constexpr int kDispatchChunk = 512;

struct Workspace {
  int32_t* hist;
  int32_t* base;
  int32_t* num_kept;
};

int64_t workspace_bytes(int64_t n, int64_t L) {
  const int64_t chunks = csort::num_chunks<kDispatchChunk>(n > 0 ? n : 1);
  return (2 * chunks * L + 64) * static_cast<int64_t>(sizeof(int32_t));
}

// Allocation-free dispatch: the counting sort's workspace (per-chunk
// histograms, bin bases, kept count; every byte is written before it is
// read, so nothing needs clearing) in a file-scope device array.  Each GPU
// holds its own copy until the process ends.  In host code `scratch` names a
// host-side stand-in, so its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and only that address is
// passed to kernels.
constexpr int64_t kNoAllocScratchBytes = int64_t{4} << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_on_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(LMOE_ERR_HIP, "dispatch_local_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(LMOE_ERR_UNSUPPORTED, "dispatch_local_noalloc: device %d >= %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(LMOE_ERR_HIP, "dispatch_local_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return LMOE_OK;
}

// The argument checks of lmoe_dispatch_local, shared with the
// allocation-free variant so that it refuses the same calls before it touches
// a device: sizes and dtypes first, then (after the workspace check) the
// pointers.
int check_dispatch_sizes(const char* name, int w_dtype, int x_dtype, int64_t T, int64_t k, int64_t lat,
                         int64_t local_start, int64_t L, int64_t m_padded) {
  LMOE_CHECK_ARG(T >= 0 && k > 0 && lat > 0 && L > 0 && m_padded >= 0 && local_start >= 0,
                 "%s: bad sizes T=%lld k=%lld lat=%lld L=%lld m_padded=%lld", name, (long long)T, (long long)k,
                 (long long)lat, (long long)L, (long long)m_padded);
  LMOE_CHECK_ARG(valid_dtype(w_dtype) && valid_dtype(x_dtype), "%s: bad dtype", name);
  LMOE_CHECK_SUPPORTED(T < (1ll << 31) && k < (1ll << 31) && T * k < (1ll << 31) && m_padded < (1ll << 31) &&
                           L < (1 << 20) && local_start < (1ll << 31) - L,
                       "%s: sizes exceed int32 indexing", name);
  LMOE_CHECK_SUPPORTED(extent_ok({T, lat}) && extent_ok({m_padded, lat}), "%s: sizes beyond device memory", name);
  LMOE_CHECK_SUPPORTED(L + 1 <= 12288, "%s: L=%lld exceeds the LDS histogram", name, (long long)L);
  return LMOE_OK;
}

int check_dispatch_pointers(const char* name, const int32_t* topk_idx, const void* topk_w, const void* x, int64_t T,
                            int64_t m_padded, const void* sorted_tokens, const int32_t* group_sizes,
                            const uint8_t* valid, const int32_t* per_expert_counts, const int32_t* padded_token_idx,
                            const void* padded_w) {
  LMOE_CHECK_ARG(group_sizes && valid && per_expert_counts && padded_token_idx && padded_w &&
                     (sorted_tokens || m_padded == 0),
                 "%s: null output", name);
  LMOE_CHECK_ARG(T == 0 || (topk_idx && topk_w), "%s: null top-k input", name);
  LMOE_CHECK_ARG(T == 0 || m_padded == 0 || x, "%s: null x", name);
  return LMOE_OK;
}

}  // namespace
}  // namespace lmoe

extern "C" int64_t lmoe_dispatch_workspace_size(int64_t T, int64_t k, int64_t L) {
  if (T < 0 || k <= 0 || L <= 0 || T >= (1ll << 31) || k >= (1ll << 31) || T * k >= (1ll << 31) || L >= (1 << 20))
    return -1;
  return lmoe::workspace_bytes(T * k, L);
}

extern "C" int lmoe_dispatch_local(const int32_t* topk_idx, const void* topk_w, int w_dtype,
                                   const void* x, int x_dtype, int64_t T, int64_t k, int64_t lat,
                                   int64_t local_start, int64_t L, int64_t m_padded,
                                   void* sorted_tokens, int32_t* group_sizes, uint8_t* valid,
                                   int32_t* per_expert_counts, int32_t* padded_token_idx,
                                   void* padded_w, int32_t* slot_pos, void* workspace,
                                   int64_t workspace_size, void* stream) {
  using namespace lmoe;
  int rc = check_dispatch_sizes("dispatch_local", w_dtype, x_dtype, T, k, lat, local_start, L, m_padded);
  if (rc != LMOE_OK) return rc;
  const int64_t need = workspace_bytes(T * k, L);
  if (!workspace || workspace_size < need)
    return fail(LMOE_ERR_WORKSPACE, "dispatch_local: workspace %lld bytes < %lld", (long long)workspace_size,
                (long long)need);
  rc = check_dispatch_pointers("dispatch_local", topk_idx, topk_w, x, T, m_padded, sorted_tokens, group_sizes, valid,
                               per_expert_counts, padded_token_idx, padded_w);
  if (rc != LMOE_OK) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t n = T * k;
  const int64_t chunks = csort::num_chunks<kDispatchChunk>(n > 0 ? n : 1);
  int32_t* ws = static_cast<int32_t*>(workspace);
  Workspace w{ws, ws + chunks * L, ws + 2 * chunks * L};
  const int Li = static_cast<int>(L);
  DispatchKey key{topk_idx, static_cast<int>(local_start), Li};
  // With n == 0 the single chunk still writes an all-zero histogram.
  csort::hist_kernel<kDispatchChunk><<<dim3(static_cast<unsigned>(chunks)), 256, (L + 1) * sizeof(int32_t), st>>>(
      key, n, Li, chunks, w.hist);
  LMOE_CHECK_LAUNCH("dispatch_hist");
  {
    DispatchSink sink{static_cast<int>(k), static_cast<const uint8_t*>(topk_w), dtype_size(w_dtype),
                      padded_token_idx, static_cast<uint8_t*>(padded_w), slot_pos, m_padded};
    if (csort::scan_and_place<kDispatchChunk>(key, n, Li, chunks, m_padded, w.hist, w.base, group_sizes,
                                              w.num_kept, sink, st) != hipSuccess)
      return fail(LMOE_ERR_HIP, "dispatch_scan: LDS attribute");
    LMOE_CHECK_LAUNCH("dispatch_scan_place");
  }
  // The gather also finalises group_sizes[L] and per_expert_counts (block 0),
  // so it runs even when m_padded == 0.
  const int64_t row_bytes = lat * dtype_size(x_dtype);
  const unsigned blocks = static_cast<unsigned>(m_padded > 0 ? ceil_div(m_padded, kGatherRows) : 1);
  if (row_bytes % 16 == 0 && aligned(x, 16) && aligned(sorted_tokens, 16)) {
    gather_kernel<uint4><<<blocks, 256, 0, st>>>(
        static_cast<const uint4*>(x), row_bytes / 16, w.num_kept, m_padded,
        static_cast<uint4*>(sorted_tokens), valid, padded_token_idx, static_cast<uint8_t*>(padded_w),
        dtype_size(w_dtype), group_sizes, per_expert_counts, Li);
  } else {
    gather_kernel<uint16_t><<<blocks, 256, 0, st>>>(
        static_cast<const uint16_t*>(x), row_bytes / 2, w.num_kept, m_padded,
        static_cast<uint16_t*>(sorted_tokens), valid, padded_token_idx,
        static_cast<uint8_t*>(padded_w), dtype_size(w_dtype), group_sizes, per_expert_counts, Li);
  }
  LMOE_CHECK_LAUNCH("dispatch_gather");
  return LMOE_OK;
}

extern "C" int lmoe_dispatch_local_noalloc(const int32_t* topk_idx, const void* topk_w, int w_dtype,
                                           const void* x, int x_dtype, int64_t T, int64_t k, int64_t lat,
                                           int64_t local_start, int64_t L, int64_t m_padded,
                                           void* sorted_tokens, int32_t* group_sizes, uint8_t* valid,
                                           int32_t* per_expert_counts, int32_t* padded_token_idx,
                                           void* padded_w, int32_t* slot_pos, void* stream) {
  using namespace lmoe;
  const char* name = "dispatch_local_noalloc";
  int rc = check_dispatch_sizes(name, w_dtype, x_dtype, T, k, lat, local_start, L, m_padded);
  if (rc != LMOE_OK) return rc;
  const int64_t need = workspace_bytes(T * k, L);
  if (need > kNoAllocScratchBytes)
    return fail(LMOE_ERR_WORKSPACE,
                "dispatch_local_noalloc: T*k=%lld, L=%lld need %lld bytes of scratch, more than the %lld-byte "
                "static array; call lmoe_dispatch_local with a workspace",
                (long long)(T * k), (long long)L, (long long)need, (long long)kNoAllocScratchBytes);
  rc = check_dispatch_pointers(name, topk_idx, topk_w, x, T, m_padded, sorted_tokens, group_sizes, valid,
                               per_expert_counts, padded_token_idx, padded_w);
  if (rc != LMOE_OK) return rc;
  void* ws = nullptr;
  rc = scratch_on_current_device(&ws);
  if (rc != LMOE_OK) return rc;
  return lmoe_dispatch_local(topk_idx, topk_w, w_dtype, x, x_dtype, T, k, lat, local_start, L, m_padded,
                             sorted_tokens, group_sizes, valid, per_expert_counts, padded_token_idx, padded_w,
                             slot_pos, ws, kNoAllocScratchBytes, stream);
}

extern "C" int lmoe_dispatch_local_rows(const int32_t* topk_idx, const void* topk_w, int w_dtype, const void* x,
                                        int x_dtype, int64_t x_ld, int64_t T, int64_t k, int64_t lat,
                                        int64_t local_start, int64_t L, int64_t m_padded, uint16_t* sorted_tokens,
                                        int32_t* group_sizes, uint8_t* valid, int32_t* per_expert_counts,
                                        int32_t* padded_token_idx, void* padded_w, int32_t* slot_pos, int flags,
                                        void* workspace, int64_t workspace_size, void* stream) {
  using namespace lmoe;
  const char* name = "dispatch_local_rows";
  LMOE_CHECK_ARG(T >= 0 && k > 0 && lat > 0 && L > 0 && m_padded >= 0 && local_start >= 0 && x_ld >= lat,
                 "%s: bad sizes", name);
  LMOE_CHECK_ARG(valid_dtype(w_dtype) && valid_dtype(x_dtype), "%s: bad dtype", name);
  LMOE_CHECK_ARG((flags & ~(LMOE_DISPATCH_FLAG_SKIP_PADDING_ROWS | LMOE_DISPATCH_FLAG_NO_ROWS)) == 0,
                 "%s: unknown flags 0x%x", name, flags);
  const bool no_rows = (flags & LMOE_DISPATCH_FLAG_NO_ROWS) != 0;
  LMOE_CHECK_SUPPORTED(T < (1ll << 31) && k < (1ll << 31) && extent_ok({T, x_ld}) && extent_ok({m_padded, lat}),
                       "%s: sizes beyond device memory (T=%lld k=%lld x_ld=%lld)", name, (long long)T, (long long)k,
                       (long long)x_ld);
  // decode-sized batches: one launch
  if (!no_rows && T * k <= 8192 && m_padded <= 8192 && L + 1 <= 1024)
    return lmoe_dispatch_local_small(topk_idx, topk_w, w_dtype, x, x_dtype, x_ld, T, k, lat, local_start, L,
                                     m_padded, sorted_tokens, group_sizes, valid, per_expert_counts,
                                     padded_token_idx, padded_w, slot_pos, flags, stream);
  LMOE_CHECK_SUPPORTED(T * k < (1ll << 31) && m_padded < (1ll << 31) && L < (1 << 20) &&
                           local_start < (1ll << 31) - L,
                       "%s: sizes exceed int32 indexing", name);
  LMOE_CHECK_SUPPORTED(L + 1 <= 12288, "%s: L=%lld exceeds the LDS histogram", name, (long long)L);
  LMOE_CHECK_SUPPORTED(no_rows || (lat % 8 == 0 && x_ld % (x_dtype == LMOE_F32 ? 4 : 8) == 0 && aligned(x, 16) &&
                                    aligned(sorted_tokens, 16)),
                       "%s: lat %% 8 == 0 and 16-byte aligned rows", name);
  const int64_t need = workspace_bytes(T * k, L);
  if (!workspace || workspace_size < need)
    return fail(LMOE_ERR_WORKSPACE, "%s: workspace %lld bytes < %lld", name, (long long)workspace_size,
                (long long)need);
  LMOE_CHECK_ARG(group_sizes && valid && per_expert_counts && padded_token_idx && padded_w &&
                     (no_rows || sorted_tokens || m_padded == 0),
                 "%s: null output", name);
  LMOE_CHECK_ARG(T == 0 || (topk_idx && topk_w), "%s: null top-k input", name);
  LMOE_CHECK_ARG(no_rows || T == 0 || m_padded == 0 || x, "%s: null x", name);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t n = T * k;
  const int64_t chunks = csort::num_chunks<kDispatchChunk>(n > 0 ? n : 1);
  int32_t* ws = static_cast<int32_t*>(workspace);
  Workspace w{ws, ws + chunks * L, ws + 2 * chunks * L};
  const int Li = static_cast<int>(L);
  DispatchKey key{topk_idx, static_cast<int>(local_start), Li};
  csort::hist_kernel<kDispatchChunk><<<dim3(static_cast<unsigned>(chunks)), 256, (L + 1) * sizeof(int32_t), st>>>(
      key, n, Li, chunks, w.hist);
  LMOE_CHECK_LAUNCH("dispatch_hist");
  // without rows the place kernel also writes the metadata when it is the
  // scanned one (few bins): no launch after it
  const bool meta_in_place = no_rows && csort::scanned_place(Li);
  {
    DispatchSink sink{static_cast<int>(k), static_cast<const uint8_t*>(topk_w), dtype_size(w_dtype),
                      padded_token_idx, static_cast<uint8_t*>(padded_w), slot_pos, m_padded};
    if (meta_in_place) {
      sink.valid = valid;
      sink.per_expert = per_expert_counts;
      sink.pad_group = group_sizes + L;
    }
    if (csort::scan_and_place<kDispatchChunk>(key, n, Li, chunks, m_padded, w.hist, w.base, group_sizes,
                                              w.num_kept, sink, st) != hipSuccess)
      return fail(LMOE_ERR_HIP, "dispatch_scan: LDS attribute");
    LMOE_CHECK_LAUNCH("dispatch_scan_place");
  }
  if (meta_in_place) return LMOE_OK;
  if (no_rows) {
    const int64_t mb = ceil_div(m_padded > 0 ? m_padded : 1, 1024);
    dispatch_meta_kernel<<<static_cast<unsigned>(mb < 64 ? mb : 64), 256, 0, st>>>(
        w.num_kept, m_padded, valid, padded_token_idx, static_cast<uint8_t*>(padded_w), dtype_size(w_dtype),
        group_sizes, per_expert_counts, Li);
    LMOE_CHECK_LAUNCH("dispatch_meta");
    return LMOE_OK;
  }
  const unsigned blocks = static_cast<unsigned>(m_padded > 0 ? ceil_div(m_padded, kGatherRows) : 1);
  const int skip = (flags & LMOE_DISPATCH_FLAG_SKIP_PADDING_ROWS) != 0;
  if (x_dtype == LMOE_F32)
    gather_rows_kernel<true><<<blocks, 256, 0, st>>>(x, x_ld, lat, w.num_kept, m_padded, sorted_tokens, skip, valid,
                                                    padded_token_idx, static_cast<uint8_t*>(padded_w),
                                                    dtype_size(w_dtype), group_sizes, per_expert_counts, Li);
  else
    gather_rows_kernel<false><<<blocks, 256, 0, st>>>(x, x_ld, lat, w.num_kept, m_padded, sorted_tokens, skip, valid,
                                                     padded_token_idx, static_cast<uint8_t*>(padded_w),
                                                     dtype_size(w_dtype), group_sizes, per_expert_counts, Li);
  LMOE_CHECK_LAUNCH("dispatch_gather");
  return LMOE_OK;
}
