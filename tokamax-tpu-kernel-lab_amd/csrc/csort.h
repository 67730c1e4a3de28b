// Stable counting sort on the GPU, the primitive behind the local-shard
// dispatch (a stable argsort by local expert id, ref.py:840) and the
// deterministic combine (rows grouped by token in ascending row order).
//
// Three launches, no host synchronisation, no atomics in the ordering:
//   1. hist  : each chunk of kChunk keys builds an LDS histogram of its keys.
//   2. scan  : one block turns the per-chunk histograms into per-chunk bases
//              base[c][b] = offset[b] + sum_{c' < c} hist[c'][b], where
//              offset[b] is the exclusive prefix of the bin totals, and the
//              kept count of each bin after truncating positions >= limit.
//   3. place : one 64-lane wavefront walks its chunk in order, 64 keys at a
//              time.  Lanes holding equal keys are found with one ballot per
//              key bit (match-any); a lane's position is
//              running[key] + popcount(peers below it), so equal keys keep
//              their input order (stability) without any sort network.
// Keys are in [0, nbins]; nbins itself is the sentinel ("not in any bin").
#pragma once

#include "lmoe_common.h"

namespace lmoe {
namespace csort {
namespace {  // kernels are instantiated per translation unit

constexpr int kChunk = 1024;
constexpr int kScanThreads = 1024;

inline int key_bits_for(int nbins) {
  int b = 0;
  while ((1 << b) <= nbins) ++b;  // sentinel nbins must be representable
  return b;
}

inline int64_t num_chunks(int64_t n) { return ceil_div(n, kChunk); }

template <class KeyFn>
__global__ __launch_bounds__(256) void hist_kernel(KeyFn key, int64_t n, int nbins,
                                                   int32_t* __restrict__ hist) {
  extern __shared__ int32_t h[];
  const int nbt = nbins + 1;
  for (int i = threadIdx.x; i < nbt; i += blockDim.x) h[i] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * kChunk;
  for (int i = threadIdx.x; i < kChunk; i += blockDim.x) {
    const int64_t s = base + i;
    if (s < n) atomicAdd(&h[key(s)], 1);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nbins; i += blockDim.x)
    hist[static_cast<int64_t>(blockIdx.x) * nbins + i] = h[i];
}

// Exclusive scan of one value per thread over a kScanThreads block.
__device__ __forceinline__ int64_t block_exclusive_scan(int64_t v, int64_t* total) {
  __shared__ int64_t wsum[kScanThreads / 64];
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  int64_t x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int64_t y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int64_t w = lane < kScanThreads / 64 ? wsum[lane] : 0;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      int64_t y = __shfl_up(w, off, 64);
      if (lane >= off) w += y;
    }
    if (lane < kScanThreads / 64) wsum[lane] = w;
  }
  __syncthreads();
  const int64_t wave_prefix = wave > 0 ? wsum[wave - 1] : 0;
  *total = wsum[kScanThreads / 64 - 1];
  __syncthreads();
  return wave_prefix + x - v;
}

// One block of kScanThreads.  bin_kept[b] = number of keys of bin b whose
// position is < limit; offsets[b] = first position of bin b; *num_kept = sum.
__global__ __launch_bounds__(kScanThreads) void scan_kernel(
    const int32_t* __restrict__ hist, int chunks, int nbins, int64_t limit,
    int32_t* __restrict__ base, int32_t* __restrict__ bin_kept, int32_t* __restrict__ offsets,
    int32_t* __restrict__ num_kept) {
  const int per = (nbins + kScanThreads - 1) / kScanThreads;
  const int b0 = threadIdx.x * per;
  int64_t local = 0;
  for (int b = b0; b < b0 + per && b < nbins; ++b)
    for (int c = 0; c < chunks; ++c) local += hist[static_cast<int64_t>(c) * nbins + b];
  int64_t total_all = 0;
  int64_t off = block_exclusive_scan(local, &total_all);
  for (int b = b0; b < b0 + per && b < nbins; ++b) {
    int64_t run = off;
    for (int c = 0; c < chunks; ++c) {
      const int64_t i = static_cast<int64_t>(c) * nbins + b;
      const int32_t hcount = hist[i];
      base[i] = static_cast<int32_t>(run);
      run += hcount;
    }
    const int64_t tot = run - off;
    int64_t kept = limit - off;
    kept = kept < 0 ? 0 : (kept > tot ? tot : kept);
    if (bin_kept) bin_kept[b] = static_cast<int32_t>(kept);
    if (offsets) offsets[b] = static_cast<int32_t>(off < limit ? off : limit);
    off = run;
  }
  if (threadIdx.x == 0) {
    const int64_t nk = total_all < limit ? total_all : limit;
    *num_kept = static_cast<int32_t>(nk);
    if (offsets) offsets[nbins] = static_cast<int32_t>(nk);
  }
}

// Sink(s, key, pos, real): called for every s < n; pos is meaningful when real.
template <class KeyFn, class Sink>
__global__ __launch_bounds__(64) void place_kernel(KeyFn key, int64_t n, int nbins, int key_bits,
                                                   const int32_t* __restrict__ base, Sink sink) {
  extern __shared__ int32_t run[];
  const int lane = threadIdx.x;
  for (int i = lane; i < nbins; i += 64) run[i] = base[static_cast<int64_t>(blockIdx.x) * nbins + i];
  __syncthreads();
  const int64_t chunk_base = static_cast<int64_t>(blockIdx.x) * kChunk;
  const uint64_t below = (1ull << lane) - 1ull;
  for (int it = 0; it < kChunk / 64; ++it) {
    const int64_t s = chunk_base + it * 64 + lane;
    if (chunk_base + it * 64 >= n) break;  // uniform across the wave
    const bool active = s < n;
    const int kk = active ? key(s) : nbins;
    const bool real = active && kk < nbins;
    uint64_t peers = __ballot(real);
    for (int b = 0; b < key_bits; ++b) {
      const bool bit = (kk >> b) & 1;
      const uint64_t bb = __ballot(bit);
      peers &= bit ? bb : ~bb;
    }
    int pos = 0;
    if (real) pos = run[kk] + __popcll(peers & below);
    __builtin_amdgcn_wave_barrier();
    __syncthreads();
    if (real && (peers & below) == 0) run[kk] = pos + __popcll(peers);
    __syncthreads();
    if (active) sink(s, kk, pos, real);
  }
}

}  // namespace
}  // namespace csort
}  // namespace lmoe
