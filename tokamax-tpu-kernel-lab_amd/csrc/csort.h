// Stable counting sort on the GPU, the primitive behind the local-shard
// dispatch (a stable argsort by local expert id, ref.py:840) and the
// deterministic combine (rows grouped by token in ascending row order).
//
// Three launches, no host synchronisation, no atomics in the ordering:
//   1. hist  : each chunk of CHUNK keys builds an LDS histogram of its keys
//              and writes it bin-major: hist[b * chunks + c].
//   2. scan  : one block computes the exclusive prefix sum of hist in that
//              (bin, chunk) order, which is exactly the first output position
//              of bin b's keys from chunk c: base[b][c] = offset[b] +
//              sum_{c' < c} hist[b][c'], offset[b] being the exclusive prefix
//              of the bin totals.  It also gives the kept count of each bin
//              after truncating positions >= limit.
//   3. place : one 64-lane wavefront walks its chunk in order, 64 keys at a
//              time.  Lanes holding equal keys are found with one ballot per
//              key bit (match-any); a lane's position is
//              running[key] + popcount(peers below it), so equal keys keep
//              their input order (stability) without any sort network.
// Keys are in [0, nbins]; nbins itself is the sentinel ("not in any bin").
// CHUNK trades parallelism in hist/place (more chunks) against the size of
// the scanned array (nbins x chunks): small for few bins (dispatch), large
// for many (the token-keyed combine).
#pragma once

#include "lmoe_common.h"

namespace lmoe {
namespace csort {
namespace {  // kernels are instantiated per translation unit

constexpr int kScanThreads = 1024;
constexpr int64_t kScanDynLds = 65536;  // dynamic LDS of the scan (bin starts + staged histogram)

inline int key_bits_for(int nbins) {
  int b = 0;
  while ((1 << b) <= nbins) ++b;  // sentinel nbins must be representable
  return b;
}

template <int CHUNK>
inline int64_t num_chunks(int64_t n) {
  return ceil_div(n, CHUNK);
}

template <int CHUNK, class KeyFn>
__global__ __launch_bounds__(256) void hist_kernel(KeyFn key, int64_t n, int nbins, int64_t chunks,
                                                   int32_t* __restrict__ hist) {
  extern __shared__ int32_t h[];
  const int nbt = nbins + 1;
  for (int i = threadIdx.x; i < nbt; i += blockDim.x) h[i] = 0;
  __syncthreads();
  const int64_t base = static_cast<int64_t>(blockIdx.x) * CHUNK;
  for (int i = threadIdx.x; i < CHUNK; i += blockDim.x) {
    const int64_t s = base + i;
    if (s < n) atomicAdd(&h[key(s)], 1);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nbins; i += blockDim.x) hist[i * chunks + blockIdx.x] = h[i];
}

// Exclusive scan of one 32-bit value per thread over a kScanThreads block
// (totals < 2^31); *total receives the block sum.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* total) {
  __shared__ uint32_t wsum[kScanThreads / 64];
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const uint32_t x = wave_scan_sat(v, 0x7fffffffu);
  if (lane == 63) wsum[wave] = x;
  __syncthreads();
  if (wave == 0) {
    const uint32_t w = lane < kScanThreads / 64 ? wsum[lane] : 0u;
    const uint32_t ws = wave_scan_sat(w, 0x7fffffffu);
    if (lane < kScanThreads / 64) wsum[lane] = ws;
  }
  __syncthreads();
  const uint32_t wave_prefix = wave > 0 ? wsum[wave - 1] : 0u;
  *total = wsum[kScanThreads / 64 - 1];
  __syncthreads();
  return wave_prefix + x - v;
}

// One block of kScanThreads; dynamic LDS (nbins + 1) ints.  Thread t scans the
// contiguous segment [t * per, (t + 1) * per) of the (bin, chunk) array; up to
// kHeld elements per thread are loaded once, all in flight together, and
// kept in registers for the second pass (one memory round trip for the usual
// sizes; larger arrays loop).  bin_kept[b] = number of keys of bin b whose
// position is < limit; offsets[b] = first position of bin b (clipped to
// limit); *num_kept = sum.
__global__ __launch_bounds__(kScanThreads) void scan_kernel(
    const int32_t* __restrict__ hist, int64_t chunks, int nbins, int64_t limit,
    int32_t* __restrict__ base, int32_t* __restrict__ bin_kept, int32_t* __restrict__ offsets,
    int32_t* __restrict__ num_kept, int staged) {
  extern __shared__ int32_t bin_start[];  // nbins + 1, then (staged) the histogram
  constexpr int kHeld = 16;
  static_assert(kScanDynLds / 4 <= kHeld * kScanThreads, "a staged histogram is copied in one pass");
  const int64_t total_n = chunks * nbins;
  const int64_t per = (total_n + kScanThreads - 1) / kScanThreads;
  const int64_t i0 = threadIdx.x * per;
  const int64_t i1 = i0 + per < total_n ? i0 + per : total_n;
  // Staged: the histogram is copied into LDS with coalesced loads, each thread
  // scans its contiguous run there (an odd run length hits distinct banks) and
  // the bases go back out coalesced.  Unstaged, the runs are read and written
  // in global memory directly (lanes 4*per bytes apart).
  int32_t* stage = bin_start + ((nbins + 4) & ~3);
  if (staged) {  // total_n <= kHeld * kScanThreads: every load in flight at once
    int32_t v[kHeld];
#pragma unroll
    for (int q = 0; q < kHeld; ++q) {
      const int64_t i = threadIdx.x + static_cast<int64_t>(q) * kScanThreads;
      v[q] = i < total_n ? hist[i] : 0;
    }
#pragma unroll
    for (int q = 0; q < kHeld; ++q) {
      const int64_t i = threadIdx.x + static_cast<int64_t>(q) * kScanThreads;
      if (i < total_n) stage[i] = v[q];
    }
    __syncthreads();
  }
  const int32_t* src = staged ? stage : hist;
  int32_t* dst = staged ? stage : base;
  int32_t held[kHeld];
#pragma unroll
  for (int q = 0; q < kHeld; ++q) held[q] = i0 + q < i1 ? src[i0 + q] : 0;
  uint32_t local = 0;
#pragma unroll
  for (int q = 0; q < kHeld; ++q) local += static_cast<uint32_t>(held[q]);
  for (int64_t i = i0 + kHeld; i < i1; ++i) local += static_cast<uint32_t>(src[i]);
  uint32_t total = 0;
  uint32_t run = block_exclusive_scan(local, &total);
  int64_t bin = i0 / chunks, chunk = i0 % chunks;  // coordinates of element i
  auto emit = [&](int64_t i, int32_t v) {
    dst[i] = static_cast<int32_t>(run);
    if (chunk == 0) bin_start[bin] = static_cast<int32_t>(run);
    run += static_cast<uint32_t>(v);
    if (++chunk == chunks) {
      chunk = 0;
      ++bin;
    }
  };
#pragma unroll
  for (int q = 0; q < kHeld; ++q)
    if (i0 + q < i1) emit(i0 + q, held[q]);
  for (int64_t i = i0 + kHeld; i < i1; ++i) emit(i, src[i]);
  if (threadIdx.x == 0) bin_start[nbins] = static_cast<int32_t>(total);
  __syncthreads();
  if (staged)
    for (int64_t i = threadIdx.x; i < total_n; i += kScanThreads) base[i] = stage[i];
  for (int b = threadIdx.x; b < nbins; b += kScanThreads) {
    const int64_t off = bin_start[b], tot = bin_start[b + 1] - off;
    int64_t kept = limit - off;
    kept = kept < 0 ? 0 : (kept > tot ? tot : kept);
    if (bin_kept) bin_kept[b] = static_cast<int32_t>(kept);
    if (offsets) offsets[b] = static_cast<int32_t>(off < limit ? off : limit);
  }
  if (threadIdx.x == 0) {
    const int64_t nk = static_cast<int64_t>(total) < limit ? static_cast<int64_t>(total) : limit;
    *num_kept = static_cast<int32_t>(nk);
    if (offsets) offsets[nbins] = static_cast<int32_t>(nk);
  }
}

// Launch the scan with (nbins + 1) ints of dynamic LDS, plus the whole
// histogram when that still fits in kScanDynLds (64 KB, beyond the default
// dynamic limit once the static wave totals are added).
inline hipError_t launch_scan(const int32_t* hist, int64_t chunks, int nbins, int64_t limit, int32_t* base,
                              int32_t* bin_kept, int32_t* offsets, int32_t* num_kept, hipStream_t st) {
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&scan_kernel),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, kScanDynLds);
  if (attr != hipSuccess) return attr;
  const int64_t head = (nbins + 4) & ~3;  // bin_start ints, the stage 16-byte aligned after them
  const int64_t staged_bytes = (head + chunks * nbins) * static_cast<int64_t>(sizeof(int32_t));
  const bool staged = staged_bytes <= kScanDynLds;
  const size_t lds = staged ? static_cast<size_t>(staged_bytes) : (nbins + 1) * sizeof(int32_t);
  scan_kernel<<<1, kScanThreads, lds, st>>>(hist, chunks, nbins, limit, base, bin_kept, offsets, num_kept,
                                            staged ? 1 : 0);
  return hipSuccess;
}

// sink.load(s) -> u32 is read for every s < n before any rank is computed;
// sink(s, key, pos, real, loaded): called for every s < n; pos is meaningful
// when real.  All the chunk's keys and loads are issued up front (one memory
// round trip per chunk, not one per 64 slots).
template <int CHUNK, class KeyFn, class Sink>
__global__ __launch_bounds__(64) void place_kernel(KeyFn key, int64_t n, int nbins, int key_bits, int64_t chunks,
                                                   const int32_t* __restrict__ base, Sink sink) {
  constexpr int IT = CHUNK / 64;
  extern __shared__ int32_t run[];
  const int lane = threadIdx.x;
  const int64_t chunk_base = static_cast<int64_t>(blockIdx.x) * CHUNK;
  int keys[IT];
  uint32_t loaded[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int64_t s = chunk_base + it * 64 + lane;
    keys[it] = s < n ? key(s) : nbins;
    loaded[it] = s < n ? sink.load(s) : 0u;
  }
  for (int i = lane; i < nbins; i += 64) run[i] = base[i * chunks + blockIdx.x];
  __syncthreads();
  const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int64_t s = chunk_base + it * 64 + lane;
    if (chunk_base + it * 64 >= n) break;  // uniform across the wave
    const bool active = s < n;
    const int kk = keys[it];
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
    if (active) sink(s, kk, pos, real, loaded[it]);
  }
}

// place with four waves per chunk: wave w takes the chunk's w-th quarter of
// slots (CHUNK / 256 rounds of 64).  A first pass finds every round's
// match-any groups and counts each wave's keys per bin in LDS; the counts
// then become per-wave starting positions (the chunk's base plus the counts
// of the earlier waves), and a second pass places the slots exactly as the
// one-wave kernel does, so the positions are the same and stable.  Four
// times the slots in flight per chunk and a quarter of the serial rounds per
// wave; LDS 16 * nbins bytes (the caller keeps it within 64 KB).
template <int CHUNK, class KeyFn, class Sink>
__global__ __launch_bounds__(256) void place4_kernel(KeyFn key, int64_t n, int nbins, int key_bits, int64_t chunks,
                                                     const int32_t* __restrict__ base, Sink sink) {
  constexpr int kW = 4, IT = CHUNK / 64 / kW;
  static_assert(CHUNK % (64 * kW) == 0, "chunk split over the waves");
  extern __shared__ int32_t off[];  // [kW][nbins]
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const int64_t wave_base = static_cast<int64_t>(blockIdx.x) * CHUNK + wave * (CHUNK / kW);
  int keys[IT];
  uint32_t loaded[IT];
  uint64_t peer_sets[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int64_t s = wave_base + it * 64 + lane;
    keys[it] = s < n ? key(s) : nbins;
    loaded[it] = s < n ? sink.load(s) : 0u;
  }
  for (int i = threadIdx.x; i < kW * nbins; i += 256) off[i] = 0;
  __syncthreads();
  const uint64_t below = (1ull << lane) - 1ull;
  int32_t* mine = off + wave * nbins;
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int64_t s = wave_base + it * 64 + lane;
    const int kk = keys[it];
    const bool real = s < n && kk < nbins;
    uint64_t peers = __ballot(real);
    for (int b = 0; b < key_bits; ++b) {
      const bool bit = (kk >> b) & 1;
      const uint64_t bb = __ballot(bit);
      peers &= bit ? bb : ~bb;
    }
    peer_sets[it] = peers;
    if (real && (peers & below) == 0) mine[kk] += __popcll(peers);
    __builtin_amdgcn_wave_barrier();
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
  }
  __syncthreads();
  for (int b = threadIdx.x; b < nbins; b += 256) {
    int32_t acc = base[b * chunks + blockIdx.x];
#pragma unroll
    for (int w = 0; w < kW; ++w) {
      const int32_t c = off[w * nbins + b];
      off[w * nbins + b] = acc;
      acc += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    if (wave_base + it * 64 >= n) break;  // uniform across the wave
    const int64_t s = wave_base + it * 64 + lane;
    const bool active = s < n;
    const int kk = keys[it];
    const bool real = active && kk < nbins;
    const uint64_t peers = peer_sets[it];
    int pos = 0;
    if (real) pos = mine[kk] + __popcll(peers & below);
    __builtin_amdgcn_wave_barrier();
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
    if (real && (peers & below) == 0) mine[kk] = pos + __popcll(peers);
    __builtin_amdgcn_wave_barrier();
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
    if (active) sink(s, kk, pos, real, loaded[it]);
  }
}

// Scan for few bins, split over the bins instead of one block: wave b scans
// bin b's chunk counts hist[b * chunks + c] in chunk order and writes their
// exclusive prefix (the position of the chunk's first key relative to the
// bin's first position) to rel[b * chunks + c], then the bin's total over
// hist[b * chunks].  Lane i owns the contiguous run [i * per, (i + 1) * per)
// of chunks; up to kHeld counts per lane are loaded at once (one memory round
// trip for up to 64 * kHeld chunks).  The bin offsets (an exclusive prefix
// over the bins) are left to place_scanned_kernel, which needs them anyway,
// so no kernel reads the whole histogram.
__global__ __launch_bounds__(64) void scan_bins_kernel(int32_t* __restrict__ hist, int64_t chunks,
                                                       int32_t* __restrict__ rel) {
  constexpr int kHeld = 16;
  const int lane = threadIdx.x;
  int32_t* h = hist + static_cast<int64_t>(blockIdx.x) * chunks;
  int32_t* r = rel + static_cast<int64_t>(blockIdx.x) * chunks;
  const int64_t per = (chunks + 63) / 64;
  const int64_t i0 = lane * per;
  const int64_t i1 = i0 + per < chunks ? i0 + per : chunks;
  int32_t held[kHeld];
#pragma unroll
  for (int q = 0; q < kHeld; ++q) held[q] = i0 + q < i1 ? h[i0 + q] : 0;
  uint32_t local = 0;
#pragma unroll
  for (int q = 0; q < kHeld; ++q) local += static_cast<uint32_t>(held[q]);
  for (int64_t i = i0 + kHeld; i < i1; ++i) local += static_cast<uint32_t>(h[i]);
  const uint32_t incl = wave_scan_sat(local, 0x7fffffffu);
  const uint32_t total = __builtin_amdgcn_readlane(incl, 63);
  uint32_t run = incl - local;
#pragma unroll
  for (int q = 0; q < kHeld; ++q)
    if (i0 + q < i1) {
      r[i0 + q] = static_cast<int32_t>(run);
      run += static_cast<uint32_t>(held[q]);
    }
  for (int64_t i = i0 + kHeld; i < i1; ++i) {
    const int32_t v = h[i];
    r[i] = static_cast<int32_t>(run);
    run += static_cast<uint32_t>(v);
  }
  if (lane == 0) h[0] = static_cast<int32_t>(total);  // only lane 0 read h[0], above
}

// place4_kernel for the scan_bins_kernel layout: every block first turns the
// bin totals (hist[b * chunks]) into bin offsets with a block-wide exclusive
// scan, so a chunk's start in bin b is offset[b] + rel[b * chunks + c].
// Block 0 also writes bin_kept[b] (positions below limit) and *num_kept, the
// outputs of the one-block scan.  Every block knows the kept total, so the
// sink may also write per-position outputs here: sink.bin_kept(b, kept) runs
// in block 0 for every bin, sink.positions(num_kept, block, blocks) in every
// block (no-ops for sinks without such outputs).  Runs for n == 0 too (one
// chunk).  LDS 20 * nbins bytes.
//
// FROM_HIST (nbins <= 256): no scan_bins_kernel before it -- `totals` is the
// raw histogram (hist[b * chunks + c]) and each block sums every bin's chunk
// counts itself (the bin total and this chunk's start in the bin; 4 * chunks
// bytes per bin, read from L2 after the histogram pass), one launch fewer.
// LDS 24 * nbins bytes.
template <int CHUNK, class KeyFn, class Sink, bool FROM_HIST = false>
__global__ __launch_bounds__(256) void place_scanned_kernel(KeyFn key, int64_t n, int nbins, int key_bits,
                                                            int64_t chunks, const int32_t* __restrict__ totals,
                                                            const int32_t* __restrict__ rel, int64_t limit,
                                                            int32_t* __restrict__ bin_kept,
                                                            int32_t* __restrict__ num_kept, Sink sink) {
  constexpr int kW = 4, IT = CHUNK / 64 / kW;
  static_assert(CHUNK % (64 * kW) == 0, "chunk split over the waves");
  extern __shared__ int32_t off[];  // [kW][nbins], the bin offsets [nbins], FROM_HIST: chunk starts [nbins]
  __shared__ uint32_t s_part[kW];
  int32_t* bin_off = off + kW * nbins;
  int32_t* rel_s = bin_off + nbins;
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const int64_t wave_base = static_cast<int64_t>(blockIdx.x) * CHUNK + wave * (CHUNK / kW);
  int keys[IT];
  uint32_t loaded[IT];
  uint64_t peer_sets[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int64_t s = wave_base + it * 64 + lane;
    keys[it] = s < n ? key(s) : nbins;
    loaded[it] = s < n ? sink.load(s) : 0u;
  }
  if constexpr (FROM_HIST) {
    // nbins <= 256: bin b's chunk counts are summed by the G adjacent lanes
    // of group b (G the largest power of two <= 64 with G * nbins <= 256),
    // each lane V counts per load with 8 loads in flight; the group's
    // partials are added by lane shuffles.  Bin total -> bin_off[b], this
    // chunk's start within the bin -> rel_s[b].
    int G = 64;
    while (G > 1 && G * nbins > 256) G >>= 1;
    const int g = threadIdx.x / G, sub = threadIdx.x % G;
    const int64_t me = blockIdx.x;
    uint32_t tot = 0, pre = 0;
    auto sum_row = [&](auto vtag) {
      constexpr int V = decltype(vtag)::value;
      const int32_t* h = totals + static_cast<int64_t>(g) * chunks;
      const int64_t nq = chunks / V;
      for (int64_t q0 = sub; q0 < nq; q0 += 8 * G) {
        uint32_t v[8][V];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int64_t q = q0 + static_cast<int64_t>(j) * G;
          if constexpr (V == 4) {
            const int4 x = q < nq ? *reinterpret_cast<const int4*>(h + 4 * q) : make_int4(0, 0, 0, 0);
            v[j][0] = static_cast<uint32_t>(x.x);
            v[j][1] = static_cast<uint32_t>(x.y);
            v[j][2] = static_cast<uint32_t>(x.z);
            v[j][3] = static_cast<uint32_t>(x.w);
          } else {
            v[j][0] = q < nq ? static_cast<uint32_t>(h[q]) : 0u;
          }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
          for (int e = 0; e < V; ++e) {
            const int64_t c = (q0 + static_cast<int64_t>(j) * G) * V + e;
            tot += v[j][e];
            pre += c < me ? v[j][e] : 0u;
          }
      }
    };
    if (g < nbins) {
      if (chunks % 4 == 0 && reinterpret_cast<uintptr_t>(totals) % 16 == 0)
        sum_row(std::integral_constant<int, 4>{});
      else
        sum_row(std::integral_constant<int, 1>{});
    }
    for (int m = 1; m < G; m <<= 1) {
      tot += __shfl_xor(tot, m);
      pre += __shfl_xor(pre, m);
    }
    if (g < nbins && sub == 0) {
      bin_off[g] = static_cast<int32_t>(tot);
      rel_s[g] = static_cast<int32_t>(pre);
    }
    __syncthreads();
  }
  // bin offsets: thread t owns the contiguous bins [t * per, (t + 1) * per)
  const int per = (nbins + 255) / 256;
  const int b0 = threadIdx.x * per, b1 = b0 + per < nbins ? b0 + per : nbins;
  uint32_t mine_sum = 0;
  for (int b = b0; b < b1; ++b) {
    const uint32_t t = FROM_HIST ? static_cast<uint32_t>(bin_off[b])
                                 : static_cast<uint32_t>(totals[static_cast<int64_t>(b) * chunks]);
    bin_off[b] = static_cast<int32_t>(t);
    mine_sum += t;
  }
  for (int i = threadIdx.x; i < kW * nbins; i += 256) off[i] = 0;
  const uint32_t incl = wave_scan_sat(mine_sum, 0x7fffffffu);
  if (lane == 63) s_part[wave] = incl;
  __syncthreads();
  uint32_t run = incl - mine_sum, grand = 0;
  for (int w = 0; w < kW; ++w) {
    if (w < wave) run += s_part[w];
    grand += s_part[w];
  }
  for (int b = b0; b < b1; ++b) {
    const uint32_t t = static_cast<uint32_t>(bin_off[b]);
    bin_off[b] = static_cast<int32_t>(run);
    if (blockIdx.x == 0) {
      int64_t kept = limit - static_cast<int64_t>(run);
      kept = kept < 0 ? 0 : (kept > t ? t : kept);
      bin_kept[b] = static_cast<int32_t>(kept);
      sink.bin_kept(b, static_cast<int32_t>(kept));
    }
    run += t;
  }
  const int64_t total_kept = static_cast<int64_t>(grand) < limit ? static_cast<int64_t>(grand) : limit;
  if (blockIdx.x == 0 && threadIdx.x == 0) *num_kept = static_cast<int32_t>(total_kept);
  sink.positions(total_kept, blockIdx.x, gridDim.x);
  __syncthreads();
  const uint64_t below = (1ull << lane) - 1ull;
  int32_t* mine = off + wave * nbins;
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int64_t s = wave_base + it * 64 + lane;
    const int kk = keys[it];
    const bool real = s < n && kk < nbins;
    uint64_t peers = __ballot(real);
    for (int b = 0; b < key_bits; ++b) {
      const bool bit = (kk >> b) & 1;
      const uint64_t bb = __ballot(bit);
      peers &= bit ? bb : ~bb;
    }
    peer_sets[it] = peers;
    if (real && (peers & below) == 0) mine[kk] += __popcll(peers);
    __builtin_amdgcn_wave_barrier();
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
  }
  __syncthreads();
  for (int b = threadIdx.x; b < nbins; b += 256) {
    int32_t acc = bin_off[b] + (FROM_HIST ? rel_s[b] : rel[static_cast<int64_t>(b) * chunks + blockIdx.x]);
#pragma unroll
    for (int w = 0; w < kW; ++w) {
      const int32_t c = off[w * nbins + b];
      off[w * nbins + b] = acc;
      acc += c;
    }
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    if (wave_base + it * 64 >= n) break;  // uniform across the wave
    const int64_t s = wave_base + it * 64 + lane;
    const bool active = s < n;
    const int kk = keys[it];
    const bool real = active && kk < nbins;
    const uint64_t peers = peer_sets[it];
    int pos = 0;
    if (real) pos = mine[kk] + __popcll(peers & below);
    __builtin_amdgcn_wave_barrier();
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
    if (real && (peers & below) == 0) mine[kk] = pos + __popcll(peers);
    __builtin_amdgcn_wave_barrier();
    asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
    if (active) sink(s, kk, pos, real, loaded[it]);
  }
}

// place over all chunks: the four-wave kernel when its per-wave counts fit
// in 64 KB of LDS, else the one-wave kernel.
template <int CHUNK, class KeyFn, class Sink>
inline void launch_place(KeyFn key, int64_t n, int nbins, int64_t chunks, const int32_t* base, Sink sink,
                         hipStream_t st) {
  const int bits = key_bits_for(nbins);
  if (static_cast<int64_t>(nbins) * 16 <= 65536)
    place4_kernel<CHUNK><<<dim3(static_cast<unsigned>(chunks)), 256, nbins * 16, st>>>(key, n, nbins, bits, chunks,
                                                                                       base, sink);
  else
    place_kernel<CHUNK><<<dim3(static_cast<unsigned>(chunks)), 64, nbins * sizeof(int32_t), st>>>(
        key, n, nbins, bits, chunks, base, sink);
}

// Scan + place of a counting sort whose histogram hist (bin-major, chunks
// per bin) is already built: bin_kept[b] and *num_kept as the one-block scan
// gives them, and sink(...) for every slot.  Few bins (20 * nbins bytes of
// LDS, with the static wave totals, fit in 64 KB): scan_bins_kernel and
// place_scanned_kernel; else the one-block scan and the place kernels.  base
// (nbins * chunks ints) receives the scanned chunk starts; hist is
// overwritten.
// scan_and_place takes scan_bins_kernel + place_scanned_kernel (whose sink
// hooks run) for this many bins
inline bool scanned_place(int nbins) { return static_cast<int64_t>(nbins) * 20 <= 65536 - 256; }

template <int CHUNK, class KeyFn, class Sink>
inline hipError_t scan_and_place(KeyFn key, int64_t n, int nbins, int64_t chunks, int64_t limit, int32_t* hist,
                                 int32_t* base, int32_t* bin_kept, int32_t* num_kept, Sink sink, hipStream_t st) {
  if (scanned_place(nbins)) {
    if (chunks <= 256 && nbins <= 256) {
      // few chunks: the place pass sums the histogram itself (no scan launch)
      place_scanned_kernel<CHUNK, KeyFn, Sink, true><<<dim3(static_cast<unsigned>(chunks)), 256, nbins * 24, st>>>(
          key, n, nbins, key_bits_for(nbins), chunks, hist, nullptr, limit, bin_kept, num_kept, sink);
      return hipSuccess;
    }
    scan_bins_kernel<<<dim3(static_cast<unsigned>(nbins)), 64, 0, st>>>(hist, chunks, base);
    place_scanned_kernel<CHUNK><<<dim3(static_cast<unsigned>(chunks)), 256, nbins * 20, st>>>(
        key, n, nbins, key_bits_for(nbins), chunks, hist, base, limit, bin_kept, num_kept, sink);
    return hipSuccess;
  }
  const hipError_t e = launch_scan(hist, chunks, nbins, limit, base, bin_kept, nullptr, num_kept, st);
  if (e != hipSuccess) return e;
  if (n > 0) launch_place<CHUNK>(key, n, nbins, chunks, base, sink, st);
  return hipSuccess;
}

}  // namespace
}  // namespace csort
}  // namespace lmoe
