// Direct-to-LDS DMA helpers shared by the grouped GEMM kernels (gfx950).
//
// global_load_lds_dwordx4 copies 16 bytes per active lane from global memory
// to LDS[M0 + 16 * lane] (global_load_lds_dword: 4 bytes to LDS[M0 + 4 * lane]).  It is issued from inline asm so the compiler neither
// tracks it nor inserts its conservative vmcnt(0) before LDS reads; the
// kernels wait for it themselves with s_waitcnt vmcnt(n), counting only these
// operations (every vector memory operation inside their K loops is one).
#pragma once

#include <type_traits>
#include <utility>

#include "lmoe_common.h"

namespace lmoe {
namespace dma {

template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (void)(f(std::integral_constant<int, I>{}) && ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)p));
}

// Load from an LDS byte address.
template <class T>
__device__ __forceinline__ T lds_load(uint32_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) T*>(static_cast<uintptr_t>(addr));
}

// x through an opaque move: the compiler keeps the value in a register
// instead of recomputing it where it is used.
__device__ __forceinline__ uint32_t opaque_u32(uint32_t x) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "v"(x));
  return r;
}

// Wave-uniform copy of a pointer (lives in an SGPR pair).
__device__ __forceinline__ const uint8_t* uniform_ptr(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const uint8_t*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// One 16-byte DMA per active lane: LDS[lds + 16 * lane] = *(sbase + off).
// `sbase` and `lds` are wave-uniform (SGPRs); M0 is written immediately
// before use (one wait state).
__device__ __forceinline__ void dma16s(uint32_t off, const uint8_t* sbase, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(off), "s"(uniform_ptr(sbase)), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

// One 4-byte DMA per active lane: LDS[lds + 4 * lane] = *(sbase + off).
__device__ __forceinline__ void dma4s(uint32_t off, const uint8_t* sbase, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :
               : "v"(off), "s"(uniform_ptr(sbase)), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// Wait until at most N of this wave's vector memory operations are in flight
// and all its LDS reads have returned.  The LDS-read wait keeps a slot's last
// fragment reads ahead of the DMA that the next step issues into it.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" : : "n"(N) : "memory");
}

__device__ __forceinline__ void barrier() { asm volatile("s_barrier" : : : "memory"); }

// Wait for the DMA of step kt when `ahead` (0 .. NS-2) later steps, of OPS
// operations each for this wave, have been issued after it.
template <int NS, int OPS>
__device__ __forceinline__ void wait_step(int ahead) {
  if (ahead >= NS - 2) {
    wait_vm_lgkm<(NS - 2) * OPS>();
  } else {
    static_for<NS - 2>([&](auto a) __attribute__((always_inline)) {
      constexpr int A = decltype(a)::value;
      if (ahead == A) wait_vm_lgkm<A * OPS>();
      return true;
    });
  }
}

}  // namespace dma
}  // namespace lmoe
