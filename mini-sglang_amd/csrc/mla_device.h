// Device helpers shared by the gfx950 MLA decode kernels.
#pragma once

#include "mla_common.h"

namespace mla {

// Row swizzle of the LDS tiles: 16-byte chunk c of token t is stored at chunk
// position c ^ swz(t & 7).
__device__ __forceinline__ int swz(int t7) { return ((t7 & 3) << 1) | ((t7 >> 2) & 1); }

__device__ __forceinline__ float wave_max_g(float v) {
  // reduce over the 4 lane groups (lanes l, l^16, l^32, l^48)
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}
__device__ __forceinline__ float wave_sum_g(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// Wait until at most N vector-memory operations of this wave are outstanding.
// The counter saturates at 63; a smaller count only waits longer, so N is clamped.
template <int N0>
__device__ __forceinline__ void wait_vmcnt() {
  constexpr int N = N0 > 63 ? 63 : N0;
  static_assert(N >= 0, "vmcnt range");
  // gfx9 encoding: vmcnt[3:0] | expcnt[6:4]=7 | lgkmcnt[11:8]=15 | vmcnt[5:4] at [15:14]
  __builtin_amdgcn_s_waitcnt((N & 15) | 0x70 | 0xF00 | ((N >> 4) << 14));
}

// 16-byte global -> LDS DMA; lane i's data lands at LDS byte address
// lds_base + 16*i. Issued as inline asm so that the compiler's wait-count
// pass does not serialise later LDS reads of other stages behind it: every
// read of a staged tile is preceded by wait_vmcnt + a workgroup barrier.
// The compiler's hazard recognizer does not look inside inline asm, so the
// wait states it would add are written here: an LDS DMA reads M0 one wait
// state after a scalar write of M0 (the compiler writes M0 just before the
// asm statement).
__device__ __forceinline__ void dma16_saddr(const char* base, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds_base) : "memory");
}
// The same with the non-temporal hint: for data read once (streamed KV rows), so the caches keep
// the lines that are reused.
__device__ __forceinline__ void dma16_saddr_nt(const char* base, uint32_t voff, uint32_t lds_base) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(base), "{m0}"(lds_base) : "memory");
}
__device__ __forceinline__ void dma16_vaddr(const char* addr, uint32_t lds_base) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(addr), "{m0}"(lds_base) : "memory");
}
// A 64-bit scalar base from a uniform vector value, for a DMA's address. A vector-ALU write of an
// SGPR needs 5 wait states before a memory instruction reads it; readfirstlane and the nops are
// volatile asm, so they stay in order with the DMA asm statements that follow.
__device__ __forceinline__ const char* uniform_ptr(uint32_t lo, uint32_t hi) {
  uint32_t slo, shi;
  asm volatile("v_readfirstlane_b32 %0, %2\n\tv_readfirstlane_b32 %1, %3\n\ts_nop 4"
               : "=s"(slo), "=s"(shi) : "v"(lo), "v"(hi));
  return reinterpret_cast<const char*>(((uint64_t)shi << 32) | slo);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  // round-to-nearest-even, matching torch's float->bfloat16 conversion; one v_cvt_pk_bf16_f32
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}


// Workgroup barrier that orders LDS only: waits for this wave's LDS ops, then
// s_barrier. Unlike __syncthreads() it never waits on vector-memory counters,
// so in-flight DMA loads and output stores stay in flight.
__device__ __forceinline__ void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Scalar (wave-uniform) 32-bit load, waited for before returning.
__device__ __forceinline__ int sload_i32(const int32_t* ptr) {
  int v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(ptr) : "memory");
  return v;
}

// Scalar load of four consecutive 32-bit values (16-byte aligned), waited for.
__device__ __forceinline__ void sload_i32x4(const int32_t* ptr, int& a, int& b, int& c, int& d) {
  typedef int i32x4_t __attribute__((__vector_size__(16)));
  i32x4_t v;
  asm volatile("s_load_dwordx4 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(ptr) : "memory");
  a = v[0];
  b = v[1];
  c = v[2];
  d = v[3];
}

// Binary tree of scalar branches over the wait count (6 compares for 0..63).
template <int Lo, int Hi>
__device__ __forceinline__ void wait_vmcnt_tree(int n) {
  if constexpr (Lo == Hi) {
    wait_vmcnt<Lo>();
  } else {
    constexpr int Mid = (Lo + Hi) / 2;
    if (n <= Mid) wait_vmcnt_tree<Lo, Mid>(n);
    else wait_vmcnt_tree<Mid + 1, Hi>(n);
  }
}

// wait_vmcnt with a run-time count, clamped to the counter range. The count is
// made wave-uniform first so that the selection compiles to scalar branches.
__device__ __forceinline__ void wait_vmcnt_dyn(int n) {
  n = __builtin_amdgcn_readfirstlane(n > 63 ? 63 : (n < 0 ? 0 : n));
  wait_vmcnt_tree<0, 63>(n);
}

}  // namespace mla
