// Measured-peak kernels of the benchmark (libmla_peaks.so, not part of the MLA library's ABI):
// a read-only HBM stream and a bf16 MFMA loop, the two yardsticks beside the published
// MI355X peaks (8 TB/s HBM, 2.5 PFLOP/s dense bf16) that the attention kernels are measured
// against.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../mla_device.h"

namespace {

using mla::bf16x8;
using mla::f32x16;
using mla::u32x4;

// Read-only stream: every thread reads 16-byte chunks, kUnroll loads in flight, grid-stride over
// the buffer; the XOR of everything read is stored once per thread so no load is dead.
template <int kUnroll, bool kNonTemporal>
__global__ __launch_bounds__(256) void hbm_read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                       uint32_t* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (; i + (kUnroll - 1) * stride < n16; i += kUnroll * stride) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if constexpr (kNonTemporal) v[u] = __builtin_nontemporal_load(src + i + u * stride);
      else v[u] = src[i + u * stride];
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u];
  }
  for (; i < n16; i += stride) acc ^= src[i];
  sink[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

// Global -> LDS DMA stream (the staging path of the decode kernel): each wave moves 1 KiB per
// instruction into a 4-stage LDS ring; one XOR of the ring per stage keeps the loads live.
template <bool kNonTemporal>
__global__ __launch_bounds__(256) void hbm_read_lds_kernel(const char* __restrict__ src, int64_t nbytes,
                                                           uint32_t* __restrict__ sink) {
  constexpr int kStage = 32768;  // bytes per CTA per stage
  __shared__ __attribute__((aligned(1024))) char ring[4 * kStage];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(MLA_LDS char*)ring;
  uint32_t acc = 0;
  int n = 0;
  for (int64_t base = (int64_t)blockIdx.x * kStage; base + kStage <= nbytes; base += (int64_t)gridDim.x * kStage, ++n) {
    const int st = n & 3;
    // 32 KiB = 32 wave-wide 1 KiB loads, 8 per wave
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int chunk = wave + 4 * k;
      const char* a = src + base + chunk * 1024 + lane * 16;
      const uint32_t l = lds0 + st * kStage + chunk * 1024;
      if constexpr (kNonTemporal)
        asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(a), "{m0}"(l) : "memory");
      else
        mla::dma16_vaddr(a, l);
    }
    if (n >= 2) {  // consume the stage issued two rounds ago; the barrier waits on LDS only
      mla::wait_vmcnt<16>();
      mla::barrier_lds();
      acc ^= *reinterpret_cast<const uint32_t*>(ring + ((n - 2) & 3) * kStage + threadIdx.x * 4);
    }
  }
  mla::wait_vmcnt<0>();
  mla::barrier_lds();
  sink[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

// bf16 MFMA loop: kChains independent 32x32x16 accumulators per wave, iters rounds.
template <int kChains>
__global__ __launch_bounds__(256) void mfma_bf16_kernel(int64_t iters, float* __restrict__ sink) {
  bf16x8 a, b;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    a[j] = (__bf16)(0.001f * (threadIdx.x + j));
    b[j] = (__bf16)(0.002f * (threadIdx.x - j));
  }
  f32x16 acc[kChains];
#pragma unroll
  for (int c = 0; c < kChains; ++c)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[c][j] = 0.f;
  for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < kChains; ++c)
#pragma unroll
    for (int j = 0; j < 16; ++j) s += acc[c][j];
  sink[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

}  // namespace

extern "C" {

// Stream `nbytes` (a multiple of 16) of `src` once on `ctas` CTAs of 256 threads. variant: 0-2 =
// 16-byte vector loads with 4 / 8 / 16 in flight per thread, 3 = 8 in flight, non-temporal;
// 4 = global->LDS DMA, 5 = the same with the non-temporal hint (nbytes a multiple of 32 KiB). `sink` holds ctas * 256 uint32.
int mla_peaks_hbm_read(const void* src, int64_t nbytes, int32_t ctas, int32_t variant, void* sink, void* stream) {
  if (src == nullptr || sink == nullptr || nbytes <= 0 || nbytes % 16 != 0 || ctas < 1) return 1;
  const hipStream_t s = (hipStream_t)stream;
  const auto* p = static_cast<const u32x4*>(src);
  auto* out = static_cast<uint32_t*>(sink);
  const int64_t n16 = nbytes / 16;
  switch (variant) {
    case 0: hipLaunchKernelGGL((hbm_read_kernel<4, false>), dim3(ctas), dim3(256), 0, s, p, n16, out); break;
    case 1: hipLaunchKernelGGL((hbm_read_kernel<8, false>), dim3(ctas), dim3(256), 0, s, p, n16, out); break;
    case 2: hipLaunchKernelGGL((hbm_read_kernel<16, false>), dim3(ctas), dim3(256), 0, s, p, n16, out); break;
    case 3: hipLaunchKernelGGL((hbm_read_kernel<8, true>), dim3(ctas), dim3(256), 0, s, p, n16, out); break;
    case 4:
    case 5:
      if (nbytes % 32768 != 0) return 1;
      if (variant == 4)
        hipLaunchKernelGGL(hbm_read_lds_kernel<false>, dim3(ctas), dim3(256), 0, s, static_cast<const char*>(src),
                           nbytes, out);
      else
        hipLaunchKernelGGL(hbm_read_lds_kernel<true>, dim3(ctas), dim3(256), 0, s, static_cast<const char*>(src),
                           nbytes, out);
      break;
    default: return 1;
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// bf16 MFMA loop on `ctas` CTAs of 256 threads (4 waves): every wave issues iters * 8
// v_mfma_f32_32x32x16_bf16 (32768 FLOP each). `sink` holds ctas * 256 floats.
int mla_peaks_mfma_bf16(int64_t iters, int32_t ctas, void* sink, void* stream) {
  if (sink == nullptr || iters < 1 || ctas < 1) return 1;
  hipLaunchKernelGGL((mfma_bf16_kernel<8>), dim3(ctas), dim3(256), 0, (hipStream_t)stream, iters,
                     static_cast<float*>(sink));
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
