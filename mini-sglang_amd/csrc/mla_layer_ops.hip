// Elementwise steps of the MLA layer around the attention kernels: RMSNorm of rows, the latent
// row of a token (RMSNorm of its 512 latent dims + RoPE of its 64 rope dims, written as one
// 576-dim row), and the queries' RoPE (plus the head-major copy of their 128 nope dims that the
// absorption GEMM reads). All three are HBM/launch bound: one wave per row or per (token, head),
// 16-byte loads, fp32 arithmetic, bf16 round-to-nearest-even on store.
#include "mla_common.h"
#include "mla_device.h"

namespace mla {
namespace {

constexpr int kRopeDim = 64;
constexpr int kNopeDim = 128;

__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ void unpack8(const u32x4 w, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return r;
}

__device__ __forceinline__ float bf(const __bf16* p) { return __uint_as_float((uint32_t)(*(const uint16_t*)p) << 16); }

__device__ __forceinline__ void store_bf(__bf16* p, float v) {
  *(uint16_t*)p = (uint16_t)(pack_bf16x2(v, 0.f) & 0xffffu);
}

// Rotates pair i of a 64-dim slice: dims (2i, 2i+1) interleaved, (i, i + 32) otherwise, by the
// angle whose cosine and sine are cos_sin[pos][i] and cos_sin[pos][32 + i].
__device__ __forceinline__ void rope_pair(const __bf16* in, __bf16* out, int i, const float* cs, int interleaved) {
  const int a = interleaved ? 2 * i : i;
  const int b = interleaved ? 2 * i + 1 : i + kRopeDim / 2;
  const float xa = bf(in + a), xb = bf(in + b);
  const float c = cs[i], s = cs[kRopeDim / 2 + i];
  store_bf(out + a, xa * c - xb * s);
  store_bf(out + b, xb * c + xa * s);
}

// out[r] = x[r] / sqrt(mean(x[r]^2) + eps) * w, one wave per row (4 rows per block). In place
// (out == x) is allowed: every lane finishes reading its chunks before the wave's reduction, and
// the second pass reads and writes only the lane's own chunks.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const __bf16* __restrict__ x, int64_t xs,
                                                      const __bf16* __restrict__ w, __bf16* out, int64_t os,
                                                      int rows, int n, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const __bf16* xr = x + (int64_t)row * xs;
  __bf16* orow = out + (int64_t)row * os;
  float ss = 0.f;
  for (int c = lane * 8; c < n; c += 512) {
    float f[8];
    unpack8(*reinterpret_cast<const u32x4*>(xr + c), f);
#pragma unroll
    for (int k = 0; k < 8; ++k) ss += f[k] * f[k];
  }
  const float inv = rsqrtf(wave_sum64(ss) / (float)n + eps);
  for (int c = lane * 8; c < n; c += 512) {
    float f[8], g[8];
    unpack8(*reinterpret_cast<const u32x4*>(xr + c), f);
    unpack8(*reinterpret_cast<const u32x4*>(w + c), g);
#pragma unroll
    for (int k = 0; k < 8; ++k) f[k] = f[k] * inv * g[k];
    *reinterpret_cast<u32x4*>(orow + c) = pack8(f);
  }
}

// Latent row of token r: out[r][0:512] = rmsnorm(kv[r][0:512]) * w, out[r][512:576] = RoPE of
// kv[r][512:576] at positions[r] (clamped into the cos/sin table). One wave per token.
__global__ __launch_bounds__(256) void latent_rows_kernel(const __bf16* __restrict__ kv, int64_t kvs,
                                                          const __bf16* __restrict__ w,
                                                          const int32_t* __restrict__ pos,
                                                          const float* __restrict__ cos_sin, int max_pos,
                                                          __bf16* __restrict__ out, int64_t os, int rows, float eps,
                                                          int interleaved) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const __bf16* r = kv + (int64_t)row * kvs;
  __bf16* orow = out + (int64_t)row * os;
  float f[8], g[8];
  unpack8(*reinterpret_cast<const u32x4*>(r + 8 * lane), f);
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) ss += f[k] * f[k];
  const float inv = rsqrtf(wave_sum64(ss) / (float)kVDim + eps);
  unpack8(*reinterpret_cast<const u32x4*>(w + 8 * lane), g);
#pragma unroll
  for (int k = 0; k < 8; ++k) f[k] = f[k] * inv * g[k];
  *reinterpret_cast<u32x4*>(orow + 8 * lane) = pack8(f);
  if (lane < kRopeDim / 2) {
    const int p = min(max(pos[row], 0), max_pos - 1);
    rope_pair(r + kVDim, orow + kVDim, lane, cos_sin + (int64_t)p * kRopeDim, interleaved);
  }
}

// The q_a / kv_a projection's rows, fused: qkv[r] = [q_a (q_rank) | kv (576)]. One wave per token
// normalises the q_a part in place (RMSNorm with q_w) and writes the token's latent row (RMSNorm
// of the kv part's 512 latent dims with kv_w, RoPE of its 64 rope dims) to out[r].
__global__ __launch_bounds__(256) void qkv_a_rows_kernel(__bf16* qkv, int64_t qkvs, int q_rank,
                                                         const __bf16* __restrict__ q_w,
                                                         const __bf16* __restrict__ kv_w,
                                                         const int32_t* __restrict__ pos,
                                                         const float* __restrict__ cos_sin, int max_pos,
                                                         __bf16* __restrict__ out, int64_t os, int rows, float eps,
                                                         int interleaved) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  __bf16* qr = qkv + (int64_t)row * qkvs;
  // q_a part: sum of squares, then scale in place (each lane rereads only its own chunks)
  float ss = 0.f;
  for (int c = lane * 8; c < q_rank; c += 512) {
    float f[8];
    unpack8(*reinterpret_cast<const u32x4*>(qr + c), f);
#pragma unroll
    for (int k = 0; k < 8; ++k) ss += f[k] * f[k];
  }
  const float qinv = rsqrtf(wave_sum64(ss) / (float)q_rank + eps);
  for (int c = lane * 8; c < q_rank; c += 512) {
    float f[8], g[8];
    unpack8(*reinterpret_cast<const u32x4*>(qr + c), f);
    unpack8(*reinterpret_cast<const u32x4*>(q_w + c), g);
#pragma unroll
    for (int k = 0; k < 8; ++k) f[k] = f[k] * qinv * g[k];
    *reinterpret_cast<u32x4*>(qr + c) = pack8(f);
  }
  // kv part: the latent row
  const __bf16* r = qr + q_rank;
  __bf16* orow = out + (int64_t)row * os;
  float f[8], g[8];
  unpack8(*reinterpret_cast<const u32x4*>(r + 8 * lane), f);
  float s2 = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) s2 += f[k] * f[k];
  const float inv = rsqrtf(wave_sum64(s2) / (float)kVDim + eps);
  unpack8(*reinterpret_cast<const u32x4*>(kv_w + 8 * lane), g);
#pragma unroll
  for (int k = 0; k < 8; ++k) f[k] = f[k] * inv * g[k];
  *reinterpret_cast<u32x4*>(orow + 8 * lane) = pack8(f);
  if (lane < kRopeDim / 2) {
    const int p = min(max(pos[row], 0), max_pos - 1);
    rope_pair(r + kVDim, orow + kVDim, lane, cos_sin + (int64_t)p * kRopeDim, interleaved);
  }
}

// Query (t, h) = q[t, h, 0:192] (128 nope + 64 rope dims): pe_out[t, h, 0:64] = RoPE of the rope
// dims at positions[t]; if nope_out is given, nope_out[t, h, 0:128] (own strides, e.g. head-major)
// = the nope dims. pe_out may alias the rope dims of q (in place: every lane writes only the
// bytes it read). One wave per (token, 8 heads): lane 8 hl + k rotates pairs 4k .. 4k + 3 of head
// 8 g + hl, one 16-byte access (interleaved pairs: dims 8k .. 8k + 7) or two 8-byte ones (halves:
// dims 4k .. 4k + 3 and 32 + 4k .. 32 + 4k + 3); the nope copy is 128 16-byte chunks per wave.
constexpr int kQRopeHeads = 8;

__global__ __launch_bounds__(256) void q_rope_kernel(const __bf16* q, int64_t qst, int64_t qsh, int tokens,
                                                     int heads, const int32_t* __restrict__ pos,
                                                     const float* __restrict__ cos_sin, int max_pos, int interleaved,
                                                     __bf16* pe, int64_t pst, int64_t psh, __bf16* __restrict__ nope,
                                                     int64_t nst, int64_t nsh) {
  const int lane = threadIdx.x & 63;
  const int groups = (heads + kQRopeHeads - 1) / kQRopeHeads;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= (int64_t)tokens * groups) return;
  const int t = (int)(item / groups), h0 = (int)(item % groups) * kQRopeHeads;
  if (nope != nullptr) {
    for (int c = lane; c < kQRopeHeads * (kNopeDim / 8); c += 64) {
      const int h = h0 + c / (kNopeDim / 8), k = c % (kNopeDim / 8);
      if (h < heads)
        *reinterpret_cast<u32x4*>(nope + (int64_t)t * nst + (int64_t)h * nsh + 8 * k) =
            *reinterpret_cast<const u32x4*>(q + (int64_t)t * qst + (int64_t)h * qsh + 8 * k);
    }
  }
  const int h = h0 + (lane >> 3), k = lane & 7;
  if (h >= heads) return;
  const int p = min(max(pos[t], 0), max_pos - 1);
  const float* cs = cos_sin + (int64_t)p * kRopeDim;
  const f32x4 cv = *reinterpret_cast<const f32x4*>(cs + 4 * k);
  const f32x4 sv = *reinterpret_cast<const f32x4*>(cs + kRopeDim / 2 + 4 * k);
  const __bf16* in = q + (int64_t)t * qst + (int64_t)h * qsh + kNopeDim;
  __bf16* out = pe + (int64_t)t * pst + (int64_t)h * psh;
  if (interleaved) {
    float f[8], g[8];
    unpack8(*reinterpret_cast<const u32x4*>(in + 8 * k), f);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      g[2 * i] = f[2 * i] * cv[i] - f[2 * i + 1] * sv[i];
      g[2 * i + 1] = f[2 * i + 1] * cv[i] + f[2 * i] * sv[i];
    }
    *reinterpret_cast<u32x4*>(out + 8 * k) = pack8(g);
  } else {
    const u32x2 a = *reinterpret_cast<const u32x2*>(in + 4 * k);
    const u32x2 b = *reinterpret_cast<const u32x2*>(in + kRopeDim / 2 + 4 * k);
    float xa[4], xb[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      xa[2 * i] = __uint_as_float(a[i] << 16);
      xa[2 * i + 1] = __uint_as_float(a[i] & 0xffff0000u);
      xb[2 * i] = __uint_as_float(b[i] << 16);
      xb[2 * i + 1] = __uint_as_float(b[i] & 0xffff0000u);
    }
    u32x2 ra, rb;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      ra[i] = pack_bf16x2(xa[2 * i] * cv[2 * i] - xb[2 * i] * sv[2 * i],
                          xa[2 * i + 1] * cv[2 * i + 1] - xb[2 * i + 1] * sv[2 * i + 1]);
      rb[i] = pack_bf16x2(xb[2 * i] * cv[2 * i] + xa[2 * i] * sv[2 * i],
                          xb[2 * i + 1] * cv[2 * i + 1] + xa[2 * i + 1] * sv[2 * i + 1]);
    }
    *reinterpret_cast<u32x2*>(out + 4 * k) = ra;
    *reinterpret_cast<u32x2*>(out + kRopeDim / 2 + 4 * k) = rb;
  }
}

}  // namespace

hipError_t launch_rmsnorm(const void* x, int64_t xs, const void* w, void* out, int64_t os, int32_t rows, int32_t n,
                          float eps, hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((rows + 3) / 4), dim3(256), 0, stream, (const __bf16*)x, xs,
                     (const __bf16*)w, (__bf16*)out, os, rows, n, eps);
  return hipGetLastError();
}

hipError_t launch_latent_rows(const void* kv, int64_t kvs, const void* w, const int32_t* pos, const float* cos_sin,
                              int32_t max_pos, void* out, int64_t os, int32_t rows, float eps, int32_t interleaved,
                              hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(latent_rows_kernel, dim3((rows + 3) / 4), dim3(256), 0, stream, (const __bf16*)kv, kvs,
                     (const __bf16*)w, pos, cos_sin, max_pos, (__bf16*)out, os, rows, eps, interleaved);
  return hipGetLastError();
}

hipError_t launch_qkv_a_rows(void* qkv, int64_t qkvs, int32_t q_rank, const void* q_w, const void* kv_w,
                             const int32_t* pos, const float* cos_sin, int32_t max_pos, void* out, int64_t os,
                             int32_t rows, float eps, int32_t interleaved, hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  hipLaunchKernelGGL(qkv_a_rows_kernel, dim3((rows + 3) / 4), dim3(256), 0, stream, (__bf16*)qkv, qkvs, q_rank,
                     (const __bf16*)q_w, (const __bf16*)kv_w, pos, cos_sin, max_pos, (__bf16*)out, os, rows, eps,
                     interleaved);
  return hipGetLastError();
}

hipError_t launch_q_rope(const void* q, int64_t qst, int64_t qsh, int32_t tokens, int32_t heads, const int32_t* pos,
                         const float* cos_sin, int32_t max_pos, int32_t interleaved, void* pe, int64_t pst, int64_t psh,
                         void* nope, int64_t nst, int64_t nsh, hipStream_t stream) {
  const int64_t items = (int64_t)tokens * ((heads + kQRopeHeads - 1) / kQRopeHeads);
  if (items == 0) return hipSuccess;
  hipLaunchKernelGGL(q_rope_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, stream, (const __bf16*)q, qst,
                     qsh, tokens, heads, pos, cos_sin, max_pos, interleaved, (__bf16*)pe, pst, psh, (__bf16*)nope,
                     nst, nsh);
  return hipGetLastError();
}

}  // namespace mla
