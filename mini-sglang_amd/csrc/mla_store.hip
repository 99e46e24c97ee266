// KV row scatter and token-table -> page-table conversion (bit-exact byte and
// integer work, HBM/launch bound).
#include "mla_common.h"

namespace mla {
namespace {

// cache[indices[i]] = x[i]: the grid covers (row, 16-byte chunk) pairs, so a
// 1152-byte latent row is 72 lanes and a wave copies 1 KiB per instruction
// whatever the row width.
template <typename Index>
__global__ __launch_bounds__(256) void store_rows_kernel(char* __restrict__ cache, int64_t cache_rows,
                                                         int64_t cache_stride,
                                                         const char* __restrict__ x, int64_t x_stride,
                                                         const Index* __restrict__ indices, int64_t rows,
                                                         int64_t chunks_per_row) {
  const int64_t total = rows * chunks_per_row;
  for (int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; id < total;
       id += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = id / chunks_per_row;
    const int64_t ch = id - r * chunks_per_row;
    const int64_t dst_row = (int64_t)indices[r];
    if (dst_row < 0 || dst_row >= cache_rows) continue;
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + r * x_stride + ch * 16);
    *reinterpret_cast<u32x4*>(cache + dst_row * cache_stride + ch * 16) = v;
  }
}

// out[i] = cache[indices[i]] (the inverse of store_rows): the grid covers (row, 16-byte chunk)
// pairs; rows whose index lies outside the cache are left untouched.
__global__ __launch_bounds__(256) void gather_rows_kernel(char* __restrict__ out, int64_t out_stride,
                                                          const char* __restrict__ cache, int64_t cache_rows,
                                                          int64_t cache_stride, const int64_t* __restrict__ indices,
                                                          int64_t rows, int64_t chunks_per_row) {
  const int64_t total = rows * chunks_per_row;
  for (int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; id < total;
       id += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = id / chunks_per_row;
    const int64_t ch = id - r * chunks_per_row;
    const int64_t src_row = indices[r];
    if (src_row < 0 || src_row >= cache_rows) continue;
    *reinterpret_cast<u32x4*>(out + r * out_stride + ch * 16) =
        *reinterpret_cast<const u32x4*>(cache + src_row * cache_stride + ch * 16);
  }
}

// out[b, j] = floor(tt[table_idx[b], j * ps] / ps)
__global__ __launch_bounds__(256) void page_table_kernel(const int32_t* __restrict__ tt, int32_t tt_rows,
                                                         int64_t tt_stride,
                                                         const int32_t* __restrict__ table_idx, int32_t cols,
                                                         int32_t ps, int32_t* __restrict__ out,
                                                         int64_t out_stride) {
  const int b = blockIdx.y;
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= cols) return;
  const int32_t row = min(max(table_idx[b], 0), tt_rows - 1);
  const int32_t v = tt[(int64_t)row * tt_stride + (int64_t)j * ps];
  int32_t q = v / ps;
  if ((v % ps) != 0 && v < 0) q -= 1;  // floor division, as torch's rounding_mode="floor"
  out[(int64_t)b * out_stride + j] = q;
}

}  // namespace

hipError_t launch_store_rows(void* cache, int64_t cache_rows, int64_t cache_stride, const void* x, int64_t x_stride,
                             const void* indices, int index_bits, int64_t rows, int64_t row_bytes,
                             hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  const int64_t cpr = row_bytes / 16;
  const int64_t total = rows * cpr;
  const int64_t want = (total + 255) / 256;
  const int grid = (int)(want < 65536 ? want : 65536);
  if (index_bits == 32)
    hipLaunchKernelGGL(store_rows_kernel<int32_t>, dim3(grid), dim3(256), 0, stream, (char*)cache, cache_rows, cache_stride,
                       (const char*)x, x_stride, (const int32_t*)indices, rows, cpr);
  else
    hipLaunchKernelGGL(store_rows_kernel<int64_t>, dim3(grid), dim3(256), 0, stream, (char*)cache, cache_rows, cache_stride,
                       (const char*)x, x_stride, (const int64_t*)indices, rows, cpr);
  return hipGetLastError();
}

hipError_t launch_gather_rows(void* out, int64_t out_stride, const void* cache, int64_t cache_rows,
                              int64_t cache_stride, const int64_t* indices, int64_t rows, int64_t row_bytes,
                              hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  const int64_t cpr = row_bytes / 16;
  const int64_t want = (rows * cpr + 255) / 256;
  const int grid = (int)(want < 65536 ? want : 65536);
  hipLaunchKernelGGL(gather_rows_kernel, dim3(grid), dim3(256), 0, stream, (char*)out, out_stride, (const char*)cache,
                     cache_rows, cache_stride, indices, rows, cpr);
  return hipGetLastError();
}

hipError_t launch_page_table(const int32_t* tt, int32_t tt_rows, int64_t tt_stride, const int32_t* table_idx,
                             int32_t batch,
                             int32_t cols, int32_t page_size, int32_t* out, int64_t out_stride,
                             hipStream_t stream) {
  if (batch == 0 || cols == 0) return hipSuccess;
  dim3 grid((cols + 255) / 256, batch);
  hipLaunchKernelGGL(page_table_kernel, grid, dim3(256), 0, stream, tt, tt_rows, tt_stride, table_idx, cols, page_size, out,
                     out_stride);
  return hipGetLastError();
}

}  // namespace mla
