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

// Latent rows of every key of a prefill batch into 64-row scratch pages, the input of the per-head
// decompression: key j of request b (pool row pt[b, j >> log2_ps] * ps + (j & (ps - 1)), page ids
// clamped into the pool) goes to scratch row 64 seg_first[b] + j, its 512 latent dims to c_out and
// its 64 rope dims to rope_out; the scratch page table gets seg_pt[b, i] = seg_first[b] + i. CTA
// (i, b) copies scratch page i of request b: 64 rows x 72 16-byte chunks, consecutive threads on
// consecutive chunks of a row. Rows at or past out_rows are not written.
__global__ __launch_bounds__(256) void prefill_gather_kernel(const char* __restrict__ kv, int64_t kv_row_bytes,
                                                             int32_t num_pages, int32_t log2_ps,
                                                             const int32_t* __restrict__ page_table, int64_t pt_stride,
                                                             const int32_t* __restrict__ seq_lens_k,
                                                             const int32_t* __restrict__ seg_first,
                                                             char* __restrict__ c_out, int64_t c_row_bytes,
                                                             char* __restrict__ rope_out, int64_t rope_row_bytes,
                                                             int64_t out_rows, int32_t* __restrict__ seg_pt,
                                                             int64_t seg_pt_stride) {
  const int b = blockIdx.y;
  const int pg = blockIdx.x;
  const int L = seq_lens_k[b];
  const int j0 = pg * 64;
  if (j0 >= L) return;
  const int first = seg_first[b];
  if (threadIdx.x == 0) seg_pt[(int64_t)b * seg_pt_stride + pg] = first + pg;
  const int rows = min(64, L - j0);
  const int ps_mask = (1 << log2_ps) - 1;
  for (int i = threadIdx.x; i < rows * 72; i += 256) {
    const int r = i / 72, ch = i - 72 * r;
    const int j = j0 + r;
    const int64_t dst = (int64_t)first * 64 + j;
    if (dst < 0 || dst >= out_rows) continue;
    const int pid = min(max(page_table[(int64_t)b * pt_stride + (j >> log2_ps)], 0), num_pages - 1);
    const int64_t src = ((int64_t)pid << log2_ps) + (j & ps_mask);
    const u32x4 v = *reinterpret_cast<const u32x4*>(kv + src * kv_row_bytes + ch * 16);
    if (ch < 64)
      *reinterpret_cast<u32x4*>(c_out + dst * c_row_bytes + ch * 16) = v;
    else
      *reinterpret_cast<u32x4*>(rope_out + dst * rope_row_bytes + (ch - 64) * 16) = v;
  }
}

}  // namespace

hipError_t launch_prefill_gather(const void* kv, int64_t kv_row_stride, int32_t num_pages, int32_t log2_ps,
                                 const int32_t* page_table, int64_t pt_stride, const int32_t* seq_lens_k,
                                 const int32_t* seg_first, int32_t batch, int32_t max_seg_pages, void* c_out,
                                 int64_t c_row_stride, void* rope_out, int64_t rope_row_stride, int64_t out_rows,
                                 int32_t* seg_pt, int64_t seg_pt_stride, hipStream_t stream) {
  if (batch == 0 || max_seg_pages == 0) return hipSuccess;
  hipLaunchKernelGGL(prefill_gather_kernel, dim3(max_seg_pages, batch), dim3(256), 0, stream, (const char*)kv,
                     kv_row_stride * 2, num_pages, log2_ps, page_table, pt_stride, seq_lens_k, seg_first,
                     (char*)c_out, c_row_stride * 2, (char*)rope_out, rope_row_stride * 2, out_rows, seg_pt,
                     seg_pt_stride);
  return hipGetLastError();
}

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
