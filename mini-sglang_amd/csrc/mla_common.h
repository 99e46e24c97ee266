// Shared types and constants of the gfx950 MLA kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mla_amd.h"

namespace mla {

typedef __bf16 bf16x8 __attribute__((__vector_size__(16)));
typedef __bf16 bf16x4 __attribute__((__vector_size__(8)));
typedef float f32x4 __attribute__((__vector_size__(16)));
typedef float f32x16 __attribute__((__vector_size__(64)));
typedef uint32_t u32x4 __attribute__((__vector_size__(16)));
typedef uint32_t u32x2 __attribute__((__vector_size__(8)));

#define MLA_LDS __attribute__((address_space(3)))

// Absorbed-MLA latent row: 512 latent dims (also the value) + 64 rope dims, bf16.
constexpr int kKvDim = 576;
constexpr int kVDim = 512;
constexpr int kRowBytes = kKvDim * 2;  // 1152
constexpr int kRowChunks = kRowBytes / 16;  // 72 16-byte chunks per row
// Decode LDS tile: 32 tokens, staged by wave-wide 16-byte DMA loads (1 KiB each).
constexpr int kTile = 32;
constexpr int kTileBytes = kTile * kRowBytes;  // 36864
constexpr int kTileDma = kTileBytes / 1024;    // 36 wave-wide DMA loads per tile
constexpr int kStages = 4;                     // LDS ring depth (147456 bytes)
constexpr int kPlanBlock = 64;                 // tokens per plan block
constexpr int kMaxPieceIds = 1024;             // page ids of one piece staged in LDS
// Per-CTA limits of a decode plan: the streaming kernel stages one page id per
// 32-token tile (2 per plan block) and the bounds of every request of its range.
constexpr int kMaxCtaBlocks = MLA_PLAN_MAX_CTA_BLOCKS;
constexpr int kMaxCtaRequests = MLA_PLAN_MAX_CTA_REQUESTS;

struct DecodeParams {
  const __bf16* q;  // [B, H, 576]
  int64_t q_stride_b, q_stride_h;
  const __bf16* kv;  // [pages * ps, 576] rows
  int64_t kv_row_stride;  // elements
  int32_t num_pages;
  int32_t log2_ps;
  const int32_t* page_table;
  int64_t pt_stride;
  const int32_t* seq_lens;
  int32_t batch, heads;
  float scale_log2;  // softmax scale * log2(e)
  const int32_t* plan;  // [num_ctas * 4] ranges, then [batch * 3] request info
  int32_t num_ctas;
  __bf16* ws_o;   // [ws_slots, H, 512] normalised bf16 partial outputs, chunk order of mla_amd.h
  float* ws_lse;  // [ws_slots, H]
  int32_t ws_slots;
  __bf16* out;  // [B, H, 512]
  int64_t out_stride_b, out_stride_h;
  float* lse;  // [B, H] or null
  int64_t lse_stride_b;
};

struct MergeParams {
  const __bf16* ws_o;  // bf16 partials, chunk order of mla_amd.h
  const float* ws_lse;
  int32_t ws_slots;
  const int32_t* req_info;  // [batch * 3]
  int32_t batch, heads;
  int32_t skip_single;  // requests with one piece were finalised by the decode kernel
  __bf16* out;
  int64_t out_stride_b, out_stride_h;
  float* lse;
  int64_t lse_stride_b;
};

// Chunked MLA prefill (non-absorbed): per-head K [.., 192] and V [.., 128] pools.
constexpr int kPrefillQkDim = 192;
constexpr int kPrefillVDim = 128;
constexpr int kPrefillRows = 256;  // query rows per CTA (64 per wave)

struct PrefillParams {
  const __bf16* q;  // [T, H, 192]
  int64_t q_stride_t, q_stride_h;
  // K row of (token row r, head h): 128 nope dims at k + r * k_row_stride + h * k_head_stride, then
  // 64 rope dims k_rope_delta0 + h * k_rope_delta_h bytes after the nope dims' start
  const __bf16* k;
  int64_t k_row_stride, k_head_stride;
  int64_t k_rope_delta0, k_rope_delta_h;
  const __bf16* v;  // V row: 128 dims at v + r * v_row_stride + h * v_head_stride
  int64_t v_row_stride, v_head_stride;
  int32_t num_pages;
  int32_t log2_ps;
  const int32_t* page_table;
  int64_t pt_stride;
  const int32_t* cu_seqlens_q;  // [B + 1]
  const int32_t* seq_lens_k;    // [B]: prefix + extend
  int32_t batch, heads;
  float scale_log2;
  __bf16* out;  // [T, H, 128]
  int64_t out_stride_t, out_stride_h;
  int32_t out_16b;  // out rows start 16-byte aligned (base and strides): 16-byte stores
  float* lse;  // [T, H] or null
  int64_t lse_stride_t;
};

// Host side of the decode entry points (mla_api.hip): the split kernel then the LSE merge over a
// caller-given workspace, and the thread-local error message of mla_last_error().
int decode_split_merge(const char* who, const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv_pool,
                       int64_t kv_row_stride, int32_t num_pages, int32_t page_size, const int32_t* page_table,
                       int64_t pt_stride, const int32_t* seq_lens, int32_t batch, int32_t heads, float scale,
                       const int32_t* plan, int32_t num_ctas, __bf16* ws_o, float* ws_lse, int32_t ws_slots, void* out,
                       int64_t out_stride_b, int64_t out_stride_h, float* lse, int64_t lse_stride_b, void* stream);
int api_error(int code, const char* fmt, ...);
// Compute units of the current device (cached per device; safe from any host thread).
int current_device_cus();

hipError_t launch_prefill(const PrefillParams& p, int32_t total_q, hipStream_t stream);
hipError_t launch_prefill_gather(const void* kv, int64_t kv_row_stride, int32_t num_pages, int32_t log2_ps,
                                 const int32_t* page_table, int64_t pt_stride, const int32_t* seq_lens_k,
                                 const int32_t* seg_first, int32_t batch, int32_t max_seg_pages, void* c_out,
                                 int64_t c_row_stride, void* rope_out, int64_t rope_row_stride, int64_t out_rows,
                                 int32_t* seg_pt, int64_t seg_pt_stride, hipStream_t stream);
hipError_t launch_decode(const DecodeParams& p, hipStream_t stream);
// The warp-specialized kernel: 64 heads, any power-of-two page size (under 32 tokens only while every
// row offset of the pool fits in 32 bits).
bool decode_ws_takes(const DecodeParams& p);
hipError_t launch_decode_ws(const DecodeParams& p, hipStream_t stream);
hipError_t launch_merge(const MergeParams& p, hipStream_t stream);
hipError_t launch_store_rows(void* cache, int64_t cache_rows, int64_t cache_stride, const void* x, int64_t x_stride,
                             const void* indices, int index_bits, int64_t rows, int64_t row_bytes,
                             hipStream_t stream);
hipError_t launch_page_table(const int32_t* tt, int32_t tt_rows, int64_t tt_stride, const int32_t* table_idx,
                             int32_t batch, int32_t cols, int32_t page_size, int32_t* out,
                             int64_t out_stride, hipStream_t stream);
hipError_t launch_rmsnorm(const void* x, int64_t xs, const void* w, void* out, int64_t os, int32_t rows, int32_t n,
                          float eps, hipStream_t stream);
hipError_t launch_latent_rows(const void* kv, int64_t kvs, const void* w, const int32_t* pos, const float* cos_sin,
                              int32_t max_pos, void* out, int64_t os, int32_t rows, float eps, int32_t interleaved,
                              hipStream_t stream);
hipError_t launch_qkv_a_rows(void* qkv, int64_t qkvs, int32_t q_rank, const void* q_w, const void* kv_w,
                             const int32_t* pos, const float* cos_sin, int32_t max_pos, void* out, int64_t os,
                             int32_t rows, float eps, int32_t interleaved, hipStream_t stream);
hipError_t launch_q_rope(const void* q, int64_t qst, int64_t qsh, int32_t tokens, int32_t heads, const int32_t* pos,
                         const float* cos_sin, int32_t max_pos, int32_t interleaved, void* pe, int64_t pst, int64_t psh,
                         void* nope, int64_t nst, int64_t nsh, hipStream_t stream);

}  // namespace mla
