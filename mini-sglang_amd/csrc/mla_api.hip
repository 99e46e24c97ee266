// extern "C" entry points of libmla_amd.so (declared in include/mla_amd.h):
// argument validation, the split-KV planner (host) and kernel launches.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <limits.h>

#include <algorithm>
#include <atomic>

#include <string>

#include "../../include/mla_amd.h"
#include "mla_common.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return MLA_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail(MLA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }
int ilog2(int64_t x) {
  int r = 0;
  while ((int64_t(1) << r) < x) ++r;
  return r;
}
// 16-byte aligned rows of at least n bf16 elements, row stride a multiple of 8 elements
bool rows_ok(const void* p, int64_t stride, int64_t n) { return aligned(p, 16) && stride % 8 == 0 && stride >= n; }

// Fixed cost of one decode piece, in 64-token blocks of KV traffic: loading the
// 64 heads' queries (73.7 KB) and writing/merging the partial output.
constexpr int kPieceOverheadBlocks = 2;

}  // namespace

extern "C" {

const char* mla_last_error(void) { return g_last_error.c_str(); }

int mla_abi_version(void) { return 9; }

int mla_device_cu_count(int device, int32_t* out) {
  if (out == nullptr) return fail(MLA_ERR_INVALID_ARG, "mla_device_cu_count: out is null");
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return hip_status(e, "hipGetDeviceProperties");
  *out = prop.multiProcessorCount;
  return ok();
}

int mla_store_rows(void* cache, int64_t cache_rows, int64_t cache_row_stride_bytes, const void* x,
                   int64_t x_row_stride_bytes, const void* indices, int32_t index_bits, int64_t num_rows,
                   int64_t row_bytes, void* stream) {
  if (num_rows < 0) return fail(MLA_ERR_INVALID_ARG, "mla_store_rows: num_rows < 0");
  if (num_rows == 0) return ok();
  if (cache == nullptr || x == nullptr || indices == nullptr)
    return fail(MLA_ERR_INVALID_ARG, "mla_store_rows: null pointer");
  if (index_bits != 32 && index_bits != 64)
    return fail(MLA_ERR_INVALID_ARG, "mla_store_rows: index_bits must be 32 or 64, got %d", index_bits);
  if (row_bytes <= 0 || row_bytes % 16 != 0)
    return fail(MLA_ERR_UNSUPPORTED, "mla_store_rows: row_bytes %lld is not a positive multiple of 16",
                (long long)row_bytes);
  if (cache_row_stride_bytes < row_bytes || cache_row_stride_bytes % 16 != 0 || x_row_stride_bytes < row_bytes ||
      x_row_stride_bytes % 16 != 0)
    return fail(MLA_ERR_INVALID_ARG, "mla_store_rows: strides must be multiples of 16 and >= row_bytes");
  if (!aligned(cache, 16) || !aligned(x, 16))
    return fail(MLA_ERR_INVALID_ARG, "mla_store_rows: cache and x must be 16-byte aligned");
  if (cache_rows <= 0) return fail(MLA_ERR_INVALID_ARG, "mla_store_rows: cache_rows must be positive");
  return hip_status(mla::launch_store_rows(cache, cache_rows, cache_row_stride_bytes, x, x_row_stride_bytes,
                                           indices, index_bits, num_rows, row_bytes, (hipStream_t)stream),
                    "mla_store_rows launch");
}

int mla_prefill_gather_bf16(const void* kv_pool, int64_t kv_row_stride, int32_t num_pages, int32_t page_size,
                            const int32_t* page_table, int64_t pt_stride, const int32_t* seq_lens_k,
                            const int32_t* seg_first, int32_t batch, int32_t max_seg_pages, void* c_out,
                            int64_t c_row_stride, void* rope_out, int64_t rope_row_stride, int64_t out_rows,
                            int32_t* seg_page_table, int64_t seg_pt_stride, void* stream) {
  const char* who = "mla_prefill_gather_bf16";
  if (batch < 0 || max_seg_pages < 0 || out_rows < 0)
    return fail(MLA_ERR_INVALID_ARG, "%s: batch %d, max_seg_pages %d, out_rows %lld", who, batch, max_seg_pages,
                (long long)out_rows);
  if (batch == 0 || max_seg_pages == 0) return ok();
  if (kv_pool == nullptr || page_table == nullptr || seq_lens_k == nullptr || seg_first == nullptr ||
      c_out == nullptr || rope_out == nullptr || seg_page_table == nullptr)
    return fail(MLA_ERR_INVALID_ARG, "%s: null pointer", who);
  if (!is_pow2(page_size)) return fail(MLA_ERR_UNSUPPORTED, "%s: page_size %d must be a power of two", who, page_size);
  if (num_pages < 1 || pt_stride < 1) return fail(MLA_ERR_INVALID_ARG, "%s: num_pages / pt_stride < 1", who);
  if (!rows_ok(kv_pool, kv_row_stride, mla::kKvDim) || !rows_ok(c_out, c_row_stride, MLA_V_DIM) ||
      !rows_ok(rope_out, rope_row_stride, mla::kKvDim - MLA_V_DIM))
    return fail(MLA_ERR_INVALID_ARG, "%s: rows must be 16-byte aligned with strides multiples of 8 holding the row", who);
  if (seg_pt_stride < max_seg_pages)
    return fail(MLA_ERR_INVALID_ARG, "%s: seg_pt_stride %lld < max_seg_pages %d", who, (long long)seg_pt_stride,
                max_seg_pages);
  return hip_status(mla::launch_prefill_gather(kv_pool, kv_row_stride, num_pages, ilog2(page_size), page_table,
                                               pt_stride, seq_lens_k, seg_first, batch, max_seg_pages, c_out,
                                               c_row_stride, rope_out, rope_row_stride, out_rows, seg_page_table,
                                               seg_pt_stride, (hipStream_t)stream),
                    who);
}

int mla_page_table_from_tokens(const int32_t* token_table, int32_t token_table_rows, int32_t token_table_cols,
                               int64_t token_table_stride, const int32_t* table_idx, int32_t batch,
                               int32_t max_seqlen_k, int32_t page_size, int32_t* out, int64_t out_stride,
                               void* stream) {
  if (batch < 0 || max_seqlen_k < 0) return fail(MLA_ERR_INVALID_ARG, "mla_page_table_from_tokens: negative size");
  if (page_size <= 0) return fail(MLA_ERR_INVALID_ARG, "mla_page_table_from_tokens: page_size must be positive");
  const int32_t cols = (max_seqlen_k + page_size - 1) / page_size;
  if (batch == 0 || cols == 0) return ok();
  if (token_table == nullptr || table_idx == nullptr || out == nullptr)
    return fail(MLA_ERR_INVALID_ARG, "mla_page_table_from_tokens: null pointer");
  if (token_table_rows <= 0 || max_seqlen_k > token_table_cols || token_table_stride < token_table_cols)
    return fail(MLA_ERR_INVALID_ARG,
                "mla_page_table_from_tokens: max_seqlen_k %d exceeds the token table (%d x %d, stride %lld)",
                max_seqlen_k, token_table_rows, token_table_cols, (long long)token_table_stride);
  if (out_stride < cols)
    return fail(MLA_ERR_INVALID_ARG, "mla_page_table_from_tokens: out_stride %lld < %d columns",
                (long long)out_stride, cols);
  return hip_status(mla::launch_page_table(token_table, token_table_rows, token_table_stride, table_idx, batch, cols,
                                           page_size, out, out_stride, (hipStream_t)stream),
                    "mla_page_table_from_tokens launch");
}

// Greedy contiguous partition of the requests' blocks with at most `cap`
// cost units (blocks + kPieceOverheadBlocks per piece) per CTA, at most
// max_blk blocks per piece, and per CTA at most mla::kMaxCtaBlocks blocks and
// mla::kMaxCtaRequests requests (the streaming kernel stages per-tile page ids
// and per-request bounds of its range in LDS). Returns the number of CTAs
// used, or INT32_MAX if the partition needs more than `limit` CTAs. Writes the
// plan when `write` is set.
static int plan_greedy(const int32_t* seq_lens, int batch, int64_t cap, int64_t max_blk, int limit, bool write,
                       int32_t* cta_ranges, int32_t* req_info, int32_t* num_slots) {
  const int B = mla::kPlanBlock;
  int w = 0;
  int64_t used = 0, blocks = 0;
  int reqs = 0;
  int32_t slots = 0;
  if (write) {
    cta_ranges[0] = 0;
    cta_ranges[1] = 0;
  }
  auto next_cta = [&](int b, int64_t blk) -> bool {
    if (w + 1 >= limit) return false;
    if (write) {
      cta_ranges[4 * w + 2] = b;
      cta_ranges[4 * w + 3] = (int32_t)blk;
      cta_ranges[4 * (w + 1) + 0] = b;
      cta_ranges[4 * (w + 1) + 1] = (int32_t)blk;
    }
    ++w;
    used = blocks = 0;
    reqs = 0;
    return true;
  };
  for (int b = 0; b < batch; ++b) {
    const int64_t nb = ((int64_t)seq_lens[b] + B - 1) / B;
    int first = w, pieces = 0;
    int64_t blk = 0;
    if (reqs >= mla::kMaxCtaRequests && !next_cta(b, 0)) return INT32_MAX;
    ++reqs;  // every request of the range (even an empty one) has an LDS entry
    while (blk < nb) {
      int64_t room = cap - used - kPieceOverheadBlocks;
      if (room > mla::kMaxCtaBlocks - blocks) room = mla::kMaxCtaBlocks - blocks;
      if (room <= 0) {
        if (used == 0) return INT32_MAX;  // cap too small for any block
        if (!next_cta(b, blk)) return INT32_MAX;
        ++reqs;
        continue;
      }
      int64_t take = nb - blk;
      if (take > room) take = room;
      if (take > max_blk) take = max_blk;
      if (pieces == 0) first = w;
      ++pieces;
      blk += take;
      used += take + kPieceOverheadBlocks;
      blocks += take;
      if (blk < nb) {
        if (!next_cta(b, blk)) return INT32_MAX;
        ++reqs;
      }
    }
    if (write) {
      req_info[3 * b + 0] = first;
      req_info[3 * b + 1] = pieces;
      req_info[3 * b + 2] = pieces >= 2 ? slots : 0;
    }
    if (pieces >= 2) slots += pieces;
  }
  if (write) {
    cta_ranges[4 * w + 2] = batch;
    cta_ranges[4 * w + 3] = 0;
    for (int e = w + 1; e < limit; ++e) {
      cta_ranges[4 * e + 0] = batch;
      cta_ranges[4 * e + 1] = 0;
      cta_ranges[4 * e + 2] = batch;
      cta_ranges[4 * e + 3] = 0;
    }
    *num_slots = slots;
  }
  return w + 1;
}

int mla_decode_plan(const int32_t* seq_lens, int32_t batch, int32_t page_size, int32_t num_ctas,
                    int32_t max_piece_pages, int32_t* cta_ranges, int32_t* req_info, int32_t* num_slots) {
  if (batch < 0) return fail(MLA_ERR_INVALID_ARG, "mla_decode_plan: batch < 0");
  if (num_ctas < 1) return fail(MLA_ERR_INVALID_ARG, "mla_decode_plan: num_ctas must be >= 1");
  if (!is_pow2(page_size)) return fail(MLA_ERR_INVALID_ARG, "mla_decode_plan: page_size %d is not a power of two", page_size);
  if (cta_ranges == nullptr || num_slots == nullptr || (batch > 0 && (seq_lens == nullptr || req_info == nullptr)))
    return fail(MLA_ERR_INVALID_ARG, "mla_decode_plan: null pointer");
  const int B = mla::kPlanBlock;
  // Longest piece in blocks such that it touches at most max_piece_pages pages (no limit if <= 0;
  // the kernels take pieces of any length).
  const int64_t max_blk = max_piece_pages <= 0 ? INT64_MAX
                          : page_size <= B     ? (int64_t)max_piece_pages * page_size / B
                                               : (int64_t)(max_piece_pages - 1) * page_size / B;
  if (max_blk < 1)
    return fail(MLA_ERR_INVALID_ARG, "mla_decode_plan: max_piece_pages %d too small for page_size %d",
                max_piece_pages, page_size);
  int64_t total = 0;
  for (int b = 0; b < batch; ++b) {
    if (seq_lens[b] < 0) return fail(MLA_ERR_INVALID_ARG, "mla_decode_plan: seq_lens[%d] < 0", b);
    const int64_t nb = ((int64_t)seq_lens[b] + B - 1) / B;
    total += nb + (nb > 0 ? kPieceOverheadBlocks : 0);
  }
  // Smallest per-CTA capacity for which the greedy partition fits num_ctas CTAs.
  int64_t lo = kPieceOverheadBlocks + 1, hi = total + kPieceOverheadBlocks + 1;
  if (plan_greedy(seq_lens, batch, hi, max_blk, num_ctas, false, nullptr, nullptr, nullptr) > num_ctas)
    return fail(MLA_ERR_UNSUPPORTED,
                "mla_decode_plan: %d CTAs cannot hold the batch (per CTA at most %d blocks and %d requests%s)",
                num_ctas, mla::kMaxCtaBlocks, mla::kMaxCtaRequests, max_piece_pages > 0 ? ", capped pieces" : "");
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo) / 2;
    if (plan_greedy(seq_lens, batch, mid, max_blk, num_ctas, false, nullptr, nullptr, nullptr) <= num_ctas)
      hi = mid;
    else
      lo = mid + 1;
  }
  plan_greedy(seq_lens, batch, lo, max_blk, num_ctas, true, cta_ranges, req_info, num_slots);
  return ok();
}

static int check_out(const void* out, int64_t sb, int64_t sh, const float* lse, int64_t lse_sb, int32_t heads,
                     const char* who) {
  if (out == nullptr) return fail(MLA_ERR_INVALID_ARG, "%s: out is null", who);
  if (!aligned(out, 16) || sb % 8 != 0 || sh % 8 != 0 || sh < 512 || sb < (int64_t)heads * sh)
    return fail(MLA_ERR_INVALID_ARG,
                "%s: out must be 16-byte aligned with strides (b=%lld, h=%lld) multiples of 8, h >= 512, "
                "b >= heads*h",
                who, (long long)sb, (long long)sh);
  if (lse != nullptr && lse_sb < heads)
    return fail(MLA_ERR_INVALID_ARG, "%s: lse row stride %lld < heads %d", who, (long long)lse_sb, heads);
  return MLA_OK;
}

static int decode_params(const char* who, const void* q, int64_t q_stride_b, int64_t q_stride_h,
                         const void* kv_pool, int64_t kv_row_stride, int32_t num_pages, int32_t page_size,
                         const int32_t* page_table, int64_t pt_stride, const int32_t* seq_lens, int32_t batch,
                         int32_t heads, float scale, const int32_t* plan, int32_t num_ctas, __bf16* ws_o,
                         float* ws_lse, int32_t ws_slots, void* out, int64_t out_stride_b, int64_t out_stride_h,
                         float* lse, int64_t lse_stride_b, mla::DecodeParams* p) {
  if (heads < 1 || heads > 64) return fail(MLA_ERR_UNSUPPORTED, "%s: heads must be in [1, 64], got %d", who, heads);
  if (q == nullptr || kv_pool == nullptr || page_table == nullptr || seq_lens == nullptr || plan == nullptr)
    return fail(MLA_ERR_INVALID_ARG, "%s: null pointer", who);
  if (!aligned(q, 16) || q_stride_h % 8 != 0 || q_stride_b % 8 != 0 || q_stride_h < MLA_KV_DIM ||
      q_stride_b < (int64_t)heads * q_stride_h)
    return fail(MLA_ERR_INVALID_ARG, "%s: q must be 16-byte aligned, row-contiguous, strides multiples of 8", who);
  if (!aligned(kv_pool, 16) || kv_row_stride % 8 != 0 || kv_row_stride < MLA_KV_DIM || kv_row_stride > (1 << 20))
    return fail(MLA_ERR_INVALID_ARG,
                "%s: kv_pool must be 16-byte aligned with row stride in [576, 2^20], multiple of 8", who);
  if (num_pages < 1) return fail(MLA_ERR_INVALID_ARG, "%s: num_pages must be >= 1", who);
  if (!is_pow2(page_size)) return fail(MLA_ERR_UNSUPPORTED, "%s: page_size %d is not a power of two", who, page_size);
  if (pt_stride < 1) return fail(MLA_ERR_INVALID_ARG, "%s: pt_stride must be >= 1", who);
  if (num_ctas < 1) return fail(MLA_ERR_INVALID_ARG, "%s: num_ctas must be >= 1", who);
  if (!(scale > 0.f) || !isfinite(scale)) return fail(MLA_ERR_INVALID_ARG, "%s: scale must be finite and > 0", who);
  if (ws_slots < 0 || (ws_slots > 0 && (ws_o == nullptr || ws_lse == nullptr)))
    return fail(MLA_ERR_INVALID_ARG, "%s: workspace pointers are null", who);
  if (ws_o != nullptr && !aligned(ws_o, 16)) return fail(MLA_ERR_INVALID_ARG, "%s: ws_o must be 16-byte aligned", who);
  if (int rc = check_out(out, out_stride_b, out_stride_h, lse, lse_stride_b, heads, who)) return rc;
  p->q = static_cast<const __bf16*>(q);
  p->q_stride_b = q_stride_b;
  p->q_stride_h = q_stride_h;
  p->kv = static_cast<const __bf16*>(kv_pool);
  p->kv_row_stride = kv_row_stride;
  p->num_pages = num_pages;
  p->log2_ps = ilog2(page_size);
  p->page_table = page_table;
  p->pt_stride = pt_stride;
  p->seq_lens = seq_lens;
  p->batch = batch;
  p->heads = heads;
  p->scale_log2 = scale * 1.4426950408889634f;
  p->plan = plan;
  p->num_ctas = num_ctas;
  p->ws_o = ws_o;
  p->ws_lse = ws_lse;
  p->ws_slots = ws_slots;
  p->out = static_cast<__bf16*>(out);
  p->out_stride_b = out_stride_b;
  p->out_stride_h = out_stride_h;
  p->lse = lse;
  p->lse_stride_b = lse_stride_b;
  return MLA_OK;
}

static mla::MergeParams merge_params(const __bf16* ws_o, const float* ws_lse, int32_t ws_slots,
                                     const int32_t* req_info, int32_t batch, int32_t heads, int32_t skip_single,
                                     void* out, int64_t out_stride_b, int64_t out_stride_h, float* lse,
                                     int64_t lse_stride_b) {
  mla::MergeParams m;
  m.ws_o = ws_o;
  m.ws_lse = ws_lse;
  m.ws_slots = ws_slots;
  m.req_info = req_info;
  m.batch = batch;
  m.heads = heads;
  m.skip_single = skip_single;
  m.out = static_cast<__bf16*>(out);
  m.out_stride_b = out_stride_b;
  m.out_stride_h = out_stride_h;
  m.lse = lse;
  m.lse_stride_b = lse_stride_b;
  return m;
}

// Decode runs in groups of at most 64 query heads (one streaming-kernel CTA holds 64 heads' state);
// a group's partials occupy its own [ws_slots, group heads, 512] block of the workspace, so the
// caller's [ws_slots, heads, 512] buffer holds every group's block back to back.
constexpr int32_t kHeadGroup = 64;
constexpr int32_t kMaxHeads = 1024;

struct HeadGroup {
  const void* q;
  __bf16* ws_o;
  float* ws_lse;
  void* out;
  float* lse;
  int32_t heads;
};

static HeadGroup head_group(int32_t h0, int32_t heads, int32_t ws_slots, const void* q, int64_t q_stride_h, __bf16* ws_o,
                            float* ws_lse, void* out, int64_t out_stride_h, float* lse) {
  HeadGroup g;
  g.heads = heads - h0 < kHeadGroup ? heads - h0 : kHeadGroup;
  g.q = q == nullptr ? nullptr : static_cast<const __bf16*>(q) + (int64_t)h0 * q_stride_h;
  g.ws_o = ws_o == nullptr ? nullptr : ws_o + (int64_t)ws_slots * h0 * MLA_V_DIM;
  g.ws_lse = ws_lse == nullptr ? nullptr : ws_lse + (int64_t)ws_slots * h0;
  g.out = static_cast<__bf16*>(out) + (int64_t)h0 * out_stride_h;
  g.lse = lse == nullptr ? nullptr : lse + h0;
  return g;
}

static int check_head_groups(const char* who, int32_t heads, int64_t q_stride_b, int64_t q_stride_h,
                             int64_t out_stride_b, int64_t out_stride_h, const float* lse, int64_t lse_stride_b) {
  if (heads < 1 || heads > kMaxHeads) return fail(MLA_ERR_UNSUPPORTED, "%s: heads must be in [1, %d], got %d", who, kMaxHeads, heads);
  if (q_stride_b < (int64_t)heads * q_stride_h || out_stride_b < (int64_t)heads * out_stride_h ||
      (lse != nullptr && lse_stride_b < heads))
    return fail(MLA_ERR_INVALID_ARG, "%s: batch strides of q / out / lse must hold %d heads", who, heads);
  return MLA_OK;
}

int mla_decode_split_bf16(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv_pool,
                          int64_t kv_row_stride, int32_t num_pages, int32_t page_size, const int32_t* page_table,
                          int64_t pt_stride, const int32_t* seq_lens, int32_t batch, int32_t heads, float scale,
                          const int32_t* plan, int32_t num_ctas, void* ws_o, float* ws_lse, int32_t ws_slots,
                          void* out, int64_t out_stride_b, int64_t out_stride_h, float* lse,
                          int64_t lse_stride_b, void* stream) {
  const char* who = "mla_decode_split_bf16";
  if (batch < 0) return fail(MLA_ERR_INVALID_ARG, "%s: batch < 0", who);
  if (batch == 0) return ok();
  if (int rc = check_head_groups(who, heads, q_stride_b, q_stride_h, out_stride_b, out_stride_h, lse, lse_stride_b))
    return rc;
  for (int32_t h0 = 0; h0 < heads; h0 += kHeadGroup) {
    const HeadGroup g = head_group(h0, heads, ws_slots, q, q_stride_h, static_cast<__bf16*>(ws_o), ws_lse, out, out_stride_h, lse);
    mla::DecodeParams p;
    if (int rc = decode_params(who, g.q, q_stride_b, q_stride_h, kv_pool, kv_row_stride, num_pages, page_size,
                               page_table, pt_stride, seq_lens, batch, g.heads, scale, plan, num_ctas, g.ws_o,
                               g.ws_lse, ws_slots, g.out, out_stride_b, out_stride_h, g.lse, lse_stride_b, &p))
      return rc;
    if (int rc = hip_status(mla::launch_decode(p, (hipStream_t)stream), "mla_decode_split_bf16 launch")) return rc;
  }
  return ok();
}

int mla_decode_bf16(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv_pool,
                    int64_t kv_row_stride, int32_t num_pages, int32_t page_size, const int32_t* page_table,
                    int64_t pt_stride, const int32_t* seq_lens, int32_t batch, int32_t heads, float scale,
                    const int32_t* plan, int32_t num_ctas, void* ws_o, float* ws_lse, int32_t ws_slots,
                    void* out, int64_t out_stride_b, int64_t out_stride_h, float* lse, int64_t lse_stride_b,
                    void* stream) {
  return mla::decode_split_merge("mla_decode_bf16", q, q_stride_b, q_stride_h, kv_pool, kv_row_stride, num_pages,
                                 page_size, page_table, pt_stride, seq_lens, batch, heads, scale, plan, num_ctas,
                                 static_cast<__bf16*>(ws_o), ws_lse, ws_slots, out, out_stride_b, out_stride_h, lse, lse_stride_b, stream);
}

}  // extern "C"

namespace mla {

int current_device_cus() {
  static std::atomic<int> cus_of[64];  // zero-initialised; a value is written once, the same by every writer
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  int cus = dev < 64 ? cus_of[dev].load(std::memory_order_relaxed) : 0;
  if (cus <= 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (dev < 64) cus_of[dev].store(cus, std::memory_order_relaxed);
  }
  return cus;
}

int api_error(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int decode_split_merge(const char* who, const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv_pool,
                       int64_t kv_row_stride, int32_t num_pages, int32_t page_size, const int32_t* page_table,
                       int64_t pt_stride, const int32_t* seq_lens, int32_t batch, int32_t heads, float scale,
                       const int32_t* plan, int32_t num_ctas, __bf16* ws_o, float* ws_lse, int32_t ws_slots, void* out,
                       int64_t out_stride_b, int64_t out_stride_h, float* lse, int64_t lse_stride_b, void* stream) {
  if (batch < 0) return fail(MLA_ERR_INVALID_ARG, "%s: batch < 0", who);
  if (batch == 0) return ok();
  if (int rc = check_head_groups(who, heads, q_stride_b, q_stride_h, out_stride_b, out_stride_h, lse, lse_stride_b))
    return rc;
  for (int32_t h0 = 0; h0 < heads; h0 += kHeadGroup) {
    const HeadGroup g = head_group(h0, heads, ws_slots, q, q_stride_h, ws_o, ws_lse, out, out_stride_h, lse);
    mla::DecodeParams p;
    if (int rc = decode_params(who, g.q, q_stride_b, q_stride_h, kv_pool, kv_row_stride, num_pages, page_size,
                               page_table, pt_stride, seq_lens, batch, g.heads, scale, plan, num_ctas, g.ws_o,
                               g.ws_lse, ws_slots, g.out, out_stride_b, out_stride_h, g.lse, lse_stride_b, &p))
      return rc;
    hipError_t e = mla::launch_decode(p, (hipStream_t)stream);
    if (e != hipSuccess) return hip_status(e, "decode split launch");
    const mla::MergeParams m = merge_params(g.ws_o, g.ws_lse, ws_slots, plan + 4 * (int64_t)num_ctas, batch, g.heads,
                                            1, g.out, out_stride_b, out_stride_h, g.lse, lse_stride_b);
    if (int rc = hip_status(mla::launch_merge(m, (hipStream_t)stream), "decode merge launch")) return rc;
  }
  return ok();
}

}  // namespace mla

extern "C" {

int mla_decode_merge_f32(const void* ws_o, const float* ws_lse, int32_t ws_slots, const int32_t* req_info,
                         int32_t batch, int32_t heads, int32_t single_piece_final, void* out, int64_t out_stride_b,
                         int64_t out_stride_h, float* lse, int64_t lse_stride_b, void* stream) {
  const char* who = "mla_decode_merge_f32";
  if (batch < 0 || heads < 1 || ws_slots < 0) return fail(MLA_ERR_INVALID_ARG, "%s: invalid sizes", who);
  if (batch == 0) return ok();
  if (req_info == nullptr || (ws_slots > 0 && (ws_o == nullptr || ws_lse == nullptr)))
    return fail(MLA_ERR_INVALID_ARG, "%s: null pointer", who);
  if (ws_o != nullptr && !aligned(ws_o, 16)) return fail(MLA_ERR_INVALID_ARG, "%s: ws_o must be 16-byte aligned", who);
  if (int rc = check_out(out, out_stride_b, out_stride_h, lse, lse_stride_b, heads, who)) return rc;
  for (int32_t h0 = 0; h0 < heads; h0 += kHeadGroup) {  // the workspace holds one [slots, group, 512] block per group
    const HeadGroup g = head_group(h0, heads, ws_slots, nullptr, 0, static_cast<__bf16*>(const_cast<void*>(ws_o)),
                                   const_cast<float*>(ws_lse), out, out_stride_h, lse);
    const mla::MergeParams m = merge_params(g.ws_o, g.ws_lse, ws_slots, req_info, batch, g.heads,
                                            single_piece_final ? 1 : 0, g.out, out_stride_b, out_stride_h, g.lse,
                                            lse_stride_b);
    if (int rc = hip_status(mla::launch_merge(m, (hipStream_t)stream), "mla_decode_merge_f32 launch")) return rc;
  }
  return ok();
}

// Shared checks and launch of the prefill entry points; K/V rows as in mla::PrefillParams.
static int prefill_launch(const char* who, const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_nope,
                          int64_t k_row_stride, int64_t k_head_stride, const void* k_rope, int64_t k_rope_head_stride,
                          const void* v, int64_t v_row_stride, int64_t v_head_stride, int32_t num_pages,
                          int32_t page_size, const int32_t* page_table, int64_t pt_stride, const int32_t* cu_seqlens_q,
                          const int32_t* seq_lens_k, int32_t batch, int32_t total_q, int32_t heads, float scale,
                          void* out, int64_t out_stride_t, int64_t out_stride_h, float* lse, int64_t lse_stride_t,
                          void* stream) {
  if (batch < 0 || total_q < 0 || heads < 1)
    return fail(MLA_ERR_INVALID_ARG, "%s: batch %d, total_q %d, heads %d", who, batch, total_q, heads);
  if (batch == 0 || total_q == 0) return ok();
  if (q == nullptr || k_nope == nullptr || k_rope == nullptr || v == nullptr || page_table == nullptr ||
      cu_seqlens_q == nullptr || seq_lens_k == nullptr || out == nullptr)
    return fail(MLA_ERR_INVALID_ARG, "%s: null pointer", who);
  if (!is_pow2(page_size) || page_size < 64)
    return fail(MLA_ERR_UNSUPPORTED, "%s: page_size %d must be a power of two >= 64", who, page_size);
  if (num_pages < 1 || pt_stride < 1) return fail(MLA_ERR_INVALID_ARG, "%s: num_pages / pt_stride < 1", who);
  if (!aligned(q, 16) || !aligned(k_nope, 16) || !aligned(k_rope, 16) || !aligned(v, 16) || !aligned(out, 8))
    return fail(MLA_ERR_INVALID_ARG, "%s: q/k/v must be 16-byte and out 8-byte aligned", who);
  if (q_stride_t % 8 || q_stride_h % 8 || q_stride_h < mla::kPrefillQkDim)
    return fail(MLA_ERR_INVALID_ARG, "%s: q strides (%lld, %lld) must be multiples of 8 with head stride >= 192", who,
                (long long)q_stride_t, (long long)q_stride_h);
  if (k_row_stride % 8 || k_head_stride % 8 || k_rope_head_stride % 8 || v_row_stride % 8 || v_head_stride % 8 ||
      k_head_stride < 0 || k_rope_head_stride < 0 || v_head_stride < 0)
    return fail(MLA_ERR_INVALID_ARG, "%s: k/v strides must be non-negative multiples of 8", who);
  if (k_row_stride < (heads - 1) * k_head_stride + 128 || v_row_stride < (heads - 1) * v_head_stride + mla::kPrefillVDim)
    return fail(MLA_ERR_INVALID_ARG, "%s: k/v row strides (%lld, %lld) must hold %d heads", who,
                (long long)k_row_stride, (long long)v_row_stride, heads);
  // the rope dims are addressed relative to the same head's nope dims, within 2 GiB after them
  const int64_t d0 = static_cast<const char*>(k_rope) - static_cast<const char*>(k_nope);
  const int64_t dh = 2 * (k_rope_head_stride - k_head_stride);
  const int64_t d_first = d0, d_last = d0 + (int64_t)(heads - 1) * dh;
  if (std::min(d_first, d_last) < 256 || std::max(d_first, d_last) >= ((int64_t)1 << 31) - 64 * k_row_stride)
    return fail(MLA_ERR_UNSUPPORTED,
                "%s: the rope dims of every head must lie between 256 bytes and 2 GiB after its nope dims", who);
  if ((int64_t)page_size * k_row_stride * 2 > (int64_t)UINT32_MAX ||
      (int64_t)page_size * v_row_stride * 2 > (int64_t)UINT32_MAX)
    return fail(MLA_ERR_UNSUPPORTED, "%s: one page of k/v rows exceeds 4 GiB", who);
  if (out_stride_t % 4 || out_stride_h % 4 || out_stride_h < mla::kPrefillVDim)
    return fail(MLA_ERR_INVALID_ARG, "%s: out strides (%lld, %lld) must be multiples of 4 with head stride >= 128",
                who, (long long)out_stride_t, (long long)out_stride_h);
  if (lse != nullptr && lse_stride_t < heads)
    return fail(MLA_ERR_INVALID_ARG, "%s: lse_stride_t %lld < heads", who, (long long)lse_stride_t);
  if (!(scale > 0.f) || !isfinite(scale)) return fail(MLA_ERR_INVALID_ARG, "%s: bad scale", who);
  mla::PrefillParams p;
  p.q = static_cast<const __bf16*>(q);
  p.q_stride_t = q_stride_t;
  p.q_stride_h = q_stride_h;
  p.k = static_cast<const __bf16*>(k_nope);
  p.k_row_stride = k_row_stride;
  p.k_head_stride = k_head_stride;
  p.k_rope_delta0 = d0;
  p.k_rope_delta_h = dh;
  p.v = static_cast<const __bf16*>(v);
  p.v_row_stride = v_row_stride;
  p.v_head_stride = v_head_stride;
  p.num_pages = num_pages;
  p.log2_ps = ilog2(page_size);
  p.page_table = page_table;
  p.pt_stride = pt_stride;
  p.cu_seqlens_q = cu_seqlens_q;
  p.seq_lens_k = seq_lens_k;
  p.batch = batch;
  p.heads = heads;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.out = static_cast<__bf16*>(out);
  p.out_stride_t = out_stride_t;
  p.out_stride_h = out_stride_h;
  p.out_16b = aligned(out, 16) && out_stride_t % 8 == 0 && out_stride_h % 8 == 0;
  p.lse = lse;
  p.lse_stride_t = lse_stride_t;
  return hip_status(mla::launch_prefill(p, total_q, (hipStream_t)stream), who);
}

int mla_prefill_bf16(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_pool, int64_t k_row_stride,
                     const void* v_pool, int64_t v_row_stride, int32_t num_pages, int32_t page_size,
                     const int32_t* page_table, int64_t pt_stride, const int32_t* cu_seqlens_q,
                     const int32_t* seq_lens_k, int32_t batch, int32_t total_q, int32_t heads, float scale, void* out,
                     int64_t out_stride_t, int64_t out_stride_h, float* lse, int64_t lse_stride_t, void* stream) {
  const char* who = "mla_prefill_bf16";
  if (heads >= 1 && (k_row_stride < (int64_t)heads * mla::kPrefillQkDim || v_row_stride < (int64_t)heads * mla::kPrefillVDim))
    return fail(MLA_ERR_INVALID_ARG, "%s: k/v row strides (%lld, %lld) must hold %d heads", who,
                (long long)k_row_stride, (long long)v_row_stride, heads);
  const void* k_rope = k_pool == nullptr ? nullptr : static_cast<const __bf16*>(k_pool) + 128;
  return prefill_launch(who, q, q_stride_t, q_stride_h, k_pool, k_row_stride, mla::kPrefillQkDim, k_rope,
                        mla::kPrefillQkDim, v_pool, v_row_stride, mla::kPrefillVDim, num_pages, page_size, page_table,
                        pt_stride, cu_seqlens_q, seq_lens_k, batch, total_q, heads, scale, out, out_stride_t,
                        out_stride_h, lse, lse_stride_t, stream);
}

int mla_prefill_strided_bf16(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_nope,
                             int64_t k_row_stride, int64_t k_head_stride, const void* k_rope, int64_t k_rope_head_stride,
                             const void* v, int64_t v_row_stride, int64_t v_head_stride, int32_t num_pages,
                             int32_t page_size, const int32_t* page_table, int64_t pt_stride,
                             const int32_t* cu_seqlens_q, const int32_t* seq_lens_k, int32_t batch, int32_t total_q,
                             int32_t heads, float scale, void* out, int64_t out_stride_t, int64_t out_stride_h,
                             float* lse, int64_t lse_stride_t, void* stream) {
  return prefill_launch("mla_prefill_strided_bf16", q, q_stride_t, q_stride_h, k_nope, k_row_stride, k_head_stride,
                        k_rope, k_rope_head_stride, v, v_row_stride, v_head_stride, num_pages, page_size, page_table,
                        pt_stride, cu_seqlens_q, seq_lens_k, batch, total_q, heads, scale, out, out_stride_t,
                        out_stride_h, lse, lse_stride_t, stream);
}

int mla_rmsnorm_bf16(const void* x, int64_t x_row_stride, const void* weight, int32_t rows, int32_t n, float eps,
                     void* out, int64_t out_row_stride, void* stream) {
  const char* who = "mla_rmsnorm_bf16";
  if (rows < 0 || n <= 0 || n % 8 != 0) return fail(MLA_ERR_INVALID_ARG, "%s: rows %d, n %d (n a positive multiple of 8)", who, rows, n);
  if (rows == 0) return ok();
  if (x == nullptr || weight == nullptr || out == nullptr) return fail(MLA_ERR_INVALID_ARG, "%s: null pointer", who);
  if (!rows_ok(x, x_row_stride, n) || !rows_ok(out, out_row_stride, n) || !aligned(weight, 16))
    return fail(MLA_ERR_INVALID_ARG, "%s: rows must be 16-byte aligned with strides multiples of 8 and >= n", who);
  return hip_status(mla::launch_rmsnorm(x, x_row_stride, weight, out, out_row_stride, rows, n, eps, (hipStream_t)stream),
                    "mla_rmsnorm_bf16 launch");
}

int mla_latent_rows_bf16(const void* kv, int64_t kv_row_stride, const void* norm_weight, const int32_t* positions,
                         const float* cos_sin, int32_t max_position, int32_t rows, float eps, int32_t interleaved,
                         void* out, int64_t out_row_stride, void* stream) {
  const char* who = "mla_latent_rows_bf16";
  if (rows < 0 || max_position <= 0) return fail(MLA_ERR_INVALID_ARG, "%s: rows %d, max_position %d", who, rows, max_position);
  if (rows == 0) return ok();
  if (kv == nullptr || norm_weight == nullptr || positions == nullptr || cos_sin == nullptr || out == nullptr)
    return fail(MLA_ERR_INVALID_ARG, "%s: null pointer", who);
  if (!rows_ok(kv, kv_row_stride, mla::kKvDim) || !rows_ok(out, out_row_stride, mla::kKvDim) || !aligned(norm_weight, 16))
    return fail(MLA_ERR_INVALID_ARG, "%s: rows must be 16-byte aligned with strides multiples of 8 and >= 576", who);
  return hip_status(mla::launch_latent_rows(kv, kv_row_stride, norm_weight, positions, cos_sin, max_position, out,
                                            out_row_stride, rows, eps, interleaved, (hipStream_t)stream),
                    "mla_latent_rows_bf16 launch");
}

int mla_qkv_a_rows_bf16(void* qkv, int64_t qkv_row_stride, int32_t q_rank, const void* q_norm_weight,
                        const void* kv_norm_weight, const int32_t* positions, const float* cos_sin,
                        int32_t max_position, int32_t rows, float eps, int32_t interleaved, void* latent_out,
                        int64_t latent_row_stride, void* stream) {
  const char* who = "mla_qkv_a_rows_bf16";
  if (rows < 0 || max_position <= 0 || q_rank <= 0 || q_rank % 8 != 0)
    return fail(MLA_ERR_INVALID_ARG, "%s: rows %d, max_position %d, q_rank %d (a positive multiple of 8)", who, rows,
                max_position, q_rank);
  if (rows == 0) return ok();
  if (qkv == nullptr || q_norm_weight == nullptr || kv_norm_weight == nullptr || positions == nullptr ||
      cos_sin == nullptr || latent_out == nullptr)
    return fail(MLA_ERR_INVALID_ARG, "%s: null pointer", who);
  if (!rows_ok(qkv, qkv_row_stride, (int64_t)q_rank + mla::kKvDim) || !rows_ok(latent_out, latent_row_stride, mla::kKvDim) ||
      !aligned(q_norm_weight, 16) || !aligned(kv_norm_weight, 16))
    return fail(MLA_ERR_INVALID_ARG, "%s: rows must be 16-byte aligned with strides multiples of 8 holding q_rank + 576",
                who);
  return hip_status(mla::launch_qkv_a_rows(qkv, qkv_row_stride, q_rank, q_norm_weight, kv_norm_weight, positions,
                                           cos_sin, max_position, latent_out, latent_row_stride, rows, eps, interleaved,
                                           (hipStream_t)stream),
                    "mla_qkv_a_rows_bf16 launch");
}

int mla_q_rope_bf16(const void* q, int64_t q_stride_t, int64_t q_stride_h, int32_t tokens, int32_t heads,
                    const int32_t* positions, const float* cos_sin, int32_t max_position, int32_t interleaved,
                    void* pe_out, int64_t pe_stride_t, int64_t pe_stride_h, void* nope_out, int64_t nope_stride_t,
                    int64_t nope_stride_h, void* stream) {
  const char* who = "mla_q_rope_bf16";
  if (tokens < 0 || heads <= 0 || max_position <= 0)
    return fail(MLA_ERR_INVALID_ARG, "%s: tokens %d, heads %d, max_position %d", who, tokens, heads, max_position);
  if (tokens == 0) return ok();
  if (q == nullptr || positions == nullptr || cos_sin == nullptr || pe_out == nullptr)
    return fail(MLA_ERR_INVALID_ARG, "%s: null pointer", who);
  if (!aligned(q, 16) || q_stride_t % 8 || q_stride_h % 8 || q_stride_h < 192 || q_stride_t < heads * q_stride_h)
    return fail(MLA_ERR_INVALID_ARG, "%s: q must be 16-byte aligned, strides multiples of 8 holding %d heads of 192",
                who, heads);
  if (!aligned(pe_out, 16) || pe_stride_t % 8 || pe_stride_h % 8 || pe_stride_h < 64 || pe_stride_t < heads * pe_stride_h)
    return fail(MLA_ERR_INVALID_ARG,
                "%s: pe_out must be 16-byte aligned, strides (%lld, %lld) multiples of 8 holding %d heads of 64", who,
                (long long)pe_stride_t, (long long)pe_stride_h, heads);
  if (nope_out != nullptr && (!aligned(nope_out, 16) || nope_stride_t % 8 || nope_stride_h % 8 ||
                              (nope_stride_t < nope_stride_h ? nope_stride_t : nope_stride_h) < 128))
    return fail(MLA_ERR_INVALID_ARG, "%s: nope_out must be 16-byte aligned with strides multiples of 8 and >= 128",
                who);
  return hip_status(mla::launch_q_rope(q, q_stride_t, q_stride_h, tokens, heads, positions, cos_sin, max_position,
                                       interleaved, pe_out, pe_stride_t, pe_stride_h, nope_out, nope_stride_t,
                                       nope_stride_h, (hipStream_t)stream),
                    "mla_q_rope_bf16 launch");
}

}  // extern "C"
