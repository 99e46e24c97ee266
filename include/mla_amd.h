/*
 * mla_amd.h -- C ABI of the MI355X (gfx950) MLA attention library
 * (libmla_amd.so, built from mini-sglang_amd/csrc).
 *
 * Conventions
 *   - Every entry point returns int: MLA_OK (0) on success, otherwise an
 *     MLA_ERR_* code; mla_last_error() then returns a thread-local message.
 *     This mirrors the reference's host::RuntimeCheck / PanicError, which
 *     carry a file:line message (python/minisgl/kernel/csrc/include/minisgl/
 *     utils.h:40-93) and surface as Python exceptions.
 *   - Device buffers are plain pointers; strides are in ELEMENTS of the
 *     buffer's own type unless the name says _bytes.
 *   - `stream` is a hipStream_t (NULL = legacy default stream). No entry
 *     point synchronises or allocates device memory, so every launch is
 *     capturable into a HIP graph; the caller owns all buffers, including the
 *     split-KV workspace, as the reference's backends own theirs
 *     (python/minisgl/attention/fi.py:90-92) -- except mla_decode_bf16_noalloc,
 *     whose partials use the library's fixed device scratch instead.
 *   - bf16 tensors are raw uint16 bit patterns (bfloat16).
 */
#ifndef MLA_AMD_H
#define MLA_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MLA_OK = 0,
  MLA_ERR_INVALID_ARG = 1, /* shape, stride, alignment or range check failed */
  MLA_ERR_HIP = 2,         /* a HIP runtime call failed (message has hipGetErrorString) */
  MLA_ERR_UNSUPPORTED = 3  /* valid request outside what the kernels implement */
};

/* Latent KV row width of absorbed MLA: 512 latent (the value) + 64 rope. */
#define MLA_KV_DIM 576
#define MLA_V_DIM 512
/* Decode work is planned in blocks of this many tokens. */
#define MLA_PLAN_BLOCK 64
/* Entries per CTA in a decode plan's cta_ranges and per request in req_info. */
#define MLA_PLAN_CTA_INTS 4
#define MLA_PLAN_REQ_INTS 3
/* A decode plan gives one CTA at most this many plan blocks and requests. */
#define MLA_PLAN_MAX_CTA_BLOCKS 512
#define MLA_PLAN_MAX_CTA_REQUESTS 128

/*
 * Split-KV partial outputs (the decode workspace ws_o): one row of 512 bf16 per (slot, head), the
 * piece's normalised output, in chunk order: 16-byte chunk c (elements 8c .. 8c+7) holds value dims
 * 32 (c / 4) + 4 (c % 4) + {0, 1, 2, 3} and then 32 (c / 4) + 16 + 4 (c % 4) + {0, 1, 2, 3}. This is
 * the order the decode kernels' registers hold them in (one 16-byte store per chunk); only the
 * library's merge reads these rows. Their LSEs (ws_lse) are fp32 natural logs.
 */

/* Message for the last failed call on this thread ("" if none). */
const char *mla_last_error(void);

/* ABI version of this header (bumped on any signature change). */
int mla_abi_version(void);

/* Number of compute units of `device` (sizes decode plans). Host only. */
int mla_device_cu_count(int device, int32_t *out);

/*
 * Row scatter: cache[indices[i]] = x[i] for i < num_rows, row_bytes each.
 * Replaces StoreKernel<...>::run / store_kv_cache
 * (python/minisgl/kernel/csrc/jit/store.cu:25-53,55-121) behind
 * MHAKVCache.store_kv (python/minisgl/kvcache/mha_pool.py:45-56). Strides are
 * in bytes; row_bytes and both strides must be multiples of 16 and the
 * pointers 16-byte aligned. index_bits is 32 or 64. Indices must be distinct
 * (the reference's own test relies on the same, tests/kernel/test_store.py:20);
 * an index outside [0, cache_rows) is skipped rather than written.
 */
int mla_store_rows(void *cache, int64_t cache_rows, int64_t cache_row_stride_bytes,
                   const void *x, int64_t x_row_stride_bytes, const void *indices,
                   int32_t index_bits, int64_t num_rows, int64_t row_bytes, void *stream);

/*
 * Latent rows of every key of a prefill batch into 64-row scratch pages, the input of the per-head
 * decompression that lets chunked prefill run over a latent-only pool (the caller role of
 * python/minisgl/layers/attention.py:47-57 for MLA; the pool it reads replaces
 * python/minisgl/kvcache/mha_pool.py:10-68). Key j < seq_lens_k[b] of request b, pool row
 * page_table[b, j / page_size] * page_size + j % page_size of kv_pool ([num_pages, page_size, 576],
 * row stride kv_row_stride; page ids clamped into [0, num_pages)), goes to scratch row
 * r = 64 * seg_first[b] + j: its 512 latent dims to c_out[r, :] (row stride c_row_stride) and its 64
 * rope dims to rope_out[r, :] (row stride rope_row_stride); rows r >= out_rows are not written.
 * seg_page_table[b, i] = seg_first[b] + i for i < ceil(seq_lens_k[b] / 64) (row stride
 * seg_pt_stride >= max_seg_pages), so the scratch rows are 64-token pages under that table.
 * max_seg_pages >= ceil(seq_lens_k[b] / 64) for every b (keys past it are not copied). Any
 * power-of-two page_size (1 included); bit-exact.
 */
int mla_prefill_gather_bf16(const void *kv_pool, int64_t kv_row_stride, int32_t num_pages,
                            int32_t page_size, const int32_t *page_table, int64_t pt_stride,
                            const int32_t *seq_lens_k, const int32_t *seg_first, int32_t batch,
                            int32_t max_seg_pages, void *c_out, int64_t c_row_stride, void *rope_out,
                            int64_t rope_row_stride, int64_t out_rows, int32_t *seg_page_table,
                            int64_t seg_pt_stride, void *stream);

/*
 * Token table -> page table, bit-exact:
 *   out[b, j] = token_table[table_idx[b], j * page_size] / page_size
 * for j < ceil(max_seqlen_k / page_size). Replaces the slicing in
 * FlashAttentionBackend.prepare_metadata (python/minisgl/attention/fa.py:92-97,
 * identical in attention/trtllm.py:116-121). token_table rows are
 * Context.page_table rows (python/minisgl/core.py:103-104); max_seqlen_k must
 * not exceed token_table_cols, and a table_idx outside [0, token_table_rows)
 * is clamped into range.
 */
int mla_page_table_from_tokens(const int32_t *token_table, int32_t token_table_rows,
                               int32_t token_table_cols, int64_t token_table_stride,
                               const int32_t *table_idx, int32_t batch, int32_t max_seqlen_k,
                               int32_t page_size, int32_t *out, int64_t out_stride,
                               void *stream);

/*
 * Split-KV decode plan (host only, no GPU needed). Balances the requests'
 * MLA_PLAN_BLOCK-token blocks over `num_ctas` CTAs, each CTA taking one
 * contiguous range of (request, block) space. Plays the role of FlashInfer's
 * plan() in the reference's backend (python/minisgl/attention/fi.py:123-166).
 *   cta_ranges[num_ctas*4] : {req_begin, blk_begin, req_end, blk_end} (end exclusive)
 *   req_info[batch*3]      : {first_cta, num_pieces, slot_base}
 *   *num_slots             : partial-result slots the plan needs in the workspace
 * A piece touches at most max_piece_pages pages (<= 0: no limit; the kernels take pieces of
 * any length). A CTA's range holds at most MLA_PLAN_MAX_CTA_BLOCKS blocks and
 * MLA_PLAN_MAX_CTA_REQUESTS requests; a batch that num_ctas CTAs cannot hold within these
 * limits fails with MLA_ERR_UNSUPPORTED ("cannot hold"). A split request's pieces sit in
 * consecutive CTAs, and no CTA holds more than two pieces of split requests, so
 * *num_slots <= 2 * num_ctas. CTAs past the last one used get the empty range
 * {batch, 0, batch, 0}; a plan for n CTAs runs unchanged on a grid of m > n CTAs once its
 * cta_ranges are extended with such empty ranges (req_info then starts at m*4).
 */
int mla_decode_plan(const int32_t *seq_lens, int32_t batch, int32_t page_size,
                    int32_t num_ctas, int32_t max_piece_pages, int32_t *cta_ranges,
                    int32_t *req_info, int32_t *num_slots);

/*
 * Absorbed-MLA paged decode (one query token per request), bf16 in, fp32
 * accumulate, bf16 out plus fp32 natural-log LSE. Replaces the attention call
 * of BaseAttnBackend.forward (python/minisgl/attention/base.py:19-22;
 * FA template python/minisgl/attention/fa.py:48-65) for MLA.
 *   q        [batch, heads, 576]  strides (q_stride_b, q_stride_h), last dim contiguous
 *   kv_pool  [num_pages, page_size, 576] latent cache, row stride kv_row_stride
 *   page_table [batch, >= ceil(seq_len/page_size)] int32, row stride pt_stride
 *   seq_lens [batch] int32 (device_len, includes the token being decoded)
 *   plan     device copy of mla_decode_plan's cta_ranges followed by req_info
 *   ws_o     [ws_slots, heads, 512] bf16 (normalised partial outputs, chunk order above),
 *            ws_lse [ws_slots, heads] fp32
 *   out      [batch, heads, 512] strides (out_stride_b, out_stride_h)
 *   lse      [batch, heads] fp32 (row stride lse_stride_b) or NULL
 * heads is 1..1024: groups of at most 64 heads run one after another (each group reads the KV
 * again) and group g's partials occupy the workspace block [ws_slots, group heads, 512] that
 * starts at ws_o + ws_slots * 64 * g * 512 (ws_lse likewise), so a [ws_slots, heads, 512] buffer
 * holds them all; within a group, one wave per 16 heads (lanes past `heads` idle). page_size a power of
 * two; page ids outside [0, num_pages) are clamped into range.
 * Launches the split kernel on num_ctas CTAs, then the LSE merge kernel.
 */
int mla_decode_bf16(const void *q, int64_t q_stride_b, int64_t q_stride_h, const void *kv_pool,
                    int64_t kv_row_stride, int32_t num_pages, int32_t page_size,
                    const int32_t *page_table, int64_t pt_stride, const int32_t *seq_lens,
                    int32_t batch, int32_t heads, float scale, const int32_t *plan,
                    int32_t num_ctas, void *ws_o, float *ws_lse, int32_t ws_slots, void *out,
                    int64_t out_stride_b, int64_t out_stride_h, float *lse, int64_t lse_stride_b,
                    void *stream);

/*
 * The split step of mla_decode_bf16 alone (same arguments): requests covered
 * by one piece get their final bf16 output and LSE, split requests leave
 * normalised partials (bf16 outputs, fp32 LSE) in ws_o / ws_lse for mla_decode_merge_f32 with
 * single_piece_final = 1. No counterpart in the reference (its decode is one
 * opaque library call); it is the unit a sequence-sharded decode distributes.
 */
int mla_decode_split_bf16(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                          const void *kv_pool, int64_t kv_row_stride, int32_t num_pages,
                          int32_t page_size, const int32_t *page_table, int64_t pt_stride,
                          const int32_t *seq_lens, int32_t batch, int32_t heads, float scale,
                          const int32_t *plan, int32_t num_ctas, void *ws_o, float *ws_lse,
                          int32_t ws_slots, void *out, int64_t out_stride_b,
                          int64_t out_stride_h, float *lse, int64_t lse_stride_b, void *stream);

/*
 * mla_decode_bf16 without a workspace argument: the split-KV partials go to a fixed scratch array
 * inside the library (static device memory, one copy per GPU, held until the process ends) of
 * MLA_NOALLOC_MAX_SLOT_HEADS slot-heads: 32 MiB of bf16 partials + 128 KiB of fp32 LSEs.
 * No counterpart in the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc); it calls no
 * allocating routine. num_slots is the plan's slot count (mla_decode_plan's *num_slots); a plan
 * with num_slots * heads > MLA_NOALLOC_MAX_SLOT_HEADS is rejected with MLA_ERR_UNSUPPORTED. The
 * scratch is laid out for 2 * num_ctas slots (the most any plan over num_ctas CTAs uses) whenever
 * they fit, so a num_slots below the plan's real count cannot drop partials; if they do not fit
 * and num_slots is too small, the merge writes NaN for the requests whose slots fall outside. Every
 * call on one GPU shares that GPU's scratch: calls that overlap on one GPU (concurrent streams)
 * race. Nothing in the scratch must start at zero (the merge reads only slots the split kernel
 * of the same call wrote).
 */
#define MLA_NOALLOC_MAX_SLOT_HEADS 32768
int mla_decode_bf16_noalloc(const void *q, int64_t q_stride_b, int64_t q_stride_h,
                            const void *kv_pool, int64_t kv_row_stride, int32_t num_pages,
                            int32_t page_size, const int32_t *page_table, int64_t pt_stride,
                            const int32_t *seq_lens, int32_t batch, int32_t heads, float scale,
                            const int32_t *plan, int32_t num_ctas, int32_t num_slots, void *out,
                            int64_t out_stride_b, int64_t out_stride_h, float *lse,
                            int64_t lse_stride_b, void *stream);

/*
 * fp32 log-sum-exp merge of split-KV partials (bf16 ws_o in the chunk order above, fp32 ws_lse; the
 * merge step of
 * mla_decode_bf16). For request b with n = req_info[3b+1] pieces in slots
 * s = req_info[3b+2] .. +n-1:
 *   lse = ln sum_i exp(ws_lse[s_i]);  out = sum_i exp(ws_lse[s_i] - lse) * ws_o[s_i]
 * n == 0 writes out = 0, lse = -inf; slots outside [0, ws_slots) write NaN. With single_piece_final != 0 requests
 * with n == 1 are skipped (the split step already wrote them); otherwise
 * their one slot is converted like any other. More than 64 heads: the workspace holds one
 * [ws_slots, group heads, 512] block per 64-head group, as mla_decode_bf16 writes it.
 */
int mla_decode_merge_f32(const void *ws_o, const float *ws_lse, int32_t ws_slots,
                         const int32_t *req_info, int32_t batch, int32_t heads,
                         int32_t single_piece_final, void *out, int64_t out_stride_b,
                         int64_t out_stride_h, float *lse, int64_t lse_stride_b, void *stream);

/*
 * MLA chunked prefill (non-absorbed form), bf16 in, fp32 accumulate, bf16 out
 * plus fp32 natural-log LSE. Causal and bottom-right aligned over a paged
 * prefix: query i of request b (absolute position P_b + i, P_b = seq_lens_k[b]
 * - extend_b) attends keys j <= P_b + i. Replaces the prefill attention call
 * of BaseAttnBackend.forward (python/minisgl/attention/base.py:19-22; FA
 * template python/minisgl/attention/fa.py:48-65 -> flash_attn_with_kvcache,
 * fa.py:157-182) for MLA.
 *   q         [total_q, heads, 192] strides (q_stride_t, q_stride_h); request b owns
 *             rows cu_seqlens_q[b] .. cu_seqlens_q[b+1]-1
 *   k_pool    [num_pages, page_size, heads, 192], token row stride k_row_stride (>= heads*192)
 *   v_pool    [num_pages, page_size, heads, 128], token row stride v_row_stride (>= heads*128)
 *   page_table [batch, >= ceil(seq_lens_k[b]/page_size)] int32, row stride pt_stride
 *   cu_seqlens_q [batch+1], seq_lens_k [batch] int32 device arrays; the K/V of all
 *             seq_lens_k[b] tokens (prefix + extend) are already in the pools
 *   out       [total_q, heads, 128] strides (out_stride_t, out_stride_h)
 *   lse       [total_q, heads] fp32 (row stride lse_stride_t) or NULL
 * page_size is a power of two >= 64 (one 64-token key tile lies in one page);
 * page ids outside [0, num_pages) are clamped into range.
 */
int mla_prefill_bf16(const void *q, int64_t q_stride_t, int64_t q_stride_h, const void *k_pool,
                     int64_t k_row_stride, const void *v_pool, int64_t v_row_stride,
                     int32_t num_pages, int32_t page_size, const int32_t *page_table,
                     int64_t pt_stride, const int32_t *cu_seqlens_q, const int32_t *seq_lens_k,
                     int32_t batch, int32_t total_q, int32_t heads, float scale, void *out,
                     int64_t out_stride_t, int64_t out_stride_h, float *lse, int64_t lse_stride_t,
                     void *stream);

/*
 * mla_prefill_bf16 with the K and V rows anywhere (same semantics, same fixed kernel): the K row of
 * (token row r = page * page_size + offset, head h) is 128 nope dims at
 * k_nope + r * k_row_stride + h * k_head_stride followed, somewhere after them, by 64 rope dims at
 * k_rope + r * k_row_stride + h * k_rope_head_stride (k_rope_head_stride 0: one rope row per token,
 * shared by all heads, as MLA's k_pe is); the V row is 128 dims at v + r * v_row_stride +
 * h * v_head_stride. The rope dims of every head must lie 256 bytes to 2 GiB after its nope dims
 * (else MLA_ERR_UNSUPPORTED). mla_prefill_bf16 is the case k_head_stride = k_rope_head_stride =
 * 192, k_rope = k_pool + 128, v_head_stride = 128. The layout of the latent decompression
 * (mla_prefill_gather_bf16, then [k_nope | v] = c W_kvb^T per head) is
 * row = [head 0: k_nope 128 | v 128, head 1: ..., rope 64]: k_head_stride = v_head_stride = 256,
 * k_rope = k_nope + 256 * heads, k_rope_head_stride = 0, v = k_nope + 128. No counterpart in the
 * reference (its FA call reads one per-head K/V layout).
 */
int mla_prefill_strided_bf16(const void *q, int64_t q_stride_t, int64_t q_stride_h,
                             const void *k_nope, int64_t k_row_stride, int64_t k_head_stride,
                             const void *k_rope, int64_t k_rope_head_stride, const void *v,
                             int64_t v_row_stride, int64_t v_head_stride, int32_t num_pages,
                             int32_t page_size, const int32_t *page_table, int64_t pt_stride,
                             const int32_t *cu_seqlens_q, const int32_t *seq_lens_k, int32_t batch,
                             int32_t total_q, int32_t heads, float scale, void *out,
                             int64_t out_stride_t, int64_t out_stride_h, float *lse,
                             int64_t lse_stride_t, void *stream);

/*
 * The elementwise steps of the DeepSeek-V3 / Kimi-K2 MLA layer around the attention calls
 * (bf16 in and out, fp32 arithmetic; strides in elements, multiples of 8; 16-byte aligned rows).
 *
 * mla_rmsnorm_bf16: out[r] = x[r] / sqrt(mean(x[r]^2) + eps) * weight over n dims (n a multiple of
 * 8), rows r < rows; out == x is allowed. Replaces the RMSNorm op of the layer (the reference's
 * RMSNorm, python/minisgl/layers/norm.py, calls flashinfer's rmsnorm).
 */
int mla_rmsnorm_bf16(const void *x, int64_t x_row_stride, const void *weight, int32_t rows, int32_t n,
                     float eps, void *out, int64_t out_row_stride, void *stream);

/*
 * mla_latent_rows_bf16: the latent row of each new token from the kv_a projection
 * kv [rows, 576]: out[r][0:512] = rmsnorm(kv[r][0:512]) * norm_weight[512],
 * out[r][512:576] = RoPE of kv[r][512:576] at positions[r]. cos_sin is the fp32 table
 * [max_position, 64] (cosines of the 32 frequencies, then their sines; the layout of
 * python/minisgl/layers/rotary.py:22-31); interleaved != 0 rotates pairs (2i, 2i+1), else
 * (i, i + 32). Positions outside [0, max_position) are clamped into range. Replaces the norm +
 * RotaryEmbedding.forward pair (rotary.py:39-51) for MLA's shared rope key.
 */
int mla_latent_rows_bf16(const void *kv, int64_t kv_row_stride, const void *norm_weight,
                         const int32_t *positions, const float *cos_sin, int32_t max_position,
                         int32_t rows, float eps, int32_t interleaved, void *out, int64_t out_row_stride,
                         void *stream);

/*
 * mla_qkv_a_rows_bf16: both halves of the fused q_a / kv_a projection output in one launch,
 * qkv [rows, q_rank + 576] (row stride qkv_row_stride): qkv[r][0:q_rank] is normalised in place
 * (RMSNorm with q_norm_weight), and latent_out[r] = the latent row of qkv[r][q_rank:] as
 * mla_latent_rows_bf16 computes it. q_rank a multiple of 8.
 */
int mla_qkv_a_rows_bf16(void *qkv, int64_t qkv_row_stride, int32_t q_rank, const void *q_norm_weight,
                        const void *kv_norm_weight, const int32_t *positions, const float *cos_sin,
                        int32_t max_position, int32_t rows, float eps, int32_t interleaved, void *latent_out,
                        int64_t latent_row_stride, void *stream);

/*
 * mla_q_rope_bf16: queries q [tokens, heads, 192] (128 nope + 64 rope dims, strides
 * (q_stride_t, q_stride_h)): pe_out[t, h, 0:64] = RoPE of q[t, h, 128:192] at positions[t]
 * (pe_out may be q + 128 with q's strides: in place); if nope_out is not NULL,
 * nope_out[t, h, 0:128] = q[t, h, 0:128] with its own strides (e.g. head-major for the W_UK
 * absorption GEMM). RoPE conventions as mla_latent_rows_bf16. q, pe_out and nope_out are
 * 16-byte aligned with strides multiples of 8 elements. Replaces the query half of
 * RotaryEmbedding.forward (rotary.py:39-51).
 */
int mla_q_rope_bf16(const void *q, int64_t q_stride_t, int64_t q_stride_h, int32_t tokens, int32_t heads,
                    const int32_t *positions, const float *cos_sin, int32_t max_position,
                    int32_t interleaved, void *pe_out, int64_t pe_stride_t, int64_t pe_stride_h,
                    void *nope_out, int64_t nope_stride_t, int64_t nope_stride_h, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MLA_AMD_H */
