// mla_decode_bf16_noalloc: the decode entry point for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). The split-KV
// partials live in `scratch`, a fixed device array of this library; every call on a GPU shares
// that GPU's copy.
//
// In host code `scratch` names a host-side stand-in, not the device array: its device address is
// taken once per device with hipGetSymbolAddress (with that device current) and only that address
// is ever passed to kernels.
#include <mutex>

#include "../../include/mla_amd.h"
#include "mla_common.h"

namespace {

constexpr int64_t kMaxSlotHeads = MLA_NOALLOC_MAX_SLOT_HEADS;
constexpr int64_t kPartialBytes = kMaxSlotHeads * MLA_V_DIM * 2;  // bf16 partial outputs
constexpr int64_t kScratchBytes = kPartialBytes + kMaxSlotHeads * 4;  // + fp32 LSEs
static_assert(kPartialBytes % 256 == 0, "LSE block alignment");

// [slot, head, 512] bf16 partial outputs (chunk order of mla_amd.h), then [slot, head] fp32 LSEs
// (slot * heads <= kMaxSlotHeads)
static __device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's `scratch`, looked up on the first call on each device.
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return mla::api_error(MLA_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return mla::api_error(MLA_ERR_UNSUPPORTED, "mla_decode_bf16_noalloc: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return mla::api_error(MLA_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MLA_OK;
}

}  // namespace

extern "C" {

int mla_decode_bf16_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* kv_pool,
                            int64_t kv_row_stride, int32_t num_pages, int32_t page_size, const int32_t* page_table,
                            int64_t pt_stride, const int32_t* seq_lens, int32_t batch, int32_t heads, float scale,
                            const int32_t* plan, int32_t num_ctas, int32_t num_slots, void* out,
                            int64_t out_stride_b, int64_t out_stride_h, float* lse, int64_t lse_stride_b,
                            void* stream) {
  const char* who = "mla_decode_bf16_noalloc";
  if (num_slots < 0 || heads < 1)
    return mla::api_error(MLA_ERR_INVALID_ARG, "%s: num_slots %d, heads %d", who, num_slots, heads);
  if ((int64_t)num_slots * heads > kMaxSlotHeads)
    return mla::api_error(MLA_ERR_UNSUPPORTED,
                          "%s: the plan's %d partial slots x %d heads exceed the fixed scratch of %lld slot-heads; "
                          "use mla_decode_bf16 with a workspace",
                          who, num_slots, heads, (long long)kMaxSlotHeads);
  if (num_ctas < 1) return mla::api_error(MLA_ERR_INVALID_ARG, "%s: num_ctas must be >= 1", who);
  void* base = nullptr;
  if (int rc = scratch_address(&base)) return rc;
  // A plan over num_ctas CTAs uses at most 2 * num_ctas slots (only a CTA's first and last piece can
  // be part of a split request). Lay the scratch out for that many whenever they fit, so a num_slots
  // below the plan's real count cannot make the split kernel drop partials; otherwise the merge
  // flags slots past num_slots with NaN.
  const int64_t most = 2 * (int64_t)num_ctas;
  const int32_t ws_slots = most * heads <= kMaxSlotHeads ? (int32_t)most : num_slots;
  // every slot the merge reads is written by the split kernel of the same call: nothing to clear
  __bf16* ws_o = static_cast<__bf16*>(base);
  float* ws_lse = reinterpret_cast<float*>(static_cast<char*>(base) + kPartialBytes);
  return mla::decode_split_merge(who, q, q_stride_b, q_stride_h, kv_pool, kv_row_stride, num_pages, page_size,
                                 page_table, pt_stride, seq_lens, batch, heads, scale, plan, num_ctas, ws_o, ws_lse,
                                 ws_slots, out, out_stride_b, out_stride_h, lse, lse_stride_b, stream);
}

}  // extern "C"
