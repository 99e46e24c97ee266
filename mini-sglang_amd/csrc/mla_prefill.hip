// Chunked MLA prefill (non-absorbed form), causal and bottom-right aligned over
// a paged prefix: query i of a request with prefix P attends keys j <= P + i.
// Per head: q [192] (128 nope + 64 rope), K [192], V [128]. A K row is read from two places: its
// 128 nope dims and, a per-head byte offset after them, its 64 rope dims (the per-head page layout
// [.., H, 192] has them adjacent; the latent-decompression scratch keeps one rope copy per token,
// shared by all heads, after the heads' [k_nope | v] blocks).
//
// One CTA per (request, 256 query rows, group of HPC = 1 or 2 heads), the heads of a group run one
// after the other (the launcher takes two when one-head CTAs would fill the GPU eight times over:
// the second head reuses the request lookup and the page-table sources, and its queries load
// during the first head's output); 8 waves x 32 query rows, two waves per SIMD (the kernel is a
// template on QS, the 32-row query sub-blocks per wave; QS = 2, 4 waves x 64 rows with one wave
// per SIMD, measured the same with a barrier per step and is kept buildable; with the current ring
// it spills and runs ~12 % slower).
//  * Keys stream in stages of 32 tokens (K 12 KB + V 8 KB) through a 7-stage
//    LDS ring filled by 16-byte DMA loads: waves 0-3 load the K tile, waves 4-7 the V tile (one
//    wave of each per SIMD); loads run four stages ahead and the CTA synchronises once per two
//    steps. K rows (384 B) are stored with the
//    16-byte chunk index XOR ((token >> 1) & 7) inside each 8-chunk group, V rows
//    (256 B) with XOR 4 * (token & 3): the K operand reads (ds_read_b128) and the
//    transposing V reads (ds_read_b64_tr_b16) are then bank-conflict free, as
//    rocprof's SQ_LDS_BANK_CONFLICT reads them on this part (XOR (token & 7) and
//    XOR 2 * (token & 3) leave both 2-way conflicted).
//  * S^T[32 keys x 32 queries] = K . Q^T and O^T[128 dims x 32 queries] +=
//    V^T . P^T on 32x32x16 bf16 MFMA; queries (the B operand) and O stay in
//    registers for the whole head.
//  * Software pipeline over the stages: step j issues the value MFMAs of stage
//    j-1 and the score MFMAs of stage j+1 while the vector ALU runs the online
//    softmax of stage j, the two instruction streams interleaved slot by slot
//    (one MFMA per slot). Every step of a wave runs this same body: a diagonal
//    step first masks its stage's scores, the first step sets the reference,
//    and the last step's score pass works on a fully masked stage.
//  * Online softmax in the log2 domain against a lazy row reference: the exact
//    max of the wave's first stage, moved (with O and l rescaled, and the
//    stage redone) only when a stage's numerators sum past 2^32.
//  * The head groups of one (request, query block) are consecutive CTAs, so the
//    query blocks of one group are H / HPC CTAs apart and, with that a multiple
//    of 8, land on the same XCD and share its L2 for K/V.
#include <type_traits>

#include "mla_common.h"
#include "mla_device.h"

namespace mla {
namespace {

typedef float f32x16_t __attribute__((__vector_size__(64)));

constexpr int kPStage = 32;                             // keys per stage
constexpr int kPKRowBytes = kPrefillQkDim * 2;          // 384
constexpr int kPVRowBytes = kPrefillVDim * 2;           // 256
constexpr int kPKBytes = kPStage * kPKRowBytes;         // 12288
constexpr int kPVBytes = kPStage * kPVRowBytes;         // 8192
constexpr int kPStageBytes = kPKBytes + kPVBytes;       // 20480
// Steps between CTA barriers (1 or 2). Step j loads stage j + kPDist; a barrier step makes
// stages up to j + kPSync visible to every wave, and the ring has kPSync - 1 more stages than one
// barrier per step needs, so that a wave one step ahead of another never refills a stage the other
// still reads.
constexpr int kPSync = 2;
constexpr int kPDist = 4;
constexpr int kPStages = kPDist + 1 + kPSync;  // ring stages
// the loop over the steps is unrolled by this: whole rounds of the ring, and an even count (the
// score and numerator registers alternate by step parity)
constexpr int kPUnroll = kPStages % 2 == 0 ? kPStages : 2 * kPStages;
// Wave-wide 1 KiB DMA loads of a stage: 12 of the K tile and 8 of the V tile; load i of a tile
// lands at i KiB. With QS = 2 (4 waves) wave w issues K loads w + 4k (k < 3) and V loads w + 4k
// (k < 2); with QS = 1 (8 waves) waves 0-3 issue the K loads (w + 4k, k < 3) and waves 4-7 the V
// loads ((w - 4) + 4k, k < 2).
constexpr int kPKDma = 3;  // K loads of a wave that issues K loads
constexpr int kPVDma = 2;  // V loads of a wave that issues V loads
constexpr int kPMaxGroups = 1024;  // stage sources of a CTA staged in LDS (else computed per stage)

// ---- the softmax of one stage as a list of micro-operations, spread over the MFMA slots of a
// pipelined step in proportion to their cost (~4-cycle units; next to running MFMAs a vector
// instruction costs ~8 cycles and exp2 ~11). QS = query sub-blocks of 32 rows per wave: 1 (8 waves
// of 32 rows, two per SIMD) or 2 (4 waves of 64 rows, one per SIMD). A step has 8 QS value MFMAs
// + 12 QS score MFMAs (its slots) and 24 QS softmax micro-ops: for u = 3 QS k + r (pair k of a
// lane's 16 scores), r < 2 QS is the exp2 of score 2k + r % 2 of sub-block r / 2 against the row
// reference, r >= 2 QS adds sub-block r - 2 QS's pair to the row sum and packs it to bf16. No exp2
// result is used by the next instruction (that would cost a wait state).
template <int QS> constexpr int kSlots = 20 * QS;
// LDS operand reads run ahead of their MFMAs: K operand ks + kAK is read in the slot of K operand
// ks, V^T operand st + kAV in the slot of V^T operand st (the first kAV by the step before)
constexpr int kAK = 4, kAV = 3;
static_assert(kAK >= 3 && kAK <= 8 && kAV >= 1 && kAV <= 12, "read-ahead outside the step's slots");
template <int QS> constexpr int kUops = 24 * QS;
template <int QS> constexpr int uop_weight(int u) { return u % (3 * QS) < 2 * QS ? 5 : 6; }
template <int QS> constexpr int uop_total() {
  int t = 0;
  for (int u = 0; u < kUops<QS>; ++u) t += uop_weight<QS>(u);
  return t;
}
template <int QS> constexpr int uop_slot(int u) {
  int t = 0;
  for (int v = 0; v < u; ++v) t += uop_weight<QS>(v);
  return t * kSlots<QS> / uop_total<QS>();
}
// The row reference m (log2 domain) is the exact max of the wave's first stage and moves only when
// a stage's numerators sum past 2^32 (a score 32 above m, in log2 units) or overflow: then that
// stage is redone against its exact max. fp32 keeps its relative precision at any scale, so the
// lagging reference costs no accuracy.
constexpr float kPLazyMax = 4294967296.0f;

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ int kswz(int c, int t) { return (c & ~7) | ((c & 7) ^ ((t >> 1) & 7)); }
__device__ __forceinline__ int vswz(int c, int t) { return c ^ (4 * (t & 3)); }
// max / sum of a lane's value with lane ^ 32 (v_permlane32_swap, no LDS traffic)
__device__ __forceinline__ float max_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// S^T += K . Q^T. A chain accumulates in place; its first k-step starts from zero. With QS = 2
// the query operand is read straight from accumulation registers (the wave holds 512 registers
// per lane, split evenly), through assembly the compiler's hazard tracking does not see; with
// QS = 1 (256 per lane) everything lives in the vector registers and the compiler places the
// MFMAs and their wait states.
template <int QS>
__device__ __forceinline__ void mfma_qk_first(f32x16_t& d, const bf16x8& k, const bf16x8& q) {
  if constexpr (QS == 2) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(k), "a"(q));
  else d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k, q, f32x16_t{}, 0, 0, 0);
}
template <int QS>
__device__ __forceinline__ void mfma_qk(f32x16_t& d, const bf16x8& k, const bf16x8& q) {
  if constexpr (QS == 2) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(k), "a"(q));
  else d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k, q, d, 0, 0, 0);
}
// keeps an output block in its register file and its MFMA in its slot
template <int QS>
__device__ __forceinline__ void pin_o(f32x16_t& o) {
  if constexpr (QS == 2) asm volatile("" : "+a"(o));
  else asm volatile("" : "+v"(o));
}
// O^T += V^T . P^T (the compiler places O and tracks its hazards).
__device__ __forceinline__ void mfma_pv(f32x16_t& o, const bf16x8& v, const u32x4& p) {
  o = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v, __builtin_bit_cast(bf16x8, p), o, 0, 0, 0);
}
// The assembly score MFMAs (QS = 2) are opaque to the compiler's hazard tracking: before the
// vector ALU reads their results, wait out the pipeline (24 wait states >= what a 16-pass MFMA
// needs).
__device__ __forceinline__ void mfma_wait_scores(f32x16_t& a, f32x16_t& b) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(a), "+v"(b));
}
template <int QS>
__device__ __forceinline__ void mfma_wait_scores(f32x16_t (&s)[QS]) {
  if constexpr (QS == 2) mfma_wait_scores(s[0], s[1]);
}

// Pin a vector-ALU result to its place in the instruction stream: the empty volatile asm is
// ordered with the MFMA asm statements, so the computation cannot drift into another slot.
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }
__device__ __forceinline__ void pin(uint32_t& x) { asm volatile("" : "+v"(x)); }

template <int N>
using ic = std::integral_constant<int, N>;
// f(ic<0>{}), ..., f(ic<N-1>{}): a loop whose index is a compile-time constant in the body
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(ic<I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

template <int QS, int HPC>  // HPC: heads per CTA, run one after the other
__global__ __launch_bounds__(8 / QS * 64, 1) void mla_prefill_kernel(const PrefillParams p) {
  constexpr int kPWaves = 8 / QS;
  constexpr int kPRowsPerWave = 32 * QS;
  // the ring, then one stage-sized area that dummy DMA groups load into
  __shared__ __attribute__((aligned(1024))) char smem[kPStages * kPStageBytes + 1024];
  __shared__ __attribute__((aligned(16))) uint32_t s_src[kPMaxGroups + 1][4];  // K and V source of stage g

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int H = p.heads;

  // ---- work item: request b, query block qb, head group hg of HPC heads (groups fastest),
  // whose heads the CTA runs one after the other on the same request metadata and page-table
  // sources; the last items (the latest query blocks, which see the most keys) are dispatched first
  const int HG = (H + HPC - 1) / HPC;
  auto items_of = [&](int r) __attribute__((always_inline)) {
    return r < p.batch ? ((p.cu_seqlens_q[r + 1] - p.cu_seqlens_q[r] + kPrefillRows - 1) / kPrefillRows) * HG : 0;
  };
  int total = 0;
  for (int c0 = 0; c0 < p.batch; c0 += 64) total += wave_sum(items_of(c0 + lane));
  total = __builtin_amdgcn_readfirstlane(total);
  const int item = total - 1 - (int)blockIdx.x;
  int b = -1, local = 0, q0 = 0, E = 0, L = 0;
  if (item >= 0) {
    int acc = 0;
    for (int c0 = 0; c0 < p.batch && b < 0; c0 += 64) {
      const int r = c0 + lane;
      const bool in = r < p.batch;
      // the request's query range and key count come with the scan (no second memory round trip)
      const int lo = in ? p.cu_seqlens_q[r] : 0, hi = in ? p.cu_seqlens_q[r + 1] : 0, lk = in ? p.seq_lens_k[r] : 0;
      const int n = in ? ((hi - lo + kPrefillRows - 1) / kPrefillRows) * HG : 0;
      int incl = n;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(incl, o);
        if (lane >= o) incl += u;
      }
      const int excl = incl - n;
      const uint64_t hit = __ballot(r < p.batch && item >= acc + excl && item < acc + incl);
      if (hit != 0) {
        const int fl = __builtin_ctzll(hit);
        b = c0 + fl;
        local = item - acc - __shfl(excl, fl);
        q0 = __shfl(lo, fl);
        E = __shfl(hi, fl) - q0;
        L = __shfl(lk, fl);
      }
      acc += __shfl(incl, 63);
    }
  }
  b = __builtin_amdgcn_readfirstlane(b);
  if (b < 0) return;  // uniform: beyond the last item
  local = __builtin_amdgcn_readfirstlane(local);
  q0 = __builtin_amdgcn_readfirstlane(q0);
  E = __builtin_amdgcn_readfirstlane(E);
  L = __builtin_amdgcn_readfirstlane(L);
  const int hg = local % HG;
  const int qb = local / HG;
  const int P = L - E;  // prefix length
  const int row0 = qb * kPrefillRows + wave * kPRowsPerWave;  // this wave's first query row in the request
  const int cta_rows_end = min(E, (qb + 1) * kPrefillRows);
  const int nkeys = P + cta_rows_end;  // keys the CTA needs
  const int nst = __builtin_amdgcn_readfirstlane((nkeys + kPStage - 1) / kPStage);
  const int wave_rows = max(0, min(E - row0, kPRowsPerWave));
  const int W =  // stages this wave needs
      __builtin_amdgcn_readfirstlane(wave_rows > 0 ? (P + row0 + wave_rows + kPStage - 1) / kPStage : 0);

  const int g32 = lane >> 5;  // half of the wave
  const int c32 = lane & 31;
  const int ps_mask = (1 << p.log2_ps) - 1;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(MLA_LDS char*)smem;

  // queries of head h: qf[qs][ks] = row row0 + 32qs + c32, dims 16ks + 8g32 .. +8 (a column past the
  // extend loads the first row: finite scores in a column whose output is not written; no select,
  // so that nothing waits for these loads before the first ring loads are issued); a head's are
  // loaded before the previous head's output is written
  bf16x8 qf[QS][12];
  auto load_q = [&](int hq) __attribute__((always_inline)) {
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
      const int row = row0 + 32 * qs + c32;
      const bool ok = row < E;
      const __bf16* qrow = p.q + (int64_t)(q0 + (ok ? row : 0)) * p.q_stride_t + (int64_t)hq * p.q_stride_h + 8 * g32;
#pragma unroll
      for (int ks = 0; ks < 12; ++ks) qf[qs][ks] = *reinterpret_cast<const bf16x8*>(qrow + 16 * ks);
    }
  };

#pragma nounroll
  for (int hi = 0; hi < HPC; ++hi) {
  const int h = HPC * hg + hi;
  if (h >= H) break;  // uniform
  if (hi > 0) barrier_lds();  // every wave is done with the previous head's ring and sources
  // a K row is 128 nope dims at kbase (+ token row) and 64 rope dims rope_delta bytes after them
  // (the host checks 0 <= rope_delta < 2^31 for every head)
  const char* kbase = reinterpret_cast<const char*>(p.k) + (int64_t)h * p.k_head_stride * 2;
  const char* vbase = reinterpret_cast<const char*>(p.v) + (int64_t)h * p.v_head_stride * 2;
  const uint32_t rope_delta = (uint32_t)(p.k_rope_delta0 + (int64_t)h * p.k_rope_delta_h);
  const int krow_bytes = (int)(p.k_row_stride * 2), vrow_bytes = (int)(p.v_row_stride * 2);
  // source byte offset of logical K chunk c (16 bytes; 0..15 nope, 16..23 rope) of a row
  auto kchunk_src = [&](int c) __attribute__((always_inline)) {
    return c < 16 ? (uint32_t)(c * 16) : rope_delta + (uint32_t)((c - 16) * 16);
  };
  // bytes of one page of K / V rows (< 4 GiB, checked by the host)
  const uint32_t kpage_bytes = (uint32_t)krow_bytes << p.log2_ps, vpage_bytes = (uint32_t)vrow_bytes << p.log2_ps;
  // first source row of the stage that starts at token t0, on page pid
  auto stage_src = [&](const char* base, uint32_t pid, int t0, uint32_t page_bytes, int row_bytes)
                       __attribute__((always_inline)) {
    return base + ((uint64_t)pid * page_bytes + (uint32_t)((t0 & ps_mask) * row_bytes));
  };

  // ---- source addresses of the CTA's full stages (s_src[n_defer]: the first stage's, the source
  // of dummy groups); a CTA with more stages than that computes each stage's source when it loads it
  const bool staged = nst <= kPMaxGroups;
  const int n_defer = staged ? min(nst, L >> 5) : 0;  // stages the pipelined step may load itself
  if (hi == 0) {
    // the page-table reads, then the first head's queries, then the table writes: the writes wait
    // for the page-table reads alone, and the queries stay in flight behind the first ring loads
    constexpr int kPer = (kPMaxGroups + kPWaves * 64) / (kPWaves * 64);  // entries per thread
    int pid_u[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int g = threadIdx.x + kPWaves * 64 * u;
      const int t0 = g < n_defer ? g * kPStage : 0;  // (an unconditional read: the first page's entry)
      pid_u[u] = p.page_table[(int64_t)b * p.pt_stride + (t0 >> p.log2_ps)];
    }
    __builtin_amdgcn_sched_barrier(0);
    load_q(h);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int g = threadIdx.x + kPWaves * 64 * u;
      if (g > n_defer) continue;
      const int t0 = g < n_defer ? g * kPStage : 0;
      const uint32_t pid = (uint32_t)min(max(pid_u[u], 0), p.num_pages - 1);
      const uint64_t ka = (uint64_t)stage_src(kbase, pid, t0, kpage_bytes, krow_bytes);
      const uint64_t va = (uint64_t)stage_src(vbase, pid, t0, vpage_bytes, vrow_bytes);
      *reinterpret_cast<MLA_LDS u32x4*>((MLA_LDS char*)s_src + 16 * g) =
          u32x4{(uint32_t)ka, (uint32_t)(ka >> 32), (uint32_t)va, (uint32_t)(va >> 32)};
    }
  } else {
    for (int g = threadIdx.x; g <= n_defer; g += kPWaves * 64) {  // the previous head's, moved by a head
      MLA_LDS u32x4* e = reinterpret_cast<MLA_LDS u32x4*>((MLA_LDS char*)s_src + 16 * g);
      const u32x4 v = *e;
      const uint64_t ka = ((uint64_t)v[1] << 32 | v[0]) + (uint64_t)(p.k_head_stride * 2);
      const uint64_t va = ((uint64_t)v[3] << 32 | v[2]) + (uint64_t)(p.v_head_stride * 2);
      *e = u32x4{(uint32_t)ka, (uint32_t)(ka >> 32), (uint32_t)va, (uint32_t)(va >> 32)};
    }
  }
  barrier_lds();  // the source table is written (the queries may still be in flight)

  // ---- DMA of stage n (32 tokens of one page: page_size >= 64); rows past the last key load the
  // last key. LDS position s (16 bytes each) of the K tile holds token s / 24, chunk kswz(s % 24);
  // of the V tile token s / 16, chunk vswz(s % 16).
  const int wq = wave & 3;
  const bool k_wave = QS == 2 || wave < 4;  // this wave issues K loads wq + 4k
  const bool v_wave = QS == 2 || wave >= 4;  // this wave issues V loads wq + 4k
  constexpr int kPDmaMax = QS == 2 ? kPKDma + kPVDma : kPKDma;  // loads per wave, at most
  uint32_t koff[kPKDma], voff[kPVDma];
#pragma unroll
  for (int k = 0; k < kPKDma; ++k) {
    const int s = (wq + 4 * k) * 64 + lane, t = s / 24;
    koff[k] = (uint32_t)(t * krow_bytes) + kchunk_src(kswz(s - 24 * t, t));
  }
#pragma unroll
  for (int k = 0; k < kPVDma; ++k) {
    const int s = (wq + 4 * k) * 64 + lane, t = s >> 4;
    voff[k] = (uint32_t)(t * vrow_bytes + vswz(s & 15, t) * 16);
  }
  // DMA groups (a wave's loads of one stage: 5 with QS = 2; 3 or 2 with QS = 1) are issued in
  // order, real stages in stage order, stage n into ring slot n % kPStages. Every step issues
  // exactly one group, one load at a time in its slots: the next stage when it is a full one with a
  // staged source, otherwise a dummy group (the first stage again, every load of it into one 1 KB
  // area past the ring), so that the slots carry no branches; a tail stage (and every stage of a
  // CTA without staged sources) is issued at once, ahead of that dummy.
  // QS = 1: a wave's loads are all K or all V, so its slot work is one list: per-lane source
  // offsets doff, the source from entry half src_sel of the stage's s_src row, the LDS destination
  // tile_off into the stage (the V-only waves' third load is absent)
  const uint32_t tile_off = k_wave || QS == 2 ? 0u : (uint32_t)kPKBytes;
  const int src_sel = k_wave ? 0 : 8;
  uint32_t doff[kPKDma];
#pragma unroll
  for (int d = 0; d < kPKDma; ++d) doff[d] = k_wave ? koff[d] : voff[d < kPVDma ? d : kPVDma - 1];
  int n_stages = 0, n_groups = 0;
  const uint32_t lds_dummy = lds0 + kPStages * kPStageBytes;
  int dma_idx = 0;       // s_src entry of the step's group
  uint32_t dma_m0w = 0;  // its LDS destination, this wave's first 1 KB
  uint32_t dma_pst = 0;  // LDS distance of its successive loads (0 for a dummy group: every load of
                         // a dummy group lands in the same 1 KB past the ring, which nothing reads)
  auto issue_now = [&]() __attribute__((always_inline)) {  // stage n_stages < nst, all loads now
    const int t0 = n_stages * kPStage;
    const int tlim = L - 1 - t0;
    const uint32_t pid = (uint32_t)min(
        max(sload_i32(p.page_table + (int64_t)b * p.pt_stride + (t0 >> p.log2_ps)), 0), p.num_pages - 1);
    // (the sources through readfirstlane: under register pressure the compiler may keep these
    // uniform values in vector registers, which the DMA's scalar base operand cannot take)
    const uint64_t ka = (uint64_t)stage_src(kbase, pid, t0, kpage_bytes, krow_bytes);
    const uint64_t va = (uint64_t)stage_src(vbase, pid, t0, vpage_bytes, vrow_bytes);
    const char* ksrc = uniform_ptr((uint32_t)ka, (uint32_t)(ka >> 32));
    const char* vsrc = uniform_ptr((uint32_t)va, (uint32_t)(va >> 32));
    const uint32_t st = lds0 + (uint32_t)(n_stages % kPStages) * kPStageBytes;
    // rows past the last key reload the last key (the lane index from a volatile asm, so that these
    // offsets are computed here and not kept in registers across the loop)
    int ln;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(ln));
    if (k_wave) {
#pragma unroll
      for (int k = 0; k < kPKDma; ++k) {
        const int s = (wq + 4 * k) * 64 + ln, t = s / 24;
        const uint32_t o = (uint32_t)(min(t, tlim) * krow_bytes) + kchunk_src(kswz(s - 24 * t, t));
        dma16_saddr(ksrc, o, st + (wq + 4 * k) * 1024);
      }
    }
    if (v_wave) {
#pragma unroll
      for (int k = 0; k < kPVDma; ++k) {
        const int s = (wq + 4 * k) * 64 + ln, t = s >> 4;
        const uint32_t o = (uint32_t)(min(t, tlim) * vrow_bytes + vswz(s & 15, t) * 16);
        dma16_saddr(vsrc, o, st + kPKBytes + (wq + 4 * k) * 1024);
      }
    }
    ++n_stages;
    ++n_groups;
  };
  // the group of a step; slot_c: the ring slot of the group when it is a real one (step j loads
  // stage j + kPDist, the unrolled loop knows j % kPStages), or -1 to compute it
  auto group_setup = [&](auto slot_c) __attribute__((always_inline)) {
    constexpr int SL = decltype(slot_c)::value;
    const bool real = n_groups < n_defer;
    dma_idx = real ? n_groups : n_defer;
    const uint32_t slot = SL >= 0 ? (uint32_t)SL * kPStageBytes : (uint32_t)(n_groups % kPStages) * kPStageBytes;
    dma_m0w = real ? lds0 + slot + wq * 1024 + tile_off : lds_dummy;
    dma_pst = real ? 4 * 1024 : 0;
    if (real) ++n_stages;
    else if (__builtin_expect(n_stages < nst, 0)) issue_now();
    ++n_groups;
  };
  // slot work of the step's group: part 0 reads its sources (in the step, so the compiler waits
  // for that LDS read alone), parts 1..kPDmaMax issue the loads (a V-only wave has no part 3)
  u32x4 dma_e;
  u32x2 dma_e1;
  const char* dma_k = kbase;
  const char* dma_v = vbase;
  auto dma_part = [&](int k) __attribute__((always_inline)) {
    if constexpr (QS == 2) {
      if (k == 0) {
        dma_e = *reinterpret_cast<const MLA_LDS u32x4*>((const MLA_LDS char*)s_src + 16 * dma_idx);
        return;
      }
      if (k == 1) {
        dma_k = uniform_ptr(dma_e[0], dma_e[1]);
        dma_v = uniform_ptr(dma_e[2], dma_e[3]);
      }
      const int d = k - 1;
      if (d < kPKDma) dma16_saddr(dma_k, koff[d], dma_m0w + d * dma_pst);
      else dma16_saddr(dma_v, voff[d - kPKDma], dma_m0w + (dma_pst != 0 ? kPKBytes : 0) + (d - kPKDma) * dma_pst);
    } else {
      if (k == 0) {
        dma_e1 = *reinterpret_cast<const MLA_LDS u32x2*>((const MLA_LDS char*)s_src + 16 * dma_idx + src_sel);
        return;
      }
      if (k == 1) dma_k = uniform_ptr(dma_e1[0], dma_e1[1]);
      const int d = k - 1;
      if (d < kPVDma || k_wave) dma16_saddr(dma_k, doff[d], dma_m0w + d * dma_pst);
    }
  };
  // all loads of the step's group at once (a wave without work in the step, and the groups before
  // the first step)
  auto group_now = [&](auto slot_c) __attribute__((always_inline)) {
    group_setup(slot_c);
#pragma unroll
    for (int k = 0; k <= kPDmaMax; ++k) dma_part(k);
  };
  // the stages before the last NG groups a wave issued have landed for every wave, and every wave
  // is done with the steps before (so the stages they finished with may be refilled). Every step
  // issues exactly one group (a step that loads a tail stage at once issues one more, which only
  // makes the wait stricter), so at most (loads per group) NG loads may still be in flight.
  auto sync_groups = [&](auto ng_c) __attribute__((always_inline)) {
    constexpr int NG = decltype(ng_c)::value;
    if (QS == 2) wait_vmcnt<(kPKDma + kPVDma) * NG>();
    else if (k_wave) wait_vmcnt<kPKDma * NG>();
    else wait_vmcnt<kPVDma * NG>();
    __builtin_amdgcn_s_barrier();
  };
  // a barrier step n: stages n + 1 .. n + kPSync landed (kPDist - 1 - kPSync groups follow them)
  auto step_sync = [&]() __attribute__((always_inline)) { sync_groups(ic<kPDist - 1 - kPSync>{}); };

  for (int g = 0; g < kPDist - 1; ++g) group_now(ic<-1>{});
  // the queries stay in registers for the whole head (with QS = 2 in the accumulation registers,
  // which the score MFMAs read) and have landed here, with the first loads of the ring issued
  // behind them. The wait is explicit and full: the compiler counts neither the DMA loads (inline
  // assembly) nor their place behind the previous head's output stores, which were issued after
  // this head's queries, so a count of its own could let a query load still be in flight.
  wait_vmcnt<0>();
#pragma unroll
  for (int qs = 0; qs < QS; ++qs)
#pragma unroll
    for (int ks = 0; ks < 12; ++ks) {
      if constexpr (QS == 2) asm volatile("" : "=a"(qf[qs][ks]) : "0"(qf[qs][ks]));
      else asm volatile("" : "+v"(qf[qs][ks]));
    }

  // ---- per-lane LDS read offsets
  // K operand of k-step ks = 4m + r: chunk 8m + 2r + g32 of key c32 at k_off[r] + 128m
  int k_off[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) k_off[r] = c32 * kPKRowBytes + kswz(2 * r + g32, c32) * 16;
  // V^T operand: 16-lane group gq = lane / 16 covers dims 16(gq & 1) .. +16 of a 32-dim block and
  // the key quarter vh = gq >> 1; lane a16 reads token 4vh + (a16 >> 2) (+ 16 ksp + 8 second), dims
  // 4(a16 & 3) .. +4; chunk 4db + y (y < 4) of token t is stored at 4(db ^ (t & 3)) + y
  const int gq = lane >> 4, a16 = lane & 15, vh = gq >> 1, vt = a16 >> 2;
  int v_off[4];
  {
    const int y = 2 * (gq & 1) + ((a16 & 3) >> 1);
#pragma unroll
    for (int db = 0; db < 4; ++db) v_off[db] = (4 * vh + vt) * kPVRowBytes + (4 * (db ^ vt) + y) * 16 + (a16 & 1) * 8;
  }
  // K operand ks of the stage at LDS byte offset `kt`
  auto kread = [&](int kt, int ks) __attribute__((always_inline)) {
    return *reinterpret_cast<const MLA_LDS bf16x8*>((const MLA_LDS char*)smem + kt + k_off[ks & 3] +
                                                   128 * (ks >> 2));
  };
  // V^T operand st = (32-dim block db = st / 2, 16-key step ksp = st % 2) of the stage at `kt`; its
  // k order (keys 16ksp + 8e + 4g32 + (0..3), e = 0, 1) matches the lanes' P^T values
  auto vop = [&](int kt, int st) __attribute__((always_inline)) {
    const int db = st >> 1, ksp = st & 1;
    const MLA_LDS char* base = (const MLA_LDS char*)smem + kt + kPKBytes + v_off[db] + 16 * ksp * kPVRowBytes;
    const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((MLA_LDS bf16x4*)base);
    const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((MLA_LDS bf16x4*)(base + 8 * kPVRowBytes));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  };

  f32x16_t O[4][QS];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) O[db][qs] = f32x16_t{};
  float m_ref[QS], l_run[QS];
#pragma unroll
  for (int qs = 0; qs < QS; ++qs) m_ref[qs] = -INFINITY, l_run[qs] = 0.f;
  f32x16_t sc[2][QS];  // [parity][qs]: scores of the stage being softmaxed / being computed
  u32x4 pb[2][QS][2];  // [parity][qs][ksp]: bf16 numerators P^T
  bf16x8 vb[kAV + 1];  // V^T operands in flight (the first kAV of a step are read by the step before)
  bf16x8 kb[kAK + 1];  // K operands in flight

  // ---- scores of stage 0 (before the first pipelined step)
  auto qk_plain = [&](f32x16_t (&dst)[QS], int kt) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 4; ++r) kb[r] = kread(kt, r);
#pragma unroll
    for (int ks = 0; ks < 12; ++ks) {
      const bf16x8 a = kb[ks & 3];
      if (ks + 4 < 12) kb[ks & 3] = kread(kt, ks + 4);
#pragma unroll
      for (int qs = 0; qs < QS; ++qs) {
        if (ks == 0) mfma_qk_first<QS>(dst[qs], a, qf[qs][0]);
        else mfma_qk<QS>(dst[qs], a, qf[qs][ks]);
      }
    }
  };
  // causal mask of stage j's scores (stages that reach past the wave's first query); all == true
  // masks every score
  auto mask_scores = [&](f32x16_t (&sv)[QS], int j, bool all) __attribute__((always_inline)) {
    mfma_wait_scores<QS>(sv);
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
      // key kfirst + 8(i/4) + 4 g32 + i%4 follows query P + row0 + 32qs + c32 when
      // 8(i/4) + i%4 > lim, lim = P + row0 + 32qs + c32 - kfirst - 4 g32
      const int lim = all ? -1 : P + row0 + 32 * qs + c32 - j * kPStage - 4 * g32;
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (8 * (i >> 2) + (i & 3) > lim) sv[qs][i] = -INFINITY;
    }
  };
  float negm[QS];  // -reference per sub-block (log2 domain)
#pragma unroll
  for (int qs = 0; qs < QS; ++qs) negm[qs] = 0.f;
  // reference of the wave's first stage: its exact row max
  auto init_ref = [&](f32x16_t (&sv)[QS]) __attribute__((always_inline)) {
    mfma_wait_scores<QS>(sv);
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
      float m = sv[qs][0];
#pragma unroll
      for (int i = 1; i < 16; ++i) m = fmaxf(m, sv[qs][i]);
      m_ref[qs] = max_halves(m) * p.scale_log2;
      negm[qs] = -m_ref[qs];
    }
  };
  // stage j again, its reference raised to its exact max (rare): from its raw (masked) scores,
  // which the pipelined step keeps; O and l (which hold the stages before it) rescaled; numerators
  // and their sum redone
  auto redo_stage = [&](f32x16_t (&sv)[QS], u32x4 (&dst)[QS][2], float (&l_step)[QS]) __attribute__((always_inline)) {
    float fr[QS];
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) {
      float m = sv[qs][0];
#pragma unroll
      for (int i = 1; i < 16; ++i) m = fmaxf(m, sv[qs][i]);
      const float m_new = fmaxf(max_halves(m) * p.scale_log2, m_ref[qs]);
      fr[qs] = __builtin_amdgcn_exp2f(m_ref[qs] - m_new);
      m_ref[qs] = m_new;
      negm[qs] = -m_new;
      l_run[qs] *= fr[qs];
      float l = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float e0 = __builtin_amdgcn_exp2f(fmaf(sv[qs][2 * k], p.scale_log2, negm[qs]));
        const float e1 = __builtin_amdgcn_exp2f(fmaf(sv[qs][2 * k + 1], p.scale_log2, negm[qs]));
        l += e0 + e1;
        dst[qs][k >> 2][k & 3] = pack_bf16x2(e0, e1);
      }
      l_step[qs] = l;
    }
    // one 16-value block at a time, so that the copies out of the accumulation registers stay few
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int qs = 0; qs < QS; ++qs) {
        O[db][qs] *= fr[qs];
        pin_o<QS>(O[db][qs]);
        __builtin_amdgcn_sched_barrier(0);
      }
  };

  // ---- pipelined step j: value MFMAs of stage j - 1 (slots 0 .. 8 QS - 1), score MFMAs of stage
  // j + 1 (the next 12 QS slots), softmax of stage j spread over all slots; one MFMA per slot, the
  // order pinned by scheduling barriers; LDS operand reads kAK / kAV operands ahead.
  // step j = j0 + U with j0 a multiple of kPStages: ring slots (U - 1, U, U + 1) % kPStages hold
  // stages j - 1, j and j + 1, and the step loads stage j + kPDist into slot (U + kPDist) % kPStages
  auto step_fast = [&](auto par_c, auto u_c) __attribute__((always_inline)) {
    constexpr int U = decltype(u_c)::value;
    constexpr int slot_prev = (U + kPStages - 1) % kPStages * kPStageBytes;
    constexpr int slot_cur = U % kPStages * kPStageBytes;
    constexpr int slot_next = (U + 1) % kPStages * kPStageBytes;
    constexpr int par = decltype(par_c)::value;
    constexpr int NS = kSlots<QS>;
    constexpr int kDmaPeriod = NS / kPDmaMax;  // DMA part p (1..) goes to slot kDmaPeriod (p - 1) + 3
    f32x16_t(&scs)[QS] = sc[par];
    f32x16_t(&scn)[QS] = sc[par ^ 1];
    u32x4(&pbw)[QS][2] = pb[par];
    const u32x4(&pbr)[QS][2] = pb[par ^ 1];
    const int kt = slot_next, vtile = slot_prev;
    float l_step[QS], ev[QS][2];  // ev: the numerators of the pair being packed (raw scores stay)
    float l_step_max;
    auto uop = [&](auto u_c) __attribute__((always_inline)) {
      constexpr int u = decltype(u_c)::value;
      constexpr int k = u / (3 * QS), r = u % (3 * QS);
      if constexpr (r < 2 * QS) {
        constexpr int qs = r >> 1, e = r & 1;
        ev[qs][e] = __builtin_amdgcn_exp2f(fmaf(scs[qs][2 * k + e], p.scale_log2, negm[qs]));
        pin(ev[qs][e]);
      } else {
        constexpr int qs = r - 2 * QS;
        l_step[qs] = k == 0 ? ev[qs][0] + ev[qs][1] : l_step[qs] + ev[qs][0] + ev[qs][1];
        uint32_t w = pack_bf16x2(ev[qs][0], ev[qs][1]);
        pin(l_step[qs]);
        pin(w);
        pbw[qs][k >> 2][k & 3] = w;
      }
    };
    static_for<NS>([&](auto s_c) __attribute__((always_inline)) {
      constexpr int s = decltype(s_c)::value;
      if constexpr (s == 0) mfma_wait_scores<QS>(scs);
      if constexpr (s < 8 * QS) {
        constexpr int st = s / QS, qs = s % QS;
        mfma_pv(O[st >> 1][qs], vb[st % (kAV + 1)], pbr[qs][st & 1]);
        pin_o<QS>(O[st >> 1][qs]);
      } else {
        constexpr int ks = (s - 8 * QS) / QS, qs = s % QS;
        if constexpr (ks == 0) mfma_qk_first<QS>(scn[qs], kb[0], qf[qs][0]);
        else mfma_qk<QS>(scn[qs], kb[ks % (kAK + 1)], qf[qs][ks]);
      }
      if constexpr (s == 0) dma_part(0);  // the stage refill, spread over the step
      if constexpr (s % kDmaPeriod == 3 && s / kDmaPeriod < kPDmaMax) dma_part(s / kDmaPeriod + 1);
      if constexpr (s % QS == 0) {  // operand reads, in units of one MFMA per sub-block
        constexpr int a = s / QS;
        constexpr int st = a + kAV, stn = a + kAV - 20, ks = a - 8 + kAK;
        if constexpr (st < 8) vb[st % (kAV + 1)] = vop(vtile, st);
        if constexpr (stn >= 0 && stn < kAV) vb[stn % (kAV + 1)] = vop(slot_cur, stn);  // the next step's
        if constexpr (ks >= 0 && ks < 12) kb[ks % (kAK + 1)] = kread(kt, ks);
      }
      static_for<kUops<QS>>([&](auto u_c) __attribute__((always_inline)) {
        if constexpr (uop_slot<QS>(decltype(u_c)::value) == s) uop(u_c);
      });
      __builtin_amdgcn_sched_barrier(0);
    });
    // any lane's sum at 2^32 or more, or infinite: one compare into a lane mask, no reduction
    uint64_t big;
    asm volatile("v_max_f32 %1, %2, %3\n\tv_cmp_le_f32_e64 %0, %4, %1"
                 : "=s"(big), "=&v"(l_step_max) : "v"(l_step[0]), "v"(l_step[QS - 1]), "v"(kPLazyMax));
    if (big != 0) redo_stage(scs, pbw, l_step);
#pragma unroll
    for (int qs = 0; qs < QS; ++qs) l_run[qs] += l_step[qs];
  };

  // step j <= W of a wave: the pipelined step. At j = 0 the value pass adds zero numerators (V of
  // stage 0, which holds finite data); at j = W - 1 the scores of stage W are computed, and at
  // j = W fully masked, so that step W only adds the values of stage W - 1.
  const int j_diag = (P + row0 + 1) >> 5;  // first stage that reaches past the wave's first query
  auto step = [&](auto u_c, int j) __attribute__((always_inline)) {
    constexpr int U = decltype(u_c)::value;
    constexpr int par = U & 1;
    using slot_c = ic<(U + kPDist) % kPStages>;
    if (j > nst) return;  // uniform over the CTA: past the last stage
    if constexpr (U % kPSync == 0) step_sync();
    if (__builtin_expect(j <= W && W > 0, 1)) {
      group_setup(slot_c{});
      if (__builtin_expect(j >= j_diag, 0)) mask_scores(sc[par], j, j == W);
      if (__builtin_expect(j == 0, 0)) init_ref(sc[par]);
      step_fast(ic<par>{}, u_c);
    } else {
      group_now(slot_c{});
    }
  };

  // step -1: scores of stage 0; then steps 0..nst (every wave takes every barrier; the unrolled
  // steps past nst are skipped). A wave without rows has W = 0 and only takes the barriers and
  // loads its groups.
#pragma unroll
  for (int qs = 0; qs < QS; ++qs) pb[1][qs][0] = pb[1][qs][1] = u32x4{};
  sync_groups(ic<kPDist - 2>{});  // stage 0 landed
  group_now(ic<-1>{});
  if (W > 0) {
    qk_plain(sc[0], 0);
#pragma unroll
    for (int st = 0; st < kAV; ++st) vb[st] = vop(0, st);
  }
  for (int j0 = 0; j0 <= nst; j0 += kPUnroll)
    static_for<kPUnroll>([&](auto u_c) __attribute__((always_inline)) { step(u_c, j0 + decltype(u_c)::value); });
  wait_vmcnt<0>();  // the last groups' loads into LDS have landed before the CTA ends
  if (hi + 1 < HPC && h + 1 < H) load_q(h + 1);  // the registers are free: the steps are done

  // ---- finalise: lane holds query column c32 and dims 32db + 8(i/4) + 4*g32 + i%4
#pragma unroll
  for (int qs = 0; qs < QS; ++qs) {
    const int row = row0 + 32 * qs + c32;
    const float l_tot = sum_halves(l_run[qs]);
    if (row >= E || wave_rows == 0) continue;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    __bf16* orow = p.out + (int64_t)(q0 + row) * p.out_stride_t + (int64_t)h * p.out_stride_h;
    auto packed = [&](int db, int i4) {  // dims 32db + 8i4 + 4g32 .. +4 of this lane's row
      u32x2 v;
      v[0] = pack_bf16x2(O[db][qs][4 * i4 + 0] * inv, O[db][qs][4 * i4 + 1] * inv);
      v[1] = pack_bf16x2(O[db][qs][4 * i4 + 2] * inv, O[db][qs][4 * i4 + 3] * inv);
      return v;
    };
    if (p.out_16b) {
      // 16-byte stores (half the store instructions): the lanes of a row (c32, g32 = 0, 1) swap
      // one 8-byte part of each 16 dims, so that lane g32 holds dims 32db + 16m + 8g32 .. +8
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const u32x2 va = packed(db, 2 * m), vb = packed(db, 2 * m + 1);
          const u32x2 x = g32 == 0 ? vb : va;
          const uint32_t y0 = (uint32_t)__shfl_xor((int)x[0], 32), y1 = (uint32_t)__shfl_xor((int)x[1], 32);
          const u32x4 v = g32 == 0 ? u32x4{va[0], va[1], y0, y1} : u32x4{y0, y1, vb[0], vb[1]};
          *reinterpret_cast<u32x4*>(orow + 32 * db + 16 * m + 8 * g32) = v;
        }
    } else {
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) *reinterpret_cast<u32x2*>(orow + 32 * db + 8 * i4 + 4 * g32) = packed(db, i4);
    }
    if (p.lse != nullptr && g32 == 0)
      p.lse[(int64_t)(q0 + row) * p.lse_stride_t + h] =
          l_tot > 0.f ? (m_ref[qs] + log2f(l_tot)) * 0.69314718055994531f : -INFINITY;
  }
  }  // heads of the group
}

}  // namespace

// query sub-blocks of 32 rows per wave: 1 (8 waves, two per SIMD) or 2 (4 waves, one per SIMD)
constexpr int kPrefillQS = 1;

hipError_t launch_prefill(const PrefillParams& p0, int32_t total_q, hipStream_t stream) {
  // upper bound on sum_b ceil(E_b / 256) over the batch
  const int64_t blocks = (int64_t)(total_q + kPrefillRows - 1) / kPrefillRows + p0.batch;
  if (blocks <= 0 || p0.heads <= 0) return hipSuccess;
  // Two heads per CTA (the second head's request metadata and page-table sources come for free,
  // its queries are loaded during the first head's output) when the one-head CTAs would fill the
  // compute units at least eight times over; a smaller batch keeps one head per CTA, whose finer
  // grain the hardware's CTA scheduling balances better (a 64-head prefill of one 256-row block
  // takes twice as long with two heads per CTA).
  if (blocks * p0.heads >= 8LL * current_device_cus())
    hipLaunchKernelGGL((mla_prefill_kernel<kPrefillQS, 2>), dim3((unsigned)(blocks * ((p0.heads + 1) / 2))),
                       dim3(8 / kPrefillQS * 64), 0, stream, p0);
  else
    hipLaunchKernelGGL((mla_prefill_kernel<kPrefillQS, 1>), dim3((unsigned)(blocks * p0.heads)),
                       dim3(8 / kPrefillQS * 64), 0, stream, p0);
  return hipGetLastError();
}

}  // namespace mla
