// Absorbed-MLA paged decode for gfx950 (MI355X), split-KV, plus the fp32
// log-sum-exp merge of the split partials (bf16 partial outputs, fp32 LSEs).
//
// Work decomposition: a CTA (one wave per 16 query heads) owns one contiguous
// range of (request, 64-token block) space from the host plan. For each piece
// of a request in its range it streams the piece's latent KV rows through a
// 4-stage LDS ring (wave-wide 16-byte global->LDS DMA loads, no register
// staging) and every wave reuses each staged row for its 16 heads:
//   S^T[32 tok x 16 heads] = K[32 x 576] . Q^T    (bf16 MFMA 16x16x32, K from LDS, Q in VGPRs)
//   O^T[512 x 16 heads]   += V^T[512 x 32] . P^T   (V^T read with ds_read_b64_tr_b16)
// with an online softmax in the log2 domain between them. A piece that covers
// its whole request writes bf16 output directly; a partial piece writes its
// normalised output (bf16, in the chunk order of mla_amd.h) and its fp32
// natural-log LSE to a workspace slot that the merge kernel folds together.
//
// LDS row layout: token t's 72 16-byte chunks are stored XOR-swizzled,
// chunk c at position c ^ swz(t & 7), so both the 16-byte K reads (8
// consecutive tokens, same chunk) and the transposing V reads (4 consecutive
// tokens, two adjacent chunks) hit 32 distinct banks.
//
// MFMA 16x16x32 bf16 lane layout (wave64, lane l, g = l/16, c = l%16):
//   A[m][k]: m = c, k = 8g + j (j = 0..7);  B[k][n]: n = c, k = 8g + j
//   D[m][n]: n = c, m = 4g + i (i = 0..3)
// ds_read_b64_tr_b16: within each 16-lane group, lane j receives element j%4
// of the 8-byte words addressed by lanes j/4 + 4k, k = 0..3.
#include "mla_common.h"
#include "mla_device.h"

namespace mla {
namespace {

// Online softmax without rescaling the output accumulators: scores are
// exponentiated against a fixed per-head reference (the piece's first-tile
// max), so exp2(x - m_ref) can exceed 1. If any score of a piece exceeds its
// reference by more than kOverflowLog2 (exp2 would approach the bf16/fp32
// range), the whole CTA re-runs the piece with the reference set to the
// piece's exact max, where every exp2 is <= 1. Both runs compute the same
// normalised result; the second one only happens for extreme logits.
constexpr float kOverflowLog2 = 64.0f;
constexpr int kKPrefetch = 8;  // K operands (16-byte LDS reads) in flight
constexpr int kVPrefetch = 4;  // V operand pairs (transposing LDS reads) in flight
constexpr int kQkChains = 3;   // independent QK accumulators per 16-token block

template <int NW, bool kPageCoversTile>
__global__ __launch_bounds__(NW * 64, 1) void mla_decode_kernel(const DecodeParams p) {
  constexpr int kDmaPerWave = kTileDma / NW;
  static_assert(kTileDma % NW == 0, "tile DMA split");
  __shared__ __attribute__((aligned(1024))) char smem[kStages * kTileBytes];
  __shared__ int s_ids[kMaxPieceIds];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4;
  const int c = lane & 15;

  // The plan's ranges w, w + gridDim.x, ... of this CTA, one after another (a launch has at most one CTA
  // per compute unit; a plan of more ranges runs as a loop). Each piece starts with a CTA barrier
  // (stage_ids) and ends with its tiles consumed, so consecutive ranges need nothing more.
  for (int w = blockIdx.x; w < p.num_ctas; w += gridDim.x) {
    const int32_t* cta = p.plan + 4 * w;
    const int rb = cta[0], kb = cta[1], re = cta[2], ke = cta[3];
    if (rb >= p.batch) break;  // the padding ranges of a plan laid out for a larger grid: all later ones too
    const int32_t* req_info = p.plan + 4 * p.num_ctas;
    const int ps_mask = (1 << p.log2_ps) - 1;
    const int row_bytes = (int)(p.kv_row_stride * 2);
    const char* kv = reinterpret_cast<const char*>(p.kv);
    const uint32_t lds_ring = (uint32_t)(uintptr_t)(MLA_LDS char*)smem;

    // per-lane LDS read offsets (bytes within a tile)
    const int xk = swz(c & 7);
    const int k_off_even = c * kRowBytes + ((g ^ xk) << 4);
    const int k_off_odd = c * kRowBytes + (((4 + g) ^ xk) << 4);
    const int v_row = (4 * g + (c >> 2)) * kRowBytes;
    int v_off[4];
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4)
      v_off[q4] = v_row + ((2 * (q4 ^ (c >> 2)) + (((c & 3) >> 1) ^ (g & 1))) << 4) + ((c & 1) << 3);

    // DMA slot s = 64 * load + lane of a tile holds token s / 72, chunk (s % 72) ^ swz(token & 7)
    auto slot_token = [&](int k) { return (((wave + k * NW) * 64 + lane) * 7282) >> 19; };  // s / 72, s < 2304
    auto slot_chunk16 = [&](int k, int t) {
      return (((wave + k * NW) * 64 + lane - t * kRowChunks) ^ swz(t & 7)) << 4;
    };
    uint32_t dma_voff[kDmaPerWave];  // byte offset of this lane's chunk from the tile's first row
#pragma unroll
    for (int k = 0; k < kDmaPerWave; ++k) {
      const int t = slot_token(k);
      dma_voff[k] = t * row_bytes + slot_chunk16(k, t);
    }

    for (int b = rb; b <= re && b < p.batch; ++b) {
      const int L = p.seq_lens[b];
      const int t0 = (b == rb) ? kb * kPlanBlock : 0;
      const int t1 = (b == re) ? min(ke * kPlanBlock, L) : L;
      if (t1 <= t0) continue;
      const int first_cta = req_info[3 * b];
      const int npieces = req_info[3 * b + 1];
      const int slot_base = req_info[3 * b + 2];

      // ---- Q^T operand (B of the QK MFMA): head c of this wave, dims ks*32 + 8g .. +8
      // A head count that is not a multiple of 16 leaves lanes of the last wave without a head:
      // they compute with a zero query (read from head 0's row, always in bounds) and store nothing.
      const int h = wave * 16 + c;
      const bool h_ok = h < p.heads;
      const __bf16* qrow = p.q + (int64_t)b * p.q_stride_b + (int64_t)(h_ok ? h : 0) * p.q_stride_h + g * 8;
      bf16x8 qf[18];
#pragma unroll
      for (int ks = 0; ks < 18; ++ks) {
        qf[ks] = *reinterpret_cast<const bf16x8*>(qrow + ks * 32);
        if (!h_ok) qf[ks] = bf16x8{};
      }
      // Consume Q here so the compiler's vmcnt wait for these loads lands before
      // the tile loop; at their first use inside the loop it would also wait for
      // every DMA load in flight (the counter is in order) on every tile.
#pragma unroll
      for (int ks = 0; ks < 18; ++ks) asm volatile("" ::"v"(qf[ks]));

      // ---- page ids of the piece -> LDS, one window of kMaxPieceIds pages at a time. t0 is a
      // multiple of the 64-token plan block, so with pages under 32 tokens it is page aligned and
      // a 32-token tile never straddles two windows (a window is a whole number of tiles); with
      // larger pages a tile lies inside one page.
      const int pg0 = t0 >> p.log2_ps;
      const int npg = ((t1 - 1) >> p.log2_ps) - pg0 + 1;
      const int32_t* pt_row = p.page_table + (int64_t)b * p.pt_stride + pg0;
      int win = -1;  // window held by s_ids
      auto tile_win = [&](int tile) { return (((t0 + tile * kTile) >> p.log2_ps) - pg0) / kMaxPieceIds; };
      // Every wave calls this at the same point. The first barrier orders it after every read of the
      // previous window (ids are read into registers when a tile is issued; DMAs already in flight do
      // not read s_ids). Loading the ids waits for this wave's DMAs in flight (the vector-memory
      // counter is in order): one drain of the ring per window.
      auto stage_ids = [&](int wdx) {
        __syncthreads();
        const int base = wdx * kMaxPieceIds;
        const int n = min(npg - base, kMaxPieceIds);
        for (int i = threadIdx.x; i < n; i += NW * 64) s_ids[i] = min(max(pt_row[base + i], 0), p.num_pages - 1);
        __syncthreads();
        win = wdx;
      };
      stage_ids(0);  // also: the previous piece is done with s_ids and the ring

      const int ntiles = (t1 - t0 + kTile - 1) / kTile;

      auto issue = [&](int tile, int stage) {
        const int tstart = t0 + tile * kTile;
        const int tlim = t1 - 1 - tstart;  // last valid token of the tile (loads clamp to it)
        const uint32_t lds_stage = lds_ring + stage * kTileBytes;
        const int id0 = pg0 + win * kMaxPieceIds;  // page of s_ids[0]
        if constexpr (kPageCoversTile) {
          const int pid = __builtin_amdgcn_readfirstlane(s_ids[(tstart >> p.log2_ps) - id0]);
          const char* tsrc = kv + ((int64_t)pid * (ps_mask + 1) + (tstart & ps_mask)) * row_bytes;
          if (tlim >= kTile - 1) {
#pragma unroll
            for (int k = 0; k < kDmaPerWave; ++k) dma16_saddr(tsrc, dma_voff[k], lds_stage + (wave + k * NW) * 1024);
          } else {
#pragma unroll
            for (int k = 0; k < kDmaPerWave; ++k) {
              const int t = slot_token(k);
              dma16_saddr(tsrc, min(t, tlim) * row_bytes + slot_chunk16(k, t), lds_stage + (wave + k * NW) * 1024);
            }
          }
        } else {
#pragma unroll
          for (int k = 0; k < kDmaPerWave; ++k) {
            const int t = slot_token(k);
            const int tok = tstart + min(t, tlim);
            const int pid = s_ids[(tok >> p.log2_ps) - id0];
            const char* src = kv + ((int64_t)pid * (ps_mask + 1) + (tok & ps_mask)) * row_bytes + slot_chunk16(k, t);
            dma16_vaddr(src, lds_stage + (wave + k * NW) * 1024);
          }
        }
      };

      float m_ref = 0.f;     // per-head exponent reference (log2 units)
      float m_max = -INFINITY;  // per-head max score of the piece
      float l_run = 0.f;
      f32x4 O[32];
      for (int attempt = 0; attempt < 2; ++attempt) {
        if (win != 0) stage_ids(0);  // a rerun restarts at the piece's first window
#pragma unroll
        for (int s = 0; s < kStages - 1; ++s)
          if (s < ntiles) issue(s, s);  // the first kStages - 1 tiles lie in window 0
#pragma unroll
        for (int i = 0; i < 32; ++i) O[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        l_run = 0.f;
        bool overflow = false;

        for (int it = 0; it < ntiles; ++it) {
          const int ahead = ntiles - 1 - it;  // tiles issued after this one (capped below)
          if (ahead >= kStages - 2) wait_vmcnt<kDmaPerWave * (kStages - 2)>();
          else if (ahead == 1) wait_vmcnt<kDmaPerWave>();
          else wait_vmcnt<0>();
          __syncthreads();
          if (it + kStages - 1 < ntiles) {
            const int nt = it + kStages - 1;
            if (tile_win(nt) != win) stage_ids(tile_win(nt));  // uniform: same tile in every wave
            issue(nt, nt % kStages);
          }

          const MLA_LDS char* T = (const MLA_LDS char*)smem + (it % kStages) * kTileBytes;

          // ---- S^T = K . Q^T : tokens 0-15 (s0) and 16-31 (s1) of the tile.
          // Read j covers k-step j>>1 of token block j&1.
          auto kread = [&](int j) {
            const int ks = j >> 1;
            const int off = ((ks & 1) ? k_off_odd : k_off_even) + 128 * (ks >> 1) + (j & 1) * 16 * kRowBytes;
            return *reinterpret_cast<const MLA_LDS bf16x8*>(T + off);
          };
          // kQkChains independent accumulators per token block keep the dependent
          // MFMA chains short; they are summed after the last k-step.
          f32x4 sacc[2][kQkChains];
#pragma unroll
          for (int u = 0; u < kQkChains; ++u) sacc[0][u] = sacc[1][u] = f32x4{0.f, 0.f, 0.f, 0.f};
          bf16x8 kbuf[kKPrefetch];
#pragma unroll
          for (int j = 0; j < kKPrefetch; ++j) kbuf[j] = kread(j);
#pragma unroll
          for (int j = 0; j < 36; ++j) {
            const bf16x8 a = kbuf[j % kKPrefetch];
            if (j + kKPrefetch < 36) kbuf[j % kKPrefetch] = kread(j + kKPrefetch);
            f32x4& acc = sacc[j & 1][(j >> 1) % kQkChains];
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[j >> 1], acc, 0, 0, 0);
          }
          f32x4 s0 = sacc[0][0], s1 = sacc[1][0];
#pragma unroll
          for (int u = 1; u < kQkChains; ++u) {
            s0 += sacc[0][u];
            s1 += sacc[1][u];
          }

          // V^T operands do not depend on P: start reading them before the softmax.
          auto vread = [&](int db, int half) {
            const int off = v_off[db & 3] + 128 * (db >> 2) + half * 16 * kRowBytes;
            return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((MLA_LDS bf16x4*)(T + off));
          };
          bf16x4 vlo[kVPrefetch], vhi[kVPrefetch];
#pragma unroll
          for (int j = 0; j < kVPrefetch; ++j) {
            vlo[j] = vread(j, 0);
            vhi[j] = vread(j, 1);
          }

          // ---- softmax numerators (log2 domain) for head c; lane holds tokens 4g+i and 16+4g+i
          float x[8];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            x[i] = s0[i] * p.scale_log2;
            x[4 + i] = s1[i] * p.scale_log2;
          }
          const int tstart = t0 + it * kTile;
          if (tstart + kTile > t1) {
            const int valid = t1 - tstart;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              if (4 * g + i >= valid) x[i] = -INFINITY;
              if (16 + 4 * g + i >= valid) x[4 + i] = -INFINITY;
            }
          }
          float mt = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
          mt = wave_max_g(mt);
          if (attempt == 0 && it == 0) m_ref = mt;
          m_max = fmaxf(m_max, mt);
          overflow |= mt > m_ref + kOverflowLog2;
          float pr[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            pr[i] = __builtin_amdgcn_exp2f(x[i] - m_ref);
            l_run += pr[i];
          }
          u32x4 pw;
          pw[0] = pack_bf16x2(pr[0], pr[1]);
          pw[1] = pack_bf16x2(pr[2], pr[3]);
          pw[2] = pack_bf16x2(pr[4], pr[5]);
          pw[3] = pack_bf16x2(pr[6], pr[7]);
          const bf16x8 pb = __builtin_bit_cast(bf16x8, pw);

          // ---- O^T += V^T . P^T over 32 blocks of 16 dims
#pragma unroll
          for (int db = 0; db < 32; ++db) {
            const bf16x8 a =
                __builtin_shufflevector(vlo[db % kVPrefetch], vhi[db % kVPrefetch], 0, 1, 2, 3, 4, 5, 6, 7);
            if (db + kVPrefetch < 32) {
              vlo[db % kVPrefetch] = vread(db + kVPrefetch, 0);
              vhi[db % kVPrefetch] = vread(db + kVPrefetch, 1);
            }
            O[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, O[db], 0, 0, 0);
          }
        }
        // every wave has drained its loads (vmcnt(0) at the last tile); agree on a re-run
        if (attempt == 0) {
          if (!__syncthreads_or(overflow)) break;
          m_ref = m_max;  // exact max of the piece: exp2(x - m_ref) <= 1 everywhere
        }
      }

      // ---- finalise: lane holds head h, dims 16*db + 4g + (0..3)
      const float l_tot = wave_sum_g(l_run);
      const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
      const float lse_nat = l_tot > 0.f ? (m_ref + log2f(l_tot)) * 0.69314718055994531f : -INFINITY;
      if (!h_ok) {
        // no head on this lane
      } else if (npieces == 1) {
        __bf16* orow = p.out + (int64_t)b * p.out_stride_b + (int64_t)h * p.out_stride_h + 4 * g;
#pragma unroll
        for (int db = 0; db < 32; ++db) {
          u32x2 v;
          v[0] = pack_bf16x2(O[db][0] * inv, O[db][1] * inv);
          v[1] = pack_bf16x2(O[db][2] * inv, O[db][3] * inv);
          *reinterpret_cast<u32x2*>(orow + 16 * db) = v;
        }
        if (p.lse != nullptr && g == 0) p.lse[(int64_t)b * p.lse_stride_b + h] = lse_nat;
      } else {
        const int slot = slot_base + (w - first_cta);
        if (slot >= 0 && slot < p.ws_slots) {
          // dim blocks 2k, 2k + 1 of this lane go to 16-byte chunk 4k + g (the chunk order of mla_amd.h)
          __bf16* orow = p.ws_o + ((int64_t)slot * p.heads + h) * kVDim + 8 * g;
#pragma unroll
          for (int k = 0; k < 16; ++k) {
            u32x4 v;
            v[0] = pack_bf16x2(O[2 * k][0] * inv, O[2 * k][1] * inv);
            v[1] = pack_bf16x2(O[2 * k][2] * inv, O[2 * k][3] * inv);
            v[2] = pack_bf16x2(O[2 * k + 1][0] * inv, O[2 * k + 1][1] * inv);
            v[3] = pack_bf16x2(O[2 * k + 1][2] * inv, O[2 * k + 1][3] * inv);
            *reinterpret_cast<u32x4*>(orow + 32 * k) = v;
          }
          if (g == 0) p.ws_lse[(int64_t)slot * p.heads + h] = lse_nat;
        }
      }
    }
  }
}

// One wave per (request, head). Lane l reads 16-byte chunk l of every piece's bf16 partial row
// (value dims 32 (l / 4) + 4 (l % 4) + {0..3, 16..19}, the chunk order of mla_amd.h) and the LSE of
// piece l (of each group of 64 pieces). The first kMergeBatch pieces are requested together with the
// LSEs, so a request of up to 8 pieces costs one memory round trip; later pieces are read 8 at a
// time. Each piece's weight exp(lse_i - lse) is computed once, by lane i, and read by the wave
// with v_readlane. fp32 arithmetic, one rounding to bf16.
constexpr int kMergeBatch = 8;

__device__ __forceinline__ void unpack_bf16x8(const u32x4 raw, float* f) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[2 * j] = __builtin_bit_cast(float, raw[j] << 16);
    f[2 * j + 1] = __builtin_bit_cast(float, raw[j] & 0xffff0000u);
  }
}

__global__ __launch_bounds__(256) void mla_merge_kernel(const MergeParams p) {
  const int b = blockIdx.x;
  const int h = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (h >= p.heads) return;
  const int n = p.req_info[3 * b + 1];
  const int base = p.req_info[3 * b + 2];
  if (n == 1 && p.skip_single) return;
  // slots outside the workspace (a caller's plan that does not match it) give NaN, never a silent result
  const bool in_ws = n <= 0 || (base >= 0 && (int64_t)base + n <= p.ws_slots);
  const int nv = in_ws && n > 0 ? n : 0;
  const __bf16* src = p.ws_o + ((int64_t)(nv > 0 ? base : 0) * p.heads + h) * kVDim + 8 * lane;
  const int64_t pstride = (int64_t)p.heads * kVDim;
  auto piece_lse = [&](int i) { return p.ws_lse[(int64_t)(base + i) * p.heads + h]; };
  u32x4 raw[kMergeBatch];
#pragma unroll
  for (int u = 0; u < kMergeBatch; ++u)
    if (u < nv) raw[u] = *reinterpret_cast<const u32x4*>(src + u * pstride);
  const float lse0 = lane < nv ? piece_lse(lane) : -INFINITY;

  constexpr float kLog2e = 1.4426950408889634f;
  float mx = lse0;
  for (int i = lane + 64; i < nv; i += 64) mx = fmaxf(mx, piece_lse(i));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  float sum = 0.f;
  if (mx > -INFINITY) {
    sum = lse0 > -INFINITY ? __builtin_amdgcn_exp2f((lse0 - mx) * kLog2e) : 0.f;
    for (int i = lane + 64; i < nv; i += 64) sum += __builtin_amdgcn_exp2f((piece_lse(i) - mx) * kLog2e);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o);
  const bool any = mx > -INFINITY && sum > 0.f;
  const float lse = any ? mx + logf(sum) : -INFINITY;

  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (any) {
#pragma unroll 1
    for (int i0 = 0; i0 < nv; i0 += 64) {
      const float l_i = i0 == 0 ? lse0 : (i0 + lane < nv ? piece_lse(i0 + lane) : -INFINITY);
      const float w_i = l_i > -INFINITY ? __builtin_amdgcn_exp2f((l_i - lse) * kLog2e) : 0.f;  // lane u: piece i0 + u
      const int cnt = min(64, nv - i0);
#pragma unroll 1
      for (int u0 = 0; u0 < cnt; u0 += kMergeBatch) {
        if (i0 + u0 > 0) {
#pragma unroll
          for (int u = 0; u < kMergeBatch; ++u)
            if (u0 + u < cnt) raw[u] = *reinterpret_cast<const u32x4*>(src + (i0 + u0 + u) * pstride);
        }
#pragma unroll
        for (int u = 0; u < kMergeBatch; ++u) {
          if (u0 + u < cnt) {
            const float wgt = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w_i), u0 + u));
            float f[8];
            unpack_bf16x8(raw[u], f);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] = fmaf(wgt, f[j], acc[j]);
          }
        }
      }
    }
  }
  const float bad = in_ws ? 0.f : __builtin_nanf("");
  __bf16* orow = p.out + (int64_t)b * p.out_stride_b + (int64_t)h * p.out_stride_h + 32 * (lane >> 2) + 4 * (lane & 3);
  *reinterpret_cast<u32x2*>(orow) = u32x2{pack_bf16x2(acc[0] + bad, acc[1] + bad), pack_bf16x2(acc[2] + bad, acc[3] + bad)};
  *reinterpret_cast<u32x2*>(orow + 16) =
      u32x2{pack_bf16x2(acc[4] + bad, acc[5] + bad), pack_bf16x2(acc[6] + bad, acc[7] + bad)};
  if (p.lse != nullptr && lane == 0) p.lse[(int64_t)b * p.lse_stride_b + h] = lse + bad;
}

template <int NW>
hipError_t launch_decode_nw(const DecodeParams& p, hipStream_t stream) {
  const int grid = p.num_ctas < current_device_cus() ? p.num_ctas : current_device_cus();
  if (p.log2_ps >= 5)
    hipLaunchKernelGGL((mla_decode_kernel<NW, true>), dim3(grid), dim3(NW * 64), 0, stream, p);
  else
    hipLaunchKernelGGL((mla_decode_kernel<NW, false>), dim3(grid), dim3(NW * 64), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_decode(const DecodeParams& p, hipStream_t stream) {
  if (decode_ws_takes(p)) return launch_decode_ws(p, stream);
  if (p.heads < 1 || p.heads > 64) return hipErrorInvalidValue;  // the entry points split larger counts
  switch ((p.heads + 15) / 16) {
    case 1: return launch_decode_nw<1>(p, stream);
    case 2: return launch_decode_nw<2>(p, stream);
    case 3: return launch_decode_nw<3>(p, stream);
    case 4: return launch_decode_nw<4>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_merge(const MergeParams& p, hipStream_t stream) {
  dim3 grid(p.batch, (p.heads + 3) / 4);
  hipLaunchKernelGGL(mla_merge_kernel, grid, dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace mla
